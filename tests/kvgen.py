"""Seeded synthetic KV workloads for the parity tests (CPU generation so the
oracle and the GPU see identical bits)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import quant as Q

FMT_NAMES = {0: "int4_sym", 1: "int4_asym", 2: "int8", 3: "fp16"}


def randn(shape, seed, dtype=torch.float16, outlier_frac=0.0, outlier_scale=20.0,
          channel_axis=(-2, -1)):
    """N(0,1) values; a fraction of (head, channel) pairs scaled by outlier_scale."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if outlier_frac > 0:
        h, d = shape[-2], shape[-1]
        n = max(1, int(round(outlier_frac * h * d)))
        idx = torch.randperm(h * d, generator=g)[:n]
        mask = torch.ones(h * d)
        mask[idx] = outlier_scale
        x = x * mask.view(h, d)
    return x.to(dtype)


def paged_table(seq_lens, block_size, num_blocks, seed, max_blocks=None):
    """Block table whose rows are consecutive slices of a random permutation
    of the block pool, and the slot of every (seq, position)."""
    g = torch.Generator().manual_seed(seed)
    need = [-(-int(n) // block_size) for n in seq_lens]
    width = max_blocks or max(max(need), 1)
    assert sum(need) <= num_blocks
    perm = torch.randperm(num_blocks, generator=g).numpy()
    bt = np.zeros((len(seq_lens), width), np.int32)
    cur = 0
    for s, nb in enumerate(need):
        bt[s, :nb] = perm[cur:cur + nb]
        cur += nb
    return bt


def token_slots(bt, seq_lens, block_size):
    """slot_mapping (int64) of all tokens of all sequences, sequence-major."""
    out = []
    for s, n in enumerate(seq_lens):
        pos = np.arange(int(n))
        out.append(bt[s, pos // block_size].astype(np.int64) * block_size + pos % block_size)
    return np.concatenate(out) if out else np.zeros(0, np.int64)


def empty_plane(fmt, num_blocks, block_size, hkv, d, gs):
    """Zero-filled numpy cache plane dict in the reference layout."""
    if fmt == 3:
        return {"format": "fp16", "data": np.zeros((num_blocks, block_size, hkv, d), np.float16),
                "scales": None, "zeros": None, "group_size": d}
    ng = d // gs
    data = np.zeros((num_blocks, block_size, hkv, d if fmt == 2 else d // 2),
                    np.int8 if fmt == 2 else np.uint8)
    return {"format": FMT_NAMES[fmt], "data": data,
            "scales": np.zeros((num_blocks, block_size, hkv, ng), np.float16),
            "zeros": np.zeros((num_blocks, block_size, hkv, ng), np.float16) if fmt == 1 else None,
            "group_size": gs}


def fill_plane(plane, x_f32, slots, clip_ratio=10.0):
    """Quantise rows ``x_f32 [num_tokens, Hkv, D]`` into ``plane`` at ``slots``
    with the oracle (in place)."""
    bs = plane["data"].shape[1]
    blk, off = slots // bs, slots % bs
    fmt = plane["format"]
    if fmt == "fp16":
        plane["data"][blk, off] = x_f32.astype(np.float16)
    elif fmt == "int8":
        c, s = Q.quantize_int8_rows(x_f32, plane["group_size"])
        plane["data"][blk, off] = c
        plane["scales"][blk, off] = s
    else:
        p, s, z = Q.quantize_int4_rows(x_f32, plane["group_size"], fmt == "int4_asym", clip_ratio)
        plane["data"][blk, off] = p
        plane["scales"][blk, off] = s
        if z is not None:
            plane["zeros"][blk, off] = z


def plane_to_torch(plane, device):
    """Device tensors (data, scales, zeros) of a numpy plane."""
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device)
    return t(plane["data"]), t(plane["scales"]), t(plane["zeros"])
