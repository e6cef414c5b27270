"""CPU restatement of the reference's dequantise-then-SDPA decode path (oracle).

References: ``_cpu_dequant_slot`` F:150-195 (F = fused-quant/fused_int4.v0.1.0.py),
the in-kernel dequantisation F:765-800 / F:853-872 (INT4) and F:1397-1423
(INT8 K), the harness oracle ``pipeline_A`` in scripts/v35_h100_bench.py:376-387
and scripts/v29_flash_bench.py:86-97 (dequantise, ``repeat_interleave`` for GQA,
``scaled_dot_product_attention``), and the kernel's output rounding F:886-894
(fp32 accumulator -> fp16 -> the query's dtype).
"""
from __future__ import annotations

import numpy as np
import torch

from .quant import unpack_nibbles

F32 = np.float32


def dequant_int4(packed, scales, zeros=None, group_size=32):
    """``packed uint8[..., D/2]`` -> float32 ``[..., D]``.

    Asymmetric: ``n * scale + zero`` with n in [0, 15]; symmetric:
    ``(n - 8) * scale`` (F:168-193).  Scale and zero are the stored fp16
    values widened to fp32.
    """
    n = unpack_nibbles(packed).astype(F32)
    if zeros is None:
        n = n - F32(8.0)
    d = n.shape[-1]
    ng = d // group_size
    n = n.reshape(n.shape[:-1] + (ng, group_size))
    out = n * np.asarray(scales, np.float16).astype(F32)[..., :ng, None]
    if zeros is not None:
        out = out + np.asarray(zeros, np.float16).astype(F32)[..., :ng, None]
    return out.reshape(n.shape[:-2] + (d,)).astype(F32)


def dequant_int8(codes, scales, group_size):
    c = np.asarray(codes, np.int8).astype(F32)
    d = c.shape[-1]
    ng = d // group_size
    c = c.reshape(c.shape[:-1] + (ng, group_size))
    out = c * np.asarray(scales, np.float16).astype(F32)[..., :ng, None]
    return out.reshape(c.shape[:-2] + (d,)).astype(F32)


def dequant_plane(plane: dict) -> np.ndarray:
    """Dequantise a whole paged cache plane to float32 ``[nb, bs, Hkv, D]``.

    ``plane`` = {"format": "int4_sym"|"int4_asym"|"int8"|"fp16", "data": ...,
    "scales": ..., "zeros": ..., "group_size": G}.
    """
    fmt = plane["format"]
    if fmt == "fp16":
        return np.asarray(plane["data"], np.float16).astype(F32)
    if fmt == "int8":
        return dequant_int8(plane["data"], plane["scales"], plane["group_size"])
    zeros = plane.get("zeros") if fmt == "int4_asym" else None
    return dequant_int4(plane["data"], plane["scales"], zeros, plane["group_size"])


def gather_sequence(cache_f32: np.ndarray, block_table_row: np.ndarray,
                    seq_len: int) -> np.ndarray:
    """Token rows ``[seq_len, Hkv, D]`` of one sequence through its block table
    (F:749-754: ``phys = block_table[seq, pos // block_size]``)."""
    bs = cache_f32.shape[1]
    pos = np.arange(seq_len)
    phys = np.asarray(block_table_row, np.int64)[pos // bs]
    return cache_f32[phys, pos % bs]


def sdpa_decode_f32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    scale: float) -> torch.Tensor:
    """One decode query per head: q ``[Hq, D]``, k/v ``[T, Hkv, D]`` (fp32).

    GQA by ``repeat_interleave`` over kv heads, then torch SDPA on the CPU in
    fp32 (the reference's P1 pipeline, V35:376-387)."""
    hq = q.shape[0]
    hkv = k.shape[1]
    rep = hq // hkv
    kk = k.permute(1, 0, 2).repeat_interleave(rep, dim=0)      # [Hq, T, D]
    vv = v.permute(1, 0, 2).repeat_interleave(rep, dim=0)
    out = torch.nn.functional.scaled_dot_product_attention(
        q[:, None, :], kk, vv, scale=scale)                      # [Hq, 1, D]
    return out[:, 0, :]


def decode_reference(query, key_plane: dict, value_plane: dict, block_table,
                     seq_lens, scale=None, out_dtype=None, round_output=True) -> np.ndarray:
    """Decode attention over paged quantised caches; returns ``[S, Hq, D]``.

    ``query``: float32 ``[num_seqs, Hq, D]`` (exact upcast of fp16/bf16).
    The fp32 result is rounded to fp16 (F:891-894) and, when ``out_dtype`` is
    ``torch.bfloat16``, converted on to bf16 as the reference's store into a
    bf16 ``empty_like(query)`` does.  ``seq_len == 0`` yields NaN, as the
    reference's ``acc / l_i`` with ``l_i = 0`` does (F:886-887).
    ``round_output=False`` returns the fp32 result before output rounding.
    """
    query = torch.as_tensor(np.asarray(query, F32))
    S, hq, d = query.shape
    if scale is None:
        scale = float(np.float32(1.0 / (d ** 0.5)))              # F:924
    kf = dequant_plane(key_plane)
    vf = dequant_plane(value_plane)
    out = np.empty((S, hq, d), F32)
    for s in range(S):
        n = int(seq_lens[s])
        if n == 0:
            out[s] = np.nan
            continue
        k = torch.from_numpy(gather_sequence(kf, block_table[s], n))
        v = torch.from_numpy(gather_sequence(vf, block_table[s], n))
        out[s] = sdpa_decode_f32(query[s], k, v, scale).numpy()
    if not round_output:
        return out
    o16 = torch.from_numpy(out).to(torch.float16)
    if out_dtype is torch.bfloat16:
        return o16.to(torch.bfloat16).to(torch.float32).numpy()
    return o16.to(torch.float32).numpy()


def decode_reference_f64(query, key_plane, value_plane, block_table, seq_lens,
                         scale=None) -> np.ndarray:
    """Same as :func:`decode_reference` but in float64 with no output rounding;
    used to bound the fp32 paths' own error."""
    query = np.asarray(query, np.float64)
    S, hq, d = query.shape
    if scale is None:
        scale = float(np.float32(1.0 / (d ** 0.5)))
    kf = dequant_plane(key_plane).astype(np.float64)
    vf = dequant_plane(value_plane).astype(np.float64)
    out = np.empty((S, hq, d))
    for s in range(S):
        n = int(seq_lens[s])
        k = gather_sequence(kf, block_table[s], n)
        v = gather_sequence(vf, block_table[s], n)
        hkv = k.shape[1]
        rep = hq // hkv
        for h in range(hq):
            sc = k[:, h // rep, :] @ query[s, h] * scale
            p = np.exp(sc - sc.max())
            out[s, h] = (p @ v[:, h // rep, :]) / p.sum()
    return out
