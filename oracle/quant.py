"""CPU restatement of knlp's INT4 / INT8 KV quantize-on-append (test oracle).

All arithmetic is numpy float32 with IEEE semantics (correctly rounded
subtraction and division, round-to-nearest-even fp32 -> fp16), which is the
normative arithmetic for bit-exact parity.  References are into
``fused-quant/fused_int4.v0.1.0.py`` (F).
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
EPS = F32(1e-8)  # the literal 1e-8 of F:314, F:335, F:342, F:1276 as fp32


def round_half_away(t: np.ndarray) -> np.ndarray:
    """``_triton_round`` (F:198-202): ``t >= 0 ? floor(t + 0.5) : ceil(t - 0.5)``.

    The +-0.5 is added in fp32, so t = 0.49999997 rounds to 1 (the fp32 sum
    rounds up to 1.0 before the floor), unlike ``rint``/``round``.
    """
    t = np.asarray(t, dtype=F32)
    half = F32(0.5)
    return np.where(t >= 0, np.floor(t + half), np.ceil(t - half)).astype(F32)


def tree_sum(x: np.ndarray) -> np.ndarray:
    """Sum over the last axis in a fixed pairwise order (fp32 at each step).

    The reference reduces with ``tl.sum`` (F:337-339), whose order is the
    compiler's.  This build fixes it to the xor-butterfly order a 64-wide
    wavefront produces with one element per lane: at each stage element i
    adds element i + stride, stride = n/2, n/4, ..., 1.  The HIP kernel uses
    the same order, so the symmetric clip path is bit-exact between them.
    """
    v = np.asarray(x, dtype=F32).copy()
    n = v.shape[-1]
    assert n & (n - 1) == 0, "group size must be a power of two"
    while n > 1:
        n //= 2
        v = (v[..., :n] + v[..., n:2 * n]).astype(F32)
    return v[..., 0]


def quantize_int4_groups(x: np.ndarray, asymmetric: bool, clip_ratio: float = 10.0):
    """Quantise ``x[..., group]`` (fp32) to INT4 codes in [0, 15].

    Restates the per-group body of ``_reshape_and_cache_int4_kernel``:
    asymmetric F:308-327, symmetric with trimmed-mean outlier clip F:328-357.
    Returns ``(codes uint8[..., group], scale_f16[...], zero_f16[...] or None)``.
    The codes are computed with the fp32 scale; the fp16 scale is what is
    stored (F:327, F:363).
    """
    x = np.asarray(x, dtype=F32)
    if asymmetric:
        mn = x.min(axis=-1)
        mx = x.max(axis=-1)
        rng = np.maximum((mx - mn).astype(F32), EPS)
        scale = (rng / F32(15.0)).astype(F32)
        zero = mn
        t = ((x - zero[..., None]).astype(F32) / scale[..., None]).astype(F32)
        q = np.clip(round_half_away(t), F32(0.0), F32(15.0))
        codes = q.astype(np.uint8)
        return codes, scale.astype(np.float16), zero.astype(np.float16)
    ax = np.abs(x)
    amax = np.maximum(ax.max(axis=-1), EPS)
    if clip_ratio > 0.0:
        below_mask = ax < amax[..., None]
        below = np.where(below_mask, ax, F32(0.0)).astype(F32)
        cnt = np.maximum(below_mask.sum(axis=-1).astype(F32), F32(1.0))
        tmean = (tree_sum(below) / cnt).astype(F32)
        clip = (tmean * F32(clip_ratio)).astype(F32)
        amax = np.minimum(amax, np.maximum(clip, EPS))
    scale = (amax / F32(7.0)).astype(F32)
    t = (x / scale[..., None]).astype(F32)
    q = np.clip(round_half_away(t), F32(-8.0), F32(7.0))
    codes = (q + F32(8.0)).astype(np.uint8)
    return codes, scale.astype(np.float16), None


def quantize_int8_groups(x: np.ndarray):
    """Symmetric INT8 per group (F:1270-1284): ``scale = max(amax,1e-8)/127``,
    ``q = clamp(round_half_away(x/scale), -128, 127)``.
    Returns ``(codes int8[..., group], scale_f16[...])``."""
    x = np.asarray(x, dtype=F32)
    amax = np.maximum(np.abs(x).max(axis=-1), EPS)
    scale = (amax / F32(127.0)).astype(F32)
    t = (x / scale[..., None]).astype(F32)
    q = np.clip(round_half_away(t), F32(-128.0), F32(127.0))
    return q.astype(np.int8), scale.astype(np.float16)


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """Two codes per byte, low nibble = even element, high = odd (F:359)."""
    codes = np.asarray(codes, dtype=np.uint8)
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed & 0x0F
    out[..., 1::2] = packed >> 4
    return out


def quantize_int4_rows(x: np.ndarray, group_size: int, asymmetric: bool,
                       clip_ratio: float = 10.0):
    """Quantise rows ``x[..., D]`` group by group and pack.

    Returns ``(packed uint8[..., D/2], scales f16[..., D/G], zeros f16 or None)``.
    """
    x = np.asarray(x, dtype=F32)
    d = x.shape[-1]
    assert d % group_size == 0
    g = x.reshape(x.shape[:-1] + (d // group_size, group_size))
    codes, sc, zp = quantize_int4_groups(g, asymmetric, clip_ratio)
    packed = pack_nibbles(codes.reshape(x.shape))
    return packed, sc, zp


def quantize_int8_rows(x: np.ndarray, group_size: int):
    x = np.asarray(x, dtype=F32)
    d = x.shape[-1]
    assert d % group_size == 0
    g = x.reshape(x.shape[:-1] + (d // group_size, group_size))
    codes, sc = quantize_int8_groups(g)
    return codes.reshape(x.shape), sc


def _slots(slot_mapping: np.ndarray, block_size: int):
    slot_mapping = np.asarray(slot_mapping, dtype=np.int64)
    valid = np.nonzero(slot_mapping >= 0)[0]          # F:266-268: slot < 0 skipped
    s = slot_mapping[valid]
    return valid, s // block_size, s % block_size      # F:270-271


def reshape_and_cache_int4(key, value, key_cache, value_cache, k_scales, v_scales,
                           slot_mapping, k_zeros=None, v_zeros=None,
                           asymmetric=False, group_size=32, clip_ratio=10.0):
    """In-place numpy restatement of ``reshape_and_cache_int4`` (F:418-472).

    ``key``/``value``: float32 ``[num_tokens, num_heads, D]`` (exact upcasts of
    the fp16/bf16 inputs).  ``key`` may be None for the V-only variant
    (F:603-647).  Caches follow the reference layout
    ``[num_blocks, block_size, num_heads, D/2]`` (uint8) and
    ``[num_blocks, block_size, num_heads, D/G]`` (fp16).
    """
    block_size = value_cache.shape[1]
    tok, blk, off = _slots(slot_mapping, block_size)
    planes = [(value, value_cache, v_scales, v_zeros)]
    if key is not None:
        planes.insert(0, (key, key_cache, k_scales, k_zeros))
    for src, cache, sc, zp in planes:
        packed, s, z = quantize_int4_rows(np.asarray(src, F32)[tok], group_size,
                                          asymmetric, clip_ratio)
        cache[blk, off] = packed
        sc[blk, off] = s
        if asymmetric:
            zp[blk, off] = z


def reshape_and_cache_k_int8(key, key_cache, k_scales, slot_mapping, group_size=32):
    """In-place numpy restatement of ``reshape_and_cache_k_int8`` (F:1287-1312)."""
    block_size = key_cache.shape[1]
    tok, blk, off = _slots(slot_mapping, block_size)
    codes, s = quantize_int8_rows(np.asarray(key, F32)[tok], group_size)
    key_cache[blk, off] = codes
    k_scales[blk, off] = s
