"""Drop-in replacements for the module functions of knlp's fused INT4 backend.

Same names, argument order, defaults and in-place / return conventions as
``fused-quant/fused_int4.v0.1.0.py`` (F): the write functions mutate the
caller's caches and return None; the decode functions return a new tensor
shaped like ``query`` (``torch.empty_like(query)``, F:932).  Every function
launches onto the current torch stream through the C ABI of
``libknlp_int4kv.so`` and performs no host synchronisation, so the calls can
be captured in a HIP graph.  There is no CPU fallback: a missing library
raises.

Extensions over the reference, all keyword-only and defaulting to the
reference's behaviour:
  * ``group_size`` / ``k_group_size`` / ``v_group_size`` -- the reference uses
    the module-wide GROUP_SIZE for K and V alike (F:1412-1418); per-plane
    sizes allow e.g. per-row INT8 K (group = head_size) with g32 INT4 V;
  * ``clip_ratio`` -- defaults to OUTLIER_CLIP_RATIO like F:470;
  * ``scale`` -- defaults to 1/sqrt(head_size) as F:924 fixes it;
  * ``split_tokens`` -- split-K length, default from the library's plan; 0 is
    the stream schedule (equal shares of all rows' tiles per CU);
  * ``total_context`` -- the batch's summed sequence lengths when the caller
    knows them on the host (0: unknown); with it the plan keeps split-K for
    uniform batches and picks the stream schedule for variable-length ones;
    unknown, it picks the stream schedule for any batch of several sequences
    the cooperative kernel takes.
``block_n`` is accepted for signature compatibility and ignored: the HIP
kernels pick their own token tiles.
"""
from __future__ import annotations

import ctypes

import torch

from . import config
from ._lib import (DT_BF16, DT_F16, DT_I32, DT_I64, KV_FP16, KV_INT4_ASYM, KV_INT4_SYM,
                   KV_INT8_SYM, KvPlane, check, lib)

GROUP_SIZE = config.GROUP_SIZE
OUTLIER_CLIP_RATIO = config.OUTLIER_CLIP_RATIO
ASYMMETRIC = config.ASYMMETRIC

_SRC_DTYPES = {torch.float16: DT_F16, torch.bfloat16: DT_BF16}


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("knlp_amd ops need device tensors (the HIP path has no CPU fallback)")


def _plane(cache: torch.Tensor, scales, zeros, fmt: int, group_size: int) -> KvPlane:
    want = {KV_INT4_SYM: torch.uint8, KV_INT4_ASYM: torch.uint8, KV_INT8_SYM: torch.int8,
            KV_FP16: torch.float16}[fmt]
    if cache.dtype != want:
        raise ValueError(f"cache dtype {cache.dtype} does not match format (want {want})")
    if cache.dim() != 4 or cache.stride(3) != 1:
        raise ValueError("cache must be [num_blocks, block_size, num_heads, packed_dim] "
                         "with a contiguous last axis")
    p = KvPlane()
    p.data = cache.data_ptr()
    p.stride_block, p.stride_page, p.stride_head = cache.stride()[:3]
    p.format = fmt
    p.group_size = group_size
    if fmt != KV_FP16:
        if scales is None or scales.dtype != torch.float16 or scales.dim() != 4 \
                or scales.stride(3) != 1:
            raise ValueError("scales must be fp16 [num_blocks, block_size, num_heads, num_groups]")
        p.scales = scales.data_ptr()
        p.s_stride_block, p.s_stride_page, p.s_stride_head = scales.stride()[:3]
    if fmt == KV_INT4_ASYM:
        if zeros is None or zeros.dtype != torch.float16 or zeros.stride(3) != 1:
            raise ValueError("asymmetric mode needs fp16 zero-points shaped like the scales")
        p.zeros = zeros.data_ptr()
        p.z_stride_block, p.z_stride_page, p.z_stride_head = zeros.stride()[:3]
    # shapes for _check_plane (the C ABI carries strides only)
    p.shape = tuple(cache.shape)
    p.s_shape = tuple(scales.shape) if fmt != KV_FP16 else None
    p.z_shape = tuple(zeros.shape) if fmt == KV_INT4_ASYM else None
    return p


def _check_plane(p: KvPlane, name: str, num_heads: int, head_size: int) -> None:
    """Raise ValueError unless the cache of plane ``p`` holds ``num_heads``
    heads of ``head_size`` elements and its scales / zero-points cover every
    (block, slot, head, group) of it.  The kernels index these tensors
    through their strides without bounds checks (as the reference's Triton
    kernels do), so a cache with fewer heads, a shorter packed axis or
    smaller scale arrays than the call implies would be read or written out
    of bounds; this is the host-side guard against that."""
    shape = getattr(p, "shape", None)
    if shape is None:
        return
    nb, bs, nh, last = shape
    packed = head_size // 2 if p.format in (KV_INT4_SYM, KV_INT4_ASYM) else head_size
    if nh < num_heads or last < packed:
        raise ValueError(f"{name} cache {list(shape)} holds fewer than {num_heads} heads of "
                         f"{packed} {'bytes' if p.format != KV_FP16 else 'halves'}")
    if p.format == KV_FP16:
        return
    ng = head_size // p.group_size if p.group_size > 0 else 0
    for what, sh in (("scales", p.s_shape), ("zeros", p.z_shape)):
        if sh is None:
            continue
        if len(sh) != 4 or sh[0] < nb or sh[1] < bs or sh[2] < num_heads or sh[3] < ng:
            raise ValueError(f"{name} {what} {list(sh)} do not cover a cache of "
                             f"{list(shape)} with {ng} groups per head")


def _src_dtype(t: torch.Tensor) -> int:
    if t.dtype not in _SRC_DTYPES:
        raise ValueError(f"key/value dtype {t.dtype} not supported (fp16 or bf16)")
    if t.dim() != 3 or t.stride(2) != 1:
        raise ValueError("key/value must be [num_tokens, num_heads, head_size], last axis contiguous")
    return _SRC_DTYPES[t.dtype]


def _slot_dtype(slot_mapping: torch.Tensor) -> int:
    if slot_mapping.dtype == torch.int64:
        return DT_I64
    if slot_mapping.dtype == torch.int32:
        return DT_I32
    raise ValueError("slot_mapping must be int32 or int64")


def _append(key, value, kplane, vplane, slot_mapping, clip_ratio, block_size) -> None:
    src = key if key is not None else value
    dt = _src_dtype(src)
    if key is not None and value is not None:
        _src_dtype(value)                      # its own layout checks too
        if key.dtype != value.dtype:
            raise ValueError("key and value must share a dtype")
        if key.shape != value.shape:
            raise ValueError("key and value must have the same shape")
    slot_mapping = slot_mapping.contiguous()
    num_tokens, num_heads, head_size = src.shape
    if slot_mapping.numel() < num_tokens:
        raise ValueError("slot_mapping shorter than num_tokens")
    if key is not None:
        _check_plane(kplane, "key", num_heads, head_size)
    if value is not None:
        _check_plane(vplane, "value", num_heads, head_size)
    if key is not None and value is not None and kplane.shape[1] != vplane.shape[1]:
        raise ValueError("key and value caches have different block sizes")
    st = lib().knlp_kv_append(
        key.data_ptr() if key is not None else None,
        value.data_ptr() if value is not None else None,
        dt, num_tokens, num_heads, head_size,
        key.stride(0) if key is not None else 0, key.stride(1) if key is not None else 0,
        value.stride(0) if value is not None else 0, value.stride(1) if value is not None else 0,
        ctypes.byref(kplane) if kplane is not None else None,
        ctypes.byref(vplane) if vplane is not None else None,
        slot_mapping.data_ptr(), _slot_dtype(slot_mapping),
        int(block_size), float(clip_ratio), _stream())
    check(st, "knlp_kv_append")


def reshape_and_cache_int4(key, value, key_cache, value_cache, k_scales, v_scales,
                           slot_mapping, k_zeros=None, v_zeros=None, asymmetric=False, *,
                           group_size=None, clip_ratio=None) -> None:
    """Quantise fp16/bf16 K and V to packed INT4 and write them at
    ``slot_mapping`` into the paged caches (F:418-472).  Symmetric mode uses
    the trimmed-mean outlier clip (F:328-357); asymmetric stores zero-points."""
    _require_cuda(key, value, key_cache, value_cache, k_scales, v_scales, slot_mapping)
    gs = group_size or GROUP_SIZE
    fmt = KV_INT4_ASYM if asymmetric else KV_INT4_SYM
    kp = _plane(key_cache, k_scales, k_zeros, fmt, gs)
    vp = _plane(value_cache, v_scales, v_zeros, fmt, gs)
    _append(key, value, kp, vp, slot_mapping,
            OUTLIER_CLIP_RATIO if clip_ratio is None else clip_ratio, key_cache.shape[1])


def reshape_and_cache_v_only_int4(value, value_cache, v_scales, slot_mapping, v_zeros=None,
                                  asymmetric=False, *, group_size=None,
                                  clip_ratio=None) -> None:
    """V-only INT4 quantise-and-cache (F:603-647)."""
    _require_cuda(value, value_cache, v_scales, slot_mapping)
    gs = group_size or GROUP_SIZE
    vp = _plane(value_cache, v_scales, v_zeros, KV_INT4_ASYM if asymmetric else KV_INT4_SYM, gs)
    _append(None, value, None, vp, slot_mapping,
            OUTLIER_CLIP_RATIO if clip_ratio is None else clip_ratio, value_cache.shape[1])


def reshape_and_cache_k_int8(key, key_cache_int8, k_scales, slot_mapping, *,
                             group_size=None) -> None:
    """Symmetric INT8 K quantise-and-cache (F:1287-1312)."""
    _require_cuda(key, key_cache_int8, k_scales, slot_mapping)
    kp = _plane(key_cache_int8, k_scales, None, KV_INT8_SYM, group_size or GROUP_SIZE)
    _append(key, None, kp, None, slot_mapping, 0.0, key_cache_int8.shape[1])


def reshape_and_cache_v_int8(value, value_cache_int8, v_scales, slot_mapping, *,
                             group_size=None) -> None:
    """Symmetric INT8 V quantise-and-cache (F:1619-1650)."""
    _require_cuda(value, value_cache_int8, v_scales, slot_mapping)
    vp = _plane(value_cache_int8, v_scales, None, KV_INT8_SYM, group_size or GROUP_SIZE)
    _append(None, value, None, vp, slot_mapping, 0.0, value_cache_int8.shape[1])


def reshape_and_cache_fp16(key, value, key_cache, value_cache, slot_mapping) -> None:
    """Plain fp16 K and V rows into fp16 paged caches at ``slot_mapping``
    (``slot < 0`` skipped).  Not a function of the reference module: it is
    the write vLLM's ``reshape_and_cache_flash`` does for the fp16 planes
    (F:2535-2544), on this library's append kernel.  Either side may be
    None."""
    _require_cuda(key, value, key_cache, value_cache, slot_mapping)
    src = key if key is not None else value
    if src is None:
        raise ValueError("reshape_and_cache_fp16 needs key or value")
    if src.dtype != torch.float16:
        raise ValueError("reshape_and_cache_fp16 writes fp16 caches from fp16 rows")
    head_size = src.shape[2]
    kp = _plane(key_cache, None, None, KV_FP16, head_size) if key is not None else None
    vp = _plane(value_cache, None, None, KV_FP16, head_size) if value is not None else None
    block_size = (key_cache if key is not None else value_cache).shape[1]
    _append(key, value, kp, vp, slot_mapping, 0.0, block_size)


def _decode(query, kp: KvPlane, vp: KvPlane, block_size, block_table, seq_lens, num_kv_heads,
            head_size, scale=None, split_tokens=None, append=None,
            total_context=0) -> torch.Tensor:
    _require_cuda(query, block_table, seq_lens)
    if query.dtype not in _SRC_DTYPES:
        raise ValueError(f"query dtype {query.dtype} not supported (fp16 or bf16)")
    if query.dim() != 3 or query.stride(2) != 1 or query.shape[2] != head_size:
        raise ValueError("query must be [num_seqs, num_heads, head_size], last axis contiguous")
    num_seqs, num_heads, _ = query.shape
    if num_heads % num_kv_heads:
        raise ValueError("num_heads must be a multiple of num_kv_heads")
    if num_seqs == 0:
        return torch.empty_like(query)
    if block_table.dtype != torch.int32:
        block_table = block_table.to(torch.int32)
    if block_table.stride(1) != 1:
        block_table = block_table.contiguous()
    if seq_lens.dtype != torch.int32 or not seq_lens.is_contiguous():
        seq_lens = seq_lens.to(torch.int32).contiguous()
    _check_plane(kp, "key", num_kv_heads, head_size)
    _check_plane(vp, "value", num_kv_heads, head_size)
    if getattr(kp, "shape", None) and getattr(vp, "shape", None) and kp.shape[1] != vp.shape[1]:
        raise ValueError("key and value caches have different block sizes")
    L = lib()
    max_context = block_table.shape[1] * block_size
    if split_tokens is None:
        split_tokens = config.DECODE_SPLIT_TOKENS or L.knlp_kv_decode_plan(
            num_seqs, num_kv_heads, num_heads, head_size, max_context, int(total_context),
            kp.format, kp.group_size, vp.format, vp.group_size)
        check(split_tokens, "knlp_kv_decode_plan")
    ws_bytes = L.knlp_kv_decode_workspace_bytes(max(num_seqs, 1), num_heads, head_size,
                                                max_context, split_tokens)
    check(ws_bytes, "knlp_kv_decode_workspace_bytes")
    ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=query.device)
    out = torch.empty_like(query)
    if scale is None:
        scale = 1.0 / (head_size ** 0.5)                  # F:924
    dt = _SRC_DTYPES[query.dtype]
    if append is None:
        st = L.knlp_kv_decode(
            query.data_ptr(), dt, query.stride(0), query.stride(1), num_seqs, num_heads,
            num_kv_heads, head_size, ctypes.byref(kp), ctypes.byref(vp),
            block_table.data_ptr(), block_table.stride(0), seq_lens.data_ptr(), block_size,
            max_context, float(scale), int(split_tokens), ws.data_ptr(), ws_bytes,
            out.data_ptr(), dt, out.stride(0), out.stride(1), _stream())
        check(st, "knlp_kv_decode")
        return out
    key, value, slot_mapping, clip_ratio = append
    src = key if key is not None else value
    for t in (key, value):
        if t is not None and (t.dim() != 3 or t.shape[0] < num_seqs or t.stride(2) != 1 or
                              t.shape[1] != num_kv_heads or t.shape[2] != head_size):
            raise ValueError("key/value must be [num_seqs, num_kv_heads, head_size], "
                             "last axis contiguous")
    if key is not None and value is not None and key.dtype != value.dtype:
        raise ValueError("key and value must share a dtype")
    slot_mapping = slot_mapping.contiguous()
    if slot_mapping.numel() < num_seqs:
        raise ValueError("slot_mapping shorter than num_seqs")
    st = L.knlp_kv_append_decode(
        query.data_ptr(), dt, query.stride(0), query.stride(1), num_seqs, num_heads,
        num_kv_heads, head_size,
        key.data_ptr() if key is not None else None,
        value.data_ptr() if value is not None else None, _src_dtype(src),
        key.stride(0) if key is not None else 0, key.stride(1) if key is not None else 0,
        value.stride(0) if value is not None else 0, value.stride(1) if value is not None else 0,
        slot_mapping.data_ptr(), _slot_dtype(slot_mapping), float(clip_ratio),
        ctypes.byref(kp), ctypes.byref(vp), block_table.data_ptr(), block_table.stride(0),
        seq_lens.data_ptr(), block_size, max_context, float(scale), int(split_tokens),
        ws.data_ptr(), ws_bytes, out.data_ptr(), dt, out.stride(0), out.stride(1), _stream())
    check(st, "knlp_kv_append_decode")
    return out


def int4_twos_to_offset(packed: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Re-encode packed INT4 codes from the gpt2 compression path's
    two's-complement nibbles (gpt2/compression/kv_plugin.py:212-257) into
    this library's offset nibbles (n = t + 8, F:359).  ``packed``: uint8
    ``[..., D/2]`` with a contiguous last axis; ``out`` may be ``packed``
    itself (in place) or None (new tensor).  With that path's per-row fp16
    scale ``[..., 1]`` the result decodes as a symmetric INT4 plane of group
    size D.  Not a function of the reference module."""
    _require_cuda(packed, out)
    if packed.dtype != torch.uint8 or packed.dim() < 1 or packed.stride(-1) != 1:
        raise ValueError("packed must be uint8 with a contiguous last axis")
    if out is None:
        out = torch.empty_like(packed)
    if out.shape != packed.shape or out.dtype != torch.uint8 or out.stride(-1) != 1:
        raise ValueError("out must be uint8 shaped like packed, last axis contiguous")
    rb = packed.shape[-1]
    src2, dst2 = packed.reshape(-1, rb), out.reshape(-1, rb)
    if dst2.data_ptr() != out.data_ptr() or (out.numel() and not _same_storage(dst2, out)):
        raise ValueError("out must be reshapeable to rows without a copy")
    st = lib().knlp_int4_twos_to_offset(src2.data_ptr(), src2.stride(0) if src2.dim() else rb,
                                         dst2.data_ptr(), dst2.stride(0) if dst2.dim() else rb,
                                         src2.shape[0], rb, _stream())
    check(st, "knlp_int4_twos_to_offset")
    return out


def _same_storage(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.untyped_storage().data_ptr() == b.untyped_storage().data_ptr()


_FORMATS = {"int8": KV_INT8_SYM, "fp16": KV_FP16}


def _fmt(name: str, asymmetric: bool) -> int:
    if name == "int4":
        return KV_INT4_ASYM if asymmetric else KV_INT4_SYM
    if name not in _FORMATS:
        raise ValueError(f"unknown cache format {name!r} (int4, int8 or fp16)")
    return _FORMATS[name]


def append_and_decode(query, key, value, slot_mapping, key_cache, value_cache, k_scales,
                      v_scales, block_table, seq_lens, num_kv_heads, head_size, *,
                      k_format="int4", v_format="int4", k_zeros=None, v_zeros=None,
                      asymmetric=False, k_group_size=None, v_group_size=None,
                      clip_ratio=None, scale=None, split_tokens=None,
                      total_context=0) -> torch.Tensor:
    """Quantise the token being decoded into the caches and decode, in the
    launches of one decode (no separate append launch).

    Not a function of the reference module: it fuses the
    ``reshape_and_cache_*`` call that F's backend makes before every decode
    (F:2600-2689) into the decode, as docs/fused-quant/latency.md:41
    proposes.  ``key`` / ``value`` are ``[num_seqs, num_kv_heads, head_size]``
    rows of the new token (either may be None), ``slot_mapping[s]`` the slot
    of position ``seq_lens[s] - 1`` (``< 0``: no write).  ``k_format`` /
    ``v_format`` are "int4" (``asymmetric`` selects zero-points), "int8" or
    "fp16"; the caches, scales and zeros are the reference's tensors.  The
    written codes equal those of the separate append; the output equals the
    decode after it."""
    _require_cuda(query, key, value, slot_mapping, key_cache, value_cache, k_scales, v_scales)
    kf, vf = _fmt(k_format, asymmetric), _fmt(v_format, asymmetric)
    kp = _plane(key_cache, k_scales, k_zeros, kf,
                head_size if kf == KV_FP16 else (k_group_size or GROUP_SIZE))
    vp = _plane(value_cache, v_scales, v_zeros, vf,
                head_size if vf == KV_FP16 else (v_group_size or GROUP_SIZE))
    clip = OUTLIER_CLIP_RATIO if clip_ratio is None else clip_ratio
    return _decode(query, kp, vp, key_cache.shape[1], block_table, seq_lens, num_kv_heads,
                   head_size, scale, split_tokens, append=(key, value, slot_mapping, clip),
                   total_context=total_context)


def fused_int4_decode(query, key_cache, value_cache, k_scales, v_scales, block_table, seq_lens,
                      num_kv_heads, head_size, block_n=64, k_zeros=None, v_zeros=None,
                      asymmetric=False, *, group_size=None, scale=None,
                      split_tokens=None, total_context=0) -> torch.Tensor:
    """Decode attention over packed INT4 K and V (F:901-979)."""
    _require_cuda(key_cache, value_cache, k_scales, v_scales)
    gs = group_size or GROUP_SIZE
    fmt = KV_INT4_ASYM if asymmetric else KV_INT4_SYM
    kp = _plane(key_cache, k_scales, k_zeros, fmt, gs)
    vp = _plane(value_cache, v_scales, v_zeros, fmt, gs)
    return _decode(query, kp, vp, key_cache.shape[1], block_table, seq_lens, num_kv_heads,
                   head_size, scale, split_tokens, total_context=total_context)


def kint8_vint4_decode(query, key_cache_int8, value_cache_int4, k_scales, v_scales, block_table,
                       seq_lens, num_kv_heads, head_size, block_n=64, v_zeros=None,
                       asymmetric=False, *, k_group_size=None, v_group_size=None, scale=None,
                       split_tokens=None, total_context=0) -> torch.Tensor:
    """Decode with symmetric INT8 K and INT4 V (F:1496-1554)."""
    _require_cuda(key_cache_int8, value_cache_int4, k_scales, v_scales)
    kp = _plane(key_cache_int8, k_scales, None, KV_INT8_SYM, k_group_size or GROUP_SIZE)
    vp = _plane(value_cache_int4, v_scales, v_zeros,
                KV_INT4_ASYM if asymmetric else KV_INT4_SYM, v_group_size or GROUP_SIZE)
    return _decode(query, kp, vp, key_cache_int8.shape[1], block_table, seq_lens, num_kv_heads,
                   head_size, scale, split_tokens, total_context=total_context)


def kfp16_vint4_decode(query, key_cache_fp16, value_cache_int4, v_scales, block_table, seq_lens,
                       num_kv_heads, head_size, block_n=64, v_zeros=None, asymmetric=False, *,
                       v_group_size=None, scale=None, split_tokens=None,
                       total_context=0) -> torch.Tensor:
    """Decode with fp16 K and INT4 V (F:1159-1225)."""
    _require_cuda(key_cache_fp16, value_cache_int4, v_scales)
    kp = _plane(key_cache_fp16, None, None, KV_FP16, head_size)
    vp = _plane(value_cache_int4, v_scales, v_zeros,
                KV_INT4_ASYM if asymmetric else KV_INT4_SYM, v_group_size or GROUP_SIZE)
    return _decode(query, kp, vp, key_cache_fp16.shape[1], block_table, seq_lens, num_kv_heads,
                   head_size, scale, split_tokens, total_context=total_context)


def kint8_vint8_decode(query, key_cache_int8, value_cache_int8, k_scales, v_scales, block_table,
                       seq_lens, num_kv_heads, head_size, block_n=64, *, k_group_size=None,
                       v_group_size=None, scale=None, split_tokens=None,
                       total_context=0) -> torch.Tensor:
    """Decode with symmetric INT8 K and V (F:1796-1848)."""
    _require_cuda(key_cache_int8, value_cache_int8, k_scales, v_scales)
    kp = _plane(key_cache_int8, k_scales, None, KV_INT8_SYM, k_group_size or GROUP_SIZE)
    vp = _plane(value_cache_int8, v_scales, None, KV_INT8_SYM, v_group_size or GROUP_SIZE)
    return _decode(query, kp, vp, key_cache_int8.shape[1], block_table, seq_lens, num_kv_heads,
                   head_size, scale, split_tokens, total_context=total_context)


def kfp16_vint8_decode(query, key_cache_fp16, value_cache_int8, v_scales, block_table, seq_lens,
                       num_kv_heads, head_size, block_n=64, *, v_group_size=None, scale=None,
                       split_tokens=None, total_context=0) -> torch.Tensor:
    """Decode with fp16 K and symmetric INT8 V (F:1975-2028)."""
    _require_cuda(key_cache_fp16, value_cache_int8, v_scales)
    kp = _plane(key_cache_fp16, None, None, KV_FP16, head_size)
    vp = _plane(value_cache_int8, v_scales, None, KV_INT8_SYM, v_group_size or GROUP_SIZE)
    return _decode(query, kp, vp, key_cache_fp16.shape[1], block_table, seq_lens, num_kv_heads,
                   head_size, scale, split_tokens, total_context=total_context)


def fp16_paged_decode(query, key_cache_fp16, value_cache_fp16, block_table, seq_lens,
                      num_kv_heads, head_size, *, scale=None, split_tokens=None,
                      total_context=0) -> torch.Tensor:
    """The same split-K decode reading plain fp16 paged K and V caches.

    Not a reference function: it is the fp16-KV instantiation of this
    library's kernel used for the INT4-vs-fp16 comparison (the reference
    compares against SDPA, scripts/spev01/tier5_fused_decode.py:341-348)."""
    _require_cuda(key_cache_fp16, value_cache_fp16)
    kp = _plane(key_cache_fp16, None, None, KV_FP16, head_size)
    vp = _plane(value_cache_fp16, None, None, KV_FP16, head_size)
    return _decode(query, kp, vp, key_cache_fp16.shape[1], block_table, seq_lens, num_kv_heads,
                   head_size, scale, split_tokens, total_context=total_context)


def decode_fp16_sdpa(query, fp16_k, fp16_v, seq_lens, num_kv_heads, num_heads,
                     head_size) -> torch.Tensor:
    """Decode attention over per-sequence fp16 K/V (F:2031-2071): ``fp16_k``
    and ``fp16_v`` are ``[max_seqs, max_ctx, num_kv_heads, head_size]``,
    sequence s holding its first ``seq_lens[s]`` positions; softmax scale
    1/sqrt(head_size), GQA head h reading kv head h // (num_heads /
    num_kv_heads), output shaped like ``query``.  The reference loops over
    the sequences with SDPA on repeat_interleave-expanded K/V; here the
    tensors are read in place as a paged cache (16-token pages when max_ctx
    allows, else one page per sequence) by the fp16 decode kernel, with no
    host synchronisation."""
    _require_cuda(query, fp16_k, fp16_v, seq_lens)
    if query.dim() != 3 or query.shape[1] != num_heads or query.shape[2] != head_size:
        raise ValueError("query must be [num_seqs, num_heads, head_size]")
    for t in (fp16_k, fp16_v):
        if t.dim() != 4 or t.shape[2] != num_kv_heads or t.shape[3] != head_size:
            raise ValueError("fp16_k / fp16_v must be [max_seqs, max_ctx, num_kv_heads, head_size]")
        if t.dtype != torch.float16:
            raise ValueError("fp16_k / fp16_v must be float16")
    num_seqs = query.shape[0]
    max_seqs, max_ctx = fp16_k.shape[:2]
    if fp16_v.shape[:2] != fp16_k.shape[:2] or num_seqs > max_seqs:
        raise ValueError("fp16_k / fp16_v shapes disagree or hold fewer sequences than query")
    page = 16 if max_ctx % 16 == 0 else max_ctx
    per_seq = max_ctx // page
    k = fp16_k.contiguous().view(max_seqs * per_seq, page, num_kv_heads, head_size)
    v = fp16_v.contiguous().view(max_seqs * per_seq, page, num_kv_heads, head_size)
    block_table = torch.arange(max_seqs * per_seq, dtype=torch.int32,
                               device=query.device).view(max_seqs, per_seq)[:num_seqs]
    return fp16_paged_decode(query, k, v, block_table, seq_lens, num_kv_heads, head_size)


def decode_kernel_kind(num_heads, num_kv_heads, head_size, k_format, k_group_size, v_format,
                       v_group_size, query_dtype=torch.float16) -> str:
    """'mfma' or 'valu': which decode kernel the library dispatches a shape to."""
    r = lib().knlp_kv_decode_kernel_kind(num_heads, num_kv_heads, head_size, k_format,
                                         k_group_size, v_format, v_group_size,
                                         _SRC_DTYPES[query_dtype])
    check(r, "knlp_kv_decode_kernel_kind")
    return "mfma" if r == 1 else "valu"
