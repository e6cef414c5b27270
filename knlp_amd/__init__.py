"""knlp_amd: MI355X (gfx950) fused INT4 KV-cache quantize-on-append and
split-K decode attention, a drop-in for the module functions of mcgrof/knlp's
fused INT4 vLLM backend (fused-quant/fused_int4.v0.1.0.py).

Import is cheap and does not touch the GPU; the HIP library is loaded on the
first operator call (:func:`knlp_amd._lib.lib`).
"""
from .ops import (  # noqa: F401
    ASYMMETRIC, GROUP_SIZE, OUTLIER_CLIP_RATIO, append_and_decode, decode_fp16_sdpa,
    decode_kernel_kind, fp16_paged_decode, int4_twos_to_offset,
    fused_int4_decode, kfp16_vint4_decode, kfp16_vint8_decode, kint8_vint4_decode,
    kint8_vint8_decode, reshape_and_cache_fp16, reshape_and_cache_int4,
    reshape_and_cache_k_int8, reshape_and_cache_v_int8, reshape_and_cache_v_only_int4,
)

__all__ = [
    "reshape_and_cache_int4", "reshape_and_cache_v_only_int4", "reshape_and_cache_k_int8",
    "reshape_and_cache_v_int8", "reshape_and_cache_fp16", "fused_int4_decode", "kint8_vint4_decode",
    "kfp16_vint4_decode", "kint8_vint8_decode", "kfp16_vint8_decode", "decode_fp16_sdpa",
    "fp16_paged_decode",
    "append_and_decode", "int4_twos_to_offset", "decode_kernel_kind", "GROUP_SIZE", "OUTLIER_CLIP_RATIO", "ASYMMETRIC",
]
