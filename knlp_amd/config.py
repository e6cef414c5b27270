"""Import-time knobs read from the same environment variables as the
reference (fused-quant/fused_int4.v0.1.0.py:55-147), so a deployment that
sets them keeps its behaviour when switching to this package."""
from __future__ import annotations

import os

GROUP_SIZE: int = int(os.environ.get("VLLM_FUSED_INT4_GROUP_SIZE", "32"))      # F:55
INT4_RANGE: int = 7                                                               # F:56
OUTLIER_CLIP_RATIO: float = float(
    os.environ.get("VLLM_FUSED_INT4_OUTLIER_CLIP_RATIO", "10.0"))               # F:70-72
ASYMMETRIC: bool = os.environ.get("VLLM_FUSED_INT4_ASYMMETRIC", "0") == "1"    # F:77
# The reference lowers its default to 999999 on CUDA compute capability < 9
# (F:101-123); that gate is about NVIDIA parts and does not apply on gfx950.
MIN_FUSED_SEQ_LEN: int = int(os.environ.get("VLLM_FUSED_INT4_MIN_SEQ_LEN", "48"))  # F:101-123
K_PRECISION: str = os.environ.get("VLLM_FUSED_INT4_K_PRECISION", "int4")        # F:131
V_PRECISION: str = os.environ.get("VLLM_FUSED_INT4_V_PRECISION", "int4")        # F:136
REPLACE_CACHE: bool = os.environ.get("VLLM_FUSED_QUANT_REPLACE_CACHE", "0") == "1"  # F:141
# Triton tuning knobs of the reference (F:144-147).  The HIP kernels choose
# their own tiling; the values are kept for callers that read them.
DECODE_BLOCK_N: int = int(os.environ.get("VLLM_FUSED_INT4_DECODE_BLOCK_N", "128"))
DECODE_NUM_WARPS: int = int(os.environ.get("VLLM_FUSED_INT4_DECODE_NUM_WARPS", "8"))
DECODE_NUM_STAGES: int = int(os.environ.get("VLLM_FUSED_INT4_DECODE_NUM_STAGES", "3"))
DECODE_GATHERED_SCALE: bool = os.environ.get(
    "VLLM_FUSED_INT4_DECODE_GATHERED_SCALE", "0") == "1"
# Split length override for the split-K decode (0 = library plan).
DECODE_SPLIT_TOKENS: int = int(os.environ.get("KNLP_DECODE_SPLIT_TOKENS", "0"))
# Softmax scale of the backend's fused decode.  The reference's fused
# kernels fix it to 1/sqrt(head_size) (F:924) whatever scale the layer was
# built with (its _fused_decode, F:2851-2928, passes none), and so does this
# package by default.  Set to 1 to use the layer's own scale instead (models
# whose attention scale is not 1/sqrt(head_size)).
FUSED_DECODE_LAYER_SCALE: bool = os.environ.get("KNLP_FUSED_DECODE_LAYER_SCALE", "0") == "1"
