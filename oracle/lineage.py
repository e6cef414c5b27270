"""CPU restatements of two other INT4 packers of the reference, for tests only.

* ``t5_quantize_and_pack_int4`` / ``t5_dequant_int4``: the standalone
  harness packer, scripts/spev01/tier5_fused_decode.py:116-145 (= v35/v29
  copies): symmetric per-group scale amax / 7, ``torch.round`` (ties to
  even), clamp [-8, 7], stored as q + 8 with element 2i in the low nibble.
  It equals F's symmetric quantiser (F:328-363) without the outlier clip,
  except at exact .5 ties, where F rounds half away from zero (F:198-202).
* ``gpt2_quantize_int4`` / ``gpt2_dequantize_int4``: the gpt2 compression
  path, gpt2/compression/kv_plugin.py:212-295: one scale per row
  (``per_channel=True``, amax / 7 over the last axis, clamped at 1e-8),
  ``torch.round`` and clamp [-7, 7], stored as two's-complement nibbles
  ``t & 0xF`` with element 2i in the low nibble; dequantisation sign-extends
  and multiplies by the scale in fp32.

Both run the same torch CPU operations, in the input's dtype, as the
reference functions they restate.  Test infrastructure only: the library
never imports this package.
"""
from __future__ import annotations

import torch


def t5_quantize_and_pack_int4(tensor: torch.Tensor, group_size: int = 32):
    """(packed uint8 [..., D/2], scales [..., D/G]) as T5:116-130."""
    shape = tensor.shape
    d = shape[-1]
    r = tensor.reshape(*shape[:-1], d // group_size, group_size)
    amax = r.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
    scale = amax / 7.0
    q = (r / scale).round().clamp(-8, 7).to(torch.int8).reshape(*shape[:-1], d)
    u = (q + 8).to(torch.uint8)
    return u[..., 0::2] | (u[..., 1::2] << 4), scale.squeeze(-1)


def t5_dequant_int4(packed: torch.Tensor, scales: torch.Tensor, group_size: int = 32):
    """fp16 [..., D] as T5:133-145 (code - 8, times the group scale, in fp16)."""
    lo = (packed & 0x0F).to(torch.int8) - 8
    hi = ((packed >> 4) & 0x0F).to(torch.int8) - 8
    d = packed.shape[-1] * 2
    out = torch.empty(*packed.shape[:-1], d, dtype=torch.float16)
    out[..., 0::2] = lo.to(torch.float16)
    out[..., 1::2] = hi.to(torch.float16)
    out = out.reshape(*packed.shape[:-1], d // group_size, group_size) * scales.unsqueeze(-1)
    return out.reshape(*packed.shape[:-1], d)


def gpt2_quantize_int4(x: torch.Tensor):
    """(packed uint8 [..., D/2] of two's-complement nibbles, scale [..., 1]) as
    kv_plugin.quantize_to_int4 with per_channel=True (kv_plugin.py:212-257)."""
    q_max = 7
    scale = (x.abs().amax(dim=-1, keepdim=True) / q_max).clamp(min=1e-8)
    q = torch.round(x / scale).clamp(-q_max, q_max).to(torch.int8)
    lo = q[..., 0::2] & 0x0F
    hi = (q[..., 1::2] & 0x0F) << 4
    return (lo | hi).to(torch.uint8), scale


def gpt2_dequantize_int4(packed: torch.Tensor, scale: torch.Tensor,
                         dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """kv_plugin.dequantize_from_int4 (kv_plugin.py:260-295): sign-extended
    nibbles times the scale in fp32, then cast to ``dtype``."""
    lo = (packed & 0x0F).to(torch.int8)
    hi = ((packed >> 4) & 0x0F).to(torch.int8)
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    d = packed.shape[-1] * 2
    x = torch.empty(*packed.shape[:-1], d, dtype=torch.int8)
    x[..., 0::2] = lo
    x[..., 1::2] = hi
    return (x.float() * scale.float()).to(dtype)
