"""Cache shapes and shadow-cache planning of the fused INT4 backend.

The reference keeps vLLM's fp16 paged cache (one or two planes) and, next to
it, "shadow" quantised caches that the backend allocates itself: packed INT4
(or INT8) codes with per-group fp16 scales (and zero-points when asymmetric).
vLLM's planner budgets those bytes through ``shadow_bytes_per_block``.  This
module restates

  * the allocator-compatible cache shape, ``get_kv_cache_shape``
    (fused-quant/fused_int4.v0.1.0.py:2122-2158);
  * the planner formula (fused-quant/support/attention.v0.1.0.py:529-591);
  * the lazy shadow allocation of ``_ensure_int4_cache`` (F:2334-2480),
    including its per-block accounting check against the planner.

No vLLM import and no GPU work: the allocation goes to whatever device the
caller names.
"""
from __future__ import annotations

from dataclasses import dataclass, fields

import torch

PRECISIONS_K = ("int4", "int8", "fp16")
PRECISIONS_V = ("int4", "int8")


def kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                   replace_cache: bool = False) -> tuple[int, ...]:
    """Shape of the allocator's fp16 paged cache: two planes (K, V), or only
    the K plane when the V plane is replaced by the quantised shadow cache
    (F:2152-2158)."""
    return (1 if replace_cache else 2, num_blocks, block_size, num_kv_heads, head_size)


def shadow_bytes_per_block(block_size: int, num_kv_heads: int, head_size: int, *,
                           k_precision: str = "int4", v_precision: str = "int4",
                           asymmetric: bool = False, group_size: int = 32) -> int:
    """Bytes of shadow cache per paged block, as the reference's planner
    counts them (support/attention.v0.1.0.py:545-584).

    V: packed INT4 codes + fp16 scales (+ zeros when asymmetric), or INT8
    codes + scales plus the 3-byte INT4 placeholder the backend keeps for its
    size guard.  K: the same INT4 layout, INT8 codes + scales, or nothing for
    fp16 K (read from the paged cache)."""
    if k_precision not in PRECISIONS_K or v_precision not in PRECISIONS_V:
        raise ValueError(f"unknown precision pair ({k_precision}, {v_precision})")
    if head_size % group_size:
        raise ValueError("head_size must be a multiple of group_size")
    rows = block_size * num_kv_heads
    groups = head_size // group_size
    scales = rows * groups * 2
    if v_precision == "int8":
        shadow = rows * head_size + scales + 1 + 2
    else:
        shadow = rows * (head_size // 2) + scales * (2 if asymmetric else 1)
    if k_precision == "int4":
        shadow += rows * (head_size // 2) + scales * (2 if asymmetric else 1)
    elif k_precision == "int8":
        shadow += rows * head_size + scales
    return shadow


@dataclass
class ShadowCaches:
    """The backend-owned quantised caches (F:2276-2290).  Unused members are
    None; ``int4_value`` / ``v_scales`` hold a 1-element placeholder when V is
    INT8, as the reference keeps one for its size guard (F:2365-2371)."""
    int4_key: torch.Tensor | None = None
    k_scales: torch.Tensor | None = None
    k_zeros: torch.Tensor | None = None
    int4_value: torch.Tensor | None = None
    v_scales: torch.Tensor | None = None
    v_zeros: torch.Tensor | None = None
    int8_key: torch.Tensor | None = None
    k_int8_scales: torch.Tensor | None = None
    int8_value: torch.Tensor | None = None
    v_int8_scales: torch.Tensor | None = None

    def nbytes(self) -> int:
        return sum(t.nelement() * t.element_size()
                   for t in (getattr(self, f.name) for f in fields(self)) if t is not None)

    def num_blocks(self, v_precision: str) -> int:
        t = self.int8_value if v_precision == "int8" else self.int4_value
        return 0 if t is None else t.shape[0]


def allocate_shadow_caches(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           *, k_precision: str = "int4", v_precision: str = "int4",
                           asymmetric: bool = False, group_size: int = 32,
                           device: torch.device | str = "cpu") -> ShadowCaches:
    """Zero-filled shadow caches for `num_blocks` paged blocks (F:2358-2425)."""
    if k_precision not in PRECISIONS_K or v_precision not in PRECISIONS_V:
        raise ValueError(f"unknown precision pair ({k_precision}, {v_precision})")
    if head_size % group_size or head_size % 2:
        raise ValueError("head_size must be even and a multiple of group_size")
    ng = head_size // group_size
    shape_codes4 = (num_blocks, block_size, num_kv_heads, head_size // 2)
    shape_codes8 = (num_blocks, block_size, num_kv_heads, head_size)
    shape_groups = (num_blocks, block_size, num_kv_heads, ng)

    def zeros(shape, dtype):
        return torch.zeros(shape, dtype=dtype, device=device)

    c = ShadowCaches()
    if v_precision == "int8":
        c.int8_value = zeros(shape_codes8, torch.int8)
        c.v_int8_scales = zeros(shape_groups, torch.float16)
        c.int4_value = zeros((1, 1, 1, 1), torch.uint8)
        c.v_scales = zeros((1, 1, 1, 1), torch.float16)
    else:
        c.int4_value = zeros(shape_codes4, torch.uint8)
        c.v_scales = zeros(shape_groups, torch.float16)
        if asymmetric:
            c.v_zeros = zeros(shape_groups, torch.float16)
    if k_precision == "int4":
        c.int4_key = zeros(shape_codes4, torch.uint8)
        c.k_scales = zeros(shape_groups, torch.float16)
        if asymmetric:
            c.k_zeros = zeros(shape_groups, torch.float16)
    elif k_precision == "int8":
        c.int8_key = zeros(shape_codes8, torch.int8)
        c.k_int8_scales = zeros(shape_groups, torch.float16)
    return c


def planner_check(caches: ShadowCaches, num_blocks: int, block_size: int, num_kv_heads: int,
                  head_size: int, **prec) -> tuple[int, int]:
    """(actual bytes per block, planner bytes per block): the reference's S1
    accounting check (F:2432-2478).  The two agree up to the 3-byte INT8-V
    placeholder, which the allocation holds once and the planner counts per
    block."""
    actual = caches.nbytes() // max(num_blocks, 1)
    expected = shadow_bytes_per_block(block_size, num_kv_heads, head_size, **prec)
    return actual, expected
