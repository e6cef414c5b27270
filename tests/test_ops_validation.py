"""Host-side shape guards of the Python ops (CPU; nothing launches).  The C
ABI takes strides only and its kernels index the caches unchecked, as the
reference's Triton kernels do, so ops._check_plane refuses caches, scales
and zero-points too small for the heads and head size of a call."""
import pytest
import torch

from knlp_amd import ops
from knlp_amd._lib import KV_FP16, KV_INT4_ASYM, KV_INT4_SYM, KV_INT8_SYM


def _int4(nb=4, bs=16, h=8, d=128, gs=32, asym=True, sg=None, zg=None):
    c = torch.zeros(nb, bs, h, d // 2, dtype=torch.uint8)
    s = torch.zeros(*(sg or (nb, bs, h, d // gs)), dtype=torch.float16)
    z = torch.zeros(*(zg or (nb, bs, h, d // gs)), dtype=torch.float16) if asym else None
    return ops._plane(c, s, z, KV_INT4_ASYM if asym else KV_INT4_SYM, gs)


def test_matching_planes_pass():
    ops._check_plane(_int4(), "key", 8, 128)
    ops._check_plane(_int4(asym=False), "key", 8, 128)
    ops._check_plane(_int4(), "key", 4, 128)          # a cache may hold more heads
    c8 = torch.zeros(4, 16, 8, 128, dtype=torch.int8)
    ops._check_plane(ops._plane(c8, torch.zeros(4, 16, 8, 1, dtype=torch.float16), None,
                                KV_INT8_SYM, 128), "key", 8, 128)
    c16 = torch.zeros(4, 16, 8, 128, dtype=torch.float16)
    ops._check_plane(ops._plane(c16, None, None, KV_FP16, 128), "value", 8, 128)


@pytest.mark.parametrize("heads,d", [(9, 128), (8, 256)])
def test_cache_too_small_for_the_call(heads, d):
    with pytest.raises(ValueError, match="fewer than"):
        ops._check_plane(_int4(), "key", heads, d)


@pytest.mark.parametrize("kw", [dict(sg=(4, 16, 8, 2)), dict(sg=(3, 16, 8, 4)),
                                dict(sg=(4, 8, 8, 4)), dict(sg=(4, 16, 4, 4)),
                                dict(zg=(4, 16, 8, 1))])
def test_scales_or_zeros_too_small(kw):
    with pytest.raises(ValueError, match="do not cover"):
        ops._check_plane(_int4(**kw), "value", 8, 128)


def test_int8_and_fp16_caches_need_full_rows():
    c8 = torch.zeros(4, 16, 8, 64, dtype=torch.int8)        # half a 128-element row
    p = ops._plane(c8, torch.zeros(4, 16, 8, 1, dtype=torch.float16), None, KV_INT8_SYM, 128)
    with pytest.raises(ValueError, match="fewer than"):
        ops._check_plane(p, "key", 8, 128)
    c16 = torch.zeros(4, 16, 8, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="fewer than"):
        ops._check_plane(ops._plane(c16, None, None, KV_FP16, 128), "key", 8, 128)
