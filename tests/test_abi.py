"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and rejects bad arguments before any launch."""
import ctypes
import os
import re

import pytest

from knlp_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "knlp_int4kv.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(knlp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    declared = _declared_functions()
    assert declared, "header parse found nothing"
    assert set(declared) == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(L, name), name


def test_abi_version_and_status_strings():
    L = _lib.lib()
    assert L.knlp_abi_version() == _lib.ABI_VERSION
    for st in (0, -1, -2, -3, -4, -5, -6):
        assert L.knlp_status_string(st)
    assert L.knlp_status_string(-99) == b"unknown status"


def test_split_plan_and_workspace():
    L = _lib.lib()
    a4 = _lib.KV_INT4_ASYM
    st = L.knlp_kv_decode_split_tokens(8, 8, 32, 128, 32768, a4, a4)
    assert st > 0 and st % 64 == 0
    assert L.knlp_kv_decode_split_tokens(0, 8, 32, 128, 32768, a4, a4) == _lib.ERR_SHAPE
    ws = L.knlp_kv_decode_workspace_bytes(8, 32, 128, 32768, st)
    ns = -(-32768 // st)
    assert ws == 8 * 32 * ns * (128 + 2) * 4


def test_kernel_kind_rejects_bad_shapes():
    L = _lib.lib()
    assert L.knlp_kv_decode_kernel_kind(32, 7, 128, 1, 32, 1, 32, 0) == _lib.ERR_SHAPE
    assert L.knlp_kv_decode_kernel_kind(32, 8, 96, 1, 32, 1, 32, 0) == _lib.ERR_SHAPE
    assert L.knlp_kv_decode_kernel_kind(32, 8, 128, 1, 32, 1, 32, 0) in (0, 1)


def _plane(fmt=_lib.KV_INT4_ASYM, gs=32, data=0x1000, scales=0x2000, zeros=0x3000):
    p = _lib.KvPlane()
    p.data, p.scales, p.zeros = data, scales, zeros
    p.stride_block, p.stride_page, p.stride_head = 16 * 8 * 64, 8 * 64, 64
    p.s_stride_block, p.s_stride_page, p.s_stride_head = 16 * 8 * 4, 8 * 4, 4
    p.z_stride_block, p.z_stride_page, p.z_stride_head = 16 * 8 * 4, 8 * 4, 4
    p.format, p.group_size = fmt, gs
    return p


def test_append_argument_validation_returns_before_launch():
    L = _lib.lib()
    kp, vp = _plane(), _plane()
    args = dict(key=0x10000, value=0x20000, src=_lib.DT_F16, nt=4, nh=8, d=128)

    def call(**kw):
        a = {**args, **kw}
        return L.knlp_kv_append(a["key"], a["value"], a["src"], a["nt"], a["nh"], a["d"],
                                1024, 128, 1024, 128, ctypes.byref(kw.get("kp", kp)),
                                ctypes.byref(kw.get("vp", vp)), a.get("slots", 0x40000),
                                kw.get("sd", _lib.DT_I64), 16, kw.get("clip", 10.0), None)

    assert call(key=None, value=None) == _lib.ERR_ARG
    assert call(slots=None) == _lib.ERR_ARG
    assert call(src=_lib.DT_I32) == _lib.ERR_DTYPE
    assert call(sd=_lib.DT_F16) == _lib.ERR_DTYPE
    assert call(d=96) == _lib.ERR_SHAPE
    assert call(clip=-1.0) == _lib.ERR_ARG
    assert call(kp=_plane(gs=48)) == _lib.ERR_SHAPE
    assert call(kp=_plane(zeros=None)) == _lib.ERR_ARG
    assert call(kp=_plane(fmt=9)) == _lib.ERR_DTYPE


def test_decode_argument_validation_returns_before_launch():
    L = _lib.lib()
    kp, vp = _plane(), _plane()

    def call(ws=0x100000, ws_bytes=1 << 40, split=256, q=0x10000, d=128, hkv=8):
        return L.knlp_kv_decode(q, _lib.DT_F16, 32 * 128, 128, 8, 32, hkv, d,
                                ctypes.byref(kp), ctypes.byref(vp), 0x50000, 2048, 0x60000,
                                16, 32768, 0.088, split, ws, ws_bytes, 0x70000, _lib.DT_F16,
                                32 * 128, 128, None)

    assert call(q=None) == _lib.ERR_ARG
    assert call(split=100) == _lib.ERR_SHAPE
    assert call(hkv=7) == _lib.ERR_SHAPE
    assert call(ws=None) == _lib.ERR_WORKSPACE
    assert call(ws_bytes=16) == _lib.ERR_WORKSPACE
    assert call(q=0x10002) == _lib.ERR_ALIGN


def test_ops_require_device_tensors():
    import torch
    from knlp_amd import ops
    q = torch.zeros(1, 4, 64, dtype=torch.float16)
    kc = torch.zeros(2, 16, 1, 32, dtype=torch.uint8)
    sc = torch.zeros(2, 16, 1, 2, dtype=torch.float16)
    with pytest.raises(ValueError):
        ops.fused_int4_decode(q, kc, kc, sc, sc, torch.zeros(1, 2, dtype=torch.int32),
                              torch.ones(1, dtype=torch.int32), 1, 64)


def test_fp16_plane_group_size_is_not_read():
    """An fp16 plane has no scales; a group_size of 0 in it must not reach a
    division (it used to end the process with SIGFPE on the dispatch path).
    Without a GPU the call gets as far as the launch and reports that."""
    L = _lib.lib()
    kp = _plane(fmt=_lib.KV_FP16, gs=0, scales=None, zeros=None)
    kp.stride_block, kp.stride_page, kp.stride_head = 16 * 8 * 128, 8 * 128, 128
    for vfmt, vgs in ((_lib.KV_INT4_ASYM, 32), (_lib.KV_INT8_SYM, 32), (_lib.KV_FP16, 0)):
        vp = _plane(fmt=vfmt, gs=vgs) if vfmt != _lib.KV_FP16 else \
            _plane(fmt=_lib.KV_FP16, gs=0, scales=None, zeros=None)
        if vfmt == _lib.KV_FP16:
            vp.stride_block, vp.stride_page, vp.stride_head = 16 * 8 * 128, 8 * 128, 128
        if vfmt == _lib.KV_INT8_SYM:
            vp.stride_block, vp.stride_page, vp.stride_head = 16 * 8 * 128, 8 * 128, 128
        st = L.knlp_kv_decode(0x10000, _lib.DT_F16, 32 * 128, 128, 8, 32, 8, 128,
                              ctypes.byref(kp), ctypes.byref(vp), 0x50000, 2048, 0x60000, 16,
                              32768, 0.088, 1024, 0x100000, 1 << 40, 0x70000, _lib.DT_F16,
                              32 * 128, 128, None)
        assert st in (_lib.OK, _lib.ERR_LAUNCH)
        assert L.knlp_kv_decode_kernel_kind(32, 8, 128, _lib.KV_FP16, 0, vfmt, vgs, 0) in (0, 1)


def test_grid_limits_return_shape_errors():
    """More sequences than a launch grid row holds (65535) is a shape error,
    not a failed launch."""
    L = _lib.lib()
    kp, vp = _plane(), _plane()
    st = L.knlp_kv_decode(0x10000, _lib.DT_F16, 32 * 128, 128, 70000, 32, 8, 128,
                          ctypes.byref(kp), ctypes.byref(vp), 0x50000, 2048, 0x60000, 16,
                          32768, 0.088, 1024, 0x100000, 1 << 40, 0x70000, _lib.DT_F16,
                          32 * 128, 128, None)
    assert st == _lib.ERR_SHAPE
    st = L.knlp_kv_decode_merge(0x100000, 1 << 40, 0x60000, 70000, 32, 128, 32768, 1024,
                                0x70000, _lib.DT_F16, 32 * 128, 128, None)
    assert st == _lib.ERR_SHAPE


def test_decode_plan_uses_group_sizes_and_total_context():
    L = _lib.lib()
    a4, i8 = _lib.KV_INT4_ASYM, _lib.KV_INT8_SYM
    legacy = L.knlp_kv_decode_split_tokens(8, 8, 32, 128, 32768, a4, a4)
    assert legacy > 0                                       # always a split length
    assert L.knlp_kv_decode_plan(8, 8, 32, 128, 32768, 8 * 32768, a4, 32, a4, 32) == legacy
    # the total unknown: the stream schedule for several sequences, a split for one
    assert L.knlp_kv_decode_plan(8, 8, 32, 128, 32768, 0, a4, 32, a4, 32) == 0
    assert L.knlp_kv_decode_plan(1, 8, 32, 128, 32768, 0, a4, 32, a4, 32) > 0
    # a variable-length batch (half the tokens of its rectangle) on the
    # cooperative kernel: the stream schedule (0)
    assert L.knlp_kv_decode_plan(64, 8, 32, 128, 16384, 64 * 8192, a4, 32, a4, 32) == 0
    assert L.knlp_kv_decode_plan(64, 8, 32, 128, 16384, 64 * 16384 * 95 // 100, a4, 32, a4,
                                 32) > 0                   # nearly uniform: split-K
    assert L.knlp_kv_decode_plan(1100, 8, 32, 128, 16384, 1100 * 8192, a4, 32, a4, 32) > 0
    # ... and on kernels without the stream schedule (Hkv % 8 != 0): shorter splits
    var = L.knlp_kv_decode_plan(64, 4, 16, 128, 16384, 64 * 8192, a4, 32, a4, 32)
    full = L.knlp_kv_decode_plan(64, 4, 16, 128, 16384, 0, a4, 32, a4, 32)
    assert 64 <= var < full and var % 64 == 0
    # INT8 V with g64 runs on the VALU kernel (two workgroups per CU): half
    # the split length of the cooperative kernel's plan for the same shape
    coop = L.knlp_kv_decode_plan(8, 8, 32, 128, 32768, 8 * 32768, i8, 128, i8, 128)
    valu = L.knlp_kv_decode_plan(8, 8, 32, 128, 32768, 8 * 32768, i8, 128, i8, 64)
    assert valu < coop
    assert L.knlp_kv_decode_plan(8, 7, 32, 128, 32768, 0, a4, 32, a4, 32) == _lib.ERR_SHAPE


def test_stream_schedule_workspace_and_limits():
    """split_tokens = 0 selects the stream schedule: its workspace is sized by
    the sequence count, not max_context, and more than 1024 sequences is a
    shape error before anything launches."""
    L = _lib.lib()
    ws = L.knlp_kv_decode_workspace_bytes(64, 32, 128, 16384, 0)
    assert ws > 0 and ws == L.knlp_kv_decode_workspace_bytes(64, 32, 128, 1 << 20, 0)
    assert L.knlp_kv_decode_workspace_bytes(1025, 32, 128, 16384, 0) > 0
    assert L.knlp_kv_decode_workspace_bytes(64, 32, 128, 16384, -64) == _lib.ERR_SHAPE
    kp, vp = _plane(), _plane()
    st = L.knlp_kv_decode(0x10000, _lib.DT_F16, 32 * 128, 128, 1025, 32, 8, 128,
                          ctypes.byref(kp), ctypes.byref(vp), 0x50000, 2048, 0x60000, 16,
                          32768, 0.088, 0, 0x100000, 1 << 40, 0x70000, _lib.DT_F16,
                          32 * 128, 128, None)
    assert st == _lib.ERR_SHAPE
    st = L.knlp_kv_decode_merge(0x100000, 1 << 40, 0x60000, 1025, 32, 128, 32768, 0,
                                0x70000, _lib.DT_F16, 32 * 128, 128, None)
    assert st == _lib.ERR_SHAPE
    # too small a workspace for the stream layout
    st = L.knlp_kv_decode_merge(0x100000, ws - 16, 0x60000, 64, 32, 128, 16384, 0,
                                0x70000, _lib.DT_F16, 32 * 128, 128, None)
    assert st == _lib.ERR_WORKSPACE


def test_argument_validation_fuzz_never_crashes():
    """Random, mostly invalid, shapes, formats, group sizes, strides and
    pointers through the host-side validation of the plan, workspace, kernel
    kind and decode entry points.  Decode gets no workspace, so every call
    returns a status before anything could launch (safe on any machine); the
    point is that no combination divides by zero or crashes on the host."""
    import random
    rng = random.Random(1234)
    L = _lib.lib()
    statuses = {0, _lib.ERR_ARG, _lib.ERR_SHAPE, _lib.ERR_DTYPE, _lib.ERR_ALIGN,
                _lib.ERR_WORKSPACE, _lib.ERR_LAUNCH}
    pick = rng.choice
    for _ in range(3000):
        S = pick([-1, 0, 1, 5, 1025, 70000])
        hq, hkv = pick([-1, 0, 1, 5, 12, 32, 40]), pick([-1, 0, 1, 4, 8, 12])
        d = pick([-1, 0, 1, 48, 64, 128, 256, 512])
        kf, vf = pick([-1, 0, 1, 2, 3, 7]), pick([-1, 0, 1, 2, 3, 7])
        kgs, vgs = pick([-5, 0, 1, 3, 16, 32, 64, 128, 256]), pick([-5, 0, 1, 3, 32, 64, 128])
        bs = pick([-1, 0, 1, 15, 16, 17, 32])
        mc = pick([-1, 0, 1, 100, 32768, (1 << 25) + 1])
        split = pick([-64, -1, 0, 1, 63, 64, 1024])
        total = pick([-1, 0, 1, 10 ** 6, 1 << 40])
        r = L.knlp_kv_decode_plan(S, hkv, hq, d, mc, total, kf, kgs, vf, vgs)
        assert r >= 0 or r in statuses
        r = L.knlp_kv_decode_workspace_bytes(S, hq, d, mc, split)
        assert r >= 0 or r in statuses
        r = L.knlp_kv_decode_kernel_kind(hq, hkv, d, kf, kgs, vf, vgs, pick([0, 1, 5]))
        assert r >= 0 or r in statuses
        kp = _plane(kf, kgs, data=pick([0, 0x1000, 0x1001]), scales=pick([0, 0x2000]),
                    zeros=pick([0, 0x3000]))
        vp = _plane(vf, vgs, data=pick([0, 0x4000]), scales=pick([0, 0x5000, 0x5002]),
                    zeros=pick([0, 0x6000]))
        for p in (kp, vp):
            p.stride_head = pick([0, 1, 64, -64, 63])
            p.s_stride_page = pick([0, 4, 3, 1 << 40])
        st = L.knlp_kv_decode(pick([0, 0x10000, 0x10002]), pick([0, 1, 5]),
                              pick([0, 4096, 4095]), pick([0, 128, 127]), S, hq, hkv, d,
                              ctypes.byref(kp), ctypes.byref(vp), pick([0, 0x50000]),
                              pick([0, 64]), pick([0, 0x60000]), bs, mc, pick([0.088, -1.0]),
                              split, None, 0, pick([0, 0x70000]), pick([0, 1]), 4096, 128, None)
        assert st in statuses and (st != 0 or S == 0), (st, S, hq, hkv, d, kf, vf, kgs, vgs)
