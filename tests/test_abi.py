"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and rejects bad arguments before any launch."""
import ctypes
import os
import re

import pytest

from knlp_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "knlp_int4kv.h")


def _gpu_visible() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


# Tests whose calls pass validation with made-up device addresses: without a
# GPU the launch itself fails (KNLP_ERR_LAUNCH); with one it would run a
# kernel on those addresses, so they run only where no GPU is visible.
no_gpu_only = pytest.mark.skipif(_gpu_visible(), reason="passes made-up device addresses "
                                                        "that a visible GPU would launch on")


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


@no_gpu_only
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


def _ws_of_plan(L, S, hkv, hq, d, mc, total, kf, kg, vf, vg):
    sp = L.knlp_kv_decode_plan(S, hkv, hq, d, mc, total, kf, kg, vf, vg)
    assert sp >= 0
    return sp, L.knlp_kv_decode_workspace_bytes(S, hq, d, mc, sp)


def test_ragged_split_plan_keeps_workspace_bounded():
    """A ragged batch that stays on split-K (no stream schedule: Hkv % 8 != 0,
    fp16 K, or more than 1024 sequences) gets splits sized from its real
    tokens, but its workspace is dense over max_context: the plan keeps it
    within about 4x of the uniform plan's (before: 1.9 GB for 256 sequences
    of 500 tokens in a 131072-token table)."""
    L = _lib.lib()
    a4, f16, i8 = _lib.KV_INT4_ASYM, _lib.KV_FP16, _lib.KV_INT8_SYM
    cases = [
        (256, 4, 28, 128, 131072, 256 * 500, a4, 32, a4, 32),       # Hkv % 8 != 0
        (256, 4, 28, 128, 131072, 256 * 100, f16, 128, a4, 32),     # fp16 K
        (1100, 8, 32, 128, 131072, 1100 * 500, a4, 32, a4, 32),     # > 1024 sequences
        (1100, 4, 28, 128, 65536, 1100 * 100, f16, 128, i8, 128),
        (2000, 8, 40, 128, 32768, 2000 * 64, i8, 128, a4, 32),
    ]
    for S, hkv, hq, d, mc, total, kf, kg, vf, vg in cases:
        sp, ws = _ws_of_plan(L, S, hkv, hq, d, mc, total, kf, kg, vf, vg)
        sp_u, ws_u = _ws_of_plan(L, S, hkv, hq, d, mc, S * mc, kf, kg, vf, vg)
        assert sp > 0 and sp_u > 0 and sp % 64 == 0
        # ceil(mc / sp) <= 4 ceil(mc / sp_u) + 4 splits
        assert ws <= 4 * ws_u + 4 * S * hq * (d + 2) * 4, (S, hkv, sp, sp_u, ws, ws_u)
        assert ws < 256 << 20, (S, hkv, ws)
    # uniform batches and ragged batches on the stream schedule are unchanged
    assert L.knlp_kv_decode_plan(8, 8, 32, 128, 32768, 8 * 32768, a4, 32, a4, 32) == 1024
    assert L.knlp_kv_decode_plan(64, 8, 32, 128, 16384, 64 * 8192, a4, 32, a4, 32) == 0
    # ... and a long sequence among short ones still gets short splits
    # relative to the table (not the uniform plan's)
    sp, _ = _ws_of_plan(L, 128, 4, 28, 128, 100000 // 64 * 64, 100000 + 127 * 500, a4, 32, a4,
                        32)
    sp_u, _ = _ws_of_plan(L, 128, 4, 28, 128, 100000 // 64 * 64, 128 * (100000 // 64 * 64),
                          a4, 32, a4, 32)
    assert sp < sp_u


@no_gpu_only
def test_stream_fallback_shape_error_comes_before_any_launch():
    """The stream schedule (split 0) on planes only split-K takes falls back to
    split-K inside the stream workspace.  When that fallback cannot serve the
    shape either (the VALU kernel takes at most 8 query heads per kv head,
    here 16 on a layout the matrix-core kernels do not take), the status is
    a shape error and nothing is launched: the fallback's header kernel,
    which once ran first, now follows the decode launch."""
    L = _lib.lib()
    kp, vp = _plane(gs=128, data=0x1004), _plane(gs=128)
    for p in (kp, vp):
        p.stride_block, p.stride_page, p.stride_head = 16 * 2 * 64, 2 * 64, 64
        p.s_stride_block, p.s_stride_page, p.s_stride_head = 16 * 2, 2, 1
        p.z_stride_block, p.z_stride_page, p.z_stride_head = 16 * 2, 2, 1
    assert L.knlp_kv_decode_kernel_kind(32, 2, 128, _lib.KV_INT4_ASYM, 128, _lib.KV_INT4_ASYM,
                                        128, 0) == 1
    for fn in ("knlp_kv_decode", "knlp_kv_decode_partial"):
        args = [0x10000, _lib.DT_F16, 32 * 128, 128, 2, 32, 2, 128, ctypes.byref(kp),
                ctypes.byref(vp), 0x50000, 2048, 0x60000, 16, 32768, 0.088, 0, 0x100000,
                1 << 40]
        if fn == "knlp_kv_decode":
            args += [0x70000, _lib.DT_F16, 32 * 128, 128]
        st = getattr(L, fn)(*args, None)
        assert st == _lib.ERR_SHAPE, (fn, st)


def test_fused_entry_points_check_the_merge_before_the_partial():
    """knlp_kv_decode and knlp_kv_append_decode validate the merge's own
    arguments (output pointer, dtype, alignment) before the partial launch,
    so a merge error is never returned after a launch."""
    L = _lib.lib()
    kp, vp = _plane(), _plane()

    def dec(out=0x70000, odt=_lib.DT_F16):
        return L.knlp_kv_decode(0x10000, _lib.DT_F16, 32 * 128, 128, 8, 32, 8, 128,
                                ctypes.byref(kp), ctypes.byref(vp), 0x50000, 2048, 0x60000,
                                16, 32768, 0.088, 1024, 0x100000, 1 << 40, out, odt,
                                32 * 128, 128, None)

    def app(out=0x70000, odt=_lib.DT_F16):
        return L.knlp_kv_append_decode(
            0x10000, _lib.DT_F16, 32 * 128, 128, 8, 32, 8, 128, 0x80000, 0x90000,
            _lib.DT_F16, 1024, 128, 1024, 128, 0xA0000, _lib.DT_I64, 0.0, ctypes.byref(kp),
            ctypes.byref(vp), 0x50000, 2048, 0x60000, 16, 32768, 0.088, 1024, 0x100000,
            1 << 40, out, odt, 32 * 128, 128, None)

    for f in (dec, app):
        assert f(out=0x70001) == _lib.ERR_ALIGN
        assert f(out=None) == _lib.ERR_ARG
        assert f(odt=_lib.DT_I32) == _lib.ERR_DTYPE


@no_gpu_only
def test_softmax_scale_of_any_sign_keeps_matrix_core_shapes():
    """Shapes that only the matrix-core kernels serve (two head sets of 16
    query heads per kv head: the VALU kernel takes at most 8) pass
    validation with a negative or zero softmax scale too: the kernels fold a
    negative scale's sign into q and treat 0 as uniform weights.  (Without a
    GPU the call gets as far as the launch.)"""
    L = _lib.lib()
    kp, vp = _plane(gs=64), _plane(gs=64)
    for p in (kp, vp):
        p.s_stride_block, p.s_stride_page, p.s_stride_head = 16 * 8 * 2, 8 * 2, 2
        p.z_stride_block, p.z_stride_page, p.z_stride_head = 16 * 8 * 2, 8 * 2, 2
    assert L.knlp_kv_decode_kernel_kind(128, 8, 128, _lib.KV_INT4_ASYM, 64, _lib.KV_INT4_ASYM,
                                        64, 0) == 1
    for scale in (0.088, -0.088, 0.0):
        st = L.knlp_kv_decode(0x10000, _lib.DT_F16, 128 * 128, 128, 8, 128, 8, 128,
                              ctypes.byref(kp), ctypes.byref(vp), 0x50000, 2048, 0x60000, 16,
                              32768, scale, 1024, 0x100000, 1 << 40, 0x70000, _lib.DT_F16,
                              128 * 128, 128, None)
        assert st in (_lib.OK, _lib.ERR_LAUNCH), (scale, st)
    for bad in (float("inf"), float("nan")):
        st = L.knlp_kv_decode(0x10000, _lib.DT_F16, 128 * 128, 128, 8, 128, 8, 128,
                              ctypes.byref(kp), ctypes.byref(vp), 0x50000, 2048, 0x60000, 16,
                              32768, bad, 1024, 0x100000, 1 << 40, 0x70000, _lib.DT_F16,
                              128 * 128, 128, None)
        assert st == _lib.ERR_ARG


def test_head_size_32_decodes():
    """D = 32 (which the append takes) decodes too, on the VALU kernel."""
    L = _lib.lib()
    a4 = _lib.KV_INT4_ASYM
    assert L.knlp_kv_decode_kernel_kind(8, 8, 32, a4, 32, a4, 32, 0) == 0
    assert L.knlp_kv_decode_kernel_kind(8, 8, 32, a4, 16, a4, 16, 0) == 0
    assert L.knlp_kv_decode_kernel_kind(8, 8, 96, a4, 32, a4, 32, 0) == _lib.ERR_SHAPE
