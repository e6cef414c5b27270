"""knlp_kv_decode_noalloc (no allocation: the split partials live in the
library's per-GPU static scratch) against knlp_kv_decode with a torch
workspace: bit-identical outputs on two calls in a row, the second with a
smaller input, and a clear error for shapes beyond the scratch."""
import ctypes

import numpy as np
import pytest
import torch

from knlp_amd import _lib, ops
from tests import kvgen

pytestmark = pytest.mark.gpu
DEV = "cuda"
BS = 16


def _noalloc():
    return _lib.lib().knlp_kv_decode_noalloc


def _case(seq_lens, hq, hkv, d, fmt, gs, seed):
    nb = sum(-(-n // BS) for n in seq_lens) + 3
    bt = kvgen.paged_table(seq_lens, BS, nb, 6000 + seed)
    slots = kvgen.token_slots(bt, seq_lens, BS)
    planes = []
    for i in range(2):
        p = kvgen.empty_plane(fmt, nb, BS, hkv, d, gs)
        kvgen.fill_plane(p, kvgen.randn((len(slots), hkv, d), 2000 + seed + i).float().numpy(),
                         slots)
        planes.append(kvgen.plane_to_torch(p, DEV))
    q = kvgen.randn((len(seq_lens), hq, d), 1000 + seed).to(DEV)
    return q, planes, torch.from_numpy(bt).to(DEV), \
        torch.tensor(seq_lens, dtype=torch.int32, device=DEV)


def _both(q, planes, bt, sl, hkv, d, fmt, gs, split):
    L = _lib.lib()
    (kd, ks, kz), (vd, vs, vz) = planes
    kp, vp = ops._plane(kd, ks, kz, fmt, gs), ops._plane(vd, vs, vz, fmt, gs)
    S, hq, _ = q.shape
    max_context = bt.shape[1] * BS
    scale = d ** -0.5
    ref = torch.empty_like(q)
    wsb = L.knlp_kv_decode_workspace_bytes(S, hq, d, max_context, split)
    ws = torch.empty(wsb // 4, dtype=torch.float32, device=DEV)
    st = L.knlp_kv_decode(q.data_ptr(), 0, q.stride(0), q.stride(1), S, hq, hkv, d,
                          ctypes.byref(kp), ctypes.byref(vp), bt.data_ptr(), bt.stride(0),
                          sl.data_ptr(), BS, max_context, scale, split, ws.data_ptr(), wsb,
                          ref.data_ptr(), 0, ref.stride(0), ref.stride(1), ops._stream())
    assert st == 0
    out = torch.full_like(q, float("nan"))
    st = _noalloc()(q.data_ptr(), 0, q.stride(0), q.stride(1), S, hq, hkv, d, ctypes.byref(kp),
                    ctypes.byref(vp), bt.data_ptr(), bt.stride(0), sl.data_ptr(), BS,
                    max_context, scale, split, out.data_ptr(), 0, out.stride(0), out.stride(1),
                    ops._stream())
    assert st == 0
    torch.cuda.synchronize()
    return ref, out


def test_noalloc_matches_workspace_decode_twice():
    # first call: a larger batch; second: fewer sequences and shorter contexts,
    # so the scratch still holds the first call's partials beyond the new shape
    for i, (lens, split) in enumerate((([3000, 1500, 2048, 77], 256), ([900, 33], 128))):
        print(f"noalloc call {i}: seq_lens={lens} split={split}", flush=True)
        q, planes, bt, sl = _case(lens, 32, 8, 128, 1, 32, 90 + i)
        ref, out = _both(q, planes, bt, sl, 8, 128, 1, 32, split)
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16))


def test_noalloc_stream_schedule_twice():
    # split_tokens = 0: the stream schedule's partials and row records in the
    # scratch; the second call has fewer rows, so stale records of the first
    # lie beyond the ones it writes
    for i, lens in enumerate(([3000, 1500, 0, 2048, 77], [900, 33])):
        print(f"noalloc stream call {i}: seq_lens={lens}", flush=True)
        q, planes, bt, sl = _case(lens, 32, 8, 128, 1, 32, 97 + i)
        ref, out = _both(q, planes, bt, sl, 8, 128, 1, 32, 0)
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("fmt,gs", [(3, 128), (2, 128)], ids=["fp16_kv", "int8_kv"])
def test_noalloc_other_planes_twice(fmt, gs):
    # fp16 K and V (the cooperative fp16-K kernel) and INT8 K and V, split and
    # stream, the second call smaller than the first
    for i, (lens, split) in enumerate((([2500, 700, 1900], 512), ([640, 17], 0))):
        print(f"noalloc fmt {fmt} call {i}: seq_lens={lens} split={split}", flush=True)
        q, planes, bt, sl = _case(lens, 32, 8, 128, fmt, gs, 120 + 10 * fmt + i)
        ref, out = _both(q, planes, bt, sl, 8, 128, fmt, gs, split)
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16))


def test_noalloc_on_a_side_stream():
    """The scratch is the copy on the stream's device, looked up through the
    stream (a non-null one here), and the call runs on that stream."""
    q, planes, bt, sl = _case([1800, 500, 64], 32, 8, 128, 1, 32, 99)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    for split in (256, 0):
        print(f"noalloc side-stream call: split={split}", flush=True)
        with torch.cuda.stream(side):
            ref, out = _both(q, planes, bt, sl, 8, 128, 1, 32, split)
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16))


def test_noalloc_rejects_shapes_beyond_the_scratch():
    L = _lib.lib()
    q, planes, bt, sl = _case([64], 32, 8, 128, 1, 32, 95)
    (kd, ks, kz), (vd, vs, vz) = planes
    kp, vp = ops._plane(kd, ks, kz, 1, 32), ops._plane(vd, vs, vz, 1, 32)
    out = torch.empty_like(q)
    # 2^20 tokens at 64-token splits: 16384 splits x 32 heads x 520 B > 16 MiB
    st = _noalloc()(q.data_ptr(), 0, q.stride(0), q.stride(1), 1, 32, 8, 128, ctypes.byref(kp),
                    ctypes.byref(vp), bt.data_ptr(), bt.stride(0), sl.data_ptr(), BS, 1 << 20,
                    0.088, 64, out.data_ptr(), 0, out.stride(0), out.stride(1), ops._stream())
    assert st == _lib.ERR_WORKSPACE
