"""Fused append + decode (knlp_kv_append_decode) against the separate append
launch followed by the decode launch: the caches must come out bit-identical
and so must the decode output, for every kernel family (cooperative MFMA,
per-head MFMA, VALU), head sizes 64/128/256, sequences of length 1, new tokens
on a split boundary and on the first position of a tile, bf16 rows, and
slot < 0 (nothing written), and the stream schedule (split_tokens = 0)."""
import numpy as np
import pytest
import torch

import knlp_amd as K
from knlp_amd import ops
from tests import kvgen

pytestmark = pytest.mark.gpu

BS = 16

CASES = [
    # name, seq_lens (incl. the new token), hq, hkv, d, kfmt, vfmt, kgs, vgs, split, src
    # dtype, kernel kind the shape dispatches to
    ("coop_int4_asym", [1, 33, 1024, 2049], 32, 8, 128, 1, 1, 32, 32, 1024, torch.float16,
     "mfma"),
    ("coop_int4_sym_split_edge", [257, 512, 513], 32, 8, 128, 0, 0, 32, 32, 256, torch.float16,
     "mfma"),
    ("perhead_mfma_hkv4", [700, 65], 16, 4, 128, 1, 1, 32, 32, 256, torch.float16, "mfma"),
    ("mfma_d64", [300, 1], 16, 8, 64, 1, 1, 32, 32, 256, torch.float16, "mfma"),
    ("coop_kint8_row_vint4_two_sets", [900, 17], 40, 8, 128, 2, 1, 128, 32, 256,
     torch.float16, "mfma"),
    ("perhead_kfp16_vint8", [400], 32, 8, 128, 3, 2, 128, 32, 256, torch.float16, "mfma"),
    ("coop_kint8_vint8", [700, 33, 1], 32, 8, 128, 2, 2, 128, 32, 256, torch.float16, "mfma"),
    ("coop_kint4_vint8", [512, 64], 32, 8, 128, 1, 2, 32, 32, 256, torch.float16, "mfma"),
    ("valu_kint8_vint4_hkv4", [300, 48], 16, 4, 128, 2, 1, 128, 32, 256, torch.float16,
     "valu"),
    ("valu_kint8_vint8_hkv4", [300, 48], 16, 4, 128, 2, 2, 32, 32, 256, torch.float16,
     "valu"),
    ("valu_kint8_g64_vint8", [420], 32, 8, 128, 2, 2, 64, 64, 256, torch.float16, "valu"),
    ("valu_d256", [333, 32], 64, 8, 256, 1, 1, 32, 32, 256, torch.float16, "valu"),
    ("bf16_rows_int4", [600, 90], 32, 8, 128, 1, 1, 32, 32, 256, torch.bfloat16, "mfma"),
    # split 0: the stream schedule (a row's last tile can sit in any block)
    ("stream_int4_asym", [1, 33, 1024, 2049, 65], 32, 8, 128, 1, 1, 32, 32, 0, torch.float16,
     "mfma"),
    ("stream_kint8_row_vint4_two_sets", [900, 17, 2], 40, 8, 128, 2, 1, 128, 32, 0,
     torch.float16, "mfma"),
    ("stream_kint8_vint8_d128", [700, 33, 1], 32, 8, 128, 2, 2, 128, 32, 0, torch.float16,
     "mfma"),
]


def _planes(fmts, gss, hkv, d, nb, dev, seed):
    """Caches pre-filled with seeded rows through the oracle, on the device."""
    out = []
    for i, (fmt, gs) in enumerate(zip(fmts, gss)):
        p = kvgen.empty_plane(fmt, nb, BS, hkv, d, gs)
        rows = kvgen.randn((nb * BS, hkv, d), seed + i).float().numpy()
        kvgen.fill_plane(p, rows, np.arange(nb * BS))
        out.append(kvgen.plane_to_torch(p, dev))
    return out


def _clone(t):
    return None if t is None else t.clone()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fused_append_matches_separate_launches(case):
    name, seq_lens, hq, hkv, d, kf, vf, kgs, vgs, split, sdt, kind = case
    dev = torch.device("cuda")
    # the kernel family this case covers (kernel_kind reports the shape's
    # kernel; Hkv % 8 != 0 or INT8 with two different groups fall back to VALU)
    assert K.decode_kernel_kind(hq, hkv, d, kf, kgs, vf, vgs) == kind, name
    if sdt == torch.bfloat16 and 3 in (kf, vf):
        pytest.skip("fp16 caches take fp16 rows")
    nb = sum(-(-n // BS) for n in seq_lens) + 2
    bt = kvgen.paged_table(seq_lens, BS, nb, seed=11)
    (kd, ks, kz), (vd, vs, vz) = _planes((kf, vf), (kgs if kf != 3 else d, vgs if vf != 3 else d),
                                         hkv, d, nb, dev, seed=20)
    S = len(seq_lens)
    q = kvgen.randn((S, hq, d), 30).to(dev)
    newk = kvgen.randn((S, hkv, d), 31, sdt, outlier_frac=0.02).to(dev)
    newv = kvgen.randn((S, hkv, d), 32, sdt, outlier_frac=0.02).to(dev)
    pos = np.array(seq_lens) - 1
    slots = bt[np.arange(S), pos // BS].astype(np.int64) * BS + pos % BS
    if name == "perhead_mfma_hkv4":
        slots[1] = -1                      # this sequence writes nothing
    slots_d = torch.from_numpy(slots).to(dev)
    bt_d = torch.from_numpy(bt).to(dev)
    sl_d = torch.tensor(seq_lens, dtype=torch.int32, device=dev)

    def planes(kd, ks, kz, vd, vs, vz):
        return (ops._plane(kd, ks, kz, kf, kgs if kf != 3 else d),
                ops._plane(vd, vs, vz, vf, vgs if vf != 3 else d))

    # separate: append launch, then decode launch
    a = [_clone(t) for t in (kd, ks, kz, vd, vs, vz)]
    kp, vp = planes(*a)
    ops._append(newk, newv, kp, vp, slots_d, 10.0, BS)
    out_sep = ops._decode(q, kp, vp, BS, bt_d, sl_d, hkv, d, split_tokens=split)
    # fused
    b = [_clone(t) for t in (kd, ks, kz, vd, vs, vz)]
    kp2, vp2 = planes(*b)
    out_fused = ops._decode(q, kp2, vp2, BS, bt_d, sl_d, hkv, d, split_tokens=split,
                            append=(newk, newv, slots_d, 10.0))
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        if x is not None:
            assert torch.equal(x, y), name
    assert torch.equal(out_sep.view(torch.int16), out_fused.view(torch.int16)), name
    if name == "perhead_mfma_hkv4":        # slot < 0: the old row is still there
        blk, off = pos[1] // BS, pos[1] % BS
        assert torch.equal(b[0][bt[1, blk], off], kd[bt[1, blk], off])


def test_append_and_decode_python_api():
    """The keyword API (reference-style tensors) against the two calls a
    reference backend makes: reshape_and_cache_int4 then fused_int4_decode."""
    dev = torch.device("cuda")
    hq, hkv, d = 32, 8, 128
    seq_lens = [513, 40]
    nb = 40
    bt = kvgen.paged_table(seq_lens, BS, nb, seed=3)
    ((kd, ks, kz), (vd, vs, vz)) = _planes((1, 1), (32, 32), hkv, d, nb, dev, seed=40)
    S = 2
    q = kvgen.randn((S, hq, d), 50).to(dev)
    newk = kvgen.randn((S, hkv, d), 51).to(dev)
    newv = kvgen.randn((S, hkv, d), 52).to(dev)
    pos = np.array(seq_lens) - 1
    slots = torch.from_numpy(bt[np.arange(S), pos // BS].astype(np.int64) * BS + pos % BS).to(dev)
    bt_d = torch.from_numpy(bt).to(dev)
    sl = torch.tensor(seq_lens, dtype=torch.int32, device=dev)
    a = [t.clone() for t in (kd, ks, kz, vd, vs, vz)]
    K.reshape_and_cache_int4(newk, newv, a[0], a[3], a[1], a[4], slots, a[2], a[5],
                             asymmetric=True)
    want = K.fused_int4_decode(q, a[0], a[3], a[1], a[4], bt_d, sl, hkv, d, k_zeros=a[2],
                               v_zeros=a[5], asymmetric=True)
    b = [t.clone() for t in (kd, ks, kz, vd, vs, vz)]
    got = K.append_and_decode(q, newk, newv, slots, b[0], b[3], b[1], b[4], bt_d, sl, hkv, d,
                              k_zeros=b[2], v_zeros=b[5], asymmetric=True)
    torch.cuda.synchronize()
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    assert torch.equal(want.view(torch.int16), got.view(torch.int16))
