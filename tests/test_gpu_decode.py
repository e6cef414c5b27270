"""GPU parity of split-K decode attention against the oracle's
dequantise-then-SDPA path (scripts/v35_h100_bench.py:376-387; F:656-979,
F:1318-1554 and the precision variants).

Tolerance (tests/tolerance.py): max |gpu - oracle| <= 2e-3 against the
oracle's fp32 result before output rounding, plus half an fp16 ulp of the
GPU's output rounding (2^-11 |oracle|) only where |oracle| > 2; bf16 outputs
carry their two roundings (fp32 -> fp16 -> bf16: (2^-8 + 2^-11) |oracle|).
Every check records its achieved max-abs error.
"""
import os
import zlib

import numpy as np
import pytest
import torch

import knlp_amd as K
from knlp_amd import _lib
from oracle import attention as A
from tests import kvgen, tolerance

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL = tolerance.ATOL


def _build(seq_lens, hq, hkv, d, kfmt, vfmt, kgs, vgs, seed, bs=16, pool=None,
           outliers=0.01, clip=10.0, vsigma=1.0):
    nb = pool or max(sum(-(-int(n) // bs) for n in seq_lens), 1) + 3
    bt = kvgen.paged_table(seq_lens, bs, nb, 6000 + seed)
    slots = kvgen.token_slots(bt, seq_lens, bs)
    nt = len(slots)
    k = kvgen.randn((nt, hkv, d), 2000 + seed, torch.float16, outliers).float().numpy()
    v = kvgen.randn((nt, hkv, d), 3000 + seed, torch.float16, outliers).float().numpy()
    if vsigma != 1.0:
        v = (v * vsigma).astype(np.float16).astype(np.float32)
    kp = kvgen.empty_plane(kfmt, nb, bs, hkv, d, kgs)
    vp = kvgen.empty_plane(vfmt, nb, bs, hkv, d, vgs)
    if nt:
        kvgen.fill_plane(kp, k, slots, clip)
        kvgen.fill_plane(vp, v, slots, clip)
    return bt, kp, vp


def _query(nseq, hq, d, seed, dtype=torch.float16):
    return kvgen.randn((nseq, hq, d), 1000 + seed, dtype)


def _run(query, kp, vp, bt, seq_lens, hkv, d, split_tokens=None):
    kd, ks, kz = kvgen.plane_to_torch(kp, DEV)
    vd, vs, vz = kvgen.plane_to_torch(vp, DEV)
    q = query.to(DEV)
    btd = torch.from_numpy(bt).to(DEV)
    sl = torch.tensor(seq_lens, dtype=torch.int32, device=DEV)
    kf, vf = kp["format"], vp["format"]
    kw = dict(split_tokens=split_tokens)
    if kf.startswith("int4") and vf.startswith("int4"):
        out = K.fused_int4_decode(q, kd, vd, ks, vs, btd, sl, hkv, d, k_zeros=kz, v_zeros=vz,
                                  asymmetric=kf == "int4_asym", group_size=kp["group_size"], **kw)
    elif kf == "int8" and vf.startswith("int4"):
        out = K.kint8_vint4_decode(q, kd, vd, ks, vs, btd, sl, hkv, d, v_zeros=vz,
                                   asymmetric=vf == "int4_asym", k_group_size=kp["group_size"],
                                   v_group_size=vp["group_size"], **kw)
    elif kf == "fp16" and vf.startswith("int4"):
        out = K.kfp16_vint4_decode(q, kd, vd, vs, btd, sl, hkv, d, v_zeros=vz,
                                   asymmetric=vf == "int4_asym", v_group_size=vp["group_size"],
                                   **kw)
    elif kf == "int8" and vf == "int8":
        out = K.kint8_vint8_decode(q, kd, vd, ks, vs, btd, sl, hkv, d,
                                   k_group_size=kp["group_size"], v_group_size=vp["group_size"],
                                   **kw)
    elif kf == "fp16" and vf == "int8":
        out = K.kfp16_vint8_decode(q, kd, vd, vs, btd, sl, hkv, d,
                                   v_group_size=vp["group_size"], **kw)
    elif kf == "fp16" and vf == "fp16":
        out = K.fp16_paged_decode(q, kd, vd, btd, sl, hkv, d, **kw)
    else:                     # pairs without a reference-named function (INT4 K, INT8 V)
        from knlp_amd import ops
        fmt = {"int4_sym": 0, "int4_asym": 1, "int8": 2, "fp16": 3}
        out = ops._decode(q, ops._plane(kd, ks, kz, fmt[kf], kp["group_size"]),
                          ops._plane(vd, vs, vz, fmt[vf], vp["group_size"]), kd.shape[1], btd,
                          sl, hkv, d, **kw)
    torch.cuda.synchronize()
    return out


def _case_name():
    return os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0].split("::")[-1]


def _check(out, query, kp, vp, bt, seq_lens, name=None):
    ref = A.decode_reference(query.float().numpy(), kp, vp, bt, seq_lens, round_output=False)
    got = out.float().cpu().numpy()
    valid = np.array([n > 0 for n in seq_lens])
    err = tolerance.check(name or _case_name(), got[valid], ref[valid],
                          bf16=out.dtype == torch.bfloat16)
    if (~valid).any():
        assert np.isnan(got[~valid]).all()       # 0/0 like the reference
    return err


CASES = [
    # name, seq_lens, hq, hkv, d, kfmt, vfmt, kgs, vgs
    ("cfg1_gpt2_small", [1024], 12, 12, 64, 1, 1, 32, 32),
    ("llama_gqa_asym", [3000, 777], 32, 8, 128, 1, 1, 32, 32),
    ("llama_gqa_sym_clip", [1, 17, 511, 2049], 32, 8, 128, 0, 0, 32, 32),
    ("g64_long", [5000], 32, 8, 128, 1, 1, 64, 64),
    ("kint8_row_vint4_g5", [1500, 64], 40, 8, 128, 2, 1, 128, 32),
    ("kint8_vint4_g32", [900], 32, 8, 128, 2, 1, 32, 32),
    ("kfp16_vint4", [1200], 32, 8, 128, 3, 1, 128, 32),
    ("kint8_vint8", [700], 32, 8, 128, 2, 2, 32, 32),
    ("kfp16_vint8", [650], 32, 8, 128, 3, 2, 128, 32),
    ("fp16_fp16", [2100, 33], 32, 8, 128, 3, 3, 128, 128),
    ("d256_g8", [600], 64, 8, 256, 1, 1, 32, 32),
    ("mha_d128_sym", [300], 8, 8, 128, 0, 0, 32, 32),
    ("g2_d64", [1000], 8, 4, 64, 1, 1, 32, 32),
    ("g1_d256_sym_g64", [333], 4, 4, 256, 0, 0, 64, 64),
    ("d64_hkv8_g2", [1500, 300], 16, 8, 64, 1, 1, 32, 32),
    ("g128_d128_hkv16", [700, 129], 64, 16, 128, 1, 1, 128, 128),
    ("sym_g64_hkv8", [999], 32, 8, 128, 0, 0, 64, 64),
    # head sets (G * groups > 16 rows) and INT8 K on the cooperative kernel,
    # and their fallbacks to the VALU kernel for non-dense layouts (Hkv % 8)
    ("int4_g5_two_sets", [1500, 300, 33], 40, 8, 128, 1, 1, 32, 32),
    ("int4_sym_g8_two_sets", [700], 64, 8, 128, 0, 0, 32, 32),
    ("int4_g10_g64_two_sets", [640], 80, 8, 128, 1, 1, 64, 64),
    ("int4_g5_hkv4_valu", [500], 20, 4, 128, 1, 1, 32, 32),
    ("kint8_row_vint4_g4", [777, 64], 32, 8, 128, 2, 1, 128, 32),
    ("kint8_row_vsym_g5", [1030], 40, 8, 128, 2, 0, 128, 32),
    ("kint8_row_hkv4_valu", [400], 20, 4, 128, 2, 1, 128, 32),
    ("kint8_row_g5_short", [1, 2, 17, 31, 32, 33], 40, 8, 128, 2, 1, 128, 32),
    ("int4_g6_two_sets_short", [1, 16, 47], 48, 8, 128, 0, 0, 32, 32),
    # INT8 V on the cooperative kernel (per-row and g32 V scales)
    ("kint8_row_vint8_g32_two_sets", [1100, 5, 33], 40, 8, 128, 2, 2, 128, 32),
    ("kint8_vint8_row", [640, 17], 32, 8, 128, 2, 2, 128, 128),
    ("kint8_vint8_hkv4_valu", [300], 16, 4, 128, 2, 2, 32, 32),
    # fp16 K with INT4 V on the per-head matrix-core kernel
    ("kfp16_vint4_sym_hkv4", [500, 17], 16, 4, 128, 3, 0, 128, 32),
    ("kfp16_vint4_d64_g2", [300, 1], 16, 8, 64, 3, 1, 64, 32),
    ("kfp16_vint4_row", [800], 32, 8, 128, 3, 1, 128, 128),
    ("kfp16_vint8_row", [700, 3], 32, 8, 128, 3, 2, 128, 128),
    ("kfp16_vint8_hkv4", [450, 33], 16, 4, 128, 3, 2, 128, 32),
    # fp16 K and V on the per-head matrix-core kernel (4 waves per block)
    ("fp16_fp16_hkv4_g5", [900, 47, 1], 20, 4, 128, 3, 3, 128, 128),
    ("fp16_fp16_d64", [700, 16], 16, 8, 64, 3, 3, 64, 64),
    ("fp16_fp16_mha", [333], 6, 6, 128, 3, 3, 128, 128),
    ("fp16_fp16_d256_valu", [400], 32, 8, 256, 3, 3, 256, 256),
    # head size 32 (VALU kernel): one group of 32 or two of 16
    ("d32_g32_asym", [700, 33, 1], 8, 2, 32, 1, 1, 32, 32),
    ("d32_g16_sym_mha", [400], 4, 4, 32, 0, 0, 16, 16),
    ("d32_kint8_vint4", [300, 65], 16, 8, 32, 2, 1, 32, 16),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_decode_matches_oracle(case):
    name, seq_lens, hq, hkv, d, kf, vf, kgs, vgs = case
    seed = zlib.crc32(name.encode()) % 1000
    bt, kp, vp = _build(seq_lens, hq, hkv, d, kf, vf, kgs, vgs, seed)
    q = _query(len(seq_lens), hq, d, seed)
    out = _run(q, kp, vp, bt, seq_lens, hkv, d)
    _check(out, q, kp, vp, bt, seq_lens)


def test_bf16_query_output_rounding():
    seq_lens = [1300, 5]
    bt, kp, vp = _build(seq_lens, 32, 8, 128, 1, 1, 32, 32, 21)
    q = _query(2, 32, 128, 21, torch.bfloat16)
    out = _run(q, kp, vp, bt, seq_lens, 8, 128)
    assert out.dtype == torch.bfloat16
    _check(out, q, kp, vp, bt, seq_lens)


BF16_CASES = [
    # name, seq_lens, hq, hkv, d, kfmt, vfmt, kgs, vgs, q magnitude
    ("coop_asym", [1300, 5, 33], 32, 8, 128, 1, 1, 32, 32, 1.0),
    ("coop_sym_large_q", [700], 32, 8, 128, 0, 0, 32, 32, 3000.0),
    ("coop_small_q", [700], 32, 8, 128, 1, 1, 32, 32, 1e-3),
    ("perhead_hkv4", [900, 17], 16, 4, 128, 1, 1, 32, 32, 1.0),
    ("d64_g2", [500], 16, 8, 64, 1, 1, 32, 32, 1.0),
    ("kint8_two_sets", [1100, 3], 40, 8, 128, 2, 1, 128, 32, 1.0),
    # the cooperative fp16-K loader (4 kv heads per block) and the wide-group
    # layout (INT4 K and V in two groups; INT8 K per row with G = 5)
    ("coop16_fp16_fp16", [900, 17], 32, 8, 128, 3, 3, 128, 128, 1.0),
    ("coop16_kfp16_vint4_g64", [700, 5], 32, 8, 128, 3, 1, 128, 64, 1.0),
    ("coop16_kfp16_vint8_g32", [600], 32, 8, 128, 3, 2, 128, 32, 1.0),
    ("wide_int4_g64", [1300, 33], 32, 8, 128, 1, 1, 64, 64, 1.0),
    ("wide_kint8_row_g5", [900, 40], 40, 8, 128, 2, 1, 128, 32, 1.0),
]


@pytest.mark.parametrize("case", BF16_CASES, ids=[c[0] for c in BF16_CASES])
def test_bf16_query_on_matrix_cores(case):
    """bf16 q on the MFMA kernels: exact conversion to fp16 under a per-head
    power-of-two scale, including q far outside [2^-14, 2^15] before it."""
    name, seq_lens, hq, hkv, d, kf, vf, kgs, vgs, mag = case
    assert K.decode_kernel_kind(hq, hkv, d, kf, kgs, vf, vgs, torch.bfloat16) == "mfma"
    bt, kp, vp = _build(seq_lens, hq, hkv, d, kf, vf, kgs, vgs, 300 + len(name))
    q = (_query(len(seq_lens), hq, d, 300 + len(name), torch.float32) * mag).to(torch.bfloat16)
    out = _run(q, kp, vp, bt, seq_lens, hkv, d)
    assert out.dtype == torch.bfloat16
    # fp32 bar plus the bf16 output rounding (relative 2^-8, half an ulp)
    _check(out, q, kp, vp, bt, seq_lens)


def test_edge_lengths_zero_one_and_boundaries():
    seq_lens = [0, 1, 63, 64, 65, 255, 256, 257]
    bt, kp, vp = _build(seq_lens, 32, 8, 128, 1, 1, 32, 32, 31)
    q = _query(len(seq_lens), 32, 128, 31)
    out = _run(q, kp, vp, bt, seq_lens, 8, 128, split_tokens=64)
    _check(out, q, kp, vp, bt, seq_lens)
    # context length 1 -> output is dequant(V_0) rounded to fp16
    v0 = A.gather_sequence(A.dequant_plane(vp), bt[1], 1)[0]
    want = np.repeat(v0, 4, axis=0).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(out[1].float().cpu().numpy(), want)


@pytest.mark.parametrize("split", [64, 128, 512, 4096])
def test_split_count_invariance(split):
    seq_lens = [4000, 1000, 2500]
    bt, kp, vp = _build(seq_lens, 32, 8, 128, 1, 1, 32, 32, 41)
    q = _query(3, 32, 128, 41)
    out = _run(q, kp, vp, bt, seq_lens, 8, 128, split_tokens=split)
    _check(out, q, kp, vp, bt, seq_lens)


def test_block_table_permutation_invariance():
    seq_lens = [2000]
    bt, kp, vp = _build(seq_lens, 32, 8, 128, 1, 1, 32, 32, 51)
    q = _query(1, 32, 128, 51)
    a = _run(q, kp, vp, bt, seq_lens, 8, 128)
    nb = kp["data"].shape[0]
    perm = np.random.default_rng(5).permutation(nb)
    inv = np.argsort(perm)
    kp2 = {**kp, **{f: kp[f][inv] for f in ("data", "scales", "zeros")}}
    vp2 = {**vp, **{f: vp[f][inv] for f in ("data", "scales", "zeros")}}
    b = _run(q, kp2, vp2, perm[bt].astype(np.int32), seq_lens, 8, 128)
    torch.testing.assert_close(a, b, atol=0, rtol=0)


def test_padded_head_layout_matches_dense():
    """Heads padded apart within a token row take the per-head loader; dense
    rows take the cooperative one.  Both meet the oracle tolerance and agree
    with each other to an fp16 ulp or so (the compiler may contract the two
    instantiations' float expressions differently)."""
    seq_lens = [2000, 77]
    hq, hkv, d = 32, 8, 128
    bt, kp, vp = _build(seq_lens, hq, hkv, d, 1, 1, 32, 32, 81)
    q = _query(2, hq, d, 81)
    dense = _run(q, kp, vp, bt, seq_lens, hkv, d)
    _check(dense, q, kp, vp, bt, seq_lens)

    def padded(t, extra):
        big = torch.zeros(t.shape[:-1] + (t.shape[-1] + extra,), dtype=t.dtype, device=DEV)
        big[..., :t.shape[-1]] = t
        return big[..., :t.shape[-1]]

    kd, ks, kz = (padded(t, e) for t, e in zip(kvgen.plane_to_torch(kp, DEV), (16, 4, 4)))
    vd, vs, vz = (padded(t, e) for t, e in zip(kvgen.plane_to_torch(vp, DEV), (16, 4, 4)))
    assert kd.stride(2) == d // 2 + 16
    out = K.fused_int4_decode(q.to(DEV), kd, vd, ks, vs, torch.from_numpy(bt).to(DEV),
                              torch.tensor(seq_lens, dtype=torch.int32, device=DEV), hkv, d,
                              k_zeros=kz, v_zeros=vz, asymmetric=True, group_size=32)
    torch.cuda.synchronize()
    _check(out, q, kp, vp, bt, seq_lens)
    torch.testing.assert_close(out, dense, atol=2e-4, rtol=2.0 ** -9)


def test_gqa_heads_equal_per_head_runs():
    """A q-group computed together equals each head computed alone (MHA)."""
    seq_lens = [800]
    hq, hkv, d = 32, 8, 128
    bt, kp, vp = _build(seq_lens, hq, hkv, d, 1, 1, 32, 32, 61)
    q = _query(1, hq, d, 61)
    out = _run(q, kp, vp, bt, seq_lens, hkv, d)
    # expand KV to one kv head per q head and rerun as MHA
    rep = hq // hkv
    kp2 = {**kp, **{f: np.repeat(kp[f], rep, axis=2) for f in ("data", "scales", "zeros")}}
    vp2 = {**vp, **{f: np.repeat(vp[f], rep, axis=2) for f in ("data", "scales", "zeros")}}
    out2 = _run(q, kp2, vp2, bt, seq_lens, hq, d)
    err = (out.float() - out2.float()).abs().max().item()
    assert err <= 2e-3


def test_deterministic_repeat():
    seq_lens = [3333, 1234]
    bt, kp, vp = _build(seq_lens, 32, 8, 128, 1, 1, 32, 32, 71)
    q = _query(2, 32, 128, 71)
    a = _run(q, kp, vp, bt, seq_lens, 8, 128)
    b = _run(q, kp, vp, bt, seq_lens, 8, 128)
    torch.testing.assert_close(a, b, atol=0, rtol=0)


def test_empty_batch_is_noop():
    kd = torch.zeros(2, 16, 8, 64, dtype=torch.uint8, device=DEV)
    ks = torch.zeros(2, 16, 8, 4, dtype=torch.float16, device=DEV)
    q = torch.zeros(0, 32, 128, dtype=torch.float16, device=DEV)
    out = K.fused_int4_decode(q, kd, kd, ks, ks, torch.zeros(0, 2, dtype=torch.int32, device=DEV),
                              torch.zeros(0, dtype=torch.int32, device=DEV), 8, 128,
                              k_zeros=ks, v_zeros=ks, asymmetric=True)
    assert out.shape == (0, 32, 128)


def test_kernel_kind_dispatch():
    """The benchmark shapes take the matrix-core kernel; others the VALU one."""
    kk = K.decode_kernel_kind
    assert kk(32, 8, 128, _lib.KV_INT4_ASYM, 32, _lib.KV_INT4_ASYM, 32) == "mfma"
    assert kk(32, 8, 128, _lib.KV_INT4_SYM, 64, _lib.KV_INT4_SYM, 64) == "mfma"
    assert kk(12, 12, 64, _lib.KV_INT4_ASYM, 32, _lib.KV_INT4_ASYM, 32) == "mfma"
    assert kk(32, 8, 128, _lib.KV_INT4_ASYM, 32, _lib.KV_INT4_ASYM, 32,
              torch.bfloat16) == "mfma"
    assert kk(64, 8, 256, _lib.KV_INT4_ASYM, 32, _lib.KV_INT4_ASYM, 32) == "valu"
    # INT8 K (per-row or V's groups) with INT4 V, and up to two 16-row head
    # sets, take the matrix cores when the caches are densely laid out
    assert kk(40, 8, 128, _lib.KV_INT8_SYM, 128, _lib.KV_INT4_ASYM, 32) == "mfma"
    assert kk(32, 8, 128, _lib.KV_INT8_SYM, 32, _lib.KV_INT4_ASYM, 32) == "mfma"
    assert kk(64, 8, 128, _lib.KV_INT4_ASYM, 32, _lib.KV_INT4_ASYM, 32) == "mfma"
    with pytest.raises(ValueError):        # 9 heads x 4 groups: neither kernel
        kk(72, 8, 128, _lib.KV_INT4_ASYM, 32, _lib.KV_INT4_ASYM, 32)
    assert kk(32, 8, 128, _lib.KV_INT8_SYM, 64, _lib.KV_INT4_ASYM, 32) == "valu"
    assert kk(32, 8, 64, _lib.KV_INT8_SYM, 64, _lib.KV_INT4_ASYM, 32) == "valu"
    assert kk(32, 8, 128, _lib.KV_INT8_SYM, 128, _lib.KV_INT8_SYM, 32) == "mfma"
    assert kk(32, 8, 64, _lib.KV_INT8_SYM, 64, _lib.KV_INT8_SYM, 32) == "valu"
    assert kk(32, 8, 128, _lib.KV_FP16, 128, _lib.KV_INT4_ASYM, 32) == "mfma"
    assert kk(32, 8, 128, _lib.KV_FP16, 128, _lib.KV_INT8_SYM, 32) == "mfma"
    # fp16 K and V: the matrix-core kernel (the like-for-like fp16 comparison)
    assert kk(32, 8, 128, _lib.KV_FP16, 128, _lib.KV_FP16, 128) == "mfma"
    assert kk(16, 4, 64, _lib.KV_FP16, 0, _lib.KV_FP16, 0) == "mfma"
    assert kk(64, 8, 256, _lib.KV_FP16, 256, _lib.KV_FP16, 256) == "valu"
    # shapes that exist only on the cooperative kernel fall back to VALU when
    # the kv heads do not come in groups of 8
    assert kk(20, 4, 128, _lib.KV_INT4_ASYM, 32, _lib.KV_INT4_ASYM, 32) == "valu"
    assert kk(20, 4, 128, _lib.KV_INT8_SYM, 128, _lib.KV_INT4_ASYM, 32) == "valu"
    assert kk(16, 4, 128, _lib.KV_INT8_SYM, 32, _lib.KV_INT8_SYM, 32) == "valu"
    assert kk(16, 4, 128, _lib.KV_FP16, 128, _lib.KV_INT8_SYM, 32) == "mfma"
    # fp16 planes: the group size field is not read
    assert kk(32, 8, 128, _lib.KV_FP16, 0, _lib.KV_INT4_ASYM, 32) == "mfma"


@pytest.mark.parametrize("kfmt,vfmt,hkv,hq", [(0, 1, 8, 32), (1, 0, 8, 40), (0, 1, 4, 16),
                                              (1, 0, 4, 16), (1, 2, 8, 32), (0, 2, 8, 40)],
                         ids=["ksym_vasym_coop", "kasym_vsym_coop_two_sets", "ksym_vasym_perhead",
                              "kasym_vsym_perhead", "kint4_vint8_coop", "kint4sym_vint8_two_sets"])
def test_mixed_int4_formats_through_the_abi(kfmt, vfmt, hkv, hq):
    """K and V planes with different INT4 encodings (the reference's Python
    API ties them to one flag; the C ABI takes one format per plane)."""
    from knlp_amd import ops
    seq_lens = [700, 33, 1]
    bt, kp, vp = _build(seq_lens, hq, hkv, 128, kfmt, vfmt, 32, 32, 77)
    q = _query(len(seq_lens), hq, 128, 77)
    kd, ks, kz = kvgen.plane_to_torch(kp, DEV)
    vd, vs, vz = kvgen.plane_to_torch(vp, DEV)
    out = ops._decode(q.to(DEV), ops._plane(kd, ks, kz, kfmt, 32), ops._plane(vd, vs, vz, vfmt, 32),
                      16, torch.from_numpy(bt).to(DEV),
                      torch.tensor(seq_lens, dtype=torch.int32, device=DEV), hkv, 128)
    torch.cuda.synchronize()
    _check(out, q, kp, vp, bt, seq_lens)


SMALL_V_CASES = [
    # name, seq_lens, hq, hkv, kfmt, vfmt, kgs, vgs
    ("coop_kint8_vint8_row", [640, 17], 32, 8, 2, 2, 128, 128),
    ("coop_kint8_vint8_g32", [700, 33], 32, 8, 2, 2, 128, 32),
    ("coop_kint4_vint8_g32", [500, 1], 32, 8, 1, 2, 32, 32),
    ("coop_int4_asym", [900, 40], 32, 8, 1, 1, 32, 32),
    ("coop_int4_sym", [900, 40], 32, 8, 0, 0, 32, 32),
    ("coop_kint8_row_vint4_g5", [700, 3], 40, 8, 2, 1, 128, 32),
    ("perhead_int4_asym_hkv4", [800, 65], 16, 4, 1, 1, 32, 32),
    ("perhead_int4_sym_hkv4", [800, 65], 16, 4, 0, 0, 32, 32),
    ("perhead_kfp16_vint8_hkv4", [600, 17], 16, 4, 3, 2, 128, 32),
    ("perhead_kfp16_vint8_row", [600, 17], 32, 8, 3, 2, 128, 128),
    ("perhead_fp16_fp16", [600, 17], 32, 8, 3, 3, 128, 128),
]


@pytest.mark.parametrize("sigma", [1e-2, 1e-3, 1e-4])
@pytest.mark.parametrize("case", SMALL_V_CASES, ids=[c[0] for c in SMALL_V_CASES])
def test_small_magnitude_v_keeps_relative_accuracy(case, sigma):
    """V of small magnitude (N(0, sigma^2), sigma down to 1e-4, so V scales
    down to ~1e-6): the output must keep the accuracy it has at sigma = 1,
    relative to its own scale.  Checked as out / sigma against oracle / sigma
    with the usual bar (the decode is linear in V).  Before P' carried a
    power-of-two factor, fp16's absolute floor in the P' = p * s_v split cost
    up to 12 % of the output at sigma = 1e-3 with INT8 V."""
    name, seq_lens, hq, hkv, kf, vf, kgs, vgs = case
    d = 128
    seed = zlib.crc32(name.encode()) % 1000
    bt, kp, vp = _build(seq_lens, hq, hkv, d, kf, vf, kgs, vgs, seed, vsigma=sigma)
    q = _query(len(seq_lens), hq, d, seed)
    out = _run(q, kp, vp, bt, seq_lens, hkv, d)
    ref = A.decode_reference(q.float().numpy(), kp, vp, bt, seq_lens, round_output=False)
    tolerance.check(f"small_v[{name}-{sigma:g}]", out.float().cpu().numpy() / sigma, ref / sigma)


@pytest.mark.parametrize("max_ctx", [2048, 1000], ids=["pages_of_16", "one_page_per_sequence"])
def test_decode_fp16_sdpa_matches_reference_sdpa(max_ctx):
    """decode_fp16_sdpa (F:2031-2071) on per-sequence fp16 K/V against the
    reference's own algorithm restated in fp32 on the CPU: per sequence, K/V
    expanded over the GQA group (repeat_interleave), softmax(q K^T / sqrt(D)) V."""
    hq, hkv, d = 32, 8, 128
    seq_lens = [min(1000, max_ctx), 1, 517]
    ms = 4
    k = kvgen.randn((ms, max_ctx, hkv, d), 81, outlier_frac=0.01)
    v = kvgen.randn((ms, max_ctx, hkv, d), 82, outlier_frac=0.01)
    q = kvgen.randn((len(seq_lens), hq, d), 83)
    out = K.decode_fp16_sdpa(q.to(DEV), k.to(DEV), v.to(DEV),
                             torch.tensor(seq_lens, dtype=torch.int32, device=DEV), hkv, hq, d)
    torch.cuda.synchronize()
    ref = []
    for s, n in enumerate(seq_lens):
        kk = k[s, :n].float().repeat_interleave(hq // hkv, dim=1).transpose(0, 1)   # [H, n, D]
        vv = v[s, :n].float().repeat_interleave(hq // hkv, dim=1).transpose(0, 1)
        p = torch.softmax((q[s].float()[:, None, :] @ kk.transpose(1, 2)) * d ** -0.5, dim=-1)
        ref.append((p @ vv)[:, 0, :])
    ref = torch.stack(ref).numpy()
    tolerance.check(f"decode_fp16_sdpa_{max_ctx}", out.float().cpu().numpy(), ref)


SCALE_CASES = [
    # name, seq_lens, hq, hkv, d, kfmt, vfmt, kgs, vgs, split (None: the plan)
    ("coop_split", [1500, 300], 32, 8, 128, 1, 1, 32, 32, 256),
    ("coop_stream", [1500, 300, 77], 32, 8, 128, 1, 1, 32, 32, 0),
    ("coop_two_sets", [700, 33], 40, 8, 128, 1, 1, 32, 32, None),
    ("coop_g16_g64_two_sets", [600], 128, 8, 128, 1, 1, 64, 64, None),
    ("coop_kint8", [900, 5], 40, 8, 128, 2, 1, 128, 32, None),
    ("perhead_hkv4", [900, 17], 16, 4, 128, 1, 1, 32, 32, None),
    ("perhead_kfp16", [500], 32, 8, 128, 3, 1, 128, 32, None),
]


@pytest.mark.parametrize("scale", [-0.125, 0.0], ids=["negative", "zero"])
@pytest.mark.parametrize("case", SCALE_CASES, ids=[c[0] for c in SCALE_CASES])
def test_softmax_scale_any_sign_on_matrix_cores(case, scale):
    """A negative softmax scale enters the matrix-core kernels as -q with
    |scale|; a zero scale as q = 0, every token weighted alike.  Negative:
    against the oracle at that scale.  Zero: against the closed form, the
    mean of the dequantised V rows of each sequence."""
    from knlp_amd import ops
    name, seq_lens, hq, hkv, d, kf, vf, kgs, vgs, split = case
    assert K.decode_kernel_kind(hq, hkv, d, kf, kgs, vf, vgs) == "mfma"
    seed = zlib.crc32(name.encode()) % 1000
    bt, kp, vp = _build(seq_lens, hq, hkv, d, kf, vf, kgs, vgs, seed)
    q = _query(len(seq_lens), hq, d, seed)
    fmt = {"int4_sym": 0, "int4_asym": 1, "int8": 2, "fp16": 3}
    kd, ks, kz = kvgen.plane_to_torch(kp, DEV)
    vd, vs, vz = kvgen.plane_to_torch(vp, DEV)
    print(f"scale case {name} scale={scale} split={split}", flush=True)
    out = ops._decode(q.to(DEV), ops._plane(kd, ks, kz, fmt[kp["format"]], kp["group_size"]),
                      ops._plane(vd, vs, vz, fmt[vp["format"]], vp["group_size"]), kd.shape[1],
                      torch.from_numpy(bt).to(DEV),
                      torch.tensor(seq_lens, dtype=torch.int32, device=DEV), hkv, d,
                      scale=scale, split_tokens=split)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    if scale != 0.0:
        ref = A.decode_reference(q.float().numpy(), kp, vp, bt, seq_lens, scale=scale,
                                 round_output=False)
    else:
        deq = A.dequant_plane(vp)
        ref = np.stack([np.repeat(A.gather_sequence(deq, bt[s], n).astype(np.float64).mean(0),
                                  hq // hkv, axis=0) for s, n in enumerate(seq_lens)])
    tolerance.check(f"scale_{name}_{scale:g}", got, ref)
