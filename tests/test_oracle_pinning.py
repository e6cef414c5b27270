"""Pin the CPU oracle against checks that do not reuse its own formulas.

* exact-rational IEEE restatement (tests/exact_fp.py) on random and
  adversarial groups, for every quantiser mode;
* closed-form groups with known codes / scales / zeros;
* brute-force optimality of codes (no other code is strictly closer);
* special values of the rounding helper;
* dequantise-then-SDPA against torch SDPA on exactly representable data,
  context length 1, identical keys, GQA equivalence and block-table
  permutation invariance.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import quant as Q
from oracle import attention as A
from tests import exact_fp as X


def _rand_groups(rng, n, gs, outliers=True):
    x = rng.standard_normal((n, gs)).astype(np.float32)
    if outliers:
        idx = rng.integers(0, gs, n)
        x[np.arange(n), idx] *= np.float32(20.0)
    return x.astype(np.float16).astype(np.float32)   # fp16-representable inputs


def _adversarial_groups(gs):
    gs_list = []
    gs_list.append(np.zeros(gs))                              # all-zero
    gs_list.append(np.full(gs, 1.5))                          # constant
    gs_list.append(np.full(gs, -3.25))
    g = np.zeros(gs); g[0] = 100.0; gs_list.append(g)         # single spike
    gs_list.append(np.linspace(-1, 1, gs))
    g = np.ones(gs); g[3] = 1000.0; gs_list.append(g)         # clip-active
    g = np.arange(gs) % 16 * 0.25 - 2.0; gs_list.append(g)    # exact grid
    g = np.full(gs, 6.1e-5); g[1] = -6.1e-5; gs_list.append(g)  # tiny range
    return np.stack(gs_list).astype(np.float16).astype(np.float32)


def test_round_half_away_special_values():
    t = np.array([0.49999997, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, -0.49999997,
                  0.0, -0.0, 3.4999998, 7.5], dtype=np.float32)
    got = Q.round_half_away(t)
    # 0.49999997 + 0.5 rounds to 1.0 in fp32 -> floor gives 1 (not 0)
    # 3.4999998 + 0.5 is exact in fp32 (3.9999998) -> 3
    want = np.array([1, 1, 2, 3, -1, -2, -3, -1, 0, 0, 3, 8], dtype=np.float32)
    np.testing.assert_array_equal(got, want)
    for v in t:
        assert Q.round_half_away(np.float32(v)) == X.round_half_away_exact(Fraction(float(v)))


@pytest.mark.parametrize("asym,clip", [(True, 0.0), (False, 10.0), (False, 0.0), (False, 3.0)])
@pytest.mark.parametrize("gs", [32, 64])
def test_int4_group_matches_exact_rational(asym, clip, gs):
    rng = np.random.default_rng(1234 + gs)
    x = np.concatenate([_rand_groups(rng, 96, gs), _adversarial_groups(gs)])
    codes, sc, zp = Q.quantize_int4_groups(x, asym, clip)
    for i in range(x.shape[0]):
        vals = [Fraction(float(v)) for v in x[i]]
        c, s, z = X.quantize_int4_group_exact(vals, asym, clip)
        assert list(codes[i]) == c, f"group {i}"
        assert Fraction(float(sc[i])) == s
        if asym:
            assert Fraction(float(zp[i])) == z


def test_int8_group_matches_exact_rational():
    rng = np.random.default_rng(99)
    x = np.concatenate([_rand_groups(rng, 64, 128), _adversarial_groups(128)])
    codes, sc = Q.quantize_int8_groups(x)
    for i in range(x.shape[0]):
        c, s = X.quantize_int8_group_exact([Fraction(float(v)) for v in x[i]])
        assert list(codes[i].astype(int)) == c
        assert Fraction(float(sc[i])) == s


def test_int4_asym_closed_form():
    # group b + c*k, k = 0..15 (twice): scale = 15c/15 = c, zero = b, codes = k
    c, b = np.float32(0.125), np.float32(-1.0)
    k = np.arange(32) % 16
    x = (b + c * k).astype(np.float32)[None]
    codes, sc, zp = Q.quantize_int4_groups(x, True)
    np.testing.assert_array_equal(codes[0], k)
    assert float(sc[0]) == 0.125 and float(zp[0]) == -1.0


def test_int4_sym_closed_form_and_clip():
    # 31 ones and one 100: amax=100, trimmed mean 1 -> clip 10 -> scale 10/7
    x = np.ones((1, 32), np.float32); x[0, 5] = 100.0
    codes, sc, _ = Q.quantize_int4_groups(x, False, 10.0)
    assert codes[0, 5] == 15                   # saturates at +7
    assert (np.delete(codes[0], 5) == 9).all()  # round(0.7) = 1 -> 1 + 8
    assert float(sc[0]) == float(np.float16(np.float32(10.0) / np.float32(7.0)))
    # no clip: scale = 100/7, the ones round to 0 -> code 8
    codes, sc, _ = Q.quantize_int4_groups(x, False, 0.0)
    assert (np.delete(codes[0], 5) == 8).all() and codes[0, 5] == 15


def test_degenerate_groups():
    x = np.full((1, 32), 2.5, np.float32)
    codes, sc, zp = Q.quantize_int4_groups(x, True)
    assert (codes == 0).all()
    assert float(sc[0]) == 0.0                 # 1e-8/15 underflows fp16
    assert float(zp[0]) == 2.5
    deq = A.dequant_int4(Q.pack_nibbles(codes), sc, zp)
    np.testing.assert_array_equal(deq, x)      # exact reconstruction


def test_codes_are_nearest_levels():
    rng = np.random.default_rng(7)
    x = _rand_groups(rng, 200, 32)
    for asym in (True, False):
        codes, _, _ = Q.quantize_int4_groups(x, asym, 0.0)
        # recompute fp32 scale/zero exactly as the quantiser uses them
        if asym:
            mn = x.min(1); sc = np.maximum(x.max(1) - mn, Q.EPS) / np.float32(15)
            lv = mn[:, None, None] + sc[:, None, None] * np.arange(16)[None, None, :]
        else:
            sc = np.maximum(np.abs(x).max(1), Q.EPS) / np.float32(7)
            lv = sc[:, None, None] * (np.arange(16)[None, None, :] - 8)
        err = np.abs(x[:, :, None].astype(np.float64) - lv)
        chosen = np.take_along_axis(err, codes[:, :, None].astype(int), 2)[..., 0]
        assert (chosen <= err.min(2) + 1e-5 * sc[:, None]).all()


def test_pack_nibble_order():
    codes = np.array([[1, 2, 3, 4, 15, 0]], np.uint8)
    packed = Q.pack_nibbles(codes)
    np.testing.assert_array_equal(packed, [[0x21, 0x43, 0x0F]])
    np.testing.assert_array_equal(Q.unpack_nibbles(packed), codes)


def test_reshape_and_cache_slots_and_padding():
    rng = np.random.default_rng(3)
    nt, h, d, bs, nb = 5, 2, 64, 4, 6
    key = rng.standard_normal((nt, h, d)).astype(np.float32)
    val = rng.standard_normal((nt, h, d)).astype(np.float32)
    kc = np.full((nb, bs, h, d // 2), 0xAB, np.uint8)
    vc = kc.copy()
    ks = np.full((nb, bs, h, d // 32), 7.0, np.float16); vs = ks.copy()
    kz = ks.copy(); vz = ks.copy()
    slots = np.array([0, 9, -1, 23, 5])
    Q.reshape_and_cache_int4(key, val, kc, vc, ks, vs, slots, kz, vz, True, 32)
    for t, s in enumerate(slots):
        if s < 0:
            continue
        p, sc, z = Q.quantize_int4_rows(key[t], 32, True)
        np.testing.assert_array_equal(kc[s // bs, s % bs], p)
        np.testing.assert_array_equal(ks[s // bs, s % bs], sc)
        np.testing.assert_array_equal(kz[s // bs, s % bs], z)
    touched = {0, 9, 23, 5}
    for s in range(nb * bs):
        if s not in touched:
            assert (kc[s // bs, s % bs] == 0xAB).all() and (ks[s // bs, s % bs] == 7.0).all()


def _plane_exact(rng, nb, bs, h, d, gs, fmt):
    """Random plane whose dequantised values are exact (power-of-two scales)."""
    if fmt == "int8":
        data = rng.integers(-128, 128, (nb, bs, h, d)).astype(np.int8)
    else:
        data = rng.integers(0, 256, (nb, bs, h, d // 2)).astype(np.uint8)
    sc = (2.0 ** rng.integers(-6, -2, (nb, bs, h, d // gs))).astype(np.float16)
    zp = (rng.integers(-8, 8, (nb, bs, h, d // gs)) * 0.25).astype(np.float16)
    return {"format": fmt, "data": data, "scales": sc, "zeros": zp, "group_size": gs}


@pytest.mark.parametrize("fmt", ["int4_asym", "int4_sym", "int8"])
def test_decode_reference_matches_textbook_sdpa(fmt):
    rng = np.random.default_rng(11)
    nb, bs, hkv, hq, d, gs = 12, 4, 2, 6, 64, 32
    kp = _plane_exact(rng, nb, bs, hkv, d, gs, fmt)
    vp = _plane_exact(rng, nb, bs, hkv, d, gs, "int4_asym")
    bt = rng.permutation(nb).reshape(2, 6).astype(np.int32)
    sl = np.array([21, 3])
    q = rng.standard_normal((2, hq, d)).astype(np.float16).astype(np.float32)
    got = A.decode_reference(q, kp, vp, bt, sl)
    kf, vf = A.dequant_plane(kp), A.dequant_plane(vp)
    for s in range(2):
        k = torch.from_numpy(A.gather_sequence(kf, bt[s], sl[s])).double()
        v = torch.from_numpy(A.gather_sequence(vf, bt[s], sl[s])).double()
        for h in range(hq):
            kh, vh = k[:, h // 3], v[:, h // 3]
            w = torch.softmax(kh @ torch.from_numpy(q[s, h]).double() / 8.0, 0)
            ref = (w @ vh).to(torch.float16).float().numpy()
            np.testing.assert_allclose(got[s, h], ref, atol=1e-3, rtol=0)
    f64 = A.decode_reference_f64(q, kp, vp, bt, sl)
    np.testing.assert_allclose(got, f64, atol=2e-3, rtol=1e-3)


def test_decode_reference_special_cases():
    rng = np.random.default_rng(5)
    nb, bs, hkv, hq, d, gs = 8, 4, 1, 2, 32, 32
    kp = _plane_exact(rng, nb, bs, hkv, d, gs, "int4_asym")
    vp = _plane_exact(rng, nb, bs, hkv, d, gs, "int4_asym")
    bt = np.arange(nb, dtype=np.int32)[None]
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    # context length 1 -> output = dequant(V_0)
    out = A.decode_reference(q, kp, vp, bt, [1])
    v0 = A.dequant_plane(vp)[0, 0, 0]
    np.testing.assert_array_equal(out[0, 0], v0.astype(np.float16).astype(np.float32))
    # identical keys -> uniform softmax -> mean of V
    kp2 = dict(kp); kp2["data"] = np.broadcast_to(kp["data"][:1, :1], kp["data"].shape).copy()
    kp2["scales"] = np.broadcast_to(kp["scales"][:1, :1], kp["scales"].shape).copy()
    kp2["zeros"] = np.broadcast_to(kp["zeros"][:1, :1], kp["zeros"].shape).copy()
    out = A.decode_reference(q, kp2, vp, bt, [13])
    vmean = A.gather_sequence(A.dequant_plane(vp), bt[0], 13).mean(0)[0]
    np.testing.assert_allclose(out[0, 1], vmean, atol=2e-3)
    # block-table permutation invariance
    perm = rng.permutation(nb)
    inv = np.argsort(perm)
    kp3 = {**kp, "data": kp["data"][inv], "scales": kp["scales"][inv], "zeros": kp["zeros"][inv]}
    vp3 = {**vp, "data": vp["data"][inv], "scales": vp["scales"][inv], "zeros": vp["zeros"][inv]}
    a = A.decode_reference(q, kp, vp, bt, [30])
    b = A.decode_reference(q, kp3, vp3, perm[None].astype(np.int32), [30])
    np.testing.assert_array_equal(a, b)
    # seq_len 0 -> NaN like the reference's 0/0
    assert np.isnan(A.decode_reference(q, kp, vp, bt, [0])).all()


def test_symmetric_dequant_closed_form():
    codes = np.arange(32, dtype=np.uint8)[None] % 16
    packed = Q.pack_nibbles(codes)
    sc = np.array([[0.5]], np.float16)
    deq = A.dequant_int4(packed, sc, None, 32)
    np.testing.assert_array_equal(deq[0], (codes[0].astype(np.float32) - 8) * 0.5)


# ---------------------------------------------------------------------------
# Dequantisation pinned from explicit floats.  The caches below are built by
# hand from integer codes and power-of-two scales / quarter-step zeros, so
# every dequantised value is an exact binary fraction that plain Python
# arithmetic computes without rounding; the bytes are packed by an explicit
# per-byte loop (low nibble = element 2i, F:169-170).  The expected values
# and the textbook softmax never go through the oracle's own dequant code.
# References: F:164-193 (asymmetric q*scale + zero, symmetric (q-8)*scale),
# F:1397-1423 (INT8 K: int8 * per-group scale).
# ---------------------------------------------------------------------------

def _hand_int4(rng, rows, d, gs, asym):
    """(packed uint8 [rows, d/2], scales fp16 [rows, ng], zeros fp16 or None,
    expected python floats [rows][d])."""
    ng = d // gs
    codes = [[int(rng.integers(0, 16)) for _ in range(d)] for _ in range(rows)]
    # distinct power-of-two scale per group and quarter-step zero-points, so a
    # scale or zero read from the wrong group changes the value
    sc = [[2.0 ** -int(rng.integers(1, 7)) for _ in range(ng)] for _ in range(rows)]
    zp = [[0.25 * int(rng.integers(-12, 12)) for _ in range(ng)] for _ in range(rows)]
    packed = np.zeros((rows, d // 2), np.uint8)
    for r in range(rows):
        for i in range(d // 2):
            packed[r, i] = codes[r][2 * i] | (codes[r][2 * i + 1] << 4)
    want = []
    for r in range(rows):
        row = []
        for e in range(d):
            g = e // gs
            if asym:
                row.append(codes[r][e] * sc[r][g] + zp[r][g])
            else:
                row.append((codes[r][e] - 8) * sc[r][g])
        want.append(row)
    scales = np.array(sc, np.float16)
    zeros = np.array(zp, np.float16) if asym else None
    return packed, scales, zeros, want


def _hand_int8(rng, rows, d, gs):
    ng = d // gs
    codes = [[int(rng.integers(-128, 128)) for _ in range(d)] for _ in range(rows)]
    sc = [[2.0 ** -int(rng.integers(3, 12)) for _ in range(ng)] for _ in range(rows)]
    want = [[codes[r][e] * sc[r][e // gs] for e in range(d)] for r in range(rows)]
    return np.array(codes, np.int8), np.array(sc, np.float16), want


def _int4_pin_holds(dequant, gs=32, d=128, rows=24) -> bool:
    rng = np.random.default_rng(4242)
    for asym in (True, False):
        packed, scales, zeros, want = _hand_int4(rng, rows, d, gs, asym)
        got = dequant(packed, scales, zeros, gs)
        if got.shape != (rows, d) or got.tolist() != want:
            return False
    return True


def _int8_pin_holds(dequant, gs=32, d=128, rows=24) -> bool:
    rng = np.random.default_rng(4343)
    for g in (gs, d):
        codes, scales, want = _hand_int8(rng, rows, d, g)
        got = dequant(codes, scales, g)
        if got.shape != (rows, d) or got.tolist() != want:
            return False
    return True


@pytest.mark.parametrize("gs,d", [(32, 128), (64, 128), (16, 64), (128, 128)])
def test_dequant_int4_from_explicit_floats(gs, d):
    assert _int4_pin_holds(A.dequant_int4, gs, d)


@pytest.mark.parametrize("gs", [32, 64, 128])
def test_dequant_int8_from_explicit_floats(gs):
    assert _int8_pin_holds(A.dequant_int8, gs)


def test_dequant_pins_reject_planted_mistakes():
    """The two pins above fail for plausible mistakes planted in a copy of
    the oracle's dequantisers (on the CPU): the symmetric -8 offset applied
    in asymmetric mode, the zero added before scaling, a per-element scale
    index, swapped nibble order, and INT8 codes read as unsigned."""
    def asym_minus8(packed, scales, zeros, gs):
        n = Q.unpack_nibbles(packed).astype(np.float32) - 8.0     # offset in both modes
        g = n.reshape(n.shape[0], -1, gs) * scales.astype(np.float32)[..., None]
        if zeros is not None:
            g = g + zeros.astype(np.float32)[..., None]
        return g.reshape(n.shape)

    def zero_before_scale(packed, scales, zeros, gs):
        n = Q.unpack_nibbles(packed).astype(np.float32)
        if zeros is None:
            return A.dequant_int4(packed, scales, None, gs)
        g = n.reshape(n.shape[0], -1, gs)
        return ((g + zeros.astype(np.float32)[..., None])
                * scales.astype(np.float32)[..., None]).reshape(n.shape)

    def per_element_scale(packed, scales, zeros, gs):
        n = Q.unpack_nibbles(packed).astype(np.float32)
        if zeros is None:
            n = n - 8.0
        idx = np.arange(n.shape[-1]) % scales.shape[-1]      # element -> scale, wrong
        out = n * scales.astype(np.float32)[:, idx]
        if zeros is not None:
            out = out + zeros.astype(np.float32)[:, idx]
        return out

    def swapped_nibbles(packed, scales, zeros, gs):
        sw = ((packed >> 4) | (packed << 4)).astype(np.uint8)
        return A.dequant_int4(sw, scales, zeros, gs)

    def int8_unsigned(codes, scales, gs):
        c = np.asarray(codes).view(np.uint8).astype(np.float32)
        g = c.reshape(c.shape[0], -1, gs) * scales.astype(np.float32)[..., None]
        return g.reshape(c.shape)

    def int8_group_off_by_one(codes, scales, gs):
        c = np.asarray(codes, np.int8).astype(np.float32)
        ng = scales.shape[-1]
        idx = np.minimum(np.arange(c.shape[-1]) // gs + 1, ng - 1)
        return c * scales.astype(np.float32)[:, idx]

    assert _int4_pin_holds(A.dequant_int4) and _int8_pin_holds(A.dequant_int8)
    for bad in (asym_minus8, zero_before_scale, per_element_scale, swapped_nibbles):
        assert not _int4_pin_holds(bad), bad.__name__
    for bad in (int8_unsigned, int8_group_off_by_one):
        assert not _int8_pin_holds(bad), bad.__name__


def _textbook_decode(q, rows_k, rows_v, hkv, hq, scale):
    """softmax(q k / sqrt(D)) v in float64 from python-float rows
    [T][Hkv][D]; one (sequence) at a time."""
    import math
    rep = hq // hkv
    out = []
    for h in range(hq):
        kv = h // rep
        sc = [scale * sum(float(q[h][e]) * rows_k[t][kv][e] for e in range(len(q[h])))
              for t in range(len(rows_k))]
        m = max(sc)
        w = [math.exp(s - m) for s in sc]
        tot = sum(w)
        out.append([sum(w[t] * rows_v[t][kv][e] for t in range(len(rows_v))) / tot
                    for e in range(len(q[h]))])
    return np.array(out)


@pytest.mark.parametrize("kfmt,vfmt", [("int4_asym", "int4_asym"), ("int4_sym", "int4_sym"),
                                       ("int8", "int4_asym"), ("int8", "int8")])
def test_decode_reference_from_explicit_floats(kfmt, vfmt):
    """decode_reference over hand-built paged caches equals a float64
    textbook softmax over the explicit floats (gathered through the block
    table by hand), to fp32 accumulation error."""
    rng = np.random.default_rng(77)
    nb, bs, hkv, hq, d, gs = 6, 4, 2, 4, 64, 32
    planes, rows = {}, {}
    for side, fmt in (("k", kfmt), ("v", vfmt)):
        if fmt == "int8":
            codes, sc, want = _hand_int8(rng, nb * bs * hkv, d, gs)
            planes[side] = {"format": "int8", "data": codes.reshape(nb, bs, hkv, d),
                            "scales": sc.reshape(nb, bs, hkv, -1), "zeros": None,
                            "group_size": gs}
        else:
            asym = fmt == "int4_asym"
            packed, sc, zp, want = _hand_int4(rng, nb * bs * hkv, d, gs, asym)
            planes[side] = {"format": fmt, "data": packed.reshape(nb, bs, hkv, d // 2),
                            "scales": sc.reshape(nb, bs, hkv, -1),
                            "zeros": None if zp is None else zp.reshape(nb, bs, hkv, -1),
                            "group_size": gs}
        # python rows indexed [block][offset][head] -> [D] floats
        rows[side] = [[[want[(b * bs + o) * hkv + h] for h in range(hkv)] for o in range(bs)]
                      for b in range(nb)]
    bt = np.array([[4, 1, 5], [2, 0, 3]], np.int32)
    sl = [11, 6]
    q = rng.standard_normal((2, hq, d)).astype(np.float16).astype(np.float32)
    got = A.decode_reference(q, planes["k"], planes["v"], bt, sl, round_output=False)
    got64 = A.decode_reference_f64(q, planes["k"], planes["v"], bt, sl)
    scale = float(np.float32(1.0 / np.sqrt(d)))
    for s in range(2):
        tk = [rows["k"][bt[s][t // bs]][t % bs] for t in range(sl[s])]
        tv = [rows["v"][bt[s][t // bs]][t % bs] for t in range(sl[s])]
        want = _textbook_decode(q[s], tk, tv, hkv, hq, scale)
        np.testing.assert_allclose(got[s], want, atol=2e-5, rtol=2e-5)
        np.testing.assert_allclose(got64[s], want, atol=1e-12, rtol=1e-12)
