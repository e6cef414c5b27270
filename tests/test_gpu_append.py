"""GPU parity of quantize-on-append: bit-exact codes, scales and zero-points
against the CPU oracle, padding slots untouched (F:210-472, F:481-647,
F:1231-1312, F:1563-1650)."""
import numpy as np
import pytest
import torch

import knlp_amd as K
from oracle import quant as Q
from tests import kvgen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(num_tokens, hkv, d, seed, dtype=torch.float16, outliers=0.01):
    k = kvgen.randn((num_tokens, hkv, d), 2000 + seed, dtype, outliers)
    v = kvgen.randn((num_tokens, hkv, d), 3000 + seed, dtype, outliers)
    return k, v


def _slots(num_tokens, num_blocks, bs, seed, pad_every=7):
    g = torch.Generator().manual_seed(6000 + seed)
    slots = torch.randperm(num_blocks * bs, generator=g)[:num_tokens].to(torch.int64)
    slots[::pad_every] = -1                       # padding tokens are skipped
    return slots


def _sentinel_caches(nb, bs, hkv, d, gs, asym, fill=0xA5):
    kc = torch.full((nb, bs, hkv, d // 2), fill, dtype=torch.uint8)
    ks = torch.full((nb, bs, hkv, d // gs), 3.0, dtype=torch.float16)
    kz = torch.full_like(ks, -7.0) if asym else None
    return kc, ks, kz


@pytest.mark.parametrize("d,gs", [(128, 32), (128, 64), (64, 32), (256, 32), (128, 128), (32, 16)])
@pytest.mark.parametrize("asym,clip", [(True, 10.0), (False, 10.0), (False, 0.0)])
def test_int4_append_bit_exact(d, gs, asym, clip):
    nt, hkv, nb, bs = 203, 8, 64, 16
    k, v = _case(nt, hkv, d, d + gs)
    slots = _slots(nt, nb, bs, d + gs)
    kc, ks, kz = _sentinel_caches(nb, bs, hkv, d, gs, asym)
    vc, vs, vz = _sentinel_caches(nb, bs, hkv, d, gs, asym)
    ref = [t.numpy().copy() if t is not None else None for t in (kc, vc, ks, vs, kz, vz)]
    Q.reshape_and_cache_int4(k.float().numpy(), v.float().numpy(), *ref[:4], slots.numpy(),
                             ref[4], ref[5], asymmetric=asym, group_size=gs, clip_ratio=clip)
    g = [t.to(DEV) if t is not None else None for t in (kc, vc, ks, vs, kz, vz)]
    K.reshape_and_cache_int4(k.to(DEV), v.to(DEV), g[0], g[1], g[2], g[3], slots.to(DEV),
                             g[4], g[5], asymmetric=asym, group_size=gs, clip_ratio=clip)
    torch.cuda.synchronize()
    for got, want, name in zip(g, ref, ("kc", "vc", "ks", "vs", "kz", "vz")):
        if want is None:
            continue
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint8),
                                      want.view(np.uint8), err_msg=name)


def test_int4_append_bf16_and_int32_slots():
    nt, hkv, d, gs, nb, bs = 77, 4, 128, 32, 16, 16
    k, v = _case(nt, hkv, d, 5, torch.bfloat16)
    slots = _slots(nt, nb, bs, 5).to(torch.int32)
    kc, ks, kz = _sentinel_caches(nb, bs, hkv, d, gs, True)
    vc, vs, vz = _sentinel_caches(nb, bs, hkv, d, gs, True)
    ref = [t.numpy().copy() for t in (kc, vc, ks, vs, kz, vz)]
    Q.reshape_and_cache_int4(k.float().numpy(), v.float().numpy(), *ref[:4], slots.numpy(),
                             ref[4], ref[5], asymmetric=True, group_size=gs)
    g = [t.to(DEV) for t in (kc, vc, ks, vs, kz, vz)]
    K.reshape_and_cache_int4(k.to(DEV), v.to(DEV), g[0], g[1], g[2], g[3], slots.to(DEV),
                             g[4], g[5], asymmetric=True, group_size=gs)
    torch.cuda.synchronize()
    for got, want in zip(g, ref):
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint8), want.view(np.uint8))


def test_v_only_int4_leaves_key_alone():
    nt, hkv, d, gs, nb, bs = 50, 8, 128, 32, 8, 16
    _, v = _case(nt, hkv, d, 9)
    slots = _slots(nt, nb, bs, 9)
    vc, vs, vz = _sentinel_caches(nb, bs, hkv, d, gs, True)
    ref = [t.numpy().copy() for t in (vc, vs, vz)]
    Q.reshape_and_cache_int4(None, v.float().numpy(), None, ref[0], None, ref[1], slots.numpy(),
                             None, ref[2], asymmetric=True, group_size=gs)
    g = [t.to(DEV) for t in (vc, vs, vz)]
    K.reshape_and_cache_v_only_int4(v.to(DEV), g[0], g[1], slots.to(DEV), g[2], asymmetric=True,
                                    group_size=gs)
    torch.cuda.synchronize()
    for got, want in zip(g, ref):
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint8), want.view(np.uint8))


@pytest.mark.parametrize("gs", [32, 128])
@pytest.mark.parametrize("plane", ["k", "v"])
def test_int8_append_bit_exact(gs, plane):
    nt, hkv, d, nb, bs = 99, 8, 128, 16, 16
    k, v = _case(nt, hkv, d, gs)
    src = k if plane == "k" else v
    slots = _slots(nt, nb, bs, gs)
    cache = torch.full((nb, bs, hkv, d), 0x5A, dtype=torch.int8)
    sc = torch.full((nb, bs, hkv, d // gs), 3.0, dtype=torch.float16)
    rc, rs = cache.numpy().copy(), sc.numpy().copy()
    Q.reshape_and_cache_k_int8(src.float().numpy(), rc, rs, slots.numpy(), group_size=gs)
    gc, gsc = cache.to(DEV), sc.to(DEV)
    if plane == "k":
        K.reshape_and_cache_k_int8(src.to(DEV), gc, gsc, slots.to(DEV), group_size=gs)
    else:
        K.reshape_and_cache_v_int8(src.to(DEV), gc, gsc, slots.to(DEV), group_size=gs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(gc.cpu().numpy(), rc)
    np.testing.assert_array_equal(gsc.cpu().numpy().view(np.uint16), rs.view(np.uint16))


def test_adversarial_groups_bit_exact():
    """Constant, all-zero, spike, tie-heavy and tiny-range rows."""
    hkv, d, gs, nb, bs = 1, 128, 32, 4, 16
    rows = []
    rows.append(np.zeros(d)); rows.append(np.full(d, 1.5)); rows.append(np.full(d, -3.25))
    r = np.zeros(d); r[0] = 100.0; rows.append(r)
    r = np.ones(d); r[3] = 1000.0; rows.append(r)
    rows.append((np.arange(d) % 16) * 0.25 - 2.0)
    rows.append(np.arange(d) * 0.5 - 10)           # many exact .5 ties
    r = np.full(d, 6.1e-5); r[1] = -6.1e-5; rows.append(r)
    x = torch.tensor(np.stack(rows)[:, None, :], dtype=torch.float16)
    nt = x.shape[0]
    slots = torch.arange(nt, dtype=torch.int64)
    for asym, clip in ((True, 0.0), (False, 10.0), (False, 0.0)):
        kc, ks, kz = _sentinel_caches(nb, bs, hkv, d, gs, asym)
        ref = [t.numpy().copy() if t is not None else None for t in (kc, ks, kz)]
        Q.reshape_and_cache_int4(x.float().numpy(), x.float().numpy(), ref[0], ref[0].copy(),
                                 ref[1], ref[1].copy(), slots.numpy(), ref[2],
                                 None if ref[2] is None else ref[2].copy(),
                                 asymmetric=asym, group_size=gs, clip_ratio=clip)
        g = [t.to(DEV) if t is not None else None for t in (kc, ks, kz)]
        vc, vs, vz = [t.clone() if t is not None else None for t in g]
        K.reshape_and_cache_int4(x.to(DEV), x.to(DEV), g[0], vc, g[1], vs, slots.to(DEV),
                                 g[2], vz, asymmetric=asym, group_size=gs, clip_ratio=clip)
        torch.cuda.synchronize()
        for got, want in zip(g, ref):
            if want is not None:
                np.testing.assert_array_equal(got.cpu().numpy().view(np.uint8), want.view(np.uint8))


def test_empty_append_is_noop():
    kc, ks, kz = _sentinel_caches(2, 16, 1, 128, 32, True)
    g = [t.to(DEV) for t in (kc, ks, kz)]
    e = torch.zeros(0, 1, 128, dtype=torch.float16, device=DEV)
    K.reshape_and_cache_int4(e, e, g[0], g[0].clone(), g[1], g[1].clone(),
                             torch.zeros(0, dtype=torch.int64, device=DEV), g[2], g[2].clone(),
                             asymmetric=True)
    torch.cuda.synchronize()
    assert (g[0].cpu() == 0xA5).all()


def _qkv_views(nt, hq, hkv, d, seed, dtype=torch.float16):
    """key / value as the reference's callers pass them: [T, H, D] views into
    one fused qkv projection, token stride (hq + 2 hkv) d (F:213-214)."""
    qkv = kvgen.randn((nt, (hq + 2 * hkv) * d), seed, dtype, 0.0).to(DEV)
    k = qkv[:, hq * d:(hq + hkv) * d].view(nt, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(nt, hkv, d)
    assert not k.is_contiguous() and k.stride() == ((hq + 2 * hkv) * d, d, 1)
    return k, v


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_append_from_qkv_views_bit_exact(dtype):
    nt, hq, hkv, d, gs, nb, bs = 61, 32, 8, 128, 32, 8, 16
    k, v = _qkv_views(nt, hq, hkv, d, 41, dtype)
    slots = _slots(nt, nb, bs, 41)
    kc, ks, kz = _sentinel_caches(nb, bs, hkv, d, gs, True)
    vc, vs, vz = _sentinel_caches(nb, bs, hkv, d, gs, True)
    ref = [t.numpy().copy() for t in (kc, vc, ks, vs, kz, vz)]
    Q.reshape_and_cache_int4(k.float().cpu().numpy(), v.float().cpu().numpy(), *ref[:4],
                             slots.numpy(), ref[4], ref[5], asymmetric=True, group_size=gs)
    g = [t.to(DEV) for t in (kc, vc, ks, vs, kz, vz)]
    K.reshape_and_cache_int4(k, v, g[0], g[1], g[2], g[3], slots.to(DEV),
                             g[4], g[5], asymmetric=True, group_size=gs)
    # INT8 K from the same strided view
    c8 = torch.full((nb, bs, hkv, d), 0x5A, dtype=torch.int8)
    s8 = torch.full((nb, bs, hkv, 1), 3.0, dtype=torch.float16)
    r8, rs8 = c8.numpy().copy(), s8.numpy().copy()
    Q.reshape_and_cache_k_int8(k.float().cpu().numpy(), r8, rs8, slots.numpy(), group_size=d)
    g8, gs8 = c8.to(DEV), s8.to(DEV)
    K.reshape_and_cache_k_int8(k, g8, gs8, slots.to(DEV), group_size=d)
    torch.cuda.synchronize()
    for got, want in zip(g, ref):
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint8), want.view(np.uint8))
    np.testing.assert_array_equal(g8.cpu().numpy(), r8)
    np.testing.assert_array_equal(gs8.cpu().numpy().view(np.uint16), rs8.view(np.uint16))


def test_fused_append_from_qkv_views_matches_separate_append():
    """append_and_decode with the new token's K/V as strided qkv views writes
    the same codes as the separate append of contiguous copies."""
    from knlp_amd import ops
    hq, hkv, d, gs, bs = 32, 8, 128, 32, 16
    lens = [300, 45]
    nb = sum(-(-n // bs) for n in lens) + 2
    bt = torch.from_numpy(kvgen.paged_table(lens, bs, nb, 77)).to(DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    slots = torch.tensor([int(bt[s, (n - 1) // bs]) * bs + (n - 1) % bs
                          for s, n in enumerate(lens)], dtype=torch.int64, device=DEV)
    k, v = _qkv_views(2, hq, hkv, d, 43)
    q = kvgen.randn((2, hq, d), 44).to(DEV)
    caches = []
    for _ in range(2):
        kc, ks, kz = _sentinel_caches(nb, bs, hkv, d, gs, True)
        vc, vs, vz = _sentinel_caches(nb, bs, hkv, d, gs, True)
        caches.append([t.to(DEV) for t in (kc, vc, ks, vs, kz, vz)])
    a, b = caches
    out = ops.append_and_decode(q, k, v, slots, a[0], a[1], a[2], a[3], bt, sl,
                                hkv, d, k_zeros=a[4], v_zeros=a[5], asymmetric=True,
                                k_group_size=gs, v_group_size=gs)
    K.reshape_and_cache_int4(k.contiguous(), v.contiguous(), b[0], b[1], b[2],
                             b[3], slots, b[4], b[5], asymmetric=True, group_size=gs)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))
    assert torch.isfinite(out.float()).all()


def test_mismatched_shapes_raise_before_launch():
    """Caches, scales or new-token rows too small for the call raise
    ValueError on the host (the kernels index them unchecked)."""
    from knlp_amd import ops
    hkv, d, gs, nb, bs = 8, 128, 32, 4, 16
    k, v = _case(5, hkv, d, 3)
    slots = torch.arange(5, device=DEV)
    small = [t.to(DEV) for t in _sentinel_caches(nb, bs, 4, d, gs, True)]   # 4 heads
    full = [t.to(DEV) for t in _sentinel_caches(nb, bs, hkv, d, gs, True)]
    with pytest.raises(ValueError, match="fewer than"):
        K.reshape_and_cache_int4(k.to(DEV), v.to(DEV), small[0], full[0], small[1], full[1],
                                 slots, small[2], full[2], asymmetric=True, group_size=gs)
    short_scales = full[1][..., :2].contiguous()
    with pytest.raises(ValueError, match="do not cover"):
        K.reshape_and_cache_int4(k.to(DEV), v.to(DEV), full[0], full[0].clone(), short_scales,
                                 full[1].clone(), slots, full[2], full[2].clone(),
                                 asymmetric=True, group_size=gs)
    bt = torch.zeros((2, 4), dtype=torch.int32, device=DEV)
    sl = torch.tensor([10, 20], dtype=torch.int32, device=DEV)
    q = torch.zeros((2, 32, d), dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="fewer than"):
        K.fused_int4_decode(q, small[0], full[0], small[1], full[1], bt, sl, hkv, d,
                            k_zeros=small[2], v_zeros=full[2], asymmetric=True, group_size=gs)
    kk = torch.zeros((2, 4, d), dtype=torch.float16, device=DEV)    # 4 of 8 kv heads
    with pytest.raises(ValueError, match="num_kv_heads"):
        ops.append_and_decode(q, kk, kk.clone(), slots[:2], full[0], full[0].clone(), full[1],
                              full[1].clone(), bt, sl, hkv, d, k_zeros=full[2],
                              v_zeros=full[2].clone(), asymmetric=True, k_group_size=gs,
                              v_group_size=gs)
    torch.cuda.synchronize()
