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
