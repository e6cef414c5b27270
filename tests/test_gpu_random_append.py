"""Seeded random quantize-on-append cases against the oracle, bit for bit:
INT4 symmetric (with and without the trimmed-mean clip) and asymmetric,
INT8 K and V, head sizes 32-256, scale groups 16-128, fp16 and bf16 sources,
int32 and int64 slots with padding (-1) slots, 16- and 32-token pages, and
sources that are strided views (token stride larger than the row).  The
hand-picked cases in test_gpu_append.py cover each format; this sweep the
products of their parameters (F:210-472, F:481-647, F:1231-1312,
F:1563-1650)."""
import numpy as np
import pytest
import torch

import knlp_amd as K
from oracle import quant as Q
from tests import kvgen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cases(n=24, seed=77):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        d = int(rng.choice([32, 64, 128, 128, 256]))
        gs = int(rng.choice([g for g in (16, 32, 64, 128) if g <= d]))
        fmt = ["int4_sym", "int4_sym_noclip", "int4_asym", "int8_k", "int8_v"][int(rng.integers(0, 5))]
        hkv = int(rng.choice([1, 2, 4, 8]))
        nt = int(rng.integers(1, 150))
        bs = int(rng.choice([16, 32]))
        bf16 = bool(rng.random() < 0.3)
        slots64 = bool(rng.random() < 0.5)
        strided = bool(rng.random() < 0.5)
        out.append((f"a{i:02d}_{fmt}_d{d}_g{gs}_h{hkv}_t{nt}_bs{bs}"
                    f"{'_bf16' if bf16 else ''}{'_i64' if slots64 else '_i32'}"
                    f"{'_strided' if strided else ''}",
                    fmt, d, gs, hkv, nt, bs, bf16, slots64, strided, 900 + i))
    return out


CASES = _cases()


def _src(nt, hkv, d, seed, dtype, strided):
    """[nt, hkv, d] rows; strided: a view whose token stride is 3 rows long."""
    x = kvgen.randn((nt, 3 * hkv, d) if strided else (nt, hkv, d), seed, dtype, 0.01)
    x = x.to(DEV)
    return x[:, hkv:2 * hkv] if strided else x


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_random_append_bit_exact(case):
    name, fmt, d, gs, hkv, nt, bs, bf16, slots64, strided, seed = case
    dtype = torch.bfloat16 if bf16 else torch.float16
    nb = -(-nt // bs) + 3
    g = torch.Generator().manual_seed(seed)
    slots = torch.randperm(nb * bs, generator=g)[:nt].to(torch.int64)
    slots[torch.randperm(nt, generator=g)[: nt // 6]] = -1
    slots = slots.to(torch.int64 if slots64 else torch.int32)
    k = _src(nt, hkv, d, 2000 + seed, dtype, strided)
    v = _src(nt, hkv, d, 3000 + seed, dtype, strided)
    kf, vf = k.float().cpu().numpy(), v.float().cpu().numpy()
    sl = slots.to(DEV)
    print(f"# {name}", flush=True)
    if fmt.startswith("int4"):
        asym = fmt == "int4_asym"
        clip = 0.0 if fmt == "int4_sym_noclip" else 10.0
        host = [torch.full((nb, bs, hkv, d // 2), 0xA5, dtype=torch.uint8) for _ in range(2)]
        host += [torch.full((nb, bs, hkv, d // gs), 3.0, dtype=torch.float16) for _ in range(2)]
        host += [torch.full((nb, bs, hkv, d // gs), -7.0, dtype=torch.float16)
                 for _ in range(2)] if asym else [None, None]
        ref = [t.numpy().copy() if t is not None else None for t in host]
        Q.reshape_and_cache_int4(kf, vf, ref[0], ref[1], ref[2], ref[3], slots.numpy(), ref[4],
                                 ref[5], asymmetric=asym, group_size=gs, clip_ratio=clip)
        dev = [t.to(DEV) if t is not None else None for t in host]
        K.reshape_and_cache_int4(k, v, dev[0], dev[1], dev[2], dev[3], sl, dev[4], dev[5],
                                 asymmetric=asym, group_size=gs, clip_ratio=clip)
    else:
        src, srcf = (k, kf) if fmt == "int8_k" else (v, vf)
        host = [torch.full((nb, bs, hkv, d), 0x5A, dtype=torch.int8),
                torch.full((nb, bs, hkv, d // gs), 3.0, dtype=torch.float16)]
        ref = [t.numpy().copy() for t in host]
        Q.reshape_and_cache_k_int8(srcf, ref[0], ref[1], slots.numpy(), group_size=gs)
        dev = [t.to(DEV) for t in host]
        fn = K.reshape_and_cache_k_int8 if fmt == "int8_k" else K.reshape_and_cache_v_int8
        fn(src, dev[0], dev[1], sl, group_size=gs)
    torch.cuda.synchronize()
    for i, (got, want) in enumerate(zip(dev, ref)):
        if want is None:
            continue
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint8), want.view(np.uint8),
                                      err_msg=f"{name}: tensor {i}")
