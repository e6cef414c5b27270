"""Seeded random decode cases against the oracle: combinations of head size,
kv heads, query-group size (including 3, 6 and 7, which fill no kernel's head
template exactly), K/V formats, scale-group sizes, page sizes, split plans
(library plan, fixed splits, the stream schedule), bf16 queries and sequence
lengths of 0 and 1.  Every combination the library accepts must match the
oracle's dequantise-then-SDPA result (scripts/v35_h100_bench.py:376-387) to
the bar of tests/tolerance.py; the hand-picked cases in test_gpu_decode.py
cover each kernel family, this sweep the products of their parameters."""
import numpy as np
import pytest
import torch

import knlp_amd as K
from tests.test_gpu_decode import _build, _check, _query, _run

pytestmark = pytest.mark.gpu

FMT_NAMES = {0: "int4_sym", 1: "int4_asym", 2: "int8", 3: "fp16"}


def _cases(n=40, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        d = int(rng.choice([64, 128, 128, 128, 256]))
        hkv = int(rng.choice([1, 2, 4, 8, 8, 16]))
        g = int(rng.integers(1, 9))
        kf = int(rng.integers(0, 4))
        vf = int(rng.integers(0, 4))
        int4_gs = [s for s in (16, 32, 64, 128) if s <= d]
        int8_gs = [s for s in (32, 64, 128) if s <= d] + ([d] if d <= 128 else [])

        def gs(f):
            if f == 3:
                return d
            return int(rng.choice(int4_gs if f in (0, 1) else int8_gs))

        kgs, vgs = gs(kf), gs(vf)
        if kf in (0, 1) and vf in (0, 1):
            # the reference's INT4 pair: one encoding and one GROUP_SIZE (F:901-915)
            vf, vgs = kf, kgs
        bs = int(rng.choice([16, 16, 32]))
        nseq = int(rng.integers(1, 5))
        lens = []
        for _ in range(nseq):
            kind = int(rng.integers(0, 6))
            lens.append([0, 1, int(rng.integers(2, 48)), int(rng.integers(48, 700)),
                         int(rng.integers(700, 2600)), int(rng.integers(700, 2600))][kind])
        if max(lens) == 0:
            lens[0] = int(rng.integers(1, 300))
        split = [None, None, 64, 256, 0][int(rng.integers(0, 5))]
        bf16 = bool(rng.random() < 0.2)
        out.append((f"r{i:02d}_d{d}_hkv{hkv}_g{g}_{FMT_NAMES[kf]}{kgs}_{FMT_NAMES[vf]}{vgs}"
                    f"_bs{bs}_s{split}{'_bf16' if bf16 else ''}",
                    lens, g * hkv, hkv, d, kf, vf, kgs, vgs, bs, split, bf16))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_random_decode_matches_oracle(case):
    name, lens, hq, hkv, d, kf, vf, kgs, vgs, bs, split, bf16 = case
    qdt = torch.bfloat16 if bf16 else torch.float16
    kind = K.decode_kernel_kind(hq, hkv, d, kf, kgs, vf, vgs, qdt)   # raises if rejected
    seed = 500 + CASES.index(case)
    bt, kp, vp = _build(lens, hq, hkv, d, kf, vf, kgs, vgs, seed, bs=bs)
    q = _query(len(lens), hq, d, seed, qdt)
    print(f"# {name}: lens {lens}, kernel {kind}", flush=True)
    out = _run(q, kp, vp, bt, lens, hkv, d, split_tokens=split)
    assert out.dtype == q.dtype
    _check(out, q, kp, vp, bt, lens, name=name)
