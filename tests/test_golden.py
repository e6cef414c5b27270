"""Committed golden fixtures (tests/golden/int4kv_golden.npz, written by
tests/golden/make_golden.py from the CPU restatement).

CPU: the oracle reproduces every stored vector (a change in the oracle shows
up here, not only as a GPU mismatch).  GPU: the append kernel reproduces the
stored cache bytes bit for bit and the decode matches the stored outputs
within the decode bar (max-abs 2e-3 against the fp32 oracle plus an fp16 ulp
of rounding)."""
import os

import numpy as np
import pytest
import torch

from oracle import attention as A
from tests import tolerance, kvgen

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "int4kv_golden.npz")
APPEND = (("asym", 1, 0.0), ("sym", 0, 10.0), ("int8", 2, 0.0))


@pytest.fixture(scope="module")
def z():
    return np.load(GOLDEN)


def _decode_planes(z):
    kp = {"format": "int4_asym", "data": z["decode_k_data"],
          "scales": z["decode_k_scales"].view(np.float16),
          "zeros": z["decode_k_zeros"].view(np.float16), "group_size": 32}
    vp = {"format": "int4_asym", "data": z["decode_v_data"],
          "scales": z["decode_v_scales"].view(np.float16),
          "zeros": z["decode_v_zeros"].view(np.float16), "group_size": 32}
    return kp, vp


def test_oracle_reproduces_append_fixtures(z):
    x = z["append_x"].view(np.float16).astype(np.float32)
    slots = z["append_slots"]
    keep = slots >= 0
    for name, fmt, clip in APPEND:
        p = kvgen.empty_plane(fmt, 6, 16, 2, 64, 32)
        kvgen.fill_plane(p, x[keep], slots[keep], clip_ratio=clip)
        assert np.array_equal(p["data"], z[f"append_{name}_data"]), name
        assert np.array_equal(p["scales"].view(np.uint16), z[f"append_{name}_scales"]), name
        if p["zeros"] is not None:
            assert np.array_equal(p["zeros"].view(np.uint16), z[f"append_{name}_zeros"]), name


def test_oracle_reproduces_decode_fixture(z):
    kp, vp = _decode_planes(z)
    q = z["decode_q"].view(np.float16).astype(np.float32)
    out = A.decode_reference(q, kp, vp, z["decode_bt"], z["decode_seq_lens"], round_output=False)
    np.testing.assert_allclose(out, z["decode_out_f32"], rtol=0, atol=1e-6)


@pytest.mark.gpu
def test_hip_append_matches_fixtures(z):
    from knlp_amd import ops
    dev = torch.device("cuda")
    x = torch.from_numpy(z["append_x"].view(np.float16).copy()).to(dev)
    slots = torch.from_numpy(z["append_slots"]).to(dev)
    for name, fmt, clip in APPEND:
        p = kvgen.empty_plane(fmt, 6, 16, 2, 64, 32)
        data, scales, zeros = kvgen.plane_to_torch(p, dev)
        plane = ops._plane(data, scales, zeros, fmt, 32)
        ops._append(None, x, None, plane, slots, clip, 16)
        torch.cuda.synchronize()
        assert np.array_equal(data.cpu().numpy(), z[f"append_{name}_data"]), name
        assert np.array_equal(scales.cpu().numpy().view(np.uint16),
                              z[f"append_{name}_scales"]), name
        if zeros is not None:
            assert np.array_equal(zeros.cpu().numpy().view(np.uint16),
                                  z[f"append_{name}_zeros"]), name


@pytest.mark.gpu
def test_hip_decode_matches_fixture(z):
    import knlp_amd as K
    dev = torch.device("cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    q = t(z["decode_q"].view(np.float16))
    out = K.fused_int4_decode(q, t(z["decode_k_data"]), t(z["decode_v_data"]),
                              t(z["decode_k_scales"].view(np.float16)),
                              t(z["decode_v_scales"].view(np.float16)), t(z["decode_bt"]),
                              t(z["decode_seq_lens"]), 8, 64,
                              k_zeros=t(z["decode_k_zeros"].view(np.float16)),
                              v_zeros=t(z["decode_v_zeros"].view(np.float16)), asymmetric=True)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = z["decode_out_f32"]
    tolerance.check("golden_decode", got, ref)
