"""vLLM backend glue end to end on the GPU (real HIP operators).

One prefill step (two sequences) then one decode step through
``FusedInt4AttentionImpl.do_kv_cache_update`` + ``forward``, as vLLM drives
it (F:2483-2843).  The decode output is checked against the oracle's
dequant -> SDPA over the backend's own shadow caches (read back), the
shadow caches against the oracle's quantiser (bit-exact), the prefill output
against causal attention in fp32, and the short-sequence path against the
oracle over the fp16 paged cache.  vLLM itself is absent: the backend is
imported against tests/vllm_stub.
"""
import os
import sys

import numpy as np
import pytest
import torch

from knlp_amd import config, kv_layout
from oracle import attention as A
from tests import kvgen, tolerance

pytestmark = pytest.mark.gpu

STUB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "vllm_stub")
H, HKV, D, BS, NB = 16, 4, 128, 16, 40
def close(got, ref, bf16=False):
    """The decode parity bar of tests/tolerance.py (asserts; records the
    achieved error under the current test's name)."""
    name = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0].split("::")[-1]
    tolerance.check(name, got, ref, bf16=bf16)
    return True


@pytest.fixture(scope="module")
def vb():
    try:
        import vllm.v1.attention.backend  # noqa: F401
    except ImportError:
        for m in [m for m in sys.modules if m == "vllm" or m.startswith("vllm.")]:
            del sys.modules[m]
        sys.path.insert(0, STUB)
    import knlp_amd.vllm_backend as vb
    return vb


def impl_for(vb, monkeypatch, k="int4", v="int4", asym=True, msl=48, scale=D ** -0.5):
    monkeypatch.setattr(config, "K_PRECISION", k)
    monkeypatch.setattr(config, "V_PRECISION", v)
    monkeypatch.setattr(config, "ASYMMETRIC", asym)
    monkeypatch.setattr(config, "MIN_FUSED_SEQ_LEN", msl)
    monkeypatch.setattr(config, "REPLACE_CACHE", False)
    return vb.FusedInt4AttentionImpl(H, D, scale, HKV)


def run_two_steps(vb, impl, dtype, prompt_lens, seed):
    """Prefill `prompt_lens`, then decode one token per sequence.  Returns
    (prefill out, decode out, q/k/v of both steps, block table, kv cache)."""
    dev = torch.device("cuda")
    bt = kvgen.paged_table([n + 1 for n in prompt_lens], BS, NB, seed)
    n_pf = sum(prompt_lens)
    q = kvgen.randn((n_pf, H, D), seed + 1, dtype)
    k = kvgen.randn((n_pf, HKV, D), seed + 2, dtype, outlier_frac=0.02)
    v = kvgen.randn((n_pf, HKV, D), seed + 3, dtype, outlier_frac=0.02)
    kv = torch.zeros(kv_layout.kv_cache_shape(NB, BS, HKV, D), dtype=dtype, device=dev)
    slots = torch.from_numpy(kvgen.token_slots(bt, prompt_lens, BS)).to(dev)
    qsl = torch.tensor(np.concatenate([[0], np.cumsum(prompt_lens)]), dtype=torch.int32,
                       device=dev)
    bt_d = torch.from_numpy(bt).to(dev)
    md = vb.FusedInt4AttentionMetadata(
        num_actual_tokens=n_pf, max_query_len=max(prompt_lens), query_start_loc=qsl,
        max_seq_len=max(prompt_lens),
        seq_lens=torch.tensor(prompt_lens, dtype=torch.int32, device=dev),
        block_table=bt_d, slot_mapping=slots)
    kd, vd = k.to(dev).view(n_pf, -1), v.to(dev).view(n_pf, -1)
    impl.do_kv_cache_update(None, kd, vd, kv, slots)
    out_pf = impl.forward(None, q.to(dev).view(n_pf, -1), kd, vd, kv, md)
    # decode: one new token per sequence at position prompt_len
    S = len(prompt_lens)
    q2 = kvgen.randn((S, H, D), seed + 4, dtype)
    k2 = kvgen.randn((S, HKV, D), seed + 5, dtype)
    v2 = kvgen.randn((S, HKV, D), seed + 6, dtype)
    pos = np.array(prompt_lens)
    slots2 = torch.from_numpy(bt[np.arange(S), pos // BS].astype(np.int64) * BS + pos % BS).to(dev)
    md2 = vb.FusedInt4AttentionMetadata(
        num_actual_tokens=S, max_query_len=1,
        query_start_loc=torch.arange(S + 1, dtype=torch.int32, device=dev),
        max_seq_len=max(prompt_lens) + 1,
        seq_lens=torch.tensor([n + 1 for n in prompt_lens], dtype=torch.int32, device=dev),
        block_table=bt_d, slot_mapping=slots2, total_context=sum(prompt_lens) + S)
    k2d, v2d = k2.to(dev).view(S, -1), v2.to(dev).view(S, -1)
    impl.do_kv_cache_update(None, k2d, v2d, kv, slots2)
    out_dec = impl.forward(None, q2.to(dev).view(S, -1), k2d, v2d, kv, md2)
    torch.cuda.synchronize()
    return dict(out_pf=out_pf.cpu(), out_dec=out_dec.cpu(), q=q, k=k, v=v, q2=q2, k2=k2, v2=v2,
                bt=bt, kv=kv, slots=slots.cpu().numpy(), slots2=slots2.cpu().numpy())


def plane(fmt, data, scales, zeros, gs):
    t = lambda x: None if x is None else x.cpu().numpy()
    return {"format": fmt, "data": t(data), "scales": t(scales), "zeros": t(zeros),
            "group_size": gs}


def causal_ref(q, k, v, lens):
    out, a = [], 0
    rep = H // HKV
    for n in lens:
        qq = q[a:a + n].float().transpose(0, 1)
        kk = k[a:a + n].float().repeat_interleave(rep, dim=1).transpose(0, 1)
        vv = v[a:a + n].float().repeat_interleave(rep, dim=1).transpose(0, 1)
        s = (qq @ kk.transpose(1, 2)) * D ** -0.5
        s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool), 1), float("-inf"))
        out.append((torch.softmax(s, -1) @ vv).transpose(0, 1))
        a += n
    return torch.cat(out)


@pytest.mark.parametrize("k,v,asym", [("int4", "int4", True), ("int4", "int4", False),
                                      ("int8", "int4", True), ("fp16", "int8", False)])
def test_prefill_then_decode_matches_oracle(vb, monkeypatch, k, v, asym):
    impl = impl_for(vb, monkeypatch, k, v, asym, msl=48)
    lens = [70, 33]
    r = run_two_steps(vb, impl, torch.float16, lens, seed=100)
    # prefill: causal attention over the fresh fp16 K/V
    want = causal_ref(r["q"], r["k"], r["v"], lens).reshape(sum(lens), -1)
    assert close(r["out_pf"].float().numpy(), want.numpy())
    # shadow caches: bit-exact with the oracle quantiser over the same rows
    c = impl.caches
    gs = config.GROUP_SIZE
    fmt_k = {"int4": 1 if asym else 0, "int8": 2, "fp16": 3}[k]
    fmt_v = {"int4": 1 if asym else 0, "int8": 2}[v]
    kp = kvgen.empty_plane(fmt_k, NB, BS, HKV, D, gs)
    vp = kvgen.empty_plane(fmt_v, NB, BS, HKV, D, gs)
    for x, y, sl in ((r["k"], r["v"], r["slots"]), (r["k2"], r["v2"], r["slots2"])):
        kvgen.fill_plane(kp, x.float().numpy(), sl, config.OUTLIER_CLIP_RATIO)
        kvgen.fill_plane(vp, y.float().numpy(), sl, config.OUTLIER_CLIP_RATIO)
    if k == "int4":
        assert np.array_equal(c.int4_key.cpu().numpy(), kp["data"])
        assert np.array_equal(c.k_scales.cpu().numpy().view(np.uint16),
                              kp["scales"].view(np.uint16))
    elif k == "int8":
        assert np.array_equal(c.int8_key.cpu().numpy(), kp["data"])
    else:
        assert np.array_equal(r["kv"][0].cpu().numpy(), kp["data"])
    vdata = c.int8_value if v == "int8" else c.int4_value
    assert np.array_equal(vdata.cpu().numpy(), vp["data"])
    # decode: oracle dequant -> SDPA over those caches
    ref = A.decode_reference(r["q2"].float().numpy(), kp, vp, r["bt"], [n + 1 for n in lens],
                             round_output=False)
    got = r["out_dec"].float().numpy().reshape(ref.shape)
    assert close(got, ref)


def test_short_sequences_read_fp16_paged_cache(vb, monkeypatch):
    """Below MIN_FUSED_SEQ_LEN the decode reads the fp16 paged cache (here
    this library's fp16 decode); compare with the oracle over that cache."""
    impl = impl_for(vb, monkeypatch, msl=10 ** 6)
    lens = [20, 9]
    r = run_two_steps(vb, impl, torch.float16, lens, seed=200)
    kc = {"format": "fp16", "data": r["kv"][0].cpu().numpy(), "scales": None, "zeros": None,
          "group_size": D}
    vc = {"format": "fp16", "data": r["kv"][1].cpu().numpy(), "scales": None, "zeros": None,
          "group_size": D}
    ref = A.decode_reference(r["q2"].float().numpy(), kc, vc, r["bt"], [n + 1 for n in lens],
                             round_output=False)
    got = r["out_dec"].float().numpy().reshape(ref.shape)
    assert close(got, ref)


def test_bf16_model_decode(vb, monkeypatch):
    """bf16 activations: quantised append from bf16 rows, bf16 query decode
    (VALU kernel), output rounded fp32 -> fp16 -> bf16 as the reference."""
    impl = impl_for(vb, monkeypatch, msl=48)
    lens = [64, 50]
    r = run_two_steps(vb, impl, torch.bfloat16, lens, seed=300)
    c = impl.caches
    kp = plane("int4_asym", c.int4_key, c.k_scales, c.k_zeros, config.GROUP_SIZE)
    vp = plane("int4_asym", c.int4_value, c.v_scales, c.v_zeros, config.GROUP_SIZE)
    ref = A.decode_reference(r["q2"].float().numpy(), kp, vp, r["bt"], [n + 1 for n in lens],
                             round_output=False)
    got = r["out_dec"].float().numpy().reshape(ref.shape)
    # bf16 output: half a bf16 ulp (relative 2^-8) on top of the fp32 bar
    assert close(got, ref, bf16=True)


def test_fp16_paged_write_matches_scatter(vb, monkeypatch):
    """reshape_and_cache_fp16 (append kernel, fp16 planes) against a torch
    scatter, with slot < 0 skipped."""
    from knlp_amd import ops
    dev = torch.device("cuda")
    n = 50
    k = kvgen.randn((n, HKV, D), 7).to(dev)
    v = kvgen.randn((n, HKV, D), 8).to(dev)
    slots = torch.randperm(NB * BS, generator=torch.Generator().manual_seed(9))[:n].to(dev)
    slots[3] = -1
    kc = torch.zeros(NB, BS, HKV, D, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    ops.reshape_and_cache_fp16(k, v, kc, vc, slots)
    kw, vw = torch.zeros_like(kc), torch.zeros_like(vc)
    keep = slots >= 0
    kw.view(-1, HKV, D)[slots[keep]] = k[keep]
    vw.view(-1, HKV, D)[slots[keep]] = v[keep]
    torch.cuda.synchronize()
    assert torch.equal(kc, kw) and torch.equal(vc, vw)


@pytest.mark.parametrize("layer_scale", [False, True], ids=["reference_scale", "layer_scale"])
def test_fused_decode_softmax_scale(vb, monkeypatch, layer_scale):
    """A layer built with a softmax scale other than 1/sqrt(D): the fused
    decode uses 1/sqrt(D) as the reference's kernels do (F:924; its
    _fused_decode passes no scale, F:2851-2928), or the layer's scale when
    KNLP_FUSED_DECODE_LAYER_SCALE asks for it."""
    monkeypatch.setattr(config, "FUSED_DECODE_LAYER_SCALE", layer_scale)
    impl = impl_for(vb, monkeypatch, msl=48, scale=0.05)
    lens = [70, 33]
    r = run_two_steps(vb, impl, torch.float16, lens, seed=400)
    c = impl.caches
    kp = plane("int4_asym", c.int4_key, c.k_scales, c.k_zeros, config.GROUP_SIZE)
    vp = plane("int4_asym", c.int4_value, c.v_scales, c.v_zeros, config.GROUP_SIZE)
    q2 = r["q2"].float().numpy()
    sl = [n + 1 for n in lens]
    want = A.decode_reference(q2, kp, vp, r["bt"], sl, scale=0.05 if layer_scale else None,
                              round_output=False)
    other = A.decode_reference(q2, kp, vp, r["bt"], sl, scale=None if layer_scale else 0.05,
                               round_output=False)
    got = r["out_dec"].float().numpy().reshape(want.shape)
    assert close(got, want)
    assert np.abs(got - other).max() > 2e-2      # the two scales give different outputs


def test_decode_stream_schedule_through_backend(vb, monkeypatch):
    """Hkv = 8 and a variable-length batch: with the host-side total context
    the plan picks the stream schedule; the backend's decode still matches
    the oracle over its shadow caches."""
    import sys as _sys
    mod = _sys.modules[__name__]
    monkeypatch.setattr(mod, "H", 32)
    monkeypatch.setattr(mod, "HKV", 8)
    from knlp_amd import _lib
    impl = impl_for(vb, monkeypatch, "int4", "int4", True, msl=48)
    lens = [300, 40, 5]
    width = max(-(-(n + 1) // BS) for n in lens)
    assert _lib.lib().knlp_kv_decode_plan(3, 8, 32, D, width * BS, sum(lens) + 3, 1, 32, 1,
                                          32) == 0
    r = run_two_steps(vb, impl, torch.float16, lens, seed=300)
    gs = config.GROUP_SIZE
    kp = kvgen.empty_plane(1, NB, BS, 8, D, gs)
    vp = kvgen.empty_plane(1, NB, BS, 8, D, gs)
    for x, y, sl in ((r["k"], r["v"], r["slots"]), (r["k2"], r["v2"], r["slots2"])):
        kvgen.fill_plane(kp, x.float().numpy(), sl, config.OUTLIER_CLIP_RATIO)
        kvgen.fill_plane(vp, y.float().numpy(), sl, config.OUTLIER_CLIP_RATIO)
    ref = A.decode_reference(r["q2"].float().numpy(), kp, vp, r["bt"], [n + 1 for n in lens],
                             round_output=False)
    assert close(r["out_dec"].float().numpy().reshape(ref.shape), ref)
