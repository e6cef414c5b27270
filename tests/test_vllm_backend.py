"""vLLM backend glue (knlp_amd.vllm_backend, knlp_amd.kv_layout) on the CPU.

vLLM is absent here, so the backend is imported against the stand-in package
under tests/vllm_stub.  The decode / write operators are replaced by
recorders, so these tests check the backend's own logic: class surface,
cache shapes, the planner's byte budget (closed-form numbers and the
allocation it budgets), the (k_precision, v_precision) dispatch of writes and
decodes (F:2600-2707, F:2851-2928), the MIN_FUSED_SEQ_LEN gate
(F:2723-2736), REPLACE_CACHE, and the placement of decode and prefill rows
in a mixed batch (F:2751-2843).
"""
import os
import sys

import pytest
import torch

from knlp_amd import _lib

from knlp_amd import config, kv_layout

STUB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "vllm_stub")

PAIRS = [("int4", "int4"), ("int8", "int4"), ("int8", "int8"), ("fp16", "int4"),
         ("fp16", "int8")]


@pytest.fixture(scope="module")
def vb():
    try:
        import vllm.v1.attention.backend  # noqa: F401  (a real vLLM install)
    except ImportError:
        for m in [m for m in sys.modules if m == "vllm" or m.startswith("vllm.")]:
            del sys.modules[m]
        sys.path.insert(0, STUB)
    import knlp_amd.vllm_backend as vb
    return vb


# ---- kv_layout: shapes and the planner's budget ---------------------------------------------

def test_kv_cache_shape():
    assert kv_layout.kv_cache_shape(10, 16, 8, 128) == (2, 10, 16, 8, 128)
    assert kv_layout.kv_cache_shape(10, 16, 8, 128, replace_cache=True) == (1, 10, 16, 8, 128)


# closed-form bytes per block for bs=16, 8 kv heads, D=128, g32 (config-2 heads):
# INT4 codes 16*8*64 = 8192, fp16 group params 16*8*4*2 = 1024 each, INT8 codes 16384,
# and the INT8-V path's 3-byte INT4 placeholder (support/attention.v0.1.0.py:556-563)
@pytest.mark.parametrize("k,v,asym,want", [
    ("int4", "int4", True, 2 * (8192 + 2 * 1024)),
    ("int4", "int4", False, 2 * (8192 + 1024)),
    ("int8", "int4", True, (16384 + 1024) + (8192 + 2 * 1024)),
    ("int8", "int8", False, (16384 + 1024) + (16384 + 1024 + 3)),
    ("fp16", "int4", True, 8192 + 2 * 1024),
    ("fp16", "int8", True, 16384 + 1024 + 3),
])
def test_shadow_bytes_per_block_known_answers(k, v, asym, want):
    got = kv_layout.shadow_bytes_per_block(16, 8, 128, k_precision=k, v_precision=v,
                                           asymmetric=asym, group_size=32)
    assert got == want


@pytest.mark.parametrize("k,v", PAIRS)
@pytest.mark.parametrize("asym", [False, True])
def test_allocation_matches_planner(k, v, asym):
    nb, bs, h, d = 7, 16, 4, 64
    c = kv_layout.allocate_shadow_caches(nb, bs, h, d, k_precision=k, v_precision=v,
                                         asymmetric=asym, group_size=32)
    actual, expected = kv_layout.planner_check(c, nb, bs, h, d, k_precision=k,
                                               v_precision=v, asymmetric=asym, group_size=32)
    # the INT8-V placeholder is allocated once but budgeted per block
    assert expected - actual == (3 if v == "int8" else 0)
    assert c.num_blocks(v) == nb
    if k == "int4":
        assert c.int4_key.shape == (nb, bs, h, d // 2) and c.int4_key.dtype == torch.uint8
        assert (c.k_zeros is not None) == asym
    if k == "int8":
        assert c.int8_key.shape == (nb, bs, h, d) and c.int8_key.dtype == torch.int8
    if k == "fp16":
        assert c.int4_key is None and c.int8_key is None
    if v == "int4":
        assert c.int4_value.shape == (nb, bs, h, d // 2)
        assert (c.v_zeros is not None) == asym


def test_planner_rejects_bad_arguments():
    with pytest.raises(ValueError):
        kv_layout.shadow_bytes_per_block(16, 8, 128, k_precision="int2")
    with pytest.raises(ValueError):
        kv_layout.shadow_bytes_per_block(16, 8, 100, group_size=32)


# ---- class surface ---------------------------------------------------------------------------

def test_backend_surface(vb, monkeypatch):
    B = vb.FusedInt4AttentionBackend
    assert B.get_name() == "FUSED_INT4"
    assert B.get_impl_cls() is vb.FusedInt4AttentionImpl
    assert B.get_builder_cls() is vb.FusedInt4AttentionMetadataBuilder
    assert B.supports_kv_cache_dtype("int4_fused") and B.supports_kv_cache_dtype(None)
    assert not B.supports_kv_cache_dtype("fp8")
    assert B.supports_head_size(128) and B.supports_head_size(64)
    assert not B.supports_head_size(100) and not B.supports_head_size(0)
    # every admitted head size is one the decode takes (D = 32 included), and
    # none it rejects (96 = 3 * 32 passes F's divisibility test alone)
    L = _lib.lib()
    for d in range(16, 513, 16):
        if B.supports_head_size(d):
            assert L.knlp_kv_decode_kernel_kind(8, 8, d, 1, 32, 1, 32, 0) in (0, 1), d
    assert B.supports_head_size(32) and not B.supports_head_size(96)
    assert not B.supports_head_size(512)
    assert B.supports_attn_type("decoder") and not B.supports_attn_type("encoder")
    assert B.get_kv_cache_shape(5, 16, 8, 128) == (2, 5, 16, 8, 128)
    monkeypatch.setattr(config, "REPLACE_CACHE", True)
    assert B.get_kv_cache_shape(5, 16, 8, 128) == (1, 5, 16, 8, 128)
    assert vb.FusedInt4AttentionMetadataBuilder._cudagraph_support.name == \
        "UNIFORM_SINGLE_TOKEN_DECODE"


def test_impl_rejects_unsupported(vb, monkeypatch):
    I = vb.FusedInt4AttentionImpl
    with pytest.raises(NotImplementedError):
        I(8, 64, 0.125, 2, alibi_slopes=[0.1] * 8)
    with pytest.raises(NotImplementedError):
        I(8, 64, 0.125, 2, sliding_window=128)
    monkeypatch.setattr(config, "K_PRECISION", "int4")
    monkeypatch.setattr(config, "V_PRECISION", "int8")
    with pytest.raises(ValueError):
        I(8, 64, 0.125, 2)


def test_builder(vb):
    from vllm.v1.attention.backend import CommonAttentionMetadata
    qsl = torch.tensor([0, 1, 2], dtype=torch.int32)
    m = CommonAttentionMetadata(query_start_loc=qsl, seq_lens=torch.tensor([5, 9]), num_reqs=2,
                                num_actual_tokens=2, max_query_len=1, max_seq_len=9,
                                block_table_tensor=torch.zeros(2, 3, dtype=torch.int32),
                                slot_mapping=torch.tensor([4, 8]))
    b = vb.FusedInt4AttentionMetadataBuilder(None, ["l0"], None, torch.device("cpu"))
    assert b.reorder_batch_threshold == 1
    md = b.build(0, m)
    assert md.max_seq_len == 9 and md.max_query_len == 1 and md.num_actual_tokens == 2
    assert md.block_table is m.block_table_tensor and md.slot_mapping is m.slot_mapping
    assert md.total_context == 0                      # no host copy of the lengths
    m.seq_lens_cpu = torch.tensor([5, 9])
    assert b.build(0, m).total_context == 14


# ---- dispatch with recording operators ---------------------------------------------------------

H, HKV, D, BS, NB = 8, 2, 64, 16, 6


class Recorder:
    """Replaces the knlp_amd.ops entry points the backend calls."""

    def __init__(self, monkeypatch, ops_mod):
        self.calls = []
        self.kwargs = {}
        for name in ("fused_int4_decode", "kint8_vint4_decode", "kint8_vint8_decode",
                     "kfp16_vint4_decode", "kfp16_vint8_decode", "fp16_paged_decode",
                     "append_and_decode"):
            monkeypatch.setattr(ops_mod, name, self._decode(name))
        for name in ("reshape_and_cache_int4", "reshape_and_cache_v_only_int4",
                     "reshape_and_cache_k_int8", "reshape_and_cache_v_int8",
                     "reshape_and_cache_fp16"):
            monkeypatch.setattr(ops_mod, name, self._write(name))

    def _decode(self, name):
        def f(q, *a, **k):
            self.calls.append(name)
            self.kwargs[name] = (a, k)
            # row s of the output is filled with 100 + s so placement is visible
            out = torch.empty_like(q)
            for s in range(q.shape[0]):
                out[s] = 100.0 + s
            return out
        return f

    def _write(self, name):
        def f(*a, **k):
            self.calls.append(name)
        return f


def make_impl(vb, monkeypatch, k="int4", v="int4", asym=True, msl=48, replace=False):
    monkeypatch.setattr(config, "K_PRECISION", k)
    monkeypatch.setattr(config, "V_PRECISION", v)
    monkeypatch.setattr(config, "ASYMMETRIC", asym)
    monkeypatch.setattr(config, "MIN_FUSED_SEQ_LEN", msl)
    monkeypatch.setattr(config, "REPLACE_CACHE", replace)
    return vb.FusedInt4AttentionImpl(H, D, D ** -0.5, HKV)


def decode_md(vb, seq_lens, slots):
    n = len(seq_lens)
    return vb.FusedInt4AttentionMetadata(
        num_actual_tokens=n, max_query_len=1,
        query_start_loc=torch.arange(n + 1, dtype=torch.int32), max_seq_len=max(seq_lens),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32),
        block_table=torch.arange(n * 3, dtype=torch.int32).view(n, 3),
        slot_mapping=torch.tensor(slots, dtype=torch.int64))


WRITES = {
    ("int4", "int4"): ["reshape_and_cache_int4"],
    ("int8", "int4"): ["reshape_and_cache_k_int8", "reshape_and_cache_v_only_int4"],
    ("int8", "int8"): ["reshape_and_cache_k_int8", "reshape_and_cache_v_int8"],
    ("fp16", "int4"): ["reshape_and_cache_v_only_int4"],
    ("fp16", "int8"): ["reshape_and_cache_v_int8"],
}


@pytest.mark.parametrize("k,v", PAIRS)
def test_decode_dispatch_table(vb, monkeypatch, k, v):
    """Mixed batch (one decode row, one 2-token prefill): the step's writes,
    then the decode kernel of the (k, v) pair (F:2701-2707)."""
    rec = Recorder(monkeypatch, vb.ops)
    impl = make_impl(vb, monkeypatch, k, v)
    kv = torch.zeros(kv_layout.kv_cache_shape(NB, BS, HKV, D), dtype=torch.float16)
    md = vb.FusedInt4AttentionMetadata(
        num_actual_tokens=3, max_query_len=2,
        query_start_loc=torch.tensor([0, 1, 3], dtype=torch.int32), max_seq_len=60,
        seq_lens=torch.tensor([60, 2], dtype=torch.int32),
        block_table=torch.arange(6, dtype=torch.int32).view(2, 3),
        slot_mapping=torch.tensor([59, 48, 49]))
    q = torch.randn(3, H * D).half()
    kk = torch.randn(3, HKV * D).half()
    out = impl.forward(None, q, kk, kk, kv, md)
    assert rec.calls == WRITES[(k, v)] + [vb.DECODE_KERNELS[(k, v)]]
    assert out.shape == (3, H * D) and float(out[0, 0]) == 100.0
    assert impl.caches.num_blocks(v) == NB


@pytest.mark.parametrize("k,v", PAIRS)
def test_pure_decode_fuses_the_append(vb, monkeypatch, k, v):
    """A pure decode step on the fused path makes one call: the new token's
    quantised append inside the decode (the separate write launch of
    F:2600-2689 disappears); fp16 K is already in the paged cache."""
    rec = Recorder(monkeypatch, vb.ops)
    impl = make_impl(vb, monkeypatch, k, v)
    kv = torch.zeros(kv_layout.kv_cache_shape(NB, BS, HKV, D), dtype=torch.float16)
    md = decode_md(vb, [60, 50], [59, 49 + 48])
    q = torch.randn(2, H * D).half()
    kk = torch.randn(2, HKV * D).half()
    out = impl.forward(None, q, kk, kk, kv, md)
    assert rec.calls == ["append_and_decode"]
    a, kw = rec.kwargs["append_and_decode"]
    assert kw["k_format"] == k and kw["v_format"] == v
    assert (a[0] is None) == (k == "fp16")          # the key rows
    assert torch.equal(a[2], md.slot_mapping)
    if k == "fp16":
        assert a[3] is kv[0] or torch.equal(a[3], kv[0])
    assert out.shape == (2, H * D) and float(out[1, 0]) == 101.0


def test_min_fused_seq_len_gate(vb, monkeypatch):
    rec = Recorder(monkeypatch, vb.ops)
    impl = make_impl(vb, monkeypatch, msl=48)
    kv = torch.zeros(kv_layout.kv_cache_shape(NB, BS, HKV, D), dtype=torch.float16)
    q = torch.randn(2, H * D).half()
    impl.forward(None, q, q[:, :HKV * D], q[:, :HKV * D], kv, decode_md(vb, [47, 10], [0, 1]))
    assert rec.calls[-1] == "fp16_paged_decode"
    impl.forward(None, q, q[:, :HKV * D], q[:, :HKV * D], kv, decode_md(vb, [48, 10], [0, 1]))
    assert rec.calls[-1] == "append_and_decode"


def test_replace_cache_always_fused(vb, monkeypatch):
    rec = Recorder(monkeypatch, vb.ops)
    impl = make_impl(vb, monkeypatch, replace=True, msl=10 ** 6)
    kv = torch.zeros(kv_layout.kv_cache_shape(NB, BS, HKV, D, True), dtype=torch.float16)
    q = torch.randn(2, H * D).half()
    impl.forward(None, q, q[:, :HKV * D], q[:, :HKV * D], kv, decode_md(vb, [5, 3], [0, 1]))
    # the quantised append happened in do_kv_cache_update, not in forward
    assert rec.calls == ["fused_int4_decode"]


def test_do_kv_cache_update(vb, monkeypatch):
    rec = Recorder(monkeypatch, vb.ops)
    impl = make_impl(vb, monkeypatch)
    kv = torch.zeros(kv_layout.kv_cache_shape(NB, BS, HKV, D), dtype=torch.float16)
    x = torch.randn(3, HKV * D).half()
    impl.do_kv_cache_update(None, x, x, kv, torch.tensor([0, 5, -1]))
    assert rec.calls == ["reshape_and_cache_fp16"]
    assert impl.caches is not None and impl.caches.num_blocks("int4") == NB


def test_bf16_paged_write_and_short_decode(vb, monkeypatch):
    """bf16 models: the fp16-plane write is a device scatter that skips
    slot < 0, and the short-sequence decode is the reference's per-sequence
    SDPA (F:3087-3125) -- checked against a direct computation."""
    Recorder(monkeypatch, vb.ops)
    impl = make_impl(vb, monkeypatch, msl=1000)
    kv = torch.zeros(kv_layout.kv_cache_shape(NB, BS, HKV, D), dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(3)
    n = 20
    k = torch.randn(n, HKV * D, generator=g).bfloat16()
    v = torch.randn(n, HKV * D, generator=g).bfloat16()
    slots = torch.arange(n) + BS          # block 1 onwards
    slots[7] = -1                          # skipped
    impl.do_kv_cache_update(None, k, v, kv, slots)
    kc, vc = kv[0].view(-1, HKV, D), kv[1].view(-1, HKV, D)
    assert torch.equal(kc[BS + 3], k[3].view(HKV, D)) and torch.equal(vc[BS + 19], v[19].view(HKV, D))
    assert float(kc[BS + 7].abs().sum()) == 0.0
    bt = torch.tensor([[1, 2, 0]], dtype=torch.int32)
    q = torch.randn(1, H * D, generator=g).bfloat16()
    md = vb.FusedInt4AttentionMetadata(1, 1, torch.tensor([0, 1], dtype=torch.int32), n,
                                       torch.tensor([n], dtype=torch.int32), bt,
                                       torch.tensor([-1]))
    out = impl.forward(None, q, k[:1], v[:1], kv, md).view(1, H, D)
    kk = kc[BS:BS + n].float().repeat_interleave(H // HKV, dim=1).transpose(0, 1)
    vv = vc[BS:BS + n].float().repeat_interleave(H // HKV, dim=1).transpose(0, 1)
    p = torch.softmax((q.view(H, 1, D).float() @ kk.transpose(1, 2)) * D ** -0.5, dim=-1)
    want = (p @ vv).view(1, H, D)
    assert torch.allclose(out.float(), want, atol=2e-2)


def test_mixed_batch_placement(vb, monkeypatch):
    """Rows 0 and 4 are decode rows (query length 1), rows 1..3 one prefill
    sequence of 3 tokens: decode outputs land at their token offsets, the
    prefill rows equal causal attention over the fresh K/V."""
    rec = Recorder(monkeypatch, vb.ops)
    impl = make_impl(vb, monkeypatch, msl=1)
    kv = torch.zeros(kv_layout.kv_cache_shape(NB, BS, HKV, D), dtype=torch.float16)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(5, H * D, generator=g).half()
    k = torch.randn(5, HKV * D, generator=g).half()
    v = torch.randn(5, HKV * D, generator=g).half()
    md = vb.FusedInt4AttentionMetadata(
        num_actual_tokens=5, max_query_len=3,
        query_start_loc=torch.tensor([0, 1, 4, 5], dtype=torch.int32), max_seq_len=40,
        seq_lens=torch.tensor([40, 3, 17], dtype=torch.int32),
        block_table=torch.arange(9, dtype=torch.int32).view(3, 3),
        slot_mapping=torch.arange(5))
    out = impl.forward(None, q, k, v, kv, md)
    assert rec.calls == ["reshape_and_cache_int4", "fused_int4_decode"]
    assert torch.all(out[0] == 100.0) and torch.all(out[4] == 101.0)
    qq = q[1:4].view(3, H, D).float().transpose(0, 1)
    kk = k[1:4].view(3, HKV, D).float().repeat_interleave(H // HKV, dim=1).transpose(0, 1)
    vv = v[1:4].view(3, HKV, D).float().repeat_interleave(H // HKV, dim=1).transpose(0, 1)
    s = (qq @ kk.transpose(1, 2)) * D ** -0.5
    s = s.masked_fill(torch.triu(torch.ones(3, 3, dtype=torch.bool), 1), float("-inf"))
    want = (torch.softmax(s, -1) @ vv).transpose(0, 1).reshape(3, H * D)
    assert torch.allclose(out[1:4].float(), want, atol=2e-3)


def test_warmup_without_metadata(vb, monkeypatch):
    Recorder(monkeypatch, vb.ops)
    impl = make_impl(vb, monkeypatch)
    q = torch.ones(3, H * D).half()
    kv = torch.zeros(kv_layout.kv_cache_shape(NB, BS, HKV, D), dtype=torch.float16)
    assert float(impl.forward(None, q, q, q, kv, None).abs().sum()) == 0.0
    o = torch.ones_like(q)
    assert impl.forward(None, q, q, q, torch.empty(0), decode_md(vb, [1], [0]), output=o) is o
    assert float(o.abs().sum()) == 0.0
