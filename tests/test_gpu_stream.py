"""The stream schedule (split_tokens = 0) of the cooperative decode kernel:
one block per CU takes an equal share of all (sequence, kv-head group) rows'
32-token tiles laid end to end, so ragged batches keep every CU busy; the
merge folds each row's per-block partials.  Checked against the oracle's
dequantise-then-SDPA path (scripts/v35_h100_bench.py:376-387) to the shared
bar (tests/tolerance.py) and against the split schedule on the same inputs.

Edge cases: zero-length sequences (NaN like the reference's 0/0, F:886-887),
lengths 1, 31, 32, 33 around the tile, batches with fewer tiles than blocks
(most blocks idle), one sequence spread over every block, several hundred
sequences (the in-kernel length scan spans several wave passes), batches
large enough that row starts are charged to the blocks, two head sets,
INT8 K and V, D = 64, bf16 q; planes the cooperative kernel does not take
(split-K inside the stream workspace) and the sequence limit."""
import numpy as np
import pytest
import torch

import knlp_amd as K
from knlp_amd import ops
from tests import kvgen, tolerance
from tests.test_gpu_decode import _build, _check, _query, _run

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lens(n, lo, hi, seed, zeros=0):
    g = np.random.default_rng(seed)
    out = g.integers(lo, hi + 1, n).tolist()
    for i in range(zeros):
        out[(7 * i + 3) % n] = 0
    return out


CASES = [
    # name, seq_lens, hq, hkv, d, kfmt, vfmt, kgs, vgs
    ("ragged_int4_asym", [1, 17, 31, 32, 33, 0, 511, 2049, 700], 32, 8, 128, 1, 1, 32, 32),
    ("sym_g64", [3000, 5, 64], 32, 8, 128, 0, 0, 64, 64),
    ("one_long_sequence", [20000], 32, 8, 128, 1, 1, 32, 32),
    ("fewer_tiles_than_blocks", [100, 3], 32, 8, 128, 1, 1, 32, 32),
    ("kint8_row_vint4_two_sets", [1100, 5, 33, 0], 40, 8, 128, 2, 1, 128, 32),
    ("kint8_vint8_row", [640, 17, 1], 32, 8, 128, 2, 2, 128, 128),
    ("kint4_vint8", [512, 64, 9], 32, 8, 128, 1, 2, 32, 32),
    ("d64_g2", [1500, 300, 1], 16, 8, 64, 1, 1, 32, 32),
    ("hkv16_two_rows_per_seq", [700, 129, 2], 64, 16, 128, 1, 1, 32, 32),
    ("int4_g6_two_sets", [1, 16, 47, 900], 48, 8, 128, 0, 0, 32, 32),
    ("many_sequences_300", _lens(300, 0, 200, 1, zeros=5), 32, 8, 128, 1, 1, 32, 32),
    ("max_sequences_1024", _lens(1024, 1, 40, 2), 32, 8, 128, 1, 1, 32, 32),
    # more than 5 tiles per block (256 CUs): each row a block starts after its
    # first is charged to it, so shares are unequal in tiles; rows shorter
    # than the charge, empty sequences, two rows per sequence
    ("charged_rows", _lens(48, 1, 3000, 3, zeros=3), 32, 8, 128, 1, 1, 32, 32),
    ("charged_short_and_long_rows", _lens(200, 1, 100, 5) + [30000, 20000, 1], 32, 8, 128, 1,
     1, 32, 32),
    ("charged_two_rows_per_seq", _lens(24, 1, 3000, 4), 64, 16, 128, 1, 1, 32, 32),
    ("charged_kint8_row_two_sets", _lens(30, 1, 3000, 6, zeros=2), 40, 8, 128, 2, 1, 128, 32),
    # fp16 K on the cooperative loader (4 kv heads per block): fp16, INT4 and
    # INT8 V; ragged rows, empty sequences, charges
    ("fp16_fp16", [1, 17, 33, 0, 900, 2049], 32, 8, 128, 3, 3, 128, 128),
    ("fp16_fp16_hkv4_g5", [700, 31, 64], 20, 4, 128, 3, 3, 128, 128),
    ("kfp16_vint4_asym", [600, 5, 0, 1500], 32, 8, 128, 3, 1, 128, 32),
    ("kfp16_vint4_sym_g64", [800, 65], 32, 8, 128, 3, 0, 128, 64),
    ("kfp16_vint8_g32", [500, 48, 1], 16, 4, 128, 3, 2, 128, 32),
    ("charged_fp16_fp16", _lens(40, 1, 3000, 7, zeros=2), 32, 8, 128, 3, 3, 128, 128),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_stream_schedule_matches_oracle(case):
    name, seq_lens, hq, hkv, d, kf, vf, kgs, vgs = case
    assert K.decode_kernel_kind(hq, hkv, d, kf, kgs, vf, vgs) == "mfma"
    print(f"stream case {name}: {len(seq_lens)} sequences, {sum(seq_lens)} tokens", flush=True)
    bt, kp, vp = _build(seq_lens, hq, hkv, d, kf, vf, kgs, vgs, seed=70)
    q = _query(len(seq_lens), hq, d, 70)
    out = _run(q, kp, vp, bt, seq_lens, hkv, d, split_tokens=0)
    _check(out, q, kp, vp, bt, seq_lens, name=f"stream_{name}")
    # the split schedule on the same inputs agrees to the bar
    split = _run(q, kp, vp, bt, seq_lens, hkv, d, split_tokens=256)
    valid = np.array([n > 0 for n in seq_lens])
    tolerance.check(f"stream_{name}_vs_split256", out.float().cpu().numpy()[valid],
                    split.float().cpu().numpy()[valid], both_rounded=True)
    again = _run(q, kp, vp, bt, seq_lens, hkv, d, split_tokens=0)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16)), "not deterministic"


def test_stream_schedule_bf16_query():
    seq_lens = [900, 1, 65]
    bt, kp, vp = _build(seq_lens, 32, 8, 128, 1, 1, 32, 32, seed=71)
    q = _query(3, 32, 128, 71, torch.bfloat16)
    out = _run(q, kp, vp, bt, seq_lens, 8, 128, split_tokens=0)
    assert out.dtype == torch.bfloat16
    _check(out, q, kp, vp, bt, seq_lens, name="stream_bf16_query")


@pytest.mark.parametrize("case", [
    # name, seq_lens, hq, hkv, d, kfmt, vfmt, kgs, vgs: planes the cooperative
    # kernel does not take run split-K inside the stream workspace (fp16 K at
    # D = 64, Hkv % 8 != 0 with packed K)
    ("fp16_k_d64_vint4", [700, 1, 0, 65], 32, 8, 64, 3, 1, 64, 32),
    ("hkv4_int4", [900, 33], 16, 4, 128, 1, 1, 32, 32),
    ("hkv4_kint8_valu", [300, 48, 0], 16, 4, 128, 2, 1, 128, 32),
], ids=lambda c: c[0])
def test_stream_request_on_other_kernels_runs_split_k(case):
    name, seq_lens, hq, hkv, d, kf, vf, kgs, vgs = case
    bt, kp, vp = _build(seq_lens, hq, hkv, d, kf, vf, kgs, vgs, seed=73)
    q = _query(len(seq_lens), hq, d, 73)
    out = _run(q, kp, vp, bt, seq_lens, hkv, d, split_tokens=0)
    _check(out, q, kp, vp, bt, seq_lens, name=f"stream_fallback_{name}")


def test_stream_schedule_sequence_limit():
    """More than 1024 sequences with split_tokens = 0 is a shape error."""
    S, hq, hkv, d, bs = 1025, 32, 8, 128, 16
    kp = kvgen.empty_plane(1, S + 1, bs, hkv, d, 32)
    vp = kvgen.empty_plane(1, S + 1, bs, hkv, d, 32)
    kd, ks, kz = kvgen.plane_to_torch(kp, DEV)
    vd, vs, vz = kvgen.plane_to_torch(vp, DEV)
    bt = torch.arange(S, dtype=torch.int32, device=DEV)[:, None]
    sl = torch.full((S,), 16, dtype=torch.int32, device=DEV)
    q = torch.zeros(S, hq, d, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="shape"):
        ops._decode(q, ops._plane(kd, ks, kz, 1, 32), ops._plane(vd, vs, vz, 1, 32), bs, bt, sl,
                    hkv, d, split_tokens=0)
    torch.cuda.synchronize()


@pytest.mark.parametrize("seq_lens", [[1, 17, 31, 32, 33, 0, 511, 2049, 700], [3000, 2, 0, 90],
                                      _lens(40, 0, 3000, 6, zeros=4)],
                         ids=["fewer_tiles_than_blocks", "more_tiles_than_blocks",
                              "charged_rows"])
def test_stream_schedule_reads_only_what_it_wrote(seq_lens):
    """The workspace filled with NaN before the call: every partial the merge
    reads was written by this launch (a stale or unwritten entry would
    surface as NaN in a sequence of nonzero length)."""
    import ctypes
    from knlp_amd import _lib
    hq, hkv, d = 32, 8, 128
    bt, kp, vp = _build(seq_lens, hq, hkv, d, 1, 1, 32, 32, seed=72)
    q = _query(len(seq_lens), hq, d, 72).to(DEV)
    kd, ks, kz = kvgen.plane_to_torch(kp, DEV)
    vd, vs, vz = kvgen.plane_to_torch(vp, DEV)
    kpl, vpl = ops._plane(kd, ks, kz, 1, 32), ops._plane(vd, vs, vz, 1, 32)
    btd = torch.from_numpy(bt).to(DEV)
    sl = torch.tensor(seq_lens, dtype=torch.int32, device=DEV)
    L = _lib.lib()
    S, mc = len(seq_lens), bt.shape[1] * 16
    nbytes = L.knlp_kv_decode_workspace_bytes(S, hq, d, mc, 0)
    assert nbytes > 0
    ws = torch.full(((nbytes + 3) // 4,), float("nan"), dtype=torch.float32, device=DEV)
    out = torch.empty_like(q)
    st = L.knlp_kv_decode(q.data_ptr(), _lib.DT_F16, q.stride(0), q.stride(1), S, hq, hkv, d,
                          ctypes.byref(kpl), ctypes.byref(vpl), btd.data_ptr(), btd.stride(0),
                          sl.data_ptr(), 16, mc, d ** -0.5, 0, ws.data_ptr(), nbytes,
                          out.data_ptr(), _lib.DT_F16, out.stride(0), out.stride(1),
                          ops._stream())
    assert st == 0
    torch.cuda.synchronize()
    _check(out.cpu(), q.cpu(), kp, vp, bt, seq_lens, name="stream_nan_workspace")


@pytest.mark.parametrize("bs", [32, 64])
def test_stream_schedule_other_block_sizes(bs):
    """Pages of 32 and 64 tokens: a 32-token tile then lies within one page
    (both 16-token halves), and a row's segment can start mid-page."""
    seq_lens = [1000, 33, 0, 517, 64]
    bt, kp, vp = _build(seq_lens, 32, 8, 128, 1, 1, 32, 32, seed=74, bs=bs)
    q = _query(len(seq_lens), 32, 128, 74)
    out = _run(q, kp, vp, bt, seq_lens, 8, 128, split_tokens=0)
    _check(out, q, kp, vp, bt, seq_lens, name=f"stream_block_size_{bs}")


def test_stream_schedule_all_sequences_empty():
    """No tiles at all: every block returns at once and every output is NaN
    (0/0, like the reference's acc / l with l = 0, F:886-887)."""
    seq_lens = [0, 0, 0]
    bt, kp, vp = _build(seq_lens, 32, 8, 128, 1, 1, 32, 32, seed=75)
    q = _query(3, 32, 128, 75)
    out = _run(q, kp, vp, bt, seq_lens, 8, 128, split_tokens=0)
    assert torch.isnan(out.float()).all()


def _random_pages(lens, hq, hkv, d, kint8, seed):
    """A paged batch with random codes and scales generated on the device (any
    byte is a valid code): sizes beyond what the oracle decodes in a test."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    bs = 16
    pages = [-(-int(n) // bs) for n in lens]
    nb = sum(pages) + 5
    width = max(max(pages), 1)
    perm = torch.randperm(nb, generator=g, device=DEV).to(torch.int32)
    bt = torch.zeros(len(lens), width, dtype=torch.int32, device=DEV)
    cur = 0
    for s, p in enumerate(pages):
        bt[s, :p] = perm[cur:cur + p]
        cur += p

    def scales(ng):
        return (0.05 + 0.15 * torch.rand(nb, bs, hkv, ng, generator=g, device=DEV)).half()

    # the planes hold raw pointers: every tensor stays referenced in `keep`
    if kint8:
        kd = torch.randint(-127, 128, (nb, bs, hkv, d), generator=g, device=DEV).to(torch.int8)
        ks, kz = scales(1), None
        kp = ops._plane(kd, ks, kz, 2, d)
    else:
        kd = torch.randint(0, 256, (nb, bs, hkv, d // 2), generator=g, device=DEV).to(torch.uint8)
        ks = scales(d // 32)
        kz = (-8 * ks.float()).half()
        kp = ops._plane(kd, ks, kz, 1, 32)
    vd = torch.randint(0, 256, (nb, bs, hkv, d // 2), generator=g, device=DEV).to(torch.uint8)
    vs = scales(d // 32)
    vz = (-8 * vs.float()).half()
    vp = ops._plane(vd, vs, vz, 1, 32)
    q = torch.randn(len(lens), hq, d, generator=g, device=DEV).half()
    keep = (kd, ks, kz, vd, vs, vz)
    return q, kp, vp, bt, torch.tensor(lens, dtype=torch.int32, device=DEV), keep


@pytest.mark.parametrize("trial", range(12))
def test_stream_matches_split_on_random_batches(trial):
    """Random batches of 1-700 sequences with lengths from three mixes
    (uniform up to 12000 tokens; extremes 0/1/31/33/100/4000/12000; heavy
    tailed), one or two kv-head groups, INT4 or INT8 K: the stream schedule,
    with or without row charges (depending on the batch's size), gives what
    split-K gives, to the bar, and the same bits twice.  A tile dropped or
    taken twice by a block's share, or a partial merged from a wrong entry,
    shows up as a difference."""
    g = np.random.default_rng(500 + trial)
    S = int(g.choice([1, 3, 17, 64, 200, 700]))
    mix = trial % 3
    if mix == 0:
        lens = g.integers(0, 12001, S)
    elif mix == 1:
        lens = g.choice([0, 1, 31, 33, 100, 4000, 12000], S)
    else:
        lens = np.minimum((g.pareto(1.2, S) * 300).astype(np.int64), 12000)
    lens = [int(x) for x in lens]
    while sum(lens) > 2_000_000:                   # bound the pool at about 2 GB
        lens = lens[: len(lens) // 2]
    hkv = 16 if trial % 4 == 3 else 8
    kint8 = trial % 5 == 4
    hq = (5 if kint8 else 4) * hkv
    tiles = sum(-(-n // 32) for n in lens) * (hkv // 8)
    print(f"random batch {trial}: {len(lens)} sequences, {sum(lens)} tokens, {tiles} row "
          f"tiles, hkv {hkv}, k {'int8' if kint8 else 'int4'}", flush=True)
    q, kp, vp, bt, sl, keep = _random_pages(lens, hq, hkv, 128, kint8, 900 + trial)

    def run(split):
        out = ops._decode(q, kp, vp, 16, bt, sl, hkv, 128, split_tokens=split)
        torch.cuda.synchronize()
        return out

    stream = run(0)
    split = run(512)
    valid = np.array([n > 0 for n in lens])
    tolerance.check(f"stream_random_{trial}_vs_split512", stream.float().cpu().numpy()[valid],
                    split.float().cpu().numpy()[valid], both_rounded=True)
    assert torch.isnan(stream.float().cpu()[~torch.from_numpy(valid)]).all()
    assert torch.equal(stream.view(torch.int16), run(0).view(torch.int16)), "not deterministic"
    del keep
