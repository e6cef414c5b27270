"""HIP-graph capture of the decode entry points (the reference's backend
captures its decode steps, F:2185; the library promises no allocation and no
synchronisation inside its calls).  Each graph is replayed several times with
eager work in between, and every replay must equal the eager result bit for
bit."""
import numpy as np
import pytest
import torch

import knlp_amd as K
from tests import kvgen

pytestmark = pytest.mark.gpu

BS = 16


def _caches(seq_lens, hq, hkv, d, seed, dev):
    nb = sum(-(-n // BS) for n in seq_lens) + 2
    bt = kvgen.paged_table(seq_lens, BS, nb, seed)
    planes = []
    for i in range(2):
        p = kvgen.empty_plane(1, nb, BS, hkv, d, 32)
        rows = kvgen.randn((nb * BS, hkv, d), seed + 1 + i).float().numpy()
        kvgen.fill_plane(p, rows, np.arange(nb * BS))
        planes.append(kvgen.plane_to_torch(p, dev))
    q = kvgen.randn((len(seq_lens), hq, d), seed + 5).to(dev)
    return planes, torch.from_numpy(bt).to(dev), q


@pytest.mark.parametrize("hkv,split", [(8, None), (4, None), (8, 0), (4, 0)],
                         ids=["cooperative", "per_head", "stream", "stream_fallback_split_k"])
def test_decode_graph_replays_match_eager(hkv, split):
    """split 0: the stream schedule (its workspace records and header are
    written by kernels, not memsets); with Hkv = 4 the planes fall back to
    split-K inside that workspace, whose header a one-wave kernel writes."""
    dev = torch.device("cuda")
    hq, d = 4 * hkv, 128
    seq_lens = [1500, 77, 4096]
    (kp, vp), bt, q = _caches(seq_lens, hq, hkv, d, 60, dev)
    sl = torch.tensor(seq_lens, dtype=torch.int32, device=dev)

    def step():
        return K.fused_int4_decode(q, kp[0], vp[0], kp[1], vp[1], bt, sl, hkv, d,
                                   k_zeros=kp[2], v_zeros=vp[2], asymmetric=True,
                                   split_tokens=split)

    want = step()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):                 # warm the caching allocator off-graph
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = step()
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {r}"
        eager = step()                         # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager.view(torch.int16), want.view(torch.int16))


def test_append_and_decode_graph():
    """The fused append inside a captured decode: replays rewrite the same
    token (idempotent) and return the eager output each time."""
    dev = torch.device("cuda")
    hq, hkv, d = 32, 8, 128
    seq_lens = [513, 1024]
    (kp, vp), bt, q = _caches(seq_lens, hq, hkv, d, 70, dev)
    sl = torch.tensor(seq_lens, dtype=torch.int32, device=dev)
    pos = np.array(seq_lens) - 1
    btn = bt.cpu().numpy()
    slots = torch.from_numpy(btn[np.arange(2), pos // BS].astype(np.int64) * BS + pos % BS).to(dev)
    nk = kvgen.randn((2, hkv, d), 71).to(dev)
    nv = kvgen.randn((2, hkv, d), 72).to(dev)

    def step():
        return K.append_and_decode(q, nk, nv, slots, kp[0], vp[0], kp[1], vp[1], bt, sl, hkv, d,
                                   k_zeros=kp[2], v_zeros=vp[2], asymmetric=True)

    want = step()
    kc = kp[0].clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = step()
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {r}"
        assert torch.equal(kp[0], kc)


@pytest.mark.parametrize("hkv,split", [(8, 256), (4, None), (8, None)],
                         ids=["cooperative_split_k", "per_head", "stream_by_plan"])
def test_decode_graph_replays_with_new_lengths_tables_and_queries(hkv, split):
    """A serving loop captures the decode once and, before every replay, writes
    the step's sequence lengths, block table and queries into the captured
    buffers (the reference's backend does this for its captured decode steps,
    F:2185).  Each replay must equal an eager call on the same buffer contents,
    so nothing of the launch may depend on the lengths seen at capture."""
    dev = torch.device("cuda")
    hq, d = 4 * hkv, 128
    steps = [[1500, 77, 4096], [4200, 1, 2048], [33, 4100, 640], [1, 1, 1], [2049, 3000, 4200]]
    width = -(-max(max(s) for s in steps) // BS)
    nb = max(sum(-(-n // BS) for n in s) for s in steps) + 3
    planes = []
    for i in range(2):
        p = kvgen.empty_plane(1, nb, BS, hkv, d, 32)
        rows = kvgen.randn((nb * BS, hkv, d), 80 + i).float().numpy()
        kvgen.fill_plane(p, rows, np.arange(nb * BS))
        planes.append(kvgen.plane_to_torch(p, dev))
    kp, vp = planes
    bt = torch.zeros((3, width), dtype=torch.int32, device=dev)
    sl = torch.zeros(3, dtype=torch.int32, device=dev)
    q = torch.zeros((3, hq, d), dtype=torch.float16, device=dev)

    def load(r):
        lens = steps[r]
        bt.copy_(torch.from_numpy(kvgen.paged_table(lens, BS, nb, 90 + r, max_blocks=width)))
        sl.copy_(torch.tensor(lens, dtype=torch.int32))
        q.copy_(kvgen.randn((3, hq, d), 100 + r))

    def step():
        return K.fused_int4_decode(q, kp[0], vp[0], kp[1], vp[1], bt, sl, hkv, d,
                                   k_zeros=kp[2], v_zeros=vp[2], asymmetric=True,
                                   split_tokens=split)

    load(0)
    step()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):                 # warm the caching allocator off-graph
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = step()
    for r in range(len(steps)):
        load(r)
        g.replay()
        torch.cuda.synchronize()
        replayed = got.clone()
        want = step()                          # eager on the same buffers
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int16), want.view(torch.int16)), \
            f"replay {r} lens {steps[r]}"
        assert torch.isfinite(replayed.float()).all()
