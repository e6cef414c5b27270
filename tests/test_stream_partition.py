"""Invariants of the stream schedule's partition, on the CPU.

The cooperative decode kernel's stream schedule (split_tokens = 0) lays all
(sequence, group of 8 kv heads) rows end to end, each row as `cost` charged
positions (no work) then its 32-token tiles, and gives block b < Pe =
min(P, T) the positions [b T / Pe, (b + 1) T / Pe).  Charges apply only when
the batch has at least (cost + 1) P tiles, and not when every non-empty row
has the same tile count and the rows divide the blocks taking part (the rows
then start on share boundaries: split-K's partition of a uniform batch).  A block writes one partial per row
it holds tiles of, at entry (b + row) * HG + head; the block holding a row's
first tile records the row's first entry and its block count, computed as
(last tile's block) - b + 1 with the last tile's block
floor((t_last Pe + Pe - 1) / T).  The merge then reads `count` entries
HG apart from the first.

This restates the partition (the position arithmetic is the kernel's; the
checks are not) and checks, over random batches up to the schedule's limits
(1024 sequences, 2^25 tokens of context), what the merge and the workspace
size rely on: every tile is computed exactly once; a row's tiles are held by
consecutive blocks, each holding at least one; the recorded count is that
number of blocks; entries are distinct and inside the workspace's
(P + num_seqs) * hq entries; with charges every block holds a tile; shares
differ by at most one position.  The GPU tests check the kernel's results
against the oracle and split-K on the same kinds of batches.
"""
import numpy as np
import pytest

COST = 6          # the library's charge (tiles) per row a block starts mid-share


def _partition(lens, max_context, nhg, P, cost_param=COST, always_charge=False):
    n = [(max(0, min(x, max_context)) + 31) // 32 for x in lens]
    tiles = nhg * sum(n)
    ne = [x for x in n if x > 0]
    aligned = len(set(ne)) == 1 and min(P, tiles) % (nhg * len(ne)) == 0
    cost = cost_param if always_charge or (not aligned and tiles >= (cost_param + 1) * P) else 0
    rows = []                        # (seq, hg, first position, n)
    pos = 0
    for s, ns in enumerate(n):
        if ns == 0:
            continue
        for hg in range(nhg):
            rows.append((s, hg, pos, ns))
            pos += cost + ns
    T = pos
    Pe = min(P, T)
    return rows, T, Pe, cost


def _count(t_last, Pe, T, b):
    return (t_last * Pe + Pe - 1) // T - b + 1


def _check(lens, max_context, nhg, P, group, count_fn=_count, always_charge=False):
    rows, T, Pe, cost = _partition(lens, max_context, nhg, P, always_charge=always_charge)
    HG = 8 * group
    hq = HG * nhg
    S = len(lens)
    bounds = [b * T // Pe for b in range(Pe + 1)] if Pe else [0]
    if Pe:
        sizes = np.diff(bounds)
        assert sizes.max() - sizes.min() <= 1
    covered = {}
    holders = {}
    entries = set()
    tiles_per_block = [0] * max(Pe, 1)
    for b in range(Pe):
        f, fe = bounds[b], bounds[b + 1]
        for r, (s, hg, start, ns) in enumerate(rows):
            r0 = start + cost                           # the row's first tile
            lo, hi = max(f, r0), min(fe, r0 + ns)
            if lo >= hi:
                continue
            row = s * nhg + hg
            for t in range(lo - r0, hi - r0):
                assert (r, t) not in covered
                covered[(r, t)] = b
            holders.setdefault(r, []).append(b)
            tiles_per_block[b] += hi - lo
            e = (b + row) * HG
            assert e not in entries
            entries.add(e)
            assert e + HG <= (P + S) * hq               # inside the workspace
            if lo == r0:                                # holds the row's first tile
                t_last = r0 + ns - 1
                count = count_fn(t_last, Pe, T, b)
                assert count >= 1
                holders.setdefault(("count", r), count)
    for r, (s, hg, start, ns) in enumerate(rows):
        for t in range(ns):
            assert (r, t) in covered                    # every tile exactly once
        hb = holders[r]
        assert hb == list(range(hb[0], hb[0] + len(hb)))   # consecutive blocks
        assert holders[("count", r)] == len(hb)
    if cost:
        assert min(tiles_per_block) >= 1
    return cost


def _lens(g, S, kind, max_context):
    if kind == 0:
        return g.integers(0, max_context + 1, S).tolist()
    if kind == 1:
        return g.choice([0, 1, 31, 32, 33, 200, max_context], S).tolist()
    x = np.minimum((g.pareto(1.1, S) * 200).astype(np.int64), max_context)
    return x.tolist()


@pytest.mark.parametrize("seed", range(40))
def test_partition_invariants_random_batches(seed):
    g = np.random.default_rng(seed)
    P = int(g.choice([8, 64, 256]))
    S = int(g.choice([1, 2, 5, 40, 200]))
    max_context = int(g.choice([100, 2048, 16384]))
    nhg = int(g.choice([1, 2]))
    group = int(g.choice([1, 4, 5]))
    for kind in range(3):
        _check(_lens(g, S, kind, max_context), max_context, nhg, P, group)


def test_partition_charges_apply_at_config3_shape():
    """Config 3's batch (bench.py's lengths: 64 sequences of 512-16384 tokens,
    256 CUs) is charged; without charges 60 of its 256 blocks hold two rows
    (the tail the charges remove)."""
    import torch
    g = torch.Generator().manual_seed(5003)
    lens = torch.randint(512, 16385, (64,), generator=g).tolist()
    assert _check(lens, 16384, 1, 256, 4) == COST
    rows, T, Pe, cost = _partition(lens, 16384, 1, 256, cost_param=0)
    assert cost == 0
    two = 0
    for b in range(Pe):
        f, fe = b * T // Pe, (b + 1) * T // Pe
        two += sum(1 for (_, _, start, ns) in rows if max(f, start) < min(fe, start + ns)) >= 2
    assert two == 60


def test_partition_checks_catch_planted_mistakes():
    """The checks fail for plausible mistakes: the block count without the
    round-up, and charges on a batch too small for every block to hold a tile."""
    g = np.random.default_rng(1)
    trunc = lambda t_last, Pe, T, b: (t_last * Pe) // T - b + 1
    failed = 0
    for _ in range(20):
        try:
            _check(_lens(g, 40, 0, 2048), 2048, 1, 256, 4, count_fn=trunc)
        except AssertionError:
            failed += 1
    assert failed > 0
    with pytest.raises(AssertionError):
        _check([100, 40, 3], 2048, 1, 256, 4, always_charge=True)


def test_partition_limits():
    """1024 sequences at the context limit (positions fit 32 bits), and
    batches with fewer tiles than blocks (uncharged, Pe = T)."""
    rows, T, Pe, cost = _partition([1 << 25] * 1024, 1 << 25, 1, 256)
    assert cost == COST and T < 2 ** 31
    assert _check([1, 17, 0, 33], 2048, 1, 256, 4) == 0
    assert _check([0, 0], 2048, 1, 256, 4) == 0
    # one sequence's two equal rows over 8 blocks: aligned, uncharged
    assert _check([5000], 8192, 2, 8, 5) == 0
    assert _check([5000, 3000], 8192, 2, 8, 5) == COST


def test_uniform_batches_get_split_k_partition():
    """Equal rows whose count divides the blocks: no charges, and block b
    holds tiles [b k, (b + 1) k) of row b // (blocks per row), which is
    split-K's partition (config 2: 8 rows of 1024 tiles over 256 blocks, 32
    tiles each; config 8: 16 rows).  Equal rows that do not divide the
    blocks (3 rows over 256) or unequal rows keep the charges.  (Shares within
    a row may differ by a tile, as split-K's splits do at the row's end.)"""
    for S, T, nhg in ((8, 32768, 1), (16, 32768, 1), (4, 32768, 2), (1, 393216, 1),
                      (64, 16384, 1), (32, 65536 + 32, 1)):
        rows, Tp, Pe, cost = _partition([T] * S, T, nhg, 256)
        assert cost == 0, (S, T)
        bpr = Pe // len(rows)                           # blocks per row
        for b in range(Pe):
            f, fe = b * Tp // Pe, (b + 1) * Tp // Pe
            held = [r for r, (_, _, st, ns) in enumerate(rows) if max(f, st) < min(fe, st + ns)]
            assert held == [b // bpr]
        _check([T] * S, T, nhg, 256, 4)
    assert _partition([65536] * 3, 65536, 1, 256)[3] == COST
    assert _partition([16384] * 63 + [16000], 16384, 1, 256)[3] == COST


def _share_bound(x, T, Pe):
    """The kernel's floor(x T / Pe) (x <= Pe <= 2^16): T = q Pe + r, then
    x q + floor(x r / Pe) with x r in 32 bits."""
    q, r = T // Pe, T % Pe
    xr = (x * r) & 0xFFFFFFFF
    assert xr == x * r                                  # fits the kernel's 32 bits
    return x * q + xr // Pe


def _block_of_position(t, T, Pe):
    """The kernel's floor((t Pe + Pe - 1) / T): an fp64 quotient when T < 2^32."""
    num = t * Pe + Pe - 1
    if T < 2 ** 32:
        return int(np.floor(np.float64(num) / np.float64(T)))
    return num // T


def test_stream_start_arithmetic_is_exact():
    """The stream schedule's share bounds and record counts use 32-bit and
    fp64 divisions in place of 64-bit ones; both equal exact integer
    arithmetic over random and boundary values (T up to 2^40, Pe up to
    1024), and the fp64 path is the one taken for T < 2^32."""
    g = np.random.default_rng(7)
    cases = []
    for _ in range(20000):
        Pe = int(g.choice([1, 7, 255, 256, 1024]))
        T = int(g.choice([Pe, Pe + 1, 2 ** 31 - 1, 2 ** 32 - 1, 2 ** 32 + 5, 2 ** 40 - 3,
                          int(g.integers(Pe, 2 ** 33))]))
        cases.append((Pe, T))
    for Pe, T in cases:
        for x in (0, 1, Pe - 1, Pe, int(g.integers(0, Pe + 1))):
            assert _share_bound(x, T, Pe) == x * T // Pe
        for t in (0, T - 1, T // 2, int(g.integers(0, T))):
            b = _block_of_position(t, T, Pe)
            assert b == (t * Pe + Pe - 1) // T
            assert b * T // Pe <= t < (b + 1) * T // Pe       # the block holding t
    # planted mistakes fail these checks: the share bound without its
    # remainder term, and the record's block without the round-up
    assert any(x * (T // Pe) != x * T // Pe for Pe, T in cases[:200] for x in (Pe - 1,))
    assert any((t * Pe) // T != (t * Pe + Pe - 1) // T
               for Pe, T in cases[:200] for t in (T - 1, T // 3) if Pe > 1)
