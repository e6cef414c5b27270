"""bench.py's byte accounting and synthetic inputs, on the CPU.

Every roofline figure divides bench.algorithmic_bytes by a time, so the byte
counts are pinned here against numbers derived by hand from the reference's
cache layout (per token and kv head: D/2 code bytes plus 2 bytes per scale and
per zero point for each of D/G groups, F:2122-2158 and the planner
fused-quant/support/attention.v0.1.0.py:545-584; D bytes plus one fp16 scale
for per-row INT8 K, F:1270-1284; 2D for fp16), not against bench's own
formula."""
import numpy as np
import pytest

import bench

BS = 16


def kv_bytes(c, kfmt=None, vfmt=None):
    cfg = bench.CONFIGS[c]
    kfmt = kfmt or cfg["kfmt"]
    vfmt = vfmt or cfg["vfmt"]
    sl = bench.make_seq_lens(cfg, 5000 + c)
    total = bench.algorithmic_bytes(cfg, sl, kfmt, vfmt, BS)
    qo = 2 * cfg["B"] * cfg["Hq"] * cfg["D"] * 2
    bt = sum(-(-int(n) // BS) for n in sl) * 4 + cfg["B"] * 4
    return total - qo - bt, sl


# K + V bytes per decode step at the BASELINE shapes, worked out by hand:
#   1: 1 seq x 1024 tok x 12 heads x 2 x (32 + 2*2*2)            =       983,040
#   2: 8 x 32768 x 8 x 2 x (64 + 4*2*2)                          =   335,544,320
#   4: 1 x 393216 x 8 x 2 x (64 + 2*2*2)                         =   452,984,832
#   5: 16 x 65537 x 8 x ((128 + 2) + (64 + 4*2*2))  (T + 1 after the append)
#   6: 8 x 32768 x 8 x 2 x (64 + 4*2)                            =   301,989,888
@pytest.mark.parametrize("c,expect", [
    (1, 983_040),
    (2, 335_544_320),
    (4, 452_984_832),
    (5, 16 * 65_537 * 8 * 210),
    (6, 301_989_888),
])
def test_kv_bytes_match_hand_counts(c, expect):
    got, _ = kv_bytes(c)
    assert got == expect


def test_fp16_leg_bytes():
    # 8 x 32768 x 8 x 2 x 256 = 1 GiB at config 2
    got, _ = kv_bytes(2, "fp16", "fp16")
    assert got == 1 << 30


def test_config2_step_and_launch_bytes():
    """The whole step adds q in, out, the block table and seq_lens; the
    partial launch is the step without the merge's output."""
    cfg = bench.CONFIGS[2]
    sl = bench.make_seq_lens(cfg, 5002)
    step = bench.algorithmic_bytes(cfg, sl, "int4_asym", "int4_asym", BS)
    q = 8 * 32 * 128 * 2
    table = 8 * (32768 // BS) * 4 + 8 * 4
    assert step == 335_544_320 + 2 * q + table == 335_740_960
    assert step - q == 335_675_424


def test_paged_config_inputs():
    cfg = bench.CONFIGS[3]
    sl = bench.make_seq_lens(cfg, 5003)
    assert sl.shape == (64,)
    assert sl.min() >= 512 and sl.max() <= 16384
    assert np.array_equal(sl, bench.make_seq_lens(cfg, 5003))          # seeded
    assert not np.array_equal(sl, bench.make_seq_lens(cfg, 5004))
    bt, pool = bench.make_block_table(cfg, sl, BS, 6003)
    assert pool == 1 << 18
    assert bt.shape == (64, -(-int(sl.max()) // BS))
    used = np.concatenate([bt[s, :-(-int(n) // BS)] for s, n in enumerate(sl)])
    assert used.min() >= 0 and used.max() < pool
    assert np.unique(used).size == used.size        # slices of one permutation
    # the permutation scatters pages over the whole pool
    assert used.max() - used.min() > pool // 2


def test_uniform_config_inputs():
    for c in (1, 2, 4, 6):
        cfg = bench.CONFIGS[c]
        sl = bench.make_seq_lens(cfg, 5000 + c)
        assert sl.shape == (cfg["B"],) and np.all(sl == cfg["T"])
    sl5 = bench.make_seq_lens(bench.CONFIGS[5], 5005)
    assert np.all(sl5 == 65_537)                       # decodes over T + 1


def test_more_than_one_gpu_is_refused():
    assert bench.main(["--gpus", "2"]) == 2
