"""The merge's three kernels and its fold's group sizes, against the oracle.

The merge folds each (sequence, q head)'s partials in groups of 8, then one
group of 4, 2 and 1 (every load in a group is of a real partial), either with
one wave per head (merge_wave_kernel: at most 2 partials, or at most 16 with
more than 2048 heads in the batch), one workgroup per 16-dim slice of a head
(merge_slice_kernel: at most 256 heads in the batch with at least 64
partials each; 16 split lanes taking every 16th partial) or four to sixteen
waves per head (merge_kernel, waves taking every 4th partial).  64-token splits over lengths
0-1024 give every partial count from 0 to 16 in one batch, so every tail of
the fold runs; empty sequences must give NaN (0/0, F:886-887).  Checked
against the oracle's dequantise -> SDPA (scripts/v35_h100_bench.py:376-387)
to the shared bar (tests/tolerance.py)."""
import numpy as np
import pytest

from tests.test_gpu_decode import _build, _check, _query, _run

pytestmark = pytest.mark.gpu


def _lens(n, lo, hi, seed, zeros=()):
    g = np.random.default_rng(seed)
    out = g.integers(lo, hi + 1, n).tolist()
    for i in zeros:
        out[i] = 0
    return out


@pytest.mark.parametrize("case", [
    # name, seq_lens, hq, d, split: one wave per head (80 x 32 heads > 2048), 0-16 partials
    ("wave_kernel_all_counts", _lens(80, 1, 1024, 11, zeros=(3, 40)) + list(range(1, 1025, 64)),
     32, 128, 64),
    # one wave per head (at most 2 partials) with few heads; D = 64 and 256 (1 and 4
    # elements per lane)
    ("wave_kernel_few_heads", [1, 64, 65, 128, 0, 100], 32, 128, 64),
    ("wave_kernel_d64", [1, 64, 100, 0, 128], 16, 64, 64),
    ("wave_kernel_d256", [1, 64, 100, 128], 64, 256, 64),
    # four waves per head (8 x 32 heads), 5-16 partials: every tail at step 4
    ("four_waves_tails", [300, 400, 449, 513, 640, 705, 900, 1024], 32, 128, 64),
    # sixteen waves per head: 80 partials over 96 heads (above the slice
    # kernel's 256 heads: 9 x 32)
    ("sixteen_waves", [5100, 77, 0, 700, 5000, 4500, 64, 3000, 1], 32, 128, 64),
    # one workgroup per 16-dim slice: 0-100 partials per head, so every split
    # lane folds 0-7 of them (each fold tail) and some fold none
    ("slice_kernel_counts", [0, 1, 64, 65, 1000, 4101, 6400], 32, 128, 64),
    ("slice_kernel_d64", [4100, 33, 0], 16, 64, 64),
    ("slice_kernel_d256", [4100, 700], 32, 256, 64),
    ("slice_kernel_d32", [4100, 129], 32, 32, 64),
], ids=lambda c: c[0])
def test_merge_kernels_and_fold_tails(case):
    name, seq_lens, hq, d, split = case
    print(f"merge case {name}: {len(seq_lens)} sequences, d {d}, split {split}", flush=True)
    bt, kp, vp = _build(seq_lens, hq, 8, d, 1, 1, 32, 32, seed=80)
    q = _query(len(seq_lens), hq, d, 80)
    out = _run(q, kp, vp, bt, seq_lens, 8, d, split_tokens=split)
    _check(out, q, kp, vp, bt, seq_lens, name=f"merge_{name}")
