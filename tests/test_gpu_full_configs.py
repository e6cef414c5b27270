"""The BASELINE configurations 2-5 at their full size on the GPU.

The oracle cannot decode whole batches of these sizes in the test budget, so
the checks are the size-independent properties the reference's own at-shape
validation relies on (scripts/v35_h100_bench.py:634-688), plus an oracle
comparison on one sampled (sequence, kv head):

* the library's plan (split-K, or the stream schedule at config 3) and other
  split lengths, and the stream schedule, agree within the bar (split-count
  invariance: the same attention, other summation orders);
* two runs are bit-identical (determinism);
* every output is finite;
* a physical permutation of the pages with the block table permuted to
  match gives bit-identical output (config 2);
* the fused append + decode equals the separate append then decode, caches
  and output bit for bit (config 5);
* the sampled (sequence, kv head) matches the oracle's dequantise -> SDPA.

Inputs follow the measurement plan's seeds (q 1000+c, K 2000+c, V 3000+c,
lengths 5000+c, page permutation 6000+c), generated on the device; the caches
are filled by the append kernel (bit-exact with the oracle elsewhere).
Config 3 uses the full 2^18-page pool (K code offsets reach 2 GiB).
"""
import numpy as np
import pytest
import torch

import knlp_amd as K
from knlp_amd import _lib, ops
from oracle import attention as A
from tests import tolerance

pytestmark = pytest.mark.gpu
DEV = "cuda"
BS = 16
FMT = {"int4_asym": 1, "int4_sym": 0, "int8": 2}

CONFIGS = {
    2: dict(B=8, Hq=32, Hkv=8, T=32768, k="int4_asym", v="int4_asym", kgs=32, vgs=32,
            outliers=0.01, paged=False),
    3: dict(B=64, Hq=32, Hkv=8, T=16384, k="int4_asym", v="int4_asym", kgs=32, vgs=32,
            outliers=0.01, paged=True),
    4: dict(B=1, Hq=32, Hkv=8, T=393216, k="int4_asym", v="int4_asym", kgs=64, vgs=64,
            outliers=0.0, paged=False),
    5: dict(B=16, Hq=40, Hkv=8, T=65536, k="int8", v="int4_asym", kgs=128, vgs=32,
            outliers=0.0, paged=False),
}
D = 128


def _rows(n, hkv, seed, outliers):
    """Seeded N(0,1) fp16 rows [n, hkv, D] on the device, 1 % of the
    (head, channel) pairs x20 when asked."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    mask = torch.ones(hkv * D, device=DEV)
    if outliers > 0:
        k = max(1, int(round(outliers * hkv * D)))
        mask[torch.randperm(hkv * D, generator=g, device=DEV)[:k]] = 20.0
    out = torch.empty(n, hkv, D, dtype=torch.float16, device=DEV)
    step = 1 << 18
    for i in range(0, n, step):
        m = min(step, n - i)
        out[i:i + m] = (torch.randn(m, hkv, D, generator=g, device=DEV) *
                        mask.view(hkv, D)).to(torch.float16)
    return out


class Plane:
    def __init__(self, fmt, gs, nb, hkv):
        self.fmt, self.gs = fmt, gs
        dt = torch.int8 if fmt == "int8" else torch.uint8
        self.data = torch.zeros(nb, BS, hkv, D if fmt == "int8" else D // 2, dtype=dt, device=DEV)
        self.scales = torch.zeros(nb, BS, hkv, D // gs, dtype=torch.float16, device=DEV)
        self.zeros = torch.zeros_like(self.scales) if fmt == "int4_asym" else None

    def fill(self, rows, slots):
        if self.fmt == "int8":
            K.reshape_and_cache_k_int8(rows, self.data, self.scales, slots, group_size=self.gs)
        else:
            K.reshape_and_cache_v_only_int4(rows, self.data, self.scales, slots, self.zeros,
                                            asymmetric=self.fmt == "int4_asym",
                                            group_size=self.gs)

    def plane(self):
        return ops._plane(self.data, self.scales, self.zeros, FMT[self.fmt], self.gs)

    def host(self, blocks, kvh):
        """numpy plane of the given blocks and one kv head (oracle input)."""
        sl = lambda t: None if t is None else t[blocks][:, :, kvh:kvh + 1].cpu().numpy()
        return {"format": self.fmt, "data": sl(self.data), "scales": sl(self.scales),
                "zeros": sl(self.zeros), "group_size": self.gs}


def _build(c):
    cfg = CONFIGS[c]
    B, hkv = cfg["B"], cfg["Hkv"]
    if cfg["paged"]:
        g = torch.Generator().manual_seed(5000 + c)
        lens = torch.randint(512, 16385, (B,), generator=g).numpy().astype(np.int64)
        pool = 1 << 18
        perm = torch.randperm(pool, generator=torch.Generator().manual_seed(6000 + c)).numpy()
    else:
        lens = np.full(B, cfg["T"], np.int64)
        pool = B * (cfg["T"] // BS)
        perm = np.arange(pool)
    width = int(-(-lens.max() // BS))
    bt = np.zeros((B, width), np.int32)
    cur = 0
    for s, n in enumerate(lens):
        nb = int(-(-n // BS))
        bt[s, :nb] = perm[cur:cur + nb]
        cur += nb
    bt_d = torch.from_numpy(bt).to(DEV)
    slots = torch.cat([bt_d[s, torch.arange(int(n), device=DEV) // BS].long() * BS +
                       torch.arange(int(n), device=DEV) % BS for s, n in enumerate(lens)])
    kp = Plane(cfg["k"], cfg["kgs"], pool, hkv)
    vp = Plane(cfg["v"], cfg["vgs"], pool, hkv)
    kp.fill(_rows(slots.numel(), hkv, 2000 + c, cfg["outliers"]), slots)
    vp.fill(_rows(slots.numel(), hkv, 3000 + c, cfg["outliers"]), slots)
    q = (torch.randn(B, cfg["Hq"], D, generator=torch.Generator().manual_seed(1000 + c))
         .to(torch.float16).to(DEV))
    sl = torch.from_numpy(lens.astype(np.int32)).to(DEV)
    torch.cuda.synchronize()
    return cfg, q, kp, vp, bt, bt_d, lens, sl


def _decode(cfg, q, kp, vp, bt_d, sl, split=None):
    out = ops._decode(q, kp.plane(), vp.plane(), BS, bt_d, sl, cfg["Hkv"], D, split_tokens=split)
    torch.cuda.synchronize()
    return out


def _plan(cfg, bt_d, lens):
    """The library's plan with the batch's total context known on the host (as
    the vLLM backend passes it): split-K for the uniform configurations, the
    stream schedule (0) for config 3's variable lengths."""
    return _lib.lib().knlp_kv_decode_plan(cfg["B"], cfg["Hkv"], cfg["Hq"], D,
                                          bt_d.shape[1] * BS, int(np.sum(lens)), FMT[cfg["k"]],
                                          cfg["kgs"], FMT[cfg["v"]], cfg["vgs"])


def _sampled_oracle(c, cfg, q, kp, vp, bt, lens, out):
    """Oracle on the longest sequence's last kv head, all its q heads."""
    s = int(np.argmax(lens))
    kvh = cfg["Hkv"] - 1
    n = int(lens[s])
    blocks = torch.from_numpy(bt[s, :-(-n // BS)].astype(np.int64)).to(DEV)
    G = cfg["Hq"] // cfg["Hkv"]
    qh = q[s:s + 1, kvh * G:(kvh + 1) * G].float().cpu().numpy()
    ref = A.decode_reference(qh, kp.host(blocks, kvh), vp.host(blocks, kvh),
                             np.arange(len(blocks), dtype=np.int32)[None], [n],
                             round_output=False)
    got = out[s:s + 1, kvh * G:(kvh + 1) * G].float().cpu().numpy()
    tolerance.check(f"full_config{c}_seq{s}_kvhead{kvh}", got, ref)


@pytest.mark.parametrize("c", [2, 3, 4, 5])
def test_full_size_config(c):
    print(f"full-size config {c}: building", flush=True)
    cfg, q, kp, vp, bt, bt_d, lens, sl = _build(c)
    kind = K.decode_kernel_kind(cfg["Hq"], cfg["Hkv"], D, FMT[cfg["k"]], cfg["kgs"],
                                FMT[cfg["v"]], cfg["vgs"])
    assert kind == "mfma"
    plan = _plan(cfg, bt_d, lens)
    print(f"config {c}: plan {plan} tokens per split (0: stream schedule)", flush=True)
    assert (plan == 0) == (c == 3)
    out = _decode(cfg, q, kp, vp, bt_d, sl, plan)
    assert torch.isfinite(out.float()).all()
    again = _decode(cfg, q, kp, vp, bt_d, sl, plan)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16)), "not deterministic"
    got = out.float().cpu().numpy()
    others = {1024, 2048} if plan == 0 else {max(64, plan // 2 // 64 * 64), plan * 2, 1024, 0}
    for other in sorted(others - {plan}):
        o2 = _decode(cfg, q, kp, vp, bt_d, sl, other).float().cpu().numpy()
        tolerance.check(f"full_config{c}_split{other}_vs_plan{plan}", o2, got, both_rounded=True)
    _sampled_oracle(c, cfg, q, kp, vp, bt, lens, out)
    if c == 2:
        # move every page and permute the table to match: bit-identical
        perm = torch.randperm(kp.data.shape[0], generator=torch.Generator().manual_seed(9))
        inv = torch.argsort(perm).to(DEV)
        for p in (kp, vp):
            p.data, p.scales = p.data[inv], p.scales[inv]
            p.zeros = None if p.zeros is None else p.zeros[inv]
        bt_p = perm.to(DEV)[bt_d.long()].to(torch.int32)
        moved = _decode(cfg, q, kp, vp, bt_p, sl, plan)
        assert torch.equal(out.view(torch.int16), moved.view(torch.int16))
    if c == 5:
        # one new token per sequence: fused append + decode against separate launches
        newk = _rows(cfg["B"], cfg["Hkv"], 7000 + c, 0.0)
        newv = _rows(cfg["B"], cfg["Hkv"], 8000 + c, 0.0)
        bt2 = np.concatenate([bt, (bt.max() + 1 + np.arange(cfg["B"], dtype=np.int32))[:, None]],
                             axis=1)
        pool = int(bt2.max()) + 1
        if pool > kp.data.shape[0]:
            for p in (kp, vp):
                grow = lambda t: None if t is None else torch.cat(
                    [t, torch.zeros((pool - t.shape[0],) + tuple(t.shape[1:]), dtype=t.dtype,
                                    device=DEV)])
                p.data, p.scales, p.zeros = grow(p.data), grow(p.scales), grow(p.zeros)
        bt2_d = torch.from_numpy(bt2).to(DEV)
        pos = torch.from_numpy(lens).to(DEV)
        slots = bt2_d[torch.arange(cfg["B"], device=DEV), pos // BS].long() * BS + pos % BS
        sl2 = sl + 1
        sep = [t.clone() for t in (kp.data, kp.scales, vp.data, vp.scales, vp.zeros)]
        K.reshape_and_cache_k_int8(newk, sep[0], sep[1], slots, group_size=cfg["kgs"])
        K.reshape_and_cache_v_only_int4(newv, sep[2], sep[3], slots, sep[4], asymmetric=True,
                                        group_size=cfg["vgs"])
        want = K.kint8_vint4_decode(q, sep[0], sep[2], sep[1], sep[3], bt2_d, sl2, cfg["Hkv"], D,
                                    v_zeros=sep[4], asymmetric=True, k_group_size=cfg["kgs"],
                                    v_group_size=cfg["vgs"], split_tokens=plan)
        fused = K.append_and_decode(q, newk, newv, slots, kp.data, vp.data, kp.scales, vp.scales,
                                    bt2_d, sl2, cfg["Hkv"], D, k_format="int8", v_format="int4",
                                    v_zeros=vp.zeros, asymmetric=True, k_group_size=cfg["kgs"],
                                    v_group_size=cfg["vgs"], split_tokens=plan)
        torch.cuda.synchronize()
        for x, y in zip(sep, (kp.data, kp.scales, vp.data, vp.scales, vp.zeros)):
            assert torch.equal(x, y)
        assert torch.equal(want.view(torch.int16), fused.view(torch.int16))
