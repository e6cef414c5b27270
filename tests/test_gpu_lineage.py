"""The gpt2 compression path's INT4 encoding on the GPU: knlp_int4_twos_to_offset
is bit-exact (new buffer, in place, strided rows), and caches quantised by that
path (two's-complement nibbles, one scale per row, kv_plugin.py:212-257)
decode through the fused kernel, after the conversion, to the oracle's
dequantise -> SDPA over the same codes (kv_plugin.py:260-295)."""
import numpy as np
import pytest
import torch

import knlp_amd as K
from oracle import attention as A
from oracle import lineage as LN
from tests import tolerance, kvgen

pytestmark = pytest.mark.gpu

BS = 16


def test_twos_to_offset_bit_exact():
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(4)
    src = torch.randint(0, 256, (1000, 64), generator=g, dtype=torch.int32).to(torch.uint8)
    want = (src ^ 0x88).numpy()
    d = src.to(dev)
    out = K.int4_twos_to_offset(d)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)
    assert np.array_equal(d.cpu().numpy(), src.numpy())           # source untouched
    K.int4_twos_to_offset(d, out=d)                                # in place
    torch.cuda.synchronize()
    assert np.array_equal(d.cpu().numpy(), want)
    big = torch.zeros(1000, 96, dtype=torch.uint8, device=dev)      # strided rows
    view = big[:, 16:80]
    view.copy_(src.to(dev))
    K.int4_twos_to_offset(view, out=view)
    torch.cuda.synchronize()
    b = big.cpu().numpy()
    assert np.array_equal(b[:, 16:80], want)
    assert not b[:, :16].any() and not b[:, 80:].any()


@pytest.mark.parametrize("hkv", [8, 4], ids=["cooperative", "per_head"])
def test_gpt2_format_caches_decode(hkv):
    dev = torch.device("cuda")
    hq, d = 4 * hkv, 128
    seq_lens = [700, 45]
    nb = sum(-(-n // BS) for n in seq_lens) + 3
    bt = kvgen.paged_table(seq_lens, BS, nb, seed=21)
    slots = kvgen.token_slots(bt, seq_lens, BS)
    n = len(slots)
    planes = []
    for i in range(2):                      # K, V quantised by the gpt2 path
        x = kvgen.randn((n, hkv, d), 30 + i, outlier_frac=0.02)
        packed, scale = LN.gpt2_quantize_int4(x)                # fp16 scale [n, hkv, 1]
        codes = torch.zeros(nb * BS, hkv, d // 2, dtype=torch.uint8)
        scales = torch.ones(nb * BS, hkv, 1, dtype=torch.float16)
        codes[slots] = packed
        scales[slots] = scale
        deq = np.zeros((nb * BS, hkv, d), np.float32)
        deq[slots] = LN.gpt2_dequantize_int4(packed, scale).numpy()
        planes.append((codes.view(nb, BS, hkv, d // 2), scales.view(nb, BS, hkv, 1),
                       deq.reshape(nb, BS, hkv, d)))
    q = kvgen.randn((len(seq_lens), hq, d), 40)
    (kc, ks, kdeq), (vc, vs, vdeq) = planes
    kd, vd = kc.to(dev), vc.to(dev)
    K.int4_twos_to_offset(kd, out=kd)
    K.int4_twos_to_offset(vd, out=vd)
    out = K.fused_int4_decode(q.to(dev), kd, vd, ks.to(dev), vs.to(dev),
                              torch.from_numpy(bt).to(dev),
                              torch.tensor(seq_lens, dtype=torch.int32, device=dev), hkv, d,
                              asymmetric=False, group_size=d)
    torch.cuda.synchronize()
    # the gpt2 dequantisation is exact in fp32 (small integer times an fp16
    # scale), so the fp32 planes stand in for fp16 caches holding those values
    ref = np.empty((len(seq_lens), hq, d), np.float32)
    for s, n_s in enumerate(seq_lens):
        kk = torch.from_numpy(A.gather_sequence(kdeq, bt[s], n_s))
        vv = torch.from_numpy(A.gather_sequence(vdeq, bt[s], n_s))
        ref[s] = A.sdpa_decode_f32(q[s].float(), kk, vv, float(np.float32(d ** -0.5))).numpy()
    got = out.float().cpu().numpy()
    tolerance.check("lineage_decode", got, ref)
