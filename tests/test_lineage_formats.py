"""The reference's other INT4 packers, restated in oracle/lineage.py, pinned on
the CPU: closed-form rows, the T5 harness packer against F's symmetric
quantiser (equal except at .5 ties), and the byte identity behind
knlp_int4_twos_to_offset (gpt2 two's-complement nibbles -> offset nibbles)."""
import numpy as np
import torch

from oracle import attention as A
from oracle import lineage as LN
from oracle import quant as Q


def test_gpt2_codes_closed_form():
    """A row whose values are k * c for k = -7..7 (and one more 7c) quantises
    to exactly k with scale c: the packed nibbles are k & 0xF, element 2i low."""
    c = 0.25
    ks = list(range(-7, 8)) + [7]
    x = torch.tensor([ks], dtype=torch.float32) * c
    packed, scale = LN.gpt2_quantize_int4(x)
    assert float(scale[0, 0]) == c
    want = [(ks[2 * i] & 0xF) | ((ks[2 * i + 1] & 0xF) << 4) for i in range(len(ks) // 2)]
    assert packed[0].tolist() == want
    assert torch.equal(LN.gpt2_dequantize_int4(packed, scale), x)


def test_gpt2_ties_to_even_and_clamp():
    """torch.round ties to even (2.5 -> 2, -0.5 -> 0) and the [-7, 7] clamp."""
    x = torch.tensor([[7.0, 2.5, -0.5, 1.5, -7.0, 3.5]])      # scale = 1
    packed, scale = LN.gpt2_quantize_int4(x)
    t = LN.gpt2_dequantize_int4(packed, scale)
    assert t[0].tolist() == [7.0, 2.0, 0.0, 2.0, -7.0, 4.0]


def test_gpt2_nibbles_map_onto_offset_nibbles():
    """For every byte b: decoding b as two gpt2 two's-complement nibbles
    equals decoding b ^ 0x88 as this library's offset nibbles ((n - 8) s)."""
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(256, 1)
    s = torch.full((256, 1), 0.375, dtype=torch.float16)
    gpt2 = LN.gpt2_dequantize_int4(b, s)
    off = A.dequant_int4((b ^ 0x88).numpy(), s.numpy(), None, group_size=2)
    assert np.array_equal(gpt2.numpy(), off)


def test_t5_packer_equals_f_symmetric_except_ties():
    """T5:116-130 and F's symmetric quantiser without the clip (F:328-363)
    share the scale amax / 7 and the [-8, 7] range; only the rounding of
    exact .5 quotients differs (ties to even vs half away from zero)."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(64, 32, generator=g) * 3
    x[0] = torch.arange(32, dtype=torch.float32) - 14.0        # amax 17: no exact ties
    x[1] = torch.tensor([7.0] + [0.5, 1.5, 2.5, -0.5, -2.5, 3.5] * 5 + [0.0])  # scale 1: ties
    packed, scale = LN.t5_quantize_and_pack_int4(x, 32)
    codes_f, scale_f, _ = Q.quantize_int4_groups(x.numpy(), asymmetric=False, clip_ratio=0.0)
    codes_t5 = np.empty((64, 32), np.uint8)
    codes_t5[:, 0::2] = (packed & 0x0F).numpy()
    codes_t5[:, 1::2] = (packed >> 4).numpy()
    diff = codes_t5 != codes_f
    q = (x / scale).numpy()                        # one group per row: scale [64, 1]
    ties = np.abs(q - np.trunc(q)) == 0.5
    assert not (diff & ~ties).any()                # every difference is a tie
    # row 1 (scale 1): ties at +-0.5 and +-2.5 round differently (20 of its
    # 30 ties); 1.5 -> 2 and 3.5 -> 4 either way
    assert diff[1].sum() == 20
    np.testing.assert_array_equal(scale[:, 0].numpy().astype(np.float16), scale_f)


def test_t5_dequant_roundtrip_closed_form():
    x = (torch.arange(32, dtype=torch.float32) - 16).reshape(1, 32) * 0.5   # amax 8
    packed, scale = LN.t5_quantize_and_pack_int4(x.half(), 32)
    y = LN.t5_dequant_int4(packed, scale.half(), 32)
    assert y.dtype == torch.float16 and y.shape == (1, 32)
    assert float((y.float() - x).abs().max()) <= float(scale) / 2 + 1e-3
