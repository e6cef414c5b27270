"""Generate tests/golden/int4kv_golden.npz from the CPU restatement (oracle/).

The fixtures pin the quantise and decode paths on small seeded inputs:

* append: fp16 rows [40 tokens, 2 heads, 64] quantised per F's rules --
  asymmetric INT4 g32, symmetric INT4 g32 with the outlier clip 10, INT8 g32
  -- into a 6-block paged cache through a permuted slot mapping with two
  padding slots (-1); stored as the raw cache bytes.
* decode: a paged INT4-asym g32 cache (D=64, 8 kv heads, 32 q heads, block
  16, sequence lengths 1, 45 and 160 over a permuted block table) and the
  oracle's decode output, fp32 before rounding and fp16 after.

Inputs are drawn with torch.Generator seeds on the CPU and stored as fp16
bits, so the test side feeds the GPU exactly these bits.  Run from the repo
root: ``python tests/golden/make_golden.py``.
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attention as A      # noqa: E402
from tests import kvgen                # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "int4kv_golden.npz")


def append_cases():
    nb, bs, h, d, gs = 6, 16, 2, 64, 32
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(40, h, d, generator=g) * 2.0)
    x[3, 0, :8] *= 40.0                                  # an outlier group for the clip
    x[7, 1, :] = 0.0                                     # a constant (zero) row
    x = x.half()
    slots = torch.randperm(nb * bs, generator=g)[:40].numpy().astype(np.int64)
    slots[[5, 23]] = -1                                  # padding tokens, skipped
    xf = x.float().numpy()
    out = {"append_x": x.numpy().view(np.uint16), "append_slots": slots}
    for name, fmt, clip in (("asym", 1, 0.0), ("sym", 0, 10.0), ("int8", 2, 0.0)):
        p = kvgen.empty_plane(fmt, nb, bs, h, d, gs)
        keep = slots >= 0
        kvgen.fill_plane(p, xf[keep], slots[keep], clip_ratio=clip)
        out[f"append_{name}_data"] = p["data"]
        out[f"append_{name}_scales"] = p["scales"].view(np.uint16)
        if p["zeros"] is not None:
            out[f"append_{name}_zeros"] = p["zeros"].view(np.uint16)
    return out


def decode_case():
    hq, hkv, d, bs, gs = 32, 8, 64, 16, 32
    seq_lens = [1, 45, 160]
    nb = sum(-(-n // bs) for n in seq_lens) + 2
    bt = kvgen.paged_table(seq_lens, bs, nb, seed=12)
    slots = kvgen.token_slots(bt, seq_lens, bs)
    k = kvgen.randn((len(slots), hkv, d), 13, outlier_frac=0.02)
    v = kvgen.randn((len(slots), hkv, d), 14, outlier_frac=0.02)
    q = kvgen.randn((len(seq_lens), hq, d), 15)
    kp = kvgen.empty_plane(1, nb, bs, hkv, d, gs)
    vp = kvgen.empty_plane(1, nb, bs, hkv, d, gs)
    kvgen.fill_plane(kp, k.float().numpy(), slots)
    kvgen.fill_plane(vp, v.float().numpy(), slots)
    ref32 = A.decode_reference(q.float().numpy(), kp, vp, bt, seq_lens, round_output=False)
    ref16 = A.decode_reference(q.float().numpy(), kp, vp, bt, seq_lens)
    return {"decode_q": q.numpy().view(np.uint16), "decode_bt": bt,
            "decode_seq_lens": np.array(seq_lens, np.int32),
            "decode_k_data": kp["data"], "decode_k_scales": kp["scales"].view(np.uint16),
            "decode_k_zeros": kp["zeros"].view(np.uint16),
            "decode_v_data": vp["data"], "decode_v_scales": vp["scales"].view(np.uint16),
            "decode_v_zeros": vp["zeros"].view(np.uint16),
            "decode_out_f32": ref32, "decode_out_f16": ref16.astype(np.float16).view(np.uint16)}


def main():
    out = {**append_cases(), **decode_case()}
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
