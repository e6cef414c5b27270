"""CPU oracle for the INT4/INT8 KV-cache quantize and decode-attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker.  The product path (``knlp_amd``) never imports it and fails loudly
when its HIP library is missing.

What is restated here (all references are into mcgrof/knlp,
``fused-quant/fused_int4.v0.1.0.py`` unless another file is named):

* ``quant.round_half_away``          -- ``_triton_round`` F:198-202
* ``quant.quantize_int4_groups``     -- the per-group body of
  ``_reshape_and_cache_int4_kernel`` F:297-363 (asymmetric F:308-327,
  symmetric + trimmed-mean clip F:328-357, nibble packing F:359-363)
* ``quant.quantize_int8_groups``     -- ``_reshape_and_cache_k_int8_kernel``
  F:1270-1284
* ``quant.reshape_and_cache_*``      -- the slot-mapped paged writes of
  F:262-296 / F:418-472 / F:519-647 / F:1287-1312
* ``attention.dequant_*``            -- ``_cpu_dequant_slot`` F:150-195 and the
  in-kernel dequantisation F:765-800, F:853-872, F:1397-1423
* ``lineage.t5_*``                   -- the harness packer, scripts/spev01/
  tier5_fused_decode.py:116-145 (ties to even, no clip)
* ``lineage.gpt2_*``                 -- the gpt2 compression path's INT4 format,
  gpt2/compression/kv_plugin.py:212-295 (two's-complement nibbles, per-row scale)
* ``attention.decode_reference``     -- the reference's own oracle, dequantise
  then ``repeat_interleave`` then SDPA: ``scripts/v35_h100_bench.py:376-387``,
  ``scripts/v29_flash_bench.py:86-97``; output rounding of F:886-894

Pinning status (how each function is checked independently of itself; the
tests live in ``tests/test_oracle_pinning.py``):

* round_half_away: special values (t = 0.49999997 -> 1, +-k.5 ties, negatives)
  and an exact-rational restatement.
* quantize_int4_groups / quantize_int8_groups: exact-rational IEEE-fp32
  recomputation (independent integer code, correctly rounded fp32 subtraction
  and division), closed-form groups, degenerate groups, brute-force code
  optimality, nibble order.
* reshape_and_cache_*: slot arithmetic and the slot < 0 skip against
  hand-built expectations.
* dequant_*: closed-form groups whose dequantisation is exact.
* lineage: closed-form rows (codes and the two's-complement bit patterns for
  every value -7..7), agreement of the T5 packer with quantize_int4_groups
  everywhere except at constructed .5 ties, and the identity that maps
  the gpt2 nibbles onto this library's offset nibbles (all 256 bytes).
* decode_reference: torch SDPA on exactly representable data, context length
  1, identical keys, GQA head equivalence, block-table permutation invariance.

The reference's Triton kernels and its vLLM backend cannot be executed here
(no vLLM, no GPU), so no function is pinned by executing the reference; the
reference repository holds no golden vectors for this path.
"""
