"""vLLM attention backend over this library: the MI355X counterpart of
``FusedInt4AttentionBackend`` / ``FusedInt4AttentionMetadataBuilder`` /
``FusedInt4AttentionImpl`` (fused-quant/fused_int4.v0.1.0.py:2072-3198).

Same class names, registry name ("FUSED_INT4"), cache-dtype string
("int4_fused"), environment knobs and control flow as the reference:

  * shadow quantised caches allocated lazily next to vLLM's fp16 paged cache
    and checked against the planner's per-block budget (F:2334-2480);
  * the quantised append of each step's K/V, dispatched on the
    (k_precision, v_precision) pair (F:2600-2689);
  * decode batches (max_query_len == 1) take the fused decode once the
    longest sequence reaches MIN_FUSED_SEQ_LEN (F:2723-2736), shorter ones
    read the fp16 paged cache; mixed batches split decode and prefill rows
    and place both outputs without Python loops over decode rows
    (F:2751-2843);
  * the fused decode dispatch table (F:2701-2707, F:2851-2928).

What differs, by design for MI355X:
  * the fused decode is this library's split-K HIP decode (knlp_amd.ops);
  * a pure decode step on the fused path quantises its new token inside the
    decode launch (ops.append_and_decode), so the separate append launch the
    reference issues before every decode disappears
    (docs/fused-quant/latency.md:41); other steps write first, as F does;
  * the fp16 paged short-sequence decode is the same HIP kernel on fp16
    planes (the reference uses FlashAttention-3, absent on ROCm); a bf16
    model's paged cache goes through the reference's own non-FA path,
    per-sequence SDPA on the device (F:3087-3125);
  * prefill is per-sequence causal SDPA on the device, the reference's
    non-FA path (F:3127-3198), since vLLM's FlashAttention wheel is CUDA-only;
  * the fp16 paged write (vLLM's ``reshape_and_cache_flash``) is this
    library's append kernel for fp16 models and a device scatter for bf16;
  * no FA3 scheduler metadata is computed.

This module imports vLLM (it plugs into vLLM's backend registry, as the
reference does); everything below the class layer lives in ``knlp_amd.ops``
and ``knlp_amd.kv_layout``, which do not need vLLM.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import ClassVar

import torch
import torch.nn.functional as F

from vllm.logger import init_logger
from vllm.v1.attention.backend import (
    AttentionBackend,
    AttentionCGSupport,
    AttentionImpl,
    AttentionLayer,
    AttentionMetadataBuilder,
    AttentionType,
    CommonAttentionMetadata,
)

from . import config, kv_layout, ops

logger = init_logger(__name__)

# the reference's (k_precision, v_precision) -> decode function table (F:2701-2707)
DECODE_KERNELS = {
    ("int4", "int4"): "fused_int4_decode",
    ("int8", "int4"): "kint8_vint4_decode",
    ("int8", "int8"): "kint8_vint8_decode",
    ("fp16", "int4"): "kfp16_vint4_decode",
    ("fp16", "int8"): "kfp16_vint8_decode",
}


@dataclass
class FusedInt4AttentionMetadata:
    """Per-step decode metadata (F:2076-2090), without the FA3 fields."""
    num_actual_tokens: int
    max_query_len: int
    query_start_loc: torch.Tensor
    max_seq_len: int
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    # summed sequence lengths, from vLLM's host copy of seq_lens when it has one
    # (0: unknown); sizes the decode plan without a device read-back
    total_context: int = 0


class FusedInt4AttentionBackend(AttentionBackend):
    """Attention backend using fused INT4 KV caches with in-kernel dequant."""

    accept_output_buffer: bool = True
    forward_includes_kv_cache_update: bool = False
    supported_dtypes: ClassVar[list[torch.dtype]] = [torch.float16, torch.bfloat16]
    supported_kv_cache_dtypes: ClassVar[list[str]] = ["int4_fused"]

    @staticmethod
    def get_name() -> str:
        return "FUSED_INT4"

    @staticmethod
    def get_impl_cls() -> type["FusedInt4AttentionImpl"]:
        return FusedInt4AttentionImpl

    @staticmethod
    def get_builder_cls() -> type["FusedInt4AttentionMetadataBuilder"]:
        return FusedInt4AttentionMetadataBuilder

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           cache_dtype_str: str = "int4_fused") -> tuple[int, ...]:
        """Allocator-compatible fp16 paged-cache shape (F:2122-2158)."""
        return kv_layout.kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size,
                                        config.REPLACE_CACHE)

    @classmethod
    def supports_kv_cache_dtype(cls, kv_cache_dtype) -> bool:
        return kv_cache_dtype is None or kv_cache_dtype == "int4_fused"

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        # F:2168-2171 asks D % GROUP_SIZE == 0; its kernels also need a power
        # of two (tl.arange(0, HALF_HD), F:729-735).  These are the head sizes
        # this library's append and decode both take.
        return head_size in (32, 64, 128, 256) and head_size % config.GROUP_SIZE == 0

    @classmethod
    def supports_attn_type(cls, attn_type: str) -> bool:
        return attn_type == AttentionType.DECODER


class FusedInt4AttentionMetadataBuilder(AttentionMetadataBuilder[FusedInt4AttentionMetadata]):
    """Builds the step metadata from vLLM's common metadata (F:2185-2262).
    Decode steps of one token per sequence are HIP-graph capturable: the
    decode allocates only torch tensors whose shapes depend on the batch."""

    _cudagraph_support = AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        self._init_reorder_batch_threshold(reorder_batch_threshold=1)

    def build(self, common_prefix_len: int, common_attn_metadata: CommonAttentionMetadata,
              fast_build: bool = False) -> FusedInt4AttentionMetadata:
        m = common_attn_metadata
        host_lens = getattr(m, "seq_lens_cpu", None)
        return FusedInt4AttentionMetadata(
            num_actual_tokens=m.num_actual_tokens, max_query_len=m.max_query_len,
            query_start_loc=m.query_start_loc, max_seq_len=m.max_seq_len,
            seq_lens=m.seq_lens, block_table=m.block_table_tensor,
            slot_mapping=m.slot_mapping,
            total_context=int(host_lens.sum()) if host_lens is not None else 0)


class FusedInt4AttentionImpl(AttentionImpl[FusedInt4AttentionMetadata]):
    """Fused INT4 attention with backend-owned shadow caches (F:2268-3198)."""

    def __init__(self, num_heads: int, head_size: int, scale: float,
                 num_kv_heads: int | None = None, alibi_slopes: list[float] | None = None,
                 sliding_window: int | None = None, kv_cache_dtype: str = "int4_fused",
                 logits_soft_cap: float | None = None, attn_type: str = AttentionType.DECODER,
                 kv_sharing_target_layer_name: str | None = None) -> None:
        if alibi_slopes is not None:
            raise NotImplementedError("FusedInt4 backend does not support ALiBi yet")
        if sliding_window is not None:
            raise NotImplementedError("FusedInt4 backend does not support sliding window yet")
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = scale
        self.num_kv_heads = num_kv_heads or num_heads
        self.kv_cache_dtype = kv_cache_dtype
        self.num_groups = head_size // config.GROUP_SIZE
        self._asymmetric = config.ASYMMETRIC
        self._k_precision = config.K_PRECISION
        self._v_precision = config.V_PRECISION
        if (self._k_precision, self._v_precision) not in DECODE_KERNELS:
            raise ValueError(f"unsupported precision pair "
                             f"({self._k_precision}, {self._v_precision})")
        self._caches: kv_layout.ShadowCaches | None = None
        self._logged_init = False

    # ---- shadow caches -----------------------------------------------------------------
    def _precision(self) -> dict:
        return dict(k_precision=self._k_precision, v_precision=self._v_precision,
                    asymmetric=self._asymmetric, group_size=config.GROUP_SIZE)

    def _ensure_int4_cache(self, num_blocks: int, block_size: int,
                           device: torch.device) -> None:
        """Allocate (or grow) the shadow caches to `num_blocks` blocks (F:2334-2480)."""
        c = self._caches
        if c is not None and c.num_blocks(self._v_precision) >= num_blocks:
            return
        if c is not None:
            logger.info("[FusedInt4] Reallocating caches: old num_blocks=%d -> new num_blocks=%d",
                        c.num_blocks(self._v_precision), num_blocks)
        self._caches = kv_layout.allocate_shadow_caches(
            num_blocks, block_size, self.num_kv_heads, self.head_size, device=device,
            **self._precision())
        actual, expected = kv_layout.planner_check(
            self._caches, num_blocks, block_size, self.num_kv_heads, self.head_size,
            **self._precision())
        logger.info("[S1] Auxiliary INT4 cache allocated (planner-visible). k_precision=%s, "
                    "per_block: actual=%d expected=%d (%s), num_blocks=%d",
                    self._k_precision, actual, expected,
                    "MATCH" if actual == expected else "MISMATCH", num_blocks)

    @property
    def caches(self) -> kv_layout.ShadowCaches | None:
        return self._caches

    # ---- cache writes --------------------------------------------------------------------
    def _write_paged_fp16(self, key, value, key_cache, value_cache, slot_mapping) -> None:
        """vLLM's reshape_and_cache_flash for the fp16 planes."""
        if key_cache.dtype == torch.float16:
            ops.reshape_and_cache_fp16(key, value, key_cache, value_cache, slot_mapping)
            return
        keep = slot_mapping >= 0
        slots = slot_mapping[keep].long()
        for rows, cache in ((key, key_cache), (value, value_cache)):
            if rows is not None and cache is not None:
                cache.view(-1, self.num_kv_heads, self.head_size)[slots] = \
                    rows[:slot_mapping.shape[0]][keep].to(cache.dtype)

    def _write_quantized(self, key_3d, value_3d, slot_mapping) -> None:
        """Quantised append of this step's K/V into the shadow caches,
        dispatched on (k_precision, v_precision) as F:2600-2689.  (The
        reference's INT4-K / INT8-V branch writes V through the INT4 writer
        into the 1-element placeholder; that pair has no decode kernel there
        and is rejected in __init__ here.)"""
        c, asym = self._caches, self._asymmetric
        kp, vp = self._k_precision, self._v_precision
        if kp == "int4":
            ops.reshape_and_cache_int4(key_3d, value_3d, c.int4_key, c.int4_value, c.k_scales,
                                       c.v_scales, slot_mapping, k_zeros=c.k_zeros,
                                       v_zeros=c.v_zeros, asymmetric=asym)
            return
        if kp == "int8":
            ops.reshape_and_cache_k_int8(key_3d, c.int8_key, c.k_int8_scales, slot_mapping)
        if vp == "int8":
            ops.reshape_and_cache_v_int8(value_3d, c.int8_value, c.v_int8_scales, slot_mapping)
        else:
            ops.reshape_and_cache_v_only_int4(value_3d, c.int4_value, c.v_scales, slot_mapping,
                                              v_zeros=c.v_zeros, asymmetric=asym)

    def do_kv_cache_update(self, layer, key: torch.Tensor, value: torch.Tensor,
                           kv_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Write this step's K/V into vLLM's paged cache (F:2483-2545).  With
        REPLACE_CACHE the cache holds only the fp16 K plane and V goes
        straight to the quantised shadow cache."""
        if kv_cache.numel() > 0:
            self._ensure_int4_cache(kv_cache.shape[1], kv_cache.shape[2], kv_cache.device)
        key_3d = key.view(-1, self.num_kv_heads, self.head_size)
        value_3d = value.view(-1, self.num_kv_heads, self.head_size)
        if config.REPLACE_CACHE:
            self._write_paged_fp16(key_3d, None, kv_cache[0], None, slot_mapping)
            c = self._caches
            if self._v_precision == "int8":
                ops.reshape_and_cache_v_int8(value_3d, c.int8_value, c.v_int8_scales,
                                             slot_mapping)
            else:
                ops.reshape_and_cache_v_only_int4(value_3d, c.int4_value, c.v_scales,
                                                  slot_mapping, v_zeros=c.v_zeros,
                                                  asymmetric=self._asymmetric)
        else:
            self._write_paged_fp16(key_3d, value_3d, kv_cache[0], kv_cache[1], slot_mapping)

    # ---- forward ---------------------------------------------------------------------------
    def forward(self, layer: AttentionLayer, query: torch.Tensor, key: torch.Tensor,
                value: torch.Tensor, kv_cache: torch.Tensor,
                attn_metadata: FusedInt4AttentionMetadata | None,
                output: torch.Tensor | None = None, output_scale=None,
                output_block_scale=None) -> torch.Tensor:
        """Prefill, decode and mixed batches over the shared cache
        architecture (F:2547-2843)."""
        if attn_metadata is None or kv_cache.numel() == 0:
            # profiling / warm-up runs
            if output is not None:
                output.zero_()
                return output
            return torch.zeros_like(query)

        key_cache_fp16 = kv_cache[0]
        value_cache_fp16 = None if config.REPLACE_CACHE else kv_cache[1]
        self._ensure_int4_cache(key_cache_fp16.shape[0], key_cache_fp16.shape[1],
                                kv_cache.device)

        n_tok = attn_metadata.num_actual_tokens
        key_3d = value_3d = None
        if not config.REPLACE_CACHE and n_tok > 0 and value.numel() > 0:
            key_3d = key.view(-1, self.num_kv_heads, self.head_size) if key.dim() == 2 else key
            value_3d = value.view(-1, self.num_kv_heads, self.head_size) \
                if value.dim() == 2 else value
        # A pure decode step on the fused path quantises its one new token per
        # sequence inside the decode launch (no separate append launch); every
        # other step writes first, as F:2600-2689.
        fuse_append = (key_3d is not None and attn_metadata.max_query_len == 1 and
                       attn_metadata.max_seq_len >= config.MIN_FUSED_SEQ_LEN)
        if key_3d is not None and not fuse_append:
            self._write_quantized(key_3d, value_3d, attn_metadata.slot_mapping)

        if not self._logged_init:
            self._logged_init = True
            logger.info("[FusedInt4] k_precision=%s, v_precision=%s, decode_kernel=%s, "
                        "group_size=%d, num_kv_heads=%d, head_size=%d, "
                        "min_fused_seq_len=%d, asymmetric=%s",
                        self._k_precision, self._v_precision,
                        DECODE_KERNELS[(self._k_precision, self._v_precision)],
                        config.GROUP_SIZE, self.num_kv_heads, self.head_size,
                        config.MIN_FUSED_SEQ_LEN, self._asymmetric)

        if query.dim() == 2:
            query = query.view(-1, self.num_heads, self.head_size)

        if attn_metadata.max_query_len == 1:
            num_seqs = attn_metadata.seq_lens.shape[0]
            dq = query[:num_seqs]
            if fuse_append:
                dout = self._append_and_decode(dq, key_3d, value_3d, key_cache_fp16,
                                               attn_metadata)
            elif config.REPLACE_CACHE or attn_metadata.max_seq_len >= config.MIN_FUSED_SEQ_LEN:
                dout = self._fused_decode(dq, key_cache_fp16, attn_metadata.block_table,
                                          attn_metadata.seq_lens, attn_metadata.total_context)
            else:
                dout = self._paged_decode(dq, key_cache_fp16, value_cache_fp16,
                                          attn_metadata.block_table, attn_metadata.seq_lens)
            if output is not None:
                output[:dout.shape[0]].copy_(dout.view(output[:dout.shape[0]].shape))
                return output
            return dout.view(dout.shape[0], -1)

        qsl = attn_metadata.query_start_loc
        num_seqs = attn_metadata.seq_lens.shape[0]
        qlens = qsl[1:num_seqs + 1] - qsl[:num_seqs]
        decode_mask = qlens == 1
        if not bool(decode_mask.any()):
            return self._prefill(query, key, value, attn_metadata, output)

        if output is None:
            output = torch.empty(query.shape[0], self.num_heads * self.head_size,
                                 dtype=query.dtype, device=query.device)
        didx = torch.where(decode_mask)[0]
        dsl = attn_metadata.seq_lens[didx]
        dbt = attn_metadata.block_table[didx]
        doff = qsl[didx]
        dq = query[doff]
        if config.REPLACE_CACHE or int(dsl.max()) >= config.MIN_FUSED_SEQ_LEN:
            dout = self._fused_decode(dq, key_cache_fp16, dbt, dsl)
        else:
            dout = self._paged_decode(dq, key_cache_fp16, value_cache_fp16, dbt, dsl)
        output.view(output.shape[0], -1).index_copy_(0, doff.long(),
                                                     dout.reshape(dout.shape[0], -1))
        pidx = torch.where(~decode_mask)[0]
        if pidx.numel():
            self._prefill_rows(query, key, value, qsl, pidx, output)
        return output

    # ---- decode kernels -------------------------------------------------------------------
    def _fused_scale(self) -> float | None:
        """Softmax scale of the fused decode: None (1/sqrt(head_size), as the
        reference's kernels fix it, F:924 with F:2851-2928 passing no scale)
        unless KNLP_FUSED_DECODE_LAYER_SCALE=1 asks for the layer's scale."""
        return self.scale if config.FUSED_DECODE_LAYER_SCALE else None

    def _fused_decode(self, q: torch.Tensor, key_cache_fp16: torch.Tensor,
                      block_table: torch.Tensor, seq_lens: torch.Tensor,
                      total_context: int = 0) -> torch.Tensor:
        """Dispatch on (k_precision, v_precision) (F:2845-2928)."""
        c, kp, vp = self._caches, self._k_precision, self._v_precision
        common = dict(num_kv_heads=self.num_kv_heads, head_size=self.head_size,
                      scale=self._fused_scale(), total_context=total_context)
        if kp == "fp16" and vp == "int8":
            return ops.kfp16_vint8_decode(q, key_cache_fp16, c.int8_value, c.v_int8_scales,
                                          block_table, seq_lens, **common)
        if kp == "fp16":
            return ops.kfp16_vint4_decode(q, key_cache_fp16, c.int4_value, c.v_scales,
                                          block_table, seq_lens, v_zeros=c.v_zeros,
                                          asymmetric=self._asymmetric, **common)
        if kp == "int8" and vp == "int8":
            return ops.kint8_vint8_decode(q, c.int8_key, c.int8_value, c.k_int8_scales,
                                          c.v_int8_scales, block_table, seq_lens, **common)
        if kp == "int8":
            return ops.kint8_vint4_decode(q, c.int8_key, c.int4_value, c.k_int8_scales,
                                          c.v_scales, block_table, seq_lens, v_zeros=c.v_zeros,
                                          asymmetric=self._asymmetric, **common)
        return ops.fused_int4_decode(q, c.int4_key, c.int4_value, c.k_scales, c.v_scales,
                                     block_table, seq_lens, k_zeros=c.k_zeros,
                                     v_zeros=c.v_zeros, asymmetric=self._asymmetric, **common)

    def _append_and_decode(self, q, key_3d, value_3d, key_cache_fp16, md) -> torch.Tensor:
        """The step's quantised append and the fused decode in one decode
        launch (ops.append_and_decode); the same writes and the same output
        as _write_quantized followed by _fused_decode."""
        c, kp, vp, asym = self._caches, self._k_precision, self._v_precision, self._asymmetric
        n = q.shape[0]
        if kp == "int4":
            kcache, ks, kz, key = c.int4_key, c.k_scales, c.k_zeros, key_3d[:n]
        elif kp == "int8":
            kcache, ks, kz, key = c.int8_key, c.k_int8_scales, None, key_3d[:n]
        else:                                  # fp16 K: already in the paged cache
            kcache, ks, kz, key = key_cache_fp16, None, None, None
        if vp == "int8":
            vcache, vs, vz = c.int8_value, c.v_int8_scales, None
        else:
            vcache, vs, vz = c.int4_value, c.v_scales, c.v_zeros
        return ops.append_and_decode(
            q, key, value_3d[:n], md.slot_mapping[:n], kcache, vcache, ks, vs, md.block_table,
            md.seq_lens, self.num_kv_heads, self.head_size, k_format=kp, v_format=vp,
            k_zeros=kz, v_zeros=vz, asymmetric=asym, scale=self._fused_scale(),
            total_context=md.total_context)

    def _paged_decode(self, q, key_cache, value_cache, block_table, seq_lens) -> torch.Tensor:
        """Short sequences from the fp16 paged cache (F:2930-3048)."""
        if key_cache.dtype == torch.float16 and value_cache is not None:
            return ops.fp16_paged_decode(q, key_cache, value_cache, block_table, seq_lens,
                                         self.num_kv_heads, self.head_size, scale=self.scale)
        return self._decode_from_paged(q, key_cache, value_cache, block_table, seq_lens)

    def _decode_from_paged(self, q, key_cache, value_cache, block_table, seq_lens):
        """Per-sequence SDPA over the paged cache, the reference's non-FA
        path (F:3087-3125)."""
        if value_cache is None:
            raise RuntimeError("REPLACE_CACHE keeps no fp16 V plane: decode is always fused")
        n_rep = self.num_heads // self.num_kv_heads
        bs = key_cache.shape[1]
        outs = []
        for s in range(q.shape[0]):
            n = int(seq_lens[s])
            blocks = block_table[s, :(n + bs - 1) // bs].long()
            k = key_cache[blocks].reshape(-1, self.num_kv_heads, self.head_size)[:n]
            v = value_cache[blocks].reshape(-1, self.num_kv_heads, self.head_size)[:n]
            k = k.float().repeat_interleave(n_rep, dim=1).transpose(0, 1)
            v = v.float().repeat_interleave(n_rep, dim=1).transpose(0, 1)
            o = F.scaled_dot_product_attention(q[s].float().unsqueeze(1), k, v,
                                               scale=self.scale)
            outs.append(o.squeeze(1).to(q.dtype))
        return torch.stack(outs) if outs else torch.empty_like(q)

    # ---- prefill ------------------------------------------------------------------------------
    def _prefill(self, query, key, value, attn_metadata, output) -> torch.Tensor:
        """Pure prefill batch (F:3050-3085)."""
        n = attn_metadata.num_actual_tokens
        if output is None:
            output = torch.empty(query.shape[0], self.num_heads * self.head_size,
                                 dtype=query.dtype, device=query.device)
        qsl = attn_metadata.query_start_loc
        rows = torch.arange(attn_metadata.seq_lens.shape[0], device=qsl.device)
        self._prefill_rows(query[:n], key[:n], value[:n], qsl, rows, output)
        return output

    def _prefill_rows(self, query, key, value, qsl, seq_rows, output) -> None:
        """Causal attention over each prefill sequence's fresh K/V, in fp32 on
        the device (the reference's non-FA path, F:3174-3198)."""
        if key.dim() == 2:
            key = key.view(-1, self.num_kv_heads, self.head_size)
            value = value.view(-1, self.num_kv_heads, self.head_size)
        n_rep = self.num_heads // self.num_kv_heads
        out3 = output.view(output.shape[0], self.num_heads, self.head_size)
        for s in seq_rows.tolist():
            a, b = int(qsl[s]), int(qsl[s + 1])
            q = query[a:b].float().transpose(0, 1)
            k = key[a:b].float().repeat_interleave(n_rep, dim=1).transpose(0, 1)
            v = value[a:b].float().repeat_interleave(n_rep, dim=1).transpose(0, 1)
            o = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=self.scale)
            out3[a:b] = o.transpose(0, 1).to(output.dtype)

