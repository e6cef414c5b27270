// extern "C" entry points: argument validation, split planning, dispatch.
// No allocation and no synchronisation happens here; every launch goes to
// the caller's stream.
#include <algorithm>
#include <atomic>
#include <cmath>

#include "kv_decode.h"

namespace knlp {
int launch_append(const void* key, const void* value, int src_bf16, int64_t num_tokens,
                  int num_heads, int head_size, int64_t kst, int64_t ksh, int64_t vst,
                  int64_t vsh, const knlp_kv_plane& KP, const knlp_kv_plane& VP,
                  const void* slots, int slots64, int block_size, float clip_ratio,
                  hipStream_t stream);
int launch_twos_to_offset(const void* src, int64_t src_stride, void* dst, int64_t dst_stride,
                          int64_t rows, int64_t row_bytes, hipStream_t stream);
int launch_hbm_read_probe(const void* src, int64_t bytes, void* sink, int blocks,
                          hipStream_t stream);
}

using namespace knlp;

namespace {

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Validate one plane for a head size.  `need_row_align` is the byte alignment
// each (block, page, head) row of codes must have for the vector loads used.
int check_plane(const knlp_kv_plane* P, int head_size, bool decode) {
  if (P == nullptr || P->data == nullptr) return KNLP_ERR_ARG;
  const int f = P->format;
  if (f < KNLP_KV_INT4_SYM || f > KNLP_KV_FP16) return KNLP_ERR_DTYPE;
  if (f != KNLP_KV_FP16) {
    const int gs = P->group_size;
    if (P->scales == nullptr) return KNLP_ERR_ARG;
    if (f == KNLP_KV_INT4_ASYM && P->zeros == nullptr) return KNLP_ERR_ARG;
    if (!is_pow2(gs) || gs < 16 || gs > 128 || gs > head_size || head_size % gs != 0)
      return KNLP_ERR_SHAPE;
  }
  // vector loads: decode reads 4 / 8 / 16 bytes per lane, append writes 1 / 2 / 4
  const int64_t eb = f == KNLP_KV_FP16 ? 2 : 1;
  const int64_t vec = decode ? (f == KNLP_KV_INT4_SYM || f == KNLP_KV_INT4_ASYM ? 4 : (f == KNLP_KV_INT8_SYM ? 8 : 16))
                             : (f == KNLP_KV_FP16 ? 4 : (f == KNLP_KV_INT8_SYM ? 2 : 1));
  if (!aligned(P->data, vec)) return KNLP_ERR_ALIGN;
  if ((P->stride_block * eb) % vec || (P->stride_page * eb) % vec || (P->stride_head * eb) % vec)
    return KNLP_ERR_ALIGN;
  if (f != KNLP_KV_FP16 && !aligned(P->scales, 2)) return KNLP_ERR_ALIGN;
  return KNLP_OK;
}

// The MFMA decode reads D/8 bytes of codes and D/G fp16 scales per lane with
// single vector loads and takes one page per 16-token sub-tile.
bool mfma_layout_ok(const knlp_kv_plane& P, int head_size, int block_size) {
  if (block_size < 16 || !is_pow2(block_size)) return false;
  const auto strides16 = [](const knlp_kv_plane& Q) {
    return (2 * Q.stride_block) % 16 == 0 && (2 * Q.stride_page) % 16 == 0 &&
           (2 * Q.stride_head) % 16 == 0;
  };
  // fp16 K: each lane reads a quarter row (D/2 bytes) with 16-byte loads
  if (P.format == KNLP_KV_FP16) return aligned(P.data, 16) && strides16(P);
  const int64_t lb = head_size / 8;
  const int64_t sb = 2 * (head_size / P.group_size);
  const auto strides_ok = [](int64_t a, int64_t b, int64_t c, int64_t m) {
    return a % m == 0 && b % m == 0 && c % m == 0;
  };
  if (!aligned(P.data, lb) || !strides_ok(P.stride_block, P.stride_page, P.stride_head, lb))
    return false;
  if (!aligned(P.scales, sb) ||
      !strides_ok(2 * P.s_stride_block, 2 * P.s_stride_page, 2 * P.s_stride_head, sb))
    return false;
  if (P.format == KNLP_KV_INT4_ASYM &&
      (!aligned(P.zeros, sb) ||
       !strides_ok(2 * P.z_stride_block, 2 * P.z_stride_page, 2 * P.z_stride_head, sb)))
    return false;
  return true;
}

// Largest grid y / z extent of a HIP launch; the decode and merge launches
// put the sequences on y.
constexpr int kMaxGridYZ = 65535;
// the stream schedule's blocks load every sequence's length at once (16 per
// lane) and count 32-token tiles in 32 bits (1024 * 2^25 / 32 = 2^30)
constexpr int kStreamMaxSeqs = 1024;
constexpr int kStreamMaxContext = 1 << 25;
// Tiles of work a stream block is charged for each row it starts after its
// first (the next row's q and block-table loads and the refill of its copy
// pipeline while the other blocks stream on).  Measured at config 3's shape
// (64 rows of 512-16384 tokens): a row boundary inside a block costs that
// block about 7 us, about four 32-token tiles of streaming; charges of 5-8
// tiles all gave 126.2 us against 129.5 us uncharged, 6 is the middle.
constexpr int kStreamRowCost = 6;

// A copy of a plane in which an fp16 plane's group_size (a field it does not
// use: it has no scales) reads head_size, so no later division sees 0.
knlp_kv_plane fp16_groups_as_rows(const knlp_kv_plane& P, int head_size) {
  knlp_kv_plane Q = P;
  if (Q.format == KNLP_KV_FP16) Q.group_size = head_size;
  return Q;
}

int check_head_size(int head_size) {
  return (head_size == 32 || head_size == 64 || head_size == 128 || head_size == 256)
             ? KNLP_OK
             : KNLP_ERR_SHAPE;
}

// CUs of the first device asked (every MI355X has 256); the stream
// schedule's grid and workspace size use it.  Threads racing on the first
// call store the same value.
int num_cus() {
  static std::atomic<int> cached{0};
  int c = cached.load(std::memory_order_relaxed);
  if (c == 0) {
    int dev = 0, n = 0;
    c = hipGetDevice(&dev) == hipSuccess &&
                hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) ==
                    hipSuccess &&
                n > 0
            ? n
            : 256;   // MI355X
    cached.store(c, std::memory_order_relaxed);
  }
  return c;
}

int heads_per_block(int num_kv_heads) {
  // all kv heads of a page in one workgroup (one wave each), up to 8 waves,
  // so every 128-byte line a workgroup touches is consumed inside it
  for (int h = 8; h >= 1; h >>= 1)
    if (num_kv_heads % h == 0) return h;
  return 1;
}

}  // namespace

extern "C" {

int knlp_abi_version(void) { return KNLP_ABI_VERSION; }

const char* knlp_status_string(int status) {
  switch (status) {
    case KNLP_OK: return "ok";
    case KNLP_ERR_SHAPE: return "unsupported or inconsistent shape";
    case KNLP_ERR_DTYPE: return "unsupported dtype or cache format";
    case KNLP_ERR_ALIGN: return "pointer or stride misaligned for vector access";
    case KNLP_ERR_WORKSPACE: return "workspace missing or too small";
    case KNLP_ERR_LAUNCH: return "HIP kernel launch failed";
    case KNLP_ERR_ARG: return "null pointer or invalid argument";
    default: return "unknown status";
  }
}

int knlp_kv_append(const void* key, const void* value, int32_t src_dtype, int64_t num_tokens,
                   int32_t num_heads, int32_t head_size, int64_t key_stride_token,
                   int64_t key_stride_head, int64_t value_stride_token,
                   int64_t value_stride_head, const knlp_kv_plane* key_cache,
                   const knlp_kv_plane* value_cache, const void* slot_mapping,
                   int32_t slot_dtype, int32_t block_size, float clip_ratio, void* stream) {
  if (src_dtype != KNLP_DT_F16 && src_dtype != KNLP_DT_BF16) return KNLP_ERR_DTYPE;
  if (slot_dtype != KNLP_DT_I32 && slot_dtype != KNLP_DT_I64) return KNLP_ERR_DTYPE;
  if (num_tokens < 0 || num_heads <= 0 || block_size <= 0) return KNLP_ERR_SHAPE;
  if (num_tokens == 0) return KNLP_OK;   // empty tensors may carry null data pointers
  if (key == nullptr && value == nullptr) return KNLP_ERR_ARG;
  if (slot_mapping == nullptr) return KNLP_ERR_ARG;
  if (!(clip_ratio >= 0.0f) || std::isinf(clip_ratio)) return KNLP_ERR_ARG;
  int st = check_head_size(head_size);
  if (st) return st;
  knlp_kv_plane kp{}, vp{};
  if (key != nullptr) {
    if ((st = check_plane(key_cache, head_size, false))) return st;
    if (key_cache->format == KNLP_KV_FP16 && src_dtype != KNLP_DT_F16) return KNLP_ERR_DTYPE;
    if (!aligned(key, 4) || key_stride_token % 2 || key_stride_head % 2) return KNLP_ERR_ALIGN;
    kp = *key_cache;
  }
  if (value != nullptr) {
    if ((st = check_plane(value_cache, head_size, false))) return st;
    if (value_cache->format == KNLP_KV_FP16 && src_dtype != KNLP_DT_F16) return KNLP_ERR_DTYPE;
    if (!aligned(value, 4) || value_stride_token % 2 || value_stride_head % 2)
      return KNLP_ERR_ALIGN;
    vp = *value_cache;
  }
  return launch_append(key, value, src_dtype == KNLP_DT_BF16, num_tokens, num_heads, head_size,
                       key_stride_token, key_stride_head, value_stride_token,
                       value_stride_head, kp, vp, slot_mapping, slot_dtype == KNLP_DT_I64,
                       block_size, clip_ratio, static_cast<hipStream_t>(stream));
}

int32_t knlp_kv_decode_plan(int32_t num_seqs, int32_t num_kv_heads, int32_t num_q_heads,
                            int32_t head_size, int32_t max_context, int64_t total_context,
                            int32_t k_format, int32_t k_group_size, int32_t v_format,
                            int32_t v_group_size) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || max_context <= 0 || head_size <= 0 ||
      num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return KNLP_ERR_SHAPE;
  // Aim for about two resident workgroups per CU over the whole batch, or one
  // when the cooperative matrix-core kernel will run (it holds one 8-wave
  // block per CU with 100-160 KB of LDS tile buffers, so every block starts in
  // the first round), in multiples of 64 tokens.  Small batches get short
  // splits down to 64 tokens (config 1, one 1024-token sequence: 9.6 us per
  // step at 64 tokens against 17 us at 256); partials cost (D+2)*4 bytes per
  // q head and split on each side of the merge, negligible at that size.
  const int g = num_q_heads / num_kv_heads;
  // the cooperative kernel takes 8 kv heads per block, or 4 with fp16 K (at
  // D = 128)
  const int coop_heads = k_format == KNLP_KV_FP16 ? 4 : 8;
  const bool wide = num_kv_heads % coop_heads == 0 &&
                    (k_format != KNLP_KV_FP16 ||
                     (head_size == 128 &&
                      (v_format == KNLP_KV_FP16 || (v_group_size > 0 && head_size / v_group_size >= 2)))) &&
                    mfma_supported(g, head_size, k_format,
                                   k_format == KNLP_KV_FP16 ? head_size : k_group_size, v_format,
                                   v_format == KNLP_KV_FP16 ? head_size : v_group_size, 0);
  const int hpb = wide ? coop_heads : heads_per_block(num_kv_heads);
  const int64_t hgroups = (num_kv_heads + hpb - 1) / hpb;
  const int64_t target = (wide ? 1LL : 2LL) * num_cus();
  // tokens over all sequences: the caller's host-side total when it has one
  // (variable-length batches), else every sequence at max_context
  const int64_t rect = static_cast<int64_t>(num_seqs) * max_context;
  const int64_t total = total_context > 0 ? total_context : rect;
  // A batch whose total falls clearly short of its rectangle has sequences
  // of different lengths: split-K leaves CUs idle at the end (the longest
  // rows run more splits than the grid's last round holds), so the
  // cooperative kernel's stream schedule (0) deals all rows' tiles out in
  // equal shares instead (config 3: 180 -> 130 us).  Uniform batches keep
  // split-K, whose start-up is about 2 us shorter.  With the total unknown
  // and several sequences the stream schedule runs too: its shares hold for
  // any mix of lengths, while splits sized for every sequence at max_context
  // leave a long sequence among short ones to a few workgroups (one
  // 100000-token sequence among 127 of 500 tokens: 1869 us per step against
  // 44 us).
  // (Two head sets with fewer than 4 V groups run out of registers in the
  // stream kernel and stay on split-K.)
  const int vng = v_format == KNLP_KV_FP16 || v_group_size <= 0 ? 1 : head_size / v_group_size;
  const bool stream_fits = g * vng <= 16 || vng == 4;
  const bool ragged = total_context > 0 ? 10 * total <= 9 * rect : num_seqs > 1;
  if (wide && stream_fits && ragged && num_seqs <= kStreamMaxSeqs &&
      max_context <= kStreamMaxContext)
    return 0;
  const auto split_of = [&](int64_t tokens) {
    int64_t t = (tokens * hgroups + target - 1) / target;
    if (t < 64) t = 64;
    return (t + 63) / 64 * 64;
  };
  int64_t tok = split_of(total);
  // A ragged batch left on split-K (planes the stream schedule does not take,
  // or more sequences than it holds) has splits sized from its real tokens,
  // but its workspace and grid stay dense: [num_seqs, hq, ceil(max_context /
  // tok)] partials.  With short sequences in a wide block table that is
  // gigabytes (256 sequences of 500 tokens in a 131072-token table at 28 q
  // heads: 1.9 GB).  The split is therefore at least a quarter of the
  // uniform plan's, which keeps the workspace within about 4x of it.
  tok = std::max(tok, (split_of(rect) / 4 + 63) / 64 * 64);
  if (tok > max_context) tok = (static_cast<int64_t>(max_context) + 63) / 64 * 64;
  return static_cast<int32_t>(tok);
}

int32_t knlp_kv_decode_split_tokens(int32_t num_seqs, int32_t num_kv_heads, int32_t num_q_heads,
                                    int32_t head_size, int32_t max_context, int32_t k_format,
                                    int32_t v_format) {
  // group sizes this entry point does not take: one scale per row for INT8,
  // 32 (the reference's default GROUP_SIZE, F:55) for INT4
  const auto gs = [&](int f) { return f == KNLP_KV_INT8_SYM ? head_size : 32; };
  if (num_q_heads <= 0) num_q_heads = num_kv_heads;
  // a split length: the batch taken as uniform (every sequence at max_context)
  return knlp_kv_decode_plan(num_seqs, num_kv_heads, num_q_heads, head_size, max_context,
                             static_cast<int64_t>(num_seqs) * max_context, k_format,
                             gs(k_format), v_format, gs(v_format));
}

int64_t knlp_kv_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads, int32_t head_size,
                                       int32_t max_context, int32_t split_tokens) {
  if (num_seqs <= 0 || num_q_heads <= 0 || head_size <= 0 || max_context <= 0 ||
      split_tokens < 0)
    return KNLP_ERR_SHAPE;
  if (split_tokens == 0)                       // stream schedule
    return stream_workspace_bytes(num_seqs, num_q_heads, head_size, num_cus());
  const int ns = (max_context + split_tokens - 1) / split_tokens;
  return workspace_floats(num_seqs, num_q_heads, head_size, ns) * 4;
}

int knlp_kv_decode_kernel_kind(int32_t num_q_heads, int32_t num_kv_heads, int32_t head_size,
                               int32_t k_format, int32_t k_group_size, int32_t v_format,
                               int32_t v_group_size, int32_t q_dtype) {
  if (num_kv_heads <= 0 || num_q_heads % num_kv_heads) return KNLP_ERR_SHAPE;
  const int g = num_q_heads / num_kv_heads;
  if (check_head_size(head_size)) return KNLP_ERR_SHAPE;
  bool mfma = mfma_supported(g, head_size, k_format, k_group_size, v_format, v_group_size,
                             q_dtype == KNLP_DT_BF16);
  // INT8 K, INT8 V (with INT4 / INT8 K) and two head sets exist only on the
  // cooperative kernel, which takes 8 kv heads per block
  const int vng = v_group_size > 0 ? head_size / v_group_size : 1;
  const bool coop_only = k_format == KNLP_KV_INT8_SYM ||
                         (v_format == KNLP_KV_INT8_SYM && k_format != KNLP_KV_FP16) ||
                         g * vng > 16;
  if (mfma && coop_only && num_kv_heads % 8 != 0) mfma = false;
  // the VALU kernel serves up to 8 query heads per kv head; the matrix-core
  // kernel up to two 16-row head sets (on dense cache layouts)
  if (g > 8 && !mfma) return KNLP_ERR_SHAPE;
  return mfma ? 1 : 0;
}

int knlp_hbm_read_probe(const void* src, int64_t bytes, void* sink, int32_t blocks,
                        void* stream) {
  if (bytes <= 0 || bytes % 16 || blocks <= 0) return KNLP_ERR_SHAPE;
  if (src == nullptr || sink == nullptr) return KNLP_ERR_ARG;
  if (!aligned(src, 16) || !aligned(sink, 4)) return KNLP_ERR_ALIGN;
  return launch_hbm_read_probe(src, bytes, sink, blocks, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

// Decode partial with an optional fused append of the token being decoded.
int decode_partial(const void* query, int32_t q_dtype, int64_t q_stride_seq,
                   int64_t q_stride_head, int32_t num_seqs, int32_t num_q_heads,
                   int32_t num_kv_heads, int32_t head_size, const knlp_kv_plane* key_cache,
                   const knlp_kv_plane* value_cache, const int32_t* block_table,
                   int64_t bt_stride_seq, const int32_t* seq_lens, int32_t block_size,
                   int32_t max_context, float softmax_scale, int32_t split_tokens,
                   void* workspace, int64_t workspace_bytes, const AppendArgs* app,
                   void* stream_ptr) {
  if (q_dtype != KNLP_DT_F16 && q_dtype != KNLP_DT_BF16) return KNLP_ERR_DTYPE;
  // split_tokens == 0: the stream schedule (one block per CU over all rows'
  // tiles); else split-K with that many tokens per split
  const bool stream = split_tokens == 0;
  if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 ||
      max_context <= 0 || split_tokens < 0 || split_tokens % 64)
    return KNLP_ERR_SHAPE;
  if (stream && (num_seqs > kStreamMaxSeqs || max_context > kStreamMaxContext))
    return KNLP_ERR_SHAPE;
  if (num_seqs == 0) return KNLP_OK;   // empty tensors may carry null data pointers
  if (num_seqs > kMaxGridYZ) return KNLP_ERR_SHAPE;   // one grid row per sequence
  if (query == nullptr || block_table == nullptr || seq_lens == nullptr) return KNLP_ERR_ARG;
  if (num_q_heads % num_kv_heads) return KNLP_ERR_SHAPE;
  if (key_cache == nullptr || value_cache == nullptr) return KNLP_ERR_ARG;
  // an fp16 plane has no scale groups: its group_size field is not read
  const knlp_kv_plane kp = fp16_groups_as_rows(*key_cache, head_size);
  const knlp_kv_plane vp = fp16_groups_as_rows(*value_cache, head_size);
  const int kind = knlp_kv_decode_kernel_kind(num_q_heads, num_kv_heads, head_size, kp.format,
                                              kp.group_size, vp.format, vp.group_size, q_dtype);
  if (kind < 0) return kind;
  int st;
  if ((st = check_plane(&kp, head_size, true))) return st;
  if ((st = check_plane(&vp, head_size, true))) return st;
  if (!std::isfinite(softmax_scale)) return KNLP_ERR_ARG;
  if (!aligned(query, 16) || q_stride_seq % 8 || q_stride_head % 8) return KNLP_ERR_ALIGN;
  const int ns = stream ? 1 : (max_context + split_tokens - 1) / split_tokens;
  if (ns > 65535) return KNLP_ERR_SHAPE;
  const int P = stream ? num_cus() : 0;
  const int64_t need = stream ? stream_workspace_bytes(num_seqs, num_q_heads, head_size, P)
                              : workspace_floats(num_seqs, num_q_heads, head_size, ns) * 4;
  if (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 16))
    return KNLP_ERR_WORKSPACE;

  DecodeArgs a{};
  a.q = static_cast<const uint16_t*>(query);
  a.q_stride_seq = q_stride_seq;
  a.q_stride_head = q_stride_head;
  a.q_bf16 = q_dtype == KNLP_DT_BF16;
  a.num_seqs = num_seqs;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.kp = kp;
  a.vp = vp;
  a.block_table = block_table;
  a.bt_stride = bt_stride_seq;
  a.seq_lens = seq_lens;
  a.block_size = block_size;
  a.block_shift = is_pow2(block_size) ? __builtin_ctz(block_size) : -1;
  a.split_tokens = split_tokens;
  a.num_splits = ns;
  a.max_context = max_context;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  if (stream) {
    const StreamViews v = stream_views(workspace, num_seqs, num_q_heads, head_size, P);
    a.part_o = v.part_o;
    a.part_ml = v.part_ml;
    a.row_meta = v.meta;
    a.stream_hdr = v.hdr;
    a.stream = P;
    a.stream_row_cost = kStreamRowCost;
  } else {
    workspace_views(workspace, num_seqs, num_q_heads, head_size, ns, &a.part_o, &a.part_ml);
  }
  if (app != nullptr) a.app = *app;
  hipStream_t hs = static_cast<hipStream_t>(stream_ptr);
  // (any finite softmax scale: the matrix-core kernels fold a negative one's
  // sign into q and treat 0 as uniform weights)
  const bool mfma = kind == 1 && mfma_layout_ok(kp, head_size, block_size) &&
                    mfma_layout_ok(vp, head_size, block_size);
  int32_t* fallback_hdr = nullptr;
  if (stream && !(mfma && stream_supported(a, head_size))) {
    // Planes only the split schedule takes (fp16 K, Hkv % 8 != 0, a sparse
    // layout): split-K inside the stream workspace, [num_seqs, hq, ns] over
    // its entries, with the split recorded in its header for the merge.
    const int64_t ns_max =
        stream_entries(num_seqs, num_q_heads, P) / (static_cast<int64_t>(num_seqs) * num_q_heads);
    int64_t split = (max_context + ns_max - 1) / ns_max;
    split = (split + 63) / 64 * 64;
    a.stream = 0;
    a.row_meta = nullptr;
    a.stream_hdr = nullptr;
    a.split_tokens = static_cast<int>(split);
    a.num_splits = static_cast<int>((max_context + split - 1) / split);
    if (a.num_splits > kMaxGridYZ) return KNLP_ERR_SHAPE;
    fallback_hdr = stream_views(workspace, num_seqs, num_q_heads, head_size, P).hdr;
  }
  // The decode launch first: a shape it cannot serve returns before anything
  // is launched.  The fallback's header (read only by the merge, later on the
  // same stream) follows it.
  st = mfma ? launch_decode_mfma(a, head_size, hs)
            : launch_decode_valu(a, head_size, heads_per_block(num_kv_heads), hs);
  if (st || fallback_hdr == nullptr) return st;
  return launch_stream_header(fallback_hdr, 0, a.split_tokens, a.num_splits, hs);
}

}  // namespace

extern "C" {

int knlp_kv_decode_partial(const void* query, int32_t q_dtype, int64_t q_stride_seq,
                           int64_t q_stride_head, int32_t num_seqs, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_size,
                           const knlp_kv_plane* key_cache, const knlp_kv_plane* value_cache,
                           const int32_t* block_table, int64_t bt_stride_seq,
                           const int32_t* seq_lens, int32_t block_size, int32_t max_context,
                           float softmax_scale, int32_t split_tokens, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  return decode_partial(query, q_dtype, q_stride_seq, q_stride_head, num_seqs, num_q_heads,
                        num_kv_heads, head_size, key_cache, value_cache, block_table,
                        bt_stride_seq, seq_lens, block_size, max_context, softmax_scale,
                        split_tokens, workspace, workspace_bytes, nullptr, stream);
}

}  // extern "C"

namespace {

// The merge launch, or with dry = true only its argument checks (the fused
// entry points run those before the partial launch, so that no negative
// status follows a launch).
int decode_merge(const void* workspace, int64_t workspace_bytes, const int32_t* seq_lens,
                 int32_t num_seqs, int32_t num_q_heads, int32_t head_size, int32_t max_context,
                 int32_t split_tokens, void* out, int32_t out_dtype, int64_t o_stride_seq,
                 int64_t o_stride_head, void* stream, bool dry) {
  if (out_dtype != KNLP_DT_F16 && out_dtype != KNLP_DT_BF16) return KNLP_ERR_DTYPE;
  if (num_seqs < 0 || num_q_heads <= 0 || max_context <= 0 || split_tokens < 0)
    return KNLP_ERR_SHAPE;
  if (check_head_size(head_size)) return KNLP_ERR_SHAPE;
  if (num_seqs == 0) return KNLP_OK;
  if (num_seqs > kMaxGridYZ) return KNLP_ERR_SHAPE;
  if (out == nullptr || seq_lens == nullptr) return KNLP_ERR_ARG;
  if (!aligned(out, 2)) return KNLP_ERR_ALIGN;
  if (split_tokens == 0) {                     // stream schedule
    if (num_seqs > kStreamMaxSeqs) return KNLP_ERR_SHAPE;
    const int P = num_cus();
    if (workspace == nullptr ||
        workspace_bytes < stream_workspace_bytes(num_seqs, num_q_heads, head_size, P))
      return KNLP_ERR_WORKSPACE;
    if (dry) return KNLP_OK;
    const StreamViews v =
        stream_views(const_cast<void*>(workspace), num_seqs, num_q_heads, head_size, P);
    // a row holds about P / rows + 1 entries, rows >= num_seqs
    const int per_row = min(P, P / max(num_seqs, 1) + 2);
    return launch_merge(v.part_o, v.part_ml, seq_lens, num_seqs, num_q_heads, head_size,
                        max_context, 1, per_row, out, out_dtype == KNLP_DT_BF16, o_stride_seq,
                        o_stride_head, static_cast<hipStream_t>(stream), v.meta, v.hdr);
  }
  const int ns = (max_context + split_tokens - 1) / split_tokens;
  const int64_t need = workspace_floats(num_seqs, num_q_heads, head_size, ns) * 4;
  if (workspace == nullptr || workspace_bytes < need) return KNLP_ERR_WORKSPACE;
  if (dry) return KNLP_OK;
  float *po, *pml;
  workspace_views(const_cast<void*>(workspace), num_seqs, num_q_heads, head_size, ns, &po, &pml);
  return launch_merge(po, pml, seq_lens, num_seqs, num_q_heads, head_size, max_context,
                      split_tokens, ns, out,
                      out_dtype == KNLP_DT_BF16, o_stride_seq, o_stride_head,
                      static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" {

int knlp_kv_decode_merge(const void* workspace, int64_t workspace_bytes, const int32_t* seq_lens,
                         int32_t num_seqs, int32_t num_q_heads, int32_t head_size,
                         int32_t max_context, int32_t split_tokens, void* out, int32_t out_dtype,
                         int64_t o_stride_seq, int64_t o_stride_head, void* stream) {
  return decode_merge(workspace, workspace_bytes, seq_lens, num_seqs, num_q_heads, head_size,
                      max_context, split_tokens, out, out_dtype, o_stride_seq, o_stride_head,
                      stream, false);
}

int knlp_kv_decode(const void* query, int32_t q_dtype, int64_t q_stride_seq,
                   int64_t q_stride_head, int32_t num_seqs, int32_t num_q_heads,
                   int32_t num_kv_heads, int32_t head_size, const knlp_kv_plane* key_cache,
                   const knlp_kv_plane* value_cache, const int32_t* block_table,
                   int64_t bt_stride_seq, const int32_t* seq_lens, int32_t block_size,
                   int32_t max_context, float softmax_scale, int32_t split_tokens,
                   void* workspace, int64_t workspace_bytes, void* out, int32_t out_dtype,
                   int64_t o_stride_seq, int64_t o_stride_head, void* stream) {
  int st = decode_merge(workspace, workspace_bytes, seq_lens, num_seqs, num_q_heads, head_size,
                        max_context, split_tokens, out, out_dtype, o_stride_seq, o_stride_head,
                        stream, true);
  if (st) return st;
  st = knlp_kv_decode_partial(query, q_dtype, q_stride_seq, q_stride_head, num_seqs,
                                  num_q_heads, num_kv_heads, head_size, key_cache, value_cache,
                                  block_table, bt_stride_seq, seq_lens, block_size, max_context,
                                  softmax_scale, split_tokens, workspace, workspace_bytes,
                                  stream);
  if (st) return st;
  return knlp_kv_decode_merge(workspace, workspace_bytes, seq_lens, num_seqs, num_q_heads,
                              head_size, max_context, split_tokens, out, out_dtype, o_stride_seq,
                              o_stride_head, stream);
}

int knlp_kv_append_decode(const void* query, int32_t q_dtype, int64_t q_stride_seq,
                          int64_t q_stride_head, int32_t num_seqs, int32_t num_q_heads,
                          int32_t num_kv_heads, int32_t head_size, const void* key,
                          const void* value, int32_t src_dtype, int64_t key_stride_seq,
                          int64_t key_stride_head, int64_t value_stride_seq,
                          int64_t value_stride_head, const void* slot_mapping,
                          int32_t slot_dtype, float clip_ratio,
                          const knlp_kv_plane* key_cache, const knlp_kv_plane* value_cache,
                          const int32_t* block_table, int64_t bt_stride_seq,
                          const int32_t* seq_lens, int32_t block_size, int32_t max_context,
                          float softmax_scale, int32_t split_tokens, void* workspace,
                          int64_t workspace_bytes, void* out, int32_t out_dtype,
                          int64_t o_stride_seq, int64_t o_stride_head, void* stream) {
  int st = decode_merge(workspace, workspace_bytes, seq_lens, num_seqs, num_q_heads, head_size,
                        max_context, split_tokens, out, out_dtype, o_stride_seq, o_stride_head,
                        stream, true);
  if (st) return st;
  if (num_seqs == 0) return KNLP_OK;
  if (src_dtype != KNLP_DT_F16 && src_dtype != KNLP_DT_BF16) return KNLP_ERR_DTYPE;
  if (slot_dtype != KNLP_DT_I32 && slot_dtype != KNLP_DT_I64) return KNLP_ERR_DTYPE;
  if (key == nullptr && value == nullptr) return KNLP_ERR_ARG;
  if (slot_mapping == nullptr) return KNLP_ERR_ARG;
  if (!(clip_ratio >= 0.0f) || std::isinf(clip_ratio)) return KNLP_ERR_ARG;
  if (key != nullptr) {
    if ((st = check_plane(key_cache, head_size, false))) return st;
    if (key_cache->format == KNLP_KV_FP16 && src_dtype != KNLP_DT_F16) return KNLP_ERR_DTYPE;
    if (!aligned(key, 4) || key_stride_seq % 2 || key_stride_head % 2) return KNLP_ERR_ALIGN;
  }
  if (value != nullptr) {
    if ((st = check_plane(value_cache, head_size, false))) return st;
    if (value_cache->format == KNLP_KV_FP16 && src_dtype != KNLP_DT_F16) return KNLP_ERR_DTYPE;
    if (!aligned(value, 4) || value_stride_seq % 2 || value_stride_head % 2)
      return KNLP_ERR_ALIGN;
  }
  AppendArgs app{};
  app.key = static_cast<const uint16_t*>(key);
  app.value = static_cast<const uint16_t*>(value);
  app.kst = key_stride_seq;
  app.ksh = key_stride_head;
  app.vst = value_stride_seq;
  app.vsh = value_stride_head;
  app.slots = slot_mapping;
  app.slots64 = slot_dtype == KNLP_DT_I64;
  app.src_bf16 = src_dtype == KNLP_DT_BF16;
  app.clip_ratio = clip_ratio;
  st = decode_partial(query, q_dtype, q_stride_seq, q_stride_head, num_seqs, num_q_heads,
                      num_kv_heads, head_size, key_cache, value_cache, block_table,
                      bt_stride_seq, seq_lens, block_size, max_context, softmax_scale,
                      split_tokens, workspace, workspace_bytes, &app, stream);
  if (st) return st;
  return knlp_kv_decode_merge(workspace, workspace_bytes, seq_lens, num_seqs, num_q_heads,
                              head_size, max_context, split_tokens, out, out_dtype, o_stride_seq,
                              o_stride_head, stream);
}

int knlp_int4_twos_to_offset(const void* src, int64_t src_stride_row, void* dst,
                             int64_t dst_stride_row, int64_t rows, int64_t row_bytes,
                             void* stream) {
  if (rows < 0 || row_bytes < 0 || row_bytes % 4) return KNLP_ERR_SHAPE;
  if (rows == 0 || row_bytes == 0) return KNLP_OK;
  if (src == nullptr || dst == nullptr) return KNLP_ERR_ARG;
  if (!aligned(src, 4) || !aligned(dst, 4) || src_stride_row % 4 || dst_stride_row % 4)
    return KNLP_ERR_ALIGN;
  if ((rows > 1 && (src_stride_row < row_bytes || dst_stride_row < row_bytes)))
    return KNLP_ERR_SHAPE;
  return launch_twos_to_offset(src, src_stride_row, dst, dst_stride_row, rows, row_bytes,
                               static_cast<hipStream_t>(stream));
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Decode with no allocation at all: the split partials live in a file-scope
// device array that each GPU holds from the library's load until the process
// ends.  In host code `scratch` names a host-side stand-in, never the device
// array: host code uses only the per-device address from
// hipGetSymbolAddress below.
// ---------------------------------------------------------------------------
namespace {

constexpr int64_t kScratchBytes = 16LL << 20;   // 16 MiB per GPU
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];

// The copy of `scratch` on the device that `stream` belongs to (the null
// stream: the current device), looked up once per device with that device
// current; nullptr on failure.
void* device_scratch(hipStream_t stream) {
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  hipDevice_t dev = cur;
  if (stream != nullptr && hipStreamGetDevice(stream, &dev) != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  // hipGetSymbolAddress answers for the current device: make the stream's
  // device current for the lookup and restore the caller's afterwards
  if (dev != cur && hipSetDevice(dev) != hipSuccess) return nullptr;
  void* q = nullptr;
  const bool ok = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) == hipSuccess && q != nullptr;
  if (dev != cur && hipSetDevice(cur) != hipSuccess) return nullptr;
  if (!ok) return nullptr;
  g_scratch[dev].store(q, std::memory_order_release);   // a racing store writes the same value
  return q;
}

}  // namespace

extern "C" int knlp_kv_decode_noalloc(const void* query, int32_t q_dtype, int64_t q_stride_seq,
                                      int64_t q_stride_head, int32_t num_seqs,
                                      int32_t num_q_heads, int32_t num_kv_heads,
                                      int32_t head_size, const knlp_kv_plane* key_cache,
                                      const knlp_kv_plane* value_cache,
                                      const int32_t* block_table, int64_t bt_stride_seq,
                                      const int32_t* seq_lens, int32_t block_size,
                                      int32_t max_context, float softmax_scale,
                                      int32_t split_tokens, void* out, int32_t out_dtype,
                                      int64_t o_stride_seq, int64_t o_stride_head,
                                      void* stream) {
  if (num_seqs < 0 || num_q_heads <= 0 || head_size <= 0 || max_context <= 0 ||
      split_tokens < 0)
    return KNLP_ERR_SHAPE;
  if (num_seqs == 0) return KNLP_OK;
  // every partial the merge reads is written by the partial kernel first, so
  // nothing in the scratch has to start at zero
  const int64_t need = knlp_kv_decode_workspace_bytes(num_seqs, num_q_heads, head_size,
                                                      max_context, split_tokens);
  if (need < 0) return static_cast<int>(need);
  if (need > kScratchBytes) return KNLP_ERR_WORKSPACE;
  void* ws = device_scratch(static_cast<hipStream_t>(stream));
  if (ws == nullptr) return KNLP_ERR_LAUNCH;
  return knlp_kv_decode(query, q_dtype, q_stride_seq, q_stride_head, num_seqs, num_q_heads,
                        num_kv_heads, head_size, key_cache, value_cache, block_table,
                        bt_stride_seq, seq_lens, block_size, max_context, softmax_scale,
                        split_tokens, ws, kScratchBytes, out, out_dtype, o_stride_seq,
                        o_stride_head, stream);
}
