// Stage 3: merge per-split partial softmax states (new; the reference has no
// split-K).  For one (sequence, q head) with splits i = 0..n-1 holding
// (o_i[D], m_i, l_i) -- unnormalised accumulator, running max in log2 units,
// running sum -- the result is
//     M = max m_i,  L = sum l_i 2^(m_i - M),  out = sum o_i 2^(m_i - M) / L,
// rounded fp32 -> fp16 (F:891-894) and then to bf16 when the output tensor is
// bf16.  n = ceil(seq_len / split_tokens); n = 0 gives 0/0 = NaN, matching the
// reference's acc / l_i with l_i = 0 (F:886-887).
//
// Few partials per (sequence, q head) in a large batch: one wave per head
// folds them (merge_wave_kernel).  Few heads with many partials each (one
// or a few sequences at long context): one workgroup per 16-dim slice of a
// head (merge_slice_kernel), so that the batch still spreads over the CUs.
// Otherwise one block of NW waves per (sequence, q head), wave w folds
// splits w, w+NW, ... with an online (max-rescaling) combine, then the NW
// wave states are combined through LDS.  NW grows with the split count (4, 8
// or 16 waves) so that a wave folds at most a few groups of U splits.
#include "kv_decode.h"

namespace knlp {

// merge_slice_kernel takes batches of at most kSliceMaxRows (sequence, q
// head) rows with at least kSliceMinSplits partials per row.  At B = 1,
// T = 32768 (32 heads of 128 partials) it shortens the decode step from
// 20.4 to 18.3 us; at config 2's 256 heads of 32 partials a threshold of 16
// made the step 1.3 us longer than merge_kernel, hence 64.
constexpr int kSliceMinSplits = 64;
constexpr int64_t kSliceMaxRows = 256;

// The partials of (seq, h): entries row0 + i * stride, i < ns.
struct MergeRows {
  int ns;
  int64_t row0, stride;
};

__device__ __forceinline__ MergeRows merge_rows(const int32_t* __restrict__ seq_lens, int seq,
                                                int h, int hq, int max_context, int split_tokens,
                                                int num_splits,
                                                const int32_t* __restrict__ stream_meta,
                                                const int32_t* __restrict__ stream_hdr) {
  const int n_len = min(seq_lens[seq], max_context);
  MergeRows r;
  if (stream_meta == nullptr) {       // split schedule: [num_seqs, hq, num_splits]
    r.ns = min(num_splits, (n_len + split_tokens - 1) / split_tokens);
    r.row0 = (static_cast<int64_t>(seq) * hq + h) * num_splits;
    r.stride = 1;
  } else {
    // a stream workspace: the record, the header and the length load
    // together (none needs another; the record is unused after a split-K run)
    const int64_t m = 2 * (static_cast<int64_t>(seq) * hq + h);
    const int first = stream_meta[m], count = stream_meta[m + 1];
    const int hg = stream_hdr[0];
    if (hg > 0) {                     // stream schedule: one entry per block segment
      r.ns = n_len > 0 ? count : 0;   // (a row of length 0 has no record)
      r.row0 = n_len > 0 ? first : 0;
      r.stride = hg;                  // query heads per row (8 kv heads' groups)
    } else {                          // split-K in the workspace (header: split, splits)
      const int st = stream_hdr[1];
      const int nsp = stream_hdr[2];
      r.ns = min(nsp, (n_len + st - 1) / st);
      r.row0 = (static_cast<int64_t>(seq) * hq + h) * nsp;
      r.stride = 1;
    }
  }
  return r;
}

// Fold N partials i = first, first + step, ... (all < ns) of one (sequence, q
// head) into the running (M, L, o) of this wave, every load issued before
// any use, so the group costs about one memory round trip.
template <int D, int N>
__device__ __forceinline__ void fold_group(const float* __restrict__ part_o,
                                           const float* __restrict__ part_ml, const MergeRows& R,
                                           int first, int step, int lane, float& M, float& L,
                                           float (&o)[D >= kWave ? D / kWave : 1]) {
  constexpr int E = D >= kWave ? D / kWave : 1;
  const bool active = lane * E < D;
  float mi[N], li[N], oi[N][E];
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int64_t ent = R.row0 + static_cast<int64_t>(first + step * u) * R.stride;
    mi[u] = part_ml[2 * ent];
    li[u] = part_ml[2 * ent + 1];
#pragma unroll
    for (int e = 0; e < E; ++e) oi[u][e] = active ? part_o[ent * D + lane * E + e] : 0.0f;
  }
  float mn = M;
#pragma unroll
  for (int u = 0; u < N; ++u) mn = fmaxf(mn, mi[u]);
  if (mn == -INFINITY) return;           // only empty partials so far
  const float a_old = exp2f(M - mn);     // 0 when M = -inf
  L *= a_old;
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] *= a_old;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const float a = exp2f(mi[u] - mn);
    L = fmaf(li[u], a, L);
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = fmaf(oi[u][e], a, o[e]);
  }
  M = mn;
}

// All partials i = first, first + step, ... < ns: groups of U while U remain,
// then of 4, 2 and 1.  Every load in a group is of a real partial:
// masked or repeated loads past the last one cost as much as real ones (one
// wave per head with 16-entry masked groups ran 6x slower at 1 partial per
// head than plain loads).
template <int D, int U>
__device__ __forceinline__ void fold_partials(const float* __restrict__ part_o,
                                              const float* __restrict__ part_ml,
                                              const MergeRows& R, int first, int step, int lane,
                                              float& M, float& L,
                                              float (&o)[D >= kWave ? D / kWave : 1]) {
  int i = first;
  for (; i + (U - 1) * step < R.ns; i += U * step)
    fold_group<D, U>(part_o, part_ml, R, i, step, lane, M, L, o);
  if (i + 3 * step < R.ns) {
    fold_group<D, 4>(part_o, part_ml, R, i, step, lane, M, L, o);
    i += 4 * step;
  }
  if (i + step < R.ns) {
    fold_group<D, 2>(part_o, part_ml, R, i, step, lane, M, L, o);
    i += 2 * step;
  }
  if (i < R.ns) fold_group<D, 1>(part_o, part_ml, R, i, step, lane, M, L, o);
}

__device__ __forceinline__ void store_out(void* out, int out_bf16, int64_t at, float r) {
  const uint16_t hb = float_to_half_bits(r);
  const uint16_t ob = out_bf16 ? float_to_bf16_bits(half_bits_to_float(hb)) : hb;
  static_cast<uint16_t*>(out)[at] = ob;
}

template <int D, int NW>
__global__ __launch_bounds__(NW * 64) void merge_kernel(const float* __restrict__ part_o,
                                                    const float* __restrict__ part_ml,
                                                    const int32_t* __restrict__ seq_lens,
                                                    int hq, int max_context,
                                                    int split_tokens, int num_splits,
                                                    void* __restrict__ out, int out_bf16,
                                                    int64_t o_stride_seq, int64_t o_stride_head,
                                                    const int32_t* __restrict__ stream_meta,
                                                    const int32_t* __restrict__ stream_hdr) {
  constexpr int E = D >= kWave ? D / kWave : 1;     // elements per lane
  __shared__ float s_o[NW][D];
  __shared__ float s_m[NW], s_l[NW];
  const int h = blockIdx.x;
  const int seq = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const MergeRows R = merge_rows(seq_lens, seq, h, hq, max_context, split_tokens, num_splits,
                                 stream_meta, stream_hdr);
  float M = -INFINITY, L = 0.0f, o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = 0.0f;
  const bool active = lane * E < D;
  fold_partials<D, 8>(part_o, part_ml, R, w, NW, lane, M, L, o);
  if (lane == 0) {
    s_m[w] = M;
    s_l[w] = L;
  }
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (active) s_o[w][lane * E + e] = o[e];
  __syncthreads();
  if (w != 0) return;
  float Mg = -INFINITY;
#pragma unroll
  for (int k = 0; k < NW; ++k) Mg = fmaxf(Mg, s_m[k]);
  float Lg = 0.0f, f[NW];
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    // a wave that saw no split has M = -inf and contributes nothing
    f[k] = s_m[k] == -INFINITY ? 0.0f : exp2f(s_m[k] - Mg);
    Lg += s_l[k] * f[k];
  }
  if (!active) return;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int d = lane * E + e;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < NW; ++k) acc += s_o[k][d] * f[k];
    store_out(out, out_bf16, seq * o_stride_seq + h * o_stride_head + d, acc / Lg);
  }
}

// Few partials per (sequence, q head) in a large batch: one wave folds each
// head's partials (8 in flight), HPW heads of one sequence per workgroup, no
// LDS: a quarter of the waves of merge_kernel, so a quarter of the rounds of
// resident waves (B = 1024, 32 heads, one partial each: 9 us; four waves
// per head with a group of 8 masked loads each took about 40 us).
template <int D, int HPW>
__global__ __launch_bounds__(HPW * 64) void merge_wave_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const int32_t* __restrict__ seq_lens, int hq, int max_context, int split_tokens,
    int num_splits, void* __restrict__ out, int out_bf16, int64_t o_stride_seq,
    int64_t o_stride_head, const int32_t* __restrict__ stream_meta,
    const int32_t* __restrict__ stream_hdr) {
  constexpr int E = D >= kWave ? D / kWave : 1;
  const int lane = threadIdx.x & (kWave - 1);
  const int h = blockIdx.x * HPW + static_cast<int>(threadIdx.x) / kWave;
  const int seq = blockIdx.y;
  if (h >= hq) return;                   // a whole wave; no barrier follows
  const MergeRows R = merge_rows(seq_lens, seq, h, hq, max_context, split_tokens, num_splits,
                                 stream_meta, stream_hdr);
  float M = -INFINITY, L = 0.0f, o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = 0.0f;
  fold_partials<D, 8>(part_o, part_ml, R, 0, 1, lane, M, L, o);
  if (lane * E >= D) return;
#pragma unroll
  for (int e = 0; e < E; ++e)
    store_out(out, out_bf16, seq * o_stride_seq + h * o_stride_head + lane * E + e, o[e] / L);
}

// Fold partials i = first, first + step, ... < ns of one (sequence, q head)
// for one dimension d: N loads in flight per group, then the remainder in
// groups of 4, 2 and 1 (every load of a real partial, as in fold_partials).
template <int D, int N>
__device__ __forceinline__ void fold_dim_group(const float* __restrict__ part_o,
                                               const float* __restrict__ part_ml,
                                               const MergeRows& R, int first, int step, int d,
                                               float& M, float& L, float& o) {
  float mi[N], li[N], oi[N];
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int64_t ent = R.row0 + static_cast<int64_t>(first + step * u) * R.stride;
    mi[u] = part_ml[2 * ent];
    li[u] = part_ml[2 * ent + 1];
    oi[u] = part_o[ent * D + d];
  }
  float mn = M;
#pragma unroll
  for (int u = 0; u < N; ++u) mn = fmaxf(mn, mi[u]);
  if (mn == -INFINITY) return;
  const float a_old = exp2f(M - mn);
  L *= a_old;
  o *= a_old;
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const float a = exp2f(mi[u] - mn);
    L = fmaf(li[u], a, L);
    o = fmaf(oi[u], a, o);
  }
  M = mn;
}

template <int D, int U>
__device__ __forceinline__ void fold_dim(const float* __restrict__ part_o,
                                         const float* __restrict__ part_ml, const MergeRows& R,
                                         int first, int step, int d, float& M, float& L,
                                         float& o) {
  int i = first;
  for (; i + (U - 1) * step < R.ns; i += U * step)
    fold_dim_group<D, U>(part_o, part_ml, R, i, step, d, M, L, o);
  if (i + 3 * step < R.ns) {
    fold_dim_group<D, 4>(part_o, part_ml, R, i, step, d, M, L, o);
    i += 4 * step;
  }
  if (i + step < R.ns) {
    fold_dim_group<D, 2>(part_o, part_ml, R, i, step, d, M, L, o);
    i += 2 * step;
  }
  if (i < R.ns) fold_dim_group<D, 1>(part_o, part_ml, R, i, step, d, M, L, o);
}

// Few (sequence, q head) rows with many partials each (one sequence at long
// context: 32 rows of 256 partials at config 4).  merge_kernel gives such a
// batch one workgroup per row, 32 in all, and each pulls its row's 133 KB
// through one CU (6.6 us for 4.3 MB).  Here a workgroup takes one 16-dim
// slice of one row, D / 16 workgroups per row: thread t folds dim
// d0 + t % 16 of partials t / 16, t / 16 + 16, ..., and the 16 split lanes
// are combined through LDS.  The 16 threads of a split lane fold the same
// (m, l) pairs (16 lanes loading one address make one request).
template <int D>
__global__ __launch_bounds__(256) void merge_slice_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const int32_t* __restrict__ seq_lens, int hq, int max_context, int split_tokens,
    int num_splits, void* __restrict__ out, int out_bf16, int64_t o_stride_seq,
    int64_t o_stride_head, const int32_t* __restrict__ stream_meta,
    const int32_t* __restrict__ stream_hdr) {
  constexpr int SD = 16;           // dims per workgroup
  constexpr int NSL = 256 / SD;    // split lanes
  static_assert(D % SD == 0, "whole slices");
  __shared__ float s_o[NSL][SD];
  __shared__ float s_m[NSL], s_l[NSL];
  const int h = blockIdx.x;
  const int seq = blockIdx.y;
  const int dl = threadIdx.x % SD;
  const int sl = threadIdx.x / SD;
  const int d = blockIdx.z * SD + dl;
  const MergeRows R = merge_rows(seq_lens, seq, h, hq, max_context, split_tokens, num_splits,
                                 stream_meta, stream_hdr);
  float M = -INFINITY, L = 0.0f, o = 0.0f;
  fold_dim<D, 8>(part_o, part_ml, R, sl, NSL, d, M, L, o);
  if (dl == 0) {
    s_m[sl] = M;
    s_l[sl] = L;
  }
  s_o[sl][dl] = o;
  __syncthreads();
  if (sl != 0) return;
  float Mg = -INFINITY;
#pragma unroll
  for (int k = 0; k < NSL; ++k) Mg = fmaxf(Mg, s_m[k]);
  float Lg = 0.0f, acc = 0.0f;
#pragma unroll
  for (int k = 0; k < NSL; ++k) {
    // a split lane that saw no partial has M = -inf and contributes nothing
    const float f = s_m[k] == -INFINITY ? 0.0f : exp2f(s_m[k] - Mg);
    Lg += s_l[k] * f;
    acc += s_o[k][dl] * f;
  }
  store_out(out, out_bf16, seq * o_stride_seq + h * o_stride_head + d, acc / Lg);
}

__global__ void stream_header_kernel(int32_t* hdr, int h0, int h1, int h2) {
  if (threadIdx.x == 0) {
    hdr[0] = h0;
    hdr[1] = h1;
    hdr[2] = h2;
  }
}

int launch_stream_header(int32_t* hdr, int h0, int h1, int h2, hipStream_t stream) {
  hipLaunchKernelGGL(stream_header_kernel, dim3(1), dim3(kWave), 0, stream, hdr, h0, h1, h2);
  return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
}

int launch_merge(const float* part_o, const float* part_ml, const int32_t* seq_lens,
                 int num_seqs, int hq, int head_size, int max_context, int split_tokens,
                 int num_splits,
                 void* out, int out_bf16, int64_t o_stride_seq, int64_t o_stride_head,
                 hipStream_t stream, const int32_t* stream_meta, const int32_t* stream_hdr) {
  // the stream schedule passes the entries a row has on average, at most its
  // block count, as num_splits.  One wave per head when a head's partials are
  // at most 2, or at most 16 and the heads alone fill the GPU's wave slots a
  // quarter over (more than 2048 of them): four waves per head then take
  // several rounds of resident waves, each a chain of memory round trips;
  // with fewer heads four waves per head fold a head in fewer round trips.
  if (num_splits <= 2 || (num_splits <= 16 && static_cast<int64_t>(num_seqs) * hq > 2048)) {
    // one wave per (sequence, q head), 8 (or 4) heads per workgroup
    const int hpw = hq % 8 == 0 ? 8 : 4;
    const dim3 wgrid((hq + hpw - 1) / hpw, num_seqs);
    switch (head_size) {
#define KNLP_MERGE_W(D, HPW)                                                              \
    hipLaunchKernelGGL((merge_wave_kernel<D, HPW>), wgrid, dim3(kWave * HPW), 0, stream,  \
                       part_o, part_ml, seq_lens, hq, max_context, split_tokens,          \
                       num_splits, out, out_bf16, o_stride_seq, o_stride_head,            \
                       stream_meta, stream_hdr);
#define KNLP_MERGE_WD(D)                                                                  \
  case D:                                                                                 \
    if (hpw == 8) { KNLP_MERGE_W(D, 8) } else { KNLP_MERGE_W(D, 4) }                      \
    break;
      KNLP_MERGE_WD(32)
      KNLP_MERGE_WD(64)
      KNLP_MERGE_WD(128)
      KNLP_MERGE_WD(256)
#undef KNLP_MERGE_WD
#undef KNLP_MERGE_W
      default:
        return KNLP_ERR_SHAPE;
    }
    return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
  }
  // few rows of many partials: one workgroup per 16-dim slice of a row
  if (num_splits >= kSliceMinSplits && static_cast<int64_t>(num_seqs) * hq <= kSliceMaxRows) {
    const dim3 sgrid(hq, num_seqs, head_size / 16);
    switch (head_size) {
#define KNLP_MERGE_S(D)                                                                   \
  case D:                                                                                 \
    hipLaunchKernelGGL((merge_slice_kernel<D>), sgrid, dim3(256), 0, stream, part_o,      \
                       part_ml, seq_lens, hq, max_context, split_tokens, num_splits, out, \
                       out_bf16, o_stride_seq, o_stride_head, stream_meta, stream_hdr);   \
    break;
      KNLP_MERGE_S(32)
      KNLP_MERGE_S(64)
      KNLP_MERGE_S(128)
      KNLP_MERGE_S(256)
#undef KNLP_MERGE_S
      default:
        return KNLP_ERR_SHAPE;
    }
    return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
  }
  const dim3 grid(hq, num_seqs);
  // waves per (sequence, q head): one group of U = 8 splits each up to 32
  // splits, then 8 and 16 waves
  const int nw = num_splits <= 32 ? 4 : num_splits <= 64 ? 8 : 16;
  const dim3 block(kWave * nw);
  switch (head_size) {
#define KNLP_MERGE_NW(D, NW)                                                            \
    hipLaunchKernelGGL((merge_kernel<D, NW>), grid, block, 0, stream, part_o, part_ml,  \
                       seq_lens, hq, max_context, split_tokens, num_splits, out, out_bf16, \
                       o_stride_seq, o_stride_head, stream_meta, stream_hdr);
#define KNLP_MERGE_D(D)                                                                 \
  case D:                                                                               \
    if (nw == 4) { KNLP_MERGE_NW(D, 4) }                                                \
    else if (nw == 8) { KNLP_MERGE_NW(D, 8) }                                           \
    else { KNLP_MERGE_NW(D, 16) }                                                       \
    break;
    KNLP_MERGE_D(32)
    KNLP_MERGE_D(64)
    KNLP_MERGE_D(128)
    KNLP_MERGE_D(256)
#undef KNLP_MERGE_D
#undef KNLP_MERGE_NW
    default:
      return KNLP_ERR_SHAPE;
  }
  return hipGetLastError() == hipSuccess ? KNLP_OK : KNLP_ERR_LAUNCH;
}

}  // namespace knlp
