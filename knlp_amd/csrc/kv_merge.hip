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
// folds them (merge_wave_kernel).  Otherwise one block of NW waves per
// (sequence, q head), wave w folds splits w, w+NW, ... with an online (max-rescaling)
// combine, then the NW wave states are combined through LDS.  NW grows with
// the split count (4, 8 or 16 waves) so that a wave folds at most a few
// groups of U splits: config 4 (one sequence, 256 splits) merges in about a
// third of the time 4 waves take.
#include "kv_decode.h"

namespace knlp {

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
