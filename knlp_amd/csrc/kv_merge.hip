// Stage 3: merge per-split partial softmax states (new; the reference has no
// split-K).  For one (sequence, q head) with splits i = 0..n-1 holding
// (o_i[D], m_i, l_i) -- unnormalised accumulator, running max in log2 units,
// running sum -- the result is
//     M = max m_i,  L = sum l_i 2^(m_i - M),  out = sum o_i 2^(m_i - M) / L,
// rounded fp32 -> fp16 (F:891-894) and then to bf16 when the output tensor is
// bf16.  n = ceil(seq_len / split_tokens); n = 0 gives 0/0 = NaN, matching the
// reference's acc / l_i with l_i = 0 (F:886-887).
//
// One block of NW waves per (sequence, q head): wave w folds splits
// w, w+NW, ... with an online (max-rescaling) combine, then the NW wave
// states are combined through LDS.  NW grows with the split count (4, 8 or
// 16 waves) so that a wave folds at most a few groups of U splits: config 4
// (one sequence, 256 splits) merges in about a third of the time 4 waves take.
#include "kv_decode.h"

namespace knlp {

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
  const int n_len = min(seq_lens[seq], max_context);
  // the partials of (seq, h): entries row0 + i * stride, i < ns
  int ns;
  int64_t row0, stride;
  if (stream_meta == nullptr) {       // split schedule: [num_seqs, hq, num_splits]
    ns = min(num_splits, (n_len + split_tokens - 1) / split_tokens);
    row0 = (static_cast<int64_t>(seq) * hq + h) * num_splits;
    stride = 1;
  } else {
    // a stream workspace: the record, the header and the length load
    // together (none needs another; the record is unused after a split-K run)
    const int64_t r = 2 * (static_cast<int64_t>(seq) * hq + h);
    const int first = stream_meta[r], count = stream_meta[r + 1];
    const int hg = stream_hdr[0];
    if (hg > 0) {                     // stream schedule: one entry per block segment
      ns = n_len > 0 ? count : 0;     // (a row of length 0 has no record)
      row0 = n_len > 0 ? first : 0;
      stride = hg;                    // query heads per row (8 kv heads' groups)
    } else {                          // split-K in the workspace (header: split, splits)
      const int st = stream_hdr[1];
      const int nsp = stream_hdr[2];
      ns = min(nsp, (n_len + st - 1) / st);
      row0 = (static_cast<int64_t>(seq) * hq + h) * nsp;
      stride = 1;
    }
  }

  // Splits are taken U at a time per wave with every load of the group issued
  // before any use, so a wave waits for about one memory round trip per
  // group instead of one per split.
  constexpr int U = 8;
  float M = -INFINITY, L = 0.0f, o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = 0.0f;
  const bool active = lane * E < D;
  for (int base = w; base < ns; base += NW * U) {
    float mi[U], li[U], oi[U][E];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + NW * u;
      const bool ok = i < ns;
      const int64_t ent = row0 + i * stride;
      mi[u] = ok ? part_ml[2 * ent] : -INFINITY;
      li[u] = ok ? part_ml[2 * ent + 1] : 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e)
        oi[u][e] = ok && active ? part_o[ent * D + lane * E + e] : 0.0f;
    }
    float mn = M;
#pragma unroll
    for (int u = 0; u < U; ++u) mn = fmaxf(mn, mi[u]);
    if (mn == -INFINITY) continue;       // nothing in this group (or all empty)
    const float a_old = exp2f(M - mn);   // 0 when M = -inf
    L *= a_old;
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] *= a_old;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float a = exp2f(mi[u] - mn);  // 0 for the padding entries
      L = fmaf(li[u], a, L);
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = fmaf(oi[u][e], a, o[e]);
    }
    M = mn;
  }
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
    const float r = acc / Lg;
    const uint16_t hb = float_to_half_bits(r);
    const uint16_t ob = out_bf16 ? float_to_bf16_bits(half_bits_to_float(hb)) : hb;
    static_cast<uint16_t*>(out)[seq * o_stride_seq + h * o_stride_head + d] = ob;
  }
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
  const dim3 grid(hq, num_seqs);
  // waves per (sequence, q head): one group of U = 8 splits each up to 32
  // splits, then 8 and 16 waves (the stream schedule passes the entries a row
  // has on average, at most its block count)
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
