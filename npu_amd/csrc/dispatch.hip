// Token -> expert dispatch: histogram, exclusive prefix-scan and a stable
// scatter of (token, slot) pairs into expert-sorted order, in one block.
//
// Equivalent of the reference's host loop over torch.unique(topk_ids) with
// (topk_ids == e).nonzero() per expert (qwen/forward.py:612, 623-629): pairs
// p = t*k + j are grouped by ascending expert id and stay in ascending p
// (hence ascending token) order inside each expert.
//
// Each of the 16 waves owns a contiguous run of pairs.  Counting: LDS
// atomics into per-wave histograms.  Scatter: a wave takes 64 consecutive
// pairs at a time; the lanes holding the same expert are found with one
// ballot per bit of the expert id, a lane's rank among them is a popcount,
// and the last of them advances the wave's running base for that expert.
// Optionally the same block cuts every expert's list (and a shared unit of
// T tokens) into segments of at most seg_tok pairs for the grouped GEMMs.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int kWaves = 16;
constexpr int kMaxE = 512;
constexpr int kBatch = 4;                   // 64-pair steps whose ids are loaded together

__global__ void __launch_bounds__(1024) k_dispatch(const int32_t* __restrict__ ids, int P, int E,
                                                   int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                   int32_t* __restrict__ sorted, int32_t* __restrict__ inv,
                                                   int32_t* __restrict__ segs, int seg_tok, int shared_T) {
  extern __shared__ int32_t cnt[];          // [kWaves][E] per-wave counts, then bases
  __shared__ int32_t wsum[kWaves];
  __shared__ int32_t nseg[kMaxE + 1];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < kWaves * E; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  const int chunk = (P + kWaves - 1) / kWaves;
  const int p0 = wave * chunk, p1 = min(P, p0 + chunk);
  int e0[kBatch];                            // the first batch's ids, kept for the scatter
  for (int b = p0; b < p1; b += 64 * kBatch) {
    int eb[kBatch];                          // every load of the batch before the first use
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int p = b + 64 * j + lane;
      eb[j] = p < p1 ? ids[p] : -1;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (b == p0) e0[j] = eb[j];
      if (eb[j] >= 0 && eb[j] < E) atomicAdd(&cnt[wave * E + eb[j]], 1);
    }
  }
  __syncthreads();
  // per-expert totals (thread e) and their exclusive scan across the block
  int tot = 0;
  if (threadIdx.x < E)
    for (int w = 0; w < kWaves; ++w) tot += cnt[w * E + threadIdx.x];
  int v = threadIdx.x < E ? tot : 0;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(v, o, 64);
    if (lane >= o) v += n;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < kWaves; ++w) { const int s = wsum[w]; wsum[w] = run; run += s; }
  }
  __syncthreads();
  v += wsum[wave];                           // inclusive prefix
  if (threadIdx.x < E) {
    const int excl = v - tot;
    counts[threadIdx.x] = tot;
    offsets[threadIdx.x] = excl;
    if (threadIdx.x == E - 1) offsets[E] = v;
    int run = excl;                          // per-wave bases: excl + counts of earlier waves
    for (int w = 0; w < kWaves; ++w) {
      const int c = cnt[w * E + threadIdx.x];
      cnt[w * E + threadIdx.x] = run;
      run += c;
    }
    if (segs) nseg[threadIdx.x] = (tot + seg_tok - 1) / seg_tok;
  }
  if (segs && threadIdx.x == E) nseg[E] = shared_T > 0 ? (shared_T + seg_tok - 1) / seg_tok : 0;
  __syncthreads();
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  for (int b0 = p0; b0 < p1; b0 += 64 * kBatch) {
    int eb[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int p = b0 + 64 * j + lane;
      eb[j] = b0 == p0 ? e0[j] : p < p1 ? ids[p] : -1;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int b = b0 + 64 * j;
      if (b >= p1) break;                      // wave-uniform
      const int p = b + lane;
      int e = eb[j];
      if (e >= E) e = -1;
      uint64_t same = __ballot(e >= 0);
      for (int i = 0; i < nbits; ++i) {
        const uint64_t m = __ballot((e >> i) & 1);
        same &= ((e >> i) & 1) ? m : ~m;
      }
      const int r = __popcll(same & ((1ull << lane) - 1ull));
      const bool last = (same >> lane) >> 1 == 0;          // no same-expert lane above
      int pos = 0;
      if (e >= 0) pos = cnt[wave * E + e] + r;
      __builtin_amdgcn_wave_barrier();
      if (e >= 0) {
        sorted[pos] = p;
        if (inv) inv[p] = pos;
        if (last) cnt[wave * E + e] = pos + 1;
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  if (!segs) return;
  // segments: unit u < E is expert u, unit E the shared one; exclusive scan of nseg
  const int n_units = E + (shared_T > 0 ? 1 : 0);
  __syncthreads();
  int ns = threadIdx.x < n_units ? nseg[threadIdx.x] : 0;
  int sv = ns;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(sv, o, 64);
    if (lane >= o) sv += n;
  }
  __syncthreads();
  if (lane == 63) wsum[wave] = sv;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < kWaves; ++w) { const int s = wsum[w]; wsum[w] = run; run += s; }
    segs[0] = run;
  }
  __syncthreads();
  if (threadIdx.x < n_units) {
    const int base = sv + wsum[wave] - ns;
    const int n = threadIdx.x < E ? tot : shared_T;
    for (int j = 0; j < ns; ++j) {
      int32_t* s = segs + 1 + 4 * (base + j);
      s[0] = threadIdx.x;
      s[1] = j * seg_tok;
      s[2] = min(seg_tok, n - j * seg_tok);
      s[3] = 0;
    }
  }
}

}  // namespace

int gm_launch_dispatch_seg(const int32_t* ids, int T, int k, int E, int32_t* counts, int32_t* offsets,
                           int32_t* sorted_pairs, int32_t* inv, int32_t* segs, int seg_tok, int shared_T,
                           hipStream_t s) {
  if (E <= 0 || E > kMaxE) return gm_fail_arg("gm_moe_dispatch: E=%d out of range (1..%d)", E, kMaxE);
  const int P = T * k;
  const size_t smem = (size_t)kWaves * E * sizeof(int32_t);
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), smem, s, ids, P, E, counts, offsets, sorted_pairs, inv, segs,
                     seg_tok, shared_T);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

int gm_launch_dispatch(const int32_t* ids, int T, int k, int E, int32_t* counts, int32_t* offsets,
                       int32_t* sorted_pairs, hipStream_t s) {
  return gm_launch_dispatch_seg(ids, T, k, E, counts, offsets, sorted_pairs, nullptr, nullptr, 1, 0, s);
}
