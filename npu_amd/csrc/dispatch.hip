// Token -> expert dispatch: histogram, exclusive prefix-scan and a stable
// scatter of (token, slot) pairs into expert-sorted order, in one block.
//
// Equivalent of the reference's host loop over torch.unique(topk_ids) with
// (topk_ids == e).nonzero() per expert (qwen/forward.py:612, 623-629): pairs
// p = t*k + j are grouped by ascending expert id and stay in ascending p
// (hence ascending token) order inside each expert.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int kWaves = 16;
constexpr int kMaxE = 512;

__global__ void __launch_bounds__(1024) k_dispatch(const int32_t* __restrict__ ids, int P, int E,
                                                   int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                                   int32_t* __restrict__ sorted, int32_t* __restrict__ inv) {
  extern __shared__ int32_t cnt[];          // [kWaves][E] per-wave counts, then bases
  __shared__ int32_t tot_scan[kMaxE + 1];
  __shared__ int32_t wsum[kWaves];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < kWaves * E; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  // contiguous chunk of pairs per wave (preserves order for the stable scatter)
  const int chunk = (P + kWaves - 1) / kWaves;
  const int p0 = wave * chunk, p1 = min(P, p0 + chunk);
  for (int p = p0 + lane; p < p1; p += 64) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[wave * E + e], 1);
  }
  __syncthreads();
  // per-expert totals and exclusive scan over experts (block-wide)
  int tot = 0;
  if (threadIdx.x < E)
    for (int w = 0; w < kWaves; ++w) tot += cnt[w * E + threadIdx.x];
  // inclusive scan of tot across threads 0..E-1 (E <= 1024): wave scan + wave sums
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
    tot_scan[threadIdx.x] = excl;
    counts[threadIdx.x] = tot;
    offsets[threadIdx.x] = excl;
    if (threadIdx.x == E - 1) offsets[E] = v;
    // per-wave bases for this expert: excl + counts of earlier waves
    int run = excl;
    for (int w = 0; w < kWaves; ++w) {
      const int c = cnt[w * E + threadIdx.x];
      cnt[w * E + threadIdx.x] = run;
      run += c;
    }
  }
  __syncthreads();
  // stable scatter: batches of 64 consecutive pairs per wave, in order
  for (int b = p0; b < p1; b += 64) {
    const int p = b + lane;
    const int e = (p < p1) ? ids[p] : -1;
    int r = 0, last = 1;
    for (int q = 0; q < 64; ++q) {
      const int eq = __shfl(e, q, 64);
      if (eq == e && e >= 0) {
        if (q < lane) r += 1;
        if (q > lane) last = 0;
      }
    }
    int pos = 0;
    if (e >= 0 && e < E) pos = cnt[wave * E + e] + r;
    __builtin_amdgcn_wave_barrier();
    if (e >= 0 && e < E) {
      sorted[pos] = p;
      if (inv) inv[p] = pos;
      if (last) cnt[wave * E + e] = pos + 1;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace

int gm_launch_dispatch_inv(const int32_t* ids, int T, int k, int E, int32_t* counts, int32_t* offsets,
                           int32_t* sorted_pairs, int32_t* inv, hipStream_t s) {
  if (E <= 0 || E > kMaxE) return gm_fail_arg("gm_moe_dispatch: E=%d out of range (1..%d)", E, kMaxE);
  const int P = T * k;
  const size_t smem = (size_t)kWaves * E * sizeof(int32_t);
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), smem, s, ids, P, E, counts, offsets, sorted_pairs, inv);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

int gm_launch_dispatch(const int32_t* ids, int T, int k, int E, int32_t* counts, int32_t* offsets,
                       int32_t* sorted_pairs, hipStream_t s) {
  return gm_launch_dispatch_inv(ids, T, k, E, counts, offsets, sorted_pairs, nullptr, s);
}
