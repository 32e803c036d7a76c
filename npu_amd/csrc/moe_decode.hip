// MoE block, decode path (T <= 8 tokens): three kernels per block.
//
//   K1 k_moe_router   router logits (bf16 W, fp32 xn) + shared scalar gate, and the
//                     shared expert's gate/up + SwiGLU (independent of routing)
//   K2 k_moe_gateup   every block recomputes top-k from the logits and the
//                     per-expert grouping of (token, slot) pairs, then computes its
//                     (expert, row-chunk) tile of silu(G x) * (U x); block 0 also
//                     publishes ids / weights / grouping for K3
//   K3 k_moe_down     per output-row tile: sum over unique experts in ascending id
//                     of w * (Down_e . h), then + sigmoid-gated shared expert
//                     (+ residual x); fixed order, no atomics -> bit-reproducible
//
// Kernel boundaries are the global synchronisation points (the three phases
// depend on all of x, all router logits and all of h respectively).
// Reference semantics: qwen/forward.py:563-665 (moe_forward).
#include "iq_decode.h"
#include "kernels.h"

namespace {

// Stage xn = rmsnorm(x) (or x) for tokens t0 .. t0+nt-1 into xs[NT][D].
// rms = 1/sqrt(mean(x^2) + eps); xn = (x * rms) * w  (qwen/forward.py:58-61).
template <int NT>
__device__ void stage_xn(const float* __restrict__ x, int t0, int nt, int D, const float* __restrict__ norm_w,
                         float eps, float* __restrict__ xs, float* __restrict__ red) {
  for (int i = threadIdx.x; i < NT * D; i += blockDim.x) {
    const int t = i / D;
    xs[i] = t < nt ? x[(int64_t)(t0 + t) * D + (i - t * D)] : 0.f;
  }
  if (norm_w != nullptr) {
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    for (int t = wave; t < nt; t += nw) {
      float ss = 0.f;
      for (int i = lane; i < D; i += 64) ss = fmaf(xs[t * D + i], xs[t * D + i], ss);
      ss = gm_wave_sum(ss);
      if (lane == 0) red[t] = 1.0f / sqrtf(ss / (float)D + eps);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nt * D; i += blockDim.x) {
      const int t = i / D;
      xs[i] = (xs[i] * red[t]) * norm_w[i - t * D];
    }
  }
  __syncthreads();
}

// One wave: top-k of E logits (descending, ties -> lower id), softmax over all E,
// renormalised top-k probabilities (qwen/forward.py:609-611).
__device__ void wave_topk(const float* __restrict__ lg, int E, int k, int32_t* __restrict__ ids,
                          float* __restrict__ wts) {
  const int lane = threadIdx.x & 63;
  constexpr int MAXV = 8;  // E <= 512
  float v[MAXV];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? lg[e] : -INFINITY;
    m = fmaxf(m, v[i]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  float z = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i)
    if (lane + 64 * i < E) z += expf(v[i] - m);
  z = gm_wave_sum(z);
  unsigned taken = 0;
  float psum = 0.f;
  float pk[8];
  int ik[8];
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !((taken >> i) & 1u) && (v[i] > bv || (v[i] == bv && e < bi))) { bv = v[i]; bi = e; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    const float p = expf(bv - m) / z;
    pk[r] = p;
    ik[r] = bi;
    psum += p;
  }
  const float den = fmaxf(psum, 1e-20f);
  if (lane == 0) {
    for (int r = 0; r < k; ++r) {
      ids[r] = ik[r];
      wts[r] = pk[r] / den;
    }
  }
}

// Lane partial of one row against several tokens picked by index.
template <int QT, int L, int NT>
__device__ __forceinline__ void row_partial_idx(const uint8_t* __restrict__ row, int nsub, int lir,
                                                const float* __restrict__ xs, int D, const int (&tok)[NT],
                                                int nt, const uint32_t* __restrict__ grid, float (&acc)[NT]) {
  for (int sub = lir; sub < nsub; sub += L) {
    const auto r = gm_load_sub<QT>(row, sub);
    float wv[32];
    const float sc = gm_decode_sub<QT>(r, sub, grid, wv);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      if (t < nt) acc[t] = fmaf(sc, gm_dot32(wv, xs + tok[t] * D + sub * GM_SUB), acc[t]);
  }
}

// ------------------------------------------------------------------- K1
template <int QTS, int L, int NT>
__global__ void __launch_bounds__(256) k_moe_router(gm_moe_layer P, const float* __restrict__ x, int T,
                                                    float* __restrict__ logits, float* __restrict__ shg,
                                                    float* __restrict__ hsh, int n_router_blocks,
                                                    int sh_rows_per_wave) {
  extern __shared__ float smem[];
  uint32_t* grid = reinterpret_cast<uint32_t*>(smem);
  float* red = smem + 256;
  float* xs = red + 16;
  const int D = P.D;
  stage_xn<NT>(x, 0, T, D, P.norm_w, P.norm_eps, xs, red);
  if constexpr (QTS == GM_QTYPE_IQ3_XXS) {
    gm_stage_grid(grid);
    __syncthreads();
  }
  constexpr int RPS = 64 / L;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nsub = D / GM_SUB;
  if ((int)blockIdx.x < n_router_blocks) {
    // router rows 0..E-1, then the shared scalar gate as row E
    const int nrows = P.E + (P.sh_gate_inp != nullptr ? 1 : 0);
    const int64_t rb = (int64_t)D * 2;
    for (int r0 = 0; r0 < RPS; r0 += RPS) {
      const int row = (blockIdx.x * 4 + wave) * RPS + lane / L;
      float acc[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = 0.f;
      if (row < nrows) {
        const uint8_t* wr = row < P.E ? reinterpret_cast<const uint8_t*>(P.router) + row * rb
                                      : reinterpret_cast<const uint8_t*>(P.sh_gate_inp);
        for (int sub = lane % L; sub < nsub; sub += L) {
          const RawBf16 r = gm_load_bf16(wr, sub);
          float wv[32];
          gm_decode_bf16(r, wv);
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[t] += gm_dot32(wv, xs + t * D + sub * GM_SUB);
        }
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = gm_group_sum<L>(acc[t]);
      if (row < nrows && (lane % L) == 0) {
        for (int t = 0; t < T && t < NT; ++t) {
          if (row < P.E) logits[t * P.E + row] = acc[t] + (P.router_bias ? P.router_bias[row] : 0.f);
          else shg[t] = gm_sigmoid(acc[t]);
        }
      }
    }
    return;
  }
  // shared expert gate/up rows
  const int FF = P.FF_sh;
  const int64_t rb = gm_row_bytes(QTS, D);
  const uint8_t* wg = static_cast<const uint8_t*>(P.gate_sh);
  const uint8_t* wu = static_cast<const uint8_t*>(P.up_sh);
  const int rbase = ((blockIdx.x - n_router_blocks) * 4 + wave) * sh_rows_per_wave;
  int tok[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) tok[t] = t;
  for (int r0 = 0; r0 < sh_rows_per_wave; r0 += RPS) {
    const int row = rbase + r0 + lane / L;
    float ag[NT], au[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) { ag[t] = 0.f; au[t] = 0.f; }
    if (row < FF) {
      row_partial_idx<QTS, L, NT>(wg + row * rb, nsub, lane % L, xs, D, tok, T, grid, ag);
      row_partial_idx<QTS, L, NT>(wu + row * rb, nsub, lane % L, xs, D, tok, T, grid, au);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) { ag[t] = gm_group_sum<L>(ag[t]); au[t] = gm_group_sum<L>(au[t]); }
    if (row < FF && (lane % L) == 0) {
      for (int t = 0; t < T && t < NT; ++t) hsh[t * FF + row] = gm_silu(ag[t]) * au[t];
    }
  }
}

// Grouping of (token, slot) pairs by expert into LDS (all threads call; pairs
// are handled by wave 0): g[0] = n_unique, g[1+u] = expert of slot u
// (ascending), g[65+u] = member count, g[129 + 8u + m] = pair index t*k + j
// of member m (tokens ascending).
__device__ void block_group(const int32_t* __restrict__ ids, int P, int E, int32_t* __restrict__ g,
                            uint32_t* __restrict__ bits) {
  const int nwords = (E + 31) / 32;
  for (int i = threadIdx.x; i < nwords; i += blockDim.x) bits[i] = 0u;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const bool w0 = threadIdx.x < 64;
  const int e = (w0 && lane < P) ? ids[lane] : -1;
  if (e >= 0) atomicOr(&bits[e >> 5], 1u << (e & 31));
  __syncthreads();
  if (w0) {
    int nu = 0, rank = 0;
    for (int w = 0; w < nwords; ++w) {
      const uint32_t b = bits[w];
      nu += __builtin_popcount(b);
      if (e >= 0 && (w << 5) < e) {
        const int hi = e - (w << 5);
        rank += hi >= 32 ? __builtin_popcount(b) : __builtin_popcount(b & ((1u << hi) - 1u));
      }
    }
    int m = 0, cnt = 0;
    for (int q = 0; q < P; ++q) {
      const int eq = __shfl(e, q, 64);
      if (eq == e) {
        cnt += 1;
        if (q < lane) m += 1;
      }
    }
    if (lane == 0) g[0] = nu;
    if (e >= 0) {
      g[1 + rank] = e;
      g[1 + GM_GRP_MAXU + rank] = cnt;
      g[1 + 2 * GM_GRP_MAXU + rank * GM_GRP_MAXM + m] = lane;
    }
  }
  __syncthreads();
}

// ------------------------------------------------------------------- K2
template <int QT, int L, int NT>
__global__ void __launch_bounds__(256) k_moe_gateup(gm_moe_layer P, const float* __restrict__ x, int T,
                                                    const float* __restrict__ logits, int32_t* __restrict__ g_ids,
                                                    float* __restrict__ g_wts, int32_t* __restrict__ g_grp,
                                                    float* __restrict__ h, int rows_per_block) {
  extern __shared__ float smem[];
  uint32_t* grid = reinterpret_cast<uint32_t*>(smem);
  float* red = smem + 256;
  int32_t* ids = reinterpret_cast<int32_t*>(red + 16);        // [64]
  float* wts = reinterpret_cast<float*>(ids + 64);           // [64]
  int32_t* grp = reinterpret_cast<int32_t*>(wts + 64);       // [GM_GRP_WORDS]
  uint32_t* bits = reinterpret_cast<uint32_t*>(grp + GM_GRP_WORDS);  // [16]
  float* xs = reinterpret_cast<float*>(bits + 16);
  const int D = P.D, E = P.E, k = P.k, FF = P.FF;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // routing (redundant per block: cheaper than another grid-wide sync)
  for (int t = wave; t < T; t += 4) wave_topk(logits + t * E, E, k, ids + t * k, wts + t * k);
  __syncthreads();
  block_group(ids, T * k, E, grp, bits);
  stage_xn<NT>(x, 0, T, D, P.norm_w, P.norm_eps, xs, red);   // contains __syncthreads
  if constexpr (QT == GM_QTYPE_IQ3_XXS) gm_stage_grid(grid);
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < T * k; i += 256) { g_ids[i] = ids[i]; g_wts[i] = wts[i]; }
    for (int i = threadIdx.x; i < GM_GRP_WORDS; i += 256) g_grp[i] = grp[i];
  }
  const int n_chunks = (FF + rows_per_block - 1) / rows_per_block;
  const int u = blockIdx.x / n_chunks, chunk = blockIdx.x - u * n_chunks;
  if (u >= grp[0]) return;
  const int e = grp[1 + u];
  const int nm = grp[1 + GM_GRP_MAXU + u];
  int tok[NT], pair[NT];
#pragma unroll
  for (int m = 0; m < NT; ++m) {
    const int p = m < nm ? grp[1 + 2 * GM_GRP_MAXU + u * GM_GRP_MAXM + m] : 0;
    pair[m] = p;
    tok[m] = p / k;
  }
  constexpr int RPS = 64 / L;
  const int nsub = D / GM_SUB;
  const int64_t rb = gm_row_bytes(QT, D);
  const uint8_t* wg = static_cast<const uint8_t*>(P.gate_exps) + (int64_t)e * FF * rb;
  const uint8_t* wu = static_cast<const uint8_t*>(P.up_exps) + (int64_t)e * FF * rb;
  const int rows_per_wave = rows_per_block / 4;
  const int rbase = chunk * rows_per_block + wave * rows_per_wave;
  for (int r0 = 0; r0 < rows_per_wave; r0 += RPS) {
    const int row = rbase + r0 + lane / L;
    float ag[NT], au[NT];
#pragma unroll
    for (int m = 0; m < NT; ++m) { ag[m] = 0.f; au[m] = 0.f; }
    if (row < FF) {
      row_partial_idx<QT, L, NT>(wg + row * rb, nsub, lane % L, xs, D, tok, nm, grid, ag);
      row_partial_idx<QT, L, NT>(wu + row * rb, nsub, lane % L, xs, D, tok, nm, grid, au);
    }
#pragma unroll
    for (int m = 0; m < NT; ++m) { ag[m] = gm_group_sum<L>(ag[m]); au[m] = gm_group_sum<L>(au[m]); }
    if (row < FF && (lane % L) == 0) {
#pragma unroll
      for (int m = 0; m < NT; ++m)
        if (m < nm) h[(int64_t)pair[m] * FF + row] = gm_silu(ag[m]) * au[m];
    }
  }
}

// ------------------------------------------------------------------- K3
template <int QTD, int QTS, int L, int NT>
__global__ void __launch_bounds__(256) k_moe_down(gm_moe_layer P, const float* __restrict__ x, int T, int flags,
                                                  const float* __restrict__ g_wts, const int32_t* __restrict__ g_grp,
                                                  const float* __restrict__ h, const float* __restrict__ shg,
                                                  const float* __restrict__ hsh, float* __restrict__ y,
                                                  int rows_per_wave) {
  __shared__ uint32_t grid[256];
  __shared__ int32_t grp[GM_GRP_WORDS];
  __shared__ float wts[64];
  __shared__ float sg[GM_DECODE_MAX_T];
  const int D = P.D, FF = P.FF, k = P.k;
  if constexpr (QTD == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS) gm_stage_grid(grid);
  for (int i = threadIdx.x; i < GM_GRP_WORDS; i += 256) grp[i] = g_grp[i];
  for (int i = threadIdx.x; i < T * k; i += 256) wts[i] = g_wts[i];
  if (threadIdx.x < T) sg[threadIdx.x] = P.down_sh ? shg[threadIdx.x] : 0.f;
  __syncthreads();
  constexpr int RPS = 64 / L;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lir = lane % L;
  const int nsub = FF / GM_SUB;
  const int64_t rbd = gm_row_bytes(QTD, FF);
  const int64_t rbs = gm_row_bytes(QTS, FF);
  const int nu = grp[0];
  const int rbase = (blockIdx.x * 4 + wave) * rows_per_wave;
  for (int r0 = 0; r0 < rows_per_wave; r0 += RPS) {
    const int row = rbase + r0 + lane / L;
    const bool live = row < D;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.f;
    for (int u = 0; u < nu; ++u) {
      const int e = grp[1 + u];
      const int nm = grp[1 + GM_GRP_MAXU + u];
      const uint8_t* wr = static_cast<const uint8_t*>(P.down_exps) + ((int64_t)e * D + (live ? row : 0)) * rbd;
      float part[NT];
#pragma unroll
      for (int m = 0; m < NT; ++m) part[m] = 0.f;
      for (int sub = lir; sub < nsub; sub += L) {
        const auto r = gm_load_sub<QTD>(wr, sub);
        float wv[32];
        const float sc = gm_decode_sub<QTD>(r, sub, grid, wv);
#pragma unroll
        for (int m = 0; m < NT; ++m) {
          if (m < nm) {
            const int p = grp[1 + 2 * GM_GRP_MAXU + u * GM_GRP_MAXM + m];
            part[m] = fmaf(sc, gm_dot32(wv, h + (int64_t)p * FF + sub * GM_SUB), part[m]);
          }
        }
      }
#pragma unroll
      for (int m = 0; m < NT; ++m) {
        if (m < nm) {
          const float s = gm_group_sum<L>(part[m]);
          const int p = grp[1 + 2 * GM_GRP_MAXU + u * GM_GRP_MAXM + m];
          const int t = p / k;
#pragma unroll
          for (int tt = 0; tt < NT; ++tt)
            if (tt == t) acc[tt] = fmaf(wts[p], s, acc[tt]);
        }
      }
    }
    if (P.down_sh != nullptr) {
      const uint8_t* wr = static_cast<const uint8_t*>(P.down_sh) + (int64_t)(live ? row : 0) * rbs;
      float part[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) part[t] = 0.f;
      for (int sub = lir; sub < nsub; sub += L) {
        const auto r = gm_load_sub<QTS>(wr, sub);
        float wv[32];
        const float sc = gm_decode_sub<QTS>(r, sub, grid, wv);
#pragma unroll
        for (int t = 0; t < NT; ++t)
          if (t < T) part[t] = fmaf(sc, gm_dot32(wv, hsh + (int64_t)t * FF + sub * GM_SUB), part[t]);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float s = gm_group_sum<L>(part[t]);
        if (t < T) acc[t] += sg[t] * s;
      }
    }
    if (live && lir == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (t < T) {
          float v = acc[t];
          if (flags & GM_MOE_RESIDUAL) v = x[(int64_t)t * D + row] + v;
          y[(int64_t)t * D + row] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------- stand-alone top-k
__global__ void __launch_bounds__(256) k_topk(const float* __restrict__ logits, int T, int E, int k,
                                              int32_t* __restrict__ ids, float* __restrict__ wts) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  wave_topk(logits + (int64_t)t * E, E, k, ids + (int64_t)t * k, wts + (int64_t)t * k);
}

template <int L, int NT>
__global__ void __launch_bounds__(256) k_router_only(const uint16_t* __restrict__ w_router,
                                                     const float* __restrict__ bias, const float* __restrict__ x,
                                                     int T, int D, int E, const uint16_t* __restrict__ w_sh,
                                                     const float* __restrict__ norm_w, float eps,
                                                     float* __restrict__ logits, float* __restrict__ shg) {
  extern __shared__ float smem[];
  float* red = smem;
  float* xs = smem + 16;
  const int t0 = blockIdx.y * NT;
  const int nt = min(NT, T - t0);
  stage_xn<NT>(x, t0, nt, D, norm_w, eps, xs, red);
  constexpr int RPS = 64 / L;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nsub = D / GM_SUB;
  const int nrows = E + (w_sh != nullptr ? 1 : 0);
  const int row = (blockIdx.x * 4 + wave) * RPS + lane / L;
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.f;
  if (row < nrows) {
    const uint8_t* wr = row < E ? reinterpret_cast<const uint8_t*>(w_router) + (int64_t)row * D * 2
                                : reinterpret_cast<const uint8_t*>(w_sh);
    for (int sub = lane % L; sub < nsub; sub += L) {
      const RawBf16 r = gm_load_bf16(wr, sub);
      float wv[32];
      gm_decode_bf16(r, wv);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] += gm_dot32(wv, xs + t * D + sub * GM_SUB);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = gm_group_sum<L>(acc[t]);
  if (row < nrows && (lane % L) == 0) {
    for (int t = 0; t < nt; ++t) {
      if (row < E) logits[(int64_t)(t0 + t) * E + row] = acc[t] + (bias ? bias[row] : 0.f);
      else shg[t0 + t] = gm_sigmoid(acc[t]);
    }
  }
}

template <int L>
int launch_router_l(const uint16_t* w, const float* bias, const float* x, int T, int D, int E,
                    const uint16_t* wsh, const float* nw, float eps, float* logits, float* shg,
                    hipStream_t s) {
  constexpr int RPS = 64 / L;
  const int nrows = E + (wsh ? 1 : 0);
  const int nb = (nrows + 4 * RPS - 1) / (4 * RPS);
  if (T == 1) {
    const size_t smem = (16 + (size_t)D) * 4;
    hipLaunchKernelGGL((k_router_only<L, 1>), dim3(nb, 1), dim3(256), smem, s, w, bias, x, T, D, E, wsh, nw,
                       eps, logits, shg);
  } else {
    const size_t smem = (16 + 8 * (size_t)D) * 4;
    int rc = gm_set_smem(k_router_only<L, 8>, smem);
    if (rc) return rc;
    hipLaunchKernelGGL((k_router_only<L, 8>), dim3(nb, (T + 7) / 8), dim3(256), smem, s, w, bias, x, T, D, E,
                       wsh, nw, eps, logits, shg);
  }
  GM_TRY(hipGetLastError());
  return GM_OK;
}

}  // namespace

int gm_launch_router(const uint16_t* w_router, const float* bias, const float* x, int T, int D, int E,
                     const uint16_t* w_sh_gate, const float* norm_w, float eps, float* logits,
                     float* sh_gate, hipStream_t s) {
  const int nsub = D / GM_SUB;
  if (nsub >= 64) return launch_router_l<64>(w_router, bias, x, T, D, E, w_sh_gate, norm_w, eps, logits, sh_gate, s);
  if (nsub >= 32) return launch_router_l<32>(w_router, bias, x, T, D, E, w_sh_gate, norm_w, eps, logits, sh_gate, s);
  if (nsub >= 16) return launch_router_l<16>(w_router, bias, x, T, D, E, w_sh_gate, norm_w, eps, logits, sh_gate, s);
  return launch_router_l<8>(w_router, bias, x, T, D, E, w_sh_gate, norm_w, eps, logits, sh_gate, s);
}

int gm_launch_topk(const float* logits, int T, int E, int k, int32_t* ids, float* wts, hipStream_t s) {
  hipLaunchKernelGGL(k_topk, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E, k, ids, wts);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

// ------------------------------------------------------------- decode driver
namespace {

template <int QTG, int QTD, int QTSG, int QTSD, int L, int LD, int NT>
int decode_t(const gm_moe_layer* P, const float* x, float* y, int T, int flags, uint8_t* ws, const GmMoeWs& lay,
             hipStream_t s, int stage) {
  const int D = P->D, FF = P->FF, E = P->E, k = P->k;
  float* logits = reinterpret_cast<float*>(ws + lay.logits);
  float* shg = reinterpret_cast<float*>(ws + lay.shg);
  int32_t* ids = reinterpret_cast<int32_t*>(ws + lay.ids);
  float* wts = reinterpret_cast<float*>(ws + lay.wts);
  int32_t* grp = reinterpret_cast<int32_t*>(ws + lay.grp);
  float* h = reinterpret_cast<float*>(ws + lay.h);
  float* hsh = reinterpret_cast<float*>(ws + lay.hsh);
  constexpr int RPS = 64 / L;
  // K1: router rows (E + shared gate) and shared gate/up rows
  if (stage == 0 || stage == 1) {
    const int nrows = E + (P->sh_gate_inp ? 1 : 0);
    const int nrb = (nrows + 4 * RPS - 1) / (4 * RPS);
    const int sh_rpw = 2 * RPS;
    const int nsb = P->gate_sh ? (P->FF_sh + 4 * sh_rpw - 1) / (4 * sh_rpw) : 0;
    const size_t smem = (256 + 16 + (size_t)NT * D) * 4;
    int rc = gm_set_smem(k_moe_router<QTSG, L, NT>, smem);
    if (rc) return rc;
    hipLaunchKernelGGL((k_moe_router<QTSG, L, NT>), dim3(nrb + nsb), dim3(256), smem, s, *P, x, T, logits, shg, hsh,
                       nrb, sh_rpw);
    GM_TRY(hipGetLastError());
  }
  // K2: routed gate/up
  if (stage == 0 || stage == 2) {
    const int max_u = T * k < E ? T * k : E;
    const int rows_per_block = 4 * 4 * RPS;
    const int n_chunks = (FF + rows_per_block - 1) / rows_per_block;
    const size_t smem = (256 + 16 + 64 + 64 + GM_GRP_WORDS + 16 + (size_t)NT * D) * 4;
    int rc = gm_set_smem(k_moe_gateup<QTG, L, NT>, smem);
    if (rc) return rc;
    hipLaunchKernelGGL((k_moe_gateup<QTG, L, NT>), dim3(max_u * n_chunks), dim3(256), smem, s, *P, x, T, logits, ids,
                       wts, grp, h, rows_per_block);
    GM_TRY(hipGetLastError());
  }
  // K3: down + combine (+ residual)
  if (stage == 0 || stage == 3) {
    constexpr int RPSD = 64 / LD;
    const int rows_per_wave = RPSD;
    const int nb = (D + 4 * rows_per_wave - 1) / (4 * rows_per_wave);
    hipLaunchKernelGGL((k_moe_down<QTD, QTSD, LD, NT>), dim3(nb), dim3(256), 0, s, *P, x, T, flags, wts, grp, h, shg,
                       hsh, y, rows_per_wave);
    GM_TRY(hipGetLastError());
  }
  return GM_OK;
}

template <int QTG, int QTD, int QTSG, int QTSD, int L, int LD>
int decode_nt(const gm_moe_layer* P, const float* x, float* y, int T, int flags, uint8_t* ws, const GmMoeWs& lay,
              hipStream_t s, int stage) {
  if (T == 1) return decode_t<QTG, QTD, QTSG, QTSD, L, LD, 1>(P, x, y, T, flags, ws, lay, s, stage);
  return decode_t<QTG, QTD, QTSG, QTSD, L, LD, 8>(P, x, y, T, flags, ws, lay, s, stage);
}

// Lanes per row: 64 for the D = 2048 rows (one sub-block per lane), 16 for the
// FF = 512 rows; 8 (several sub-blocks per lane) covers any other size.
template <int QTG, int QTD, int QTSG, int QTSD>
int decode_q(const gm_moe_layer* P, const float* x, float* y, int T, int flags, uint8_t* ws, const GmMoeWs& lay,
             hipStream_t s, int stage) {
  const int nd = P->D / GM_SUB, nf = P->FF / GM_SUB;
  if (nd < 8 || nf < 8) return gm_fail_arg("gm_moe_forward: decode kernels need D, FF >= 256");
  if (nd >= 64) {
    if (nf >= 16) return decode_nt<QTG, QTD, QTSG, QTSD, 64, 16>(P, x, y, T, flags, ws, lay, s, stage);
    return decode_nt<QTG, QTD, QTSG, QTSD, 64, 8>(P, x, y, T, flags, ws, lay, s, stage);
  }
  if (nf >= 16) return decode_nt<QTG, QTD, QTSG, QTSD, 8, 16>(P, x, y, T, flags, ws, lay, s, stage);
  return decode_nt<QTG, QTD, QTSG, QTSD, 8, 8>(P, x, y, T, flags, ws, lay, s, stage);
}

// The shared expert either mirrors the routed formats (BASELINE's config) or is
// dense bf16 (the reference model dequantises it at load, qwen/forward.py:465-468).
template <int QTG, int QTD>
int decode_s(const gm_moe_layer* P, const float* x, float* y, int T, int flags, uint8_t* ws, const GmMoeWs& lay,
             hipStream_t s, int stage) {
  if (!P->gate_sh || (P->q_gate_sh == QTG && P->q_down_sh == QTD))
    return decode_q<QTG, QTD, QTG, QTD>(P, x, y, T, flags, ws, lay, s, stage);
  if (P->q_gate_sh == GM_QTYPE_BF16 && P->q_down_sh == GM_QTYPE_BF16)
    return decode_q<QTG, QTD, GM_QTYPE_BF16, GM_QTYPE_BF16>(P, x, y, T, flags, ws, lay, s, stage);
  return gm_fail_arg("gm_moe_forward: shared-expert formats gate/up %d down %d unsupported (use the routed "
                     "formats or BF16/BF16)", P->q_gate_sh, P->q_down_sh);
}

}  // namespace

int gm_moe_decode(const gm_moe_layer* P, const float* x, float* y, int T, int flags, uint8_t* ws,
                  const GmMoeWs& lay, hipStream_t s, int stage) {
  const int qg = P->q_gate, qd = P->q_down;
  if (qg == GM_QTYPE_IQ4_XS && qd == GM_QTYPE_IQ3_XXS) return decode_s<GM_QTYPE_IQ4_XS, GM_QTYPE_IQ3_XXS>(P, x, y, T, flags, ws, lay, s, stage);
  if (qg == GM_QTYPE_IQ3_XXS && qd == GM_QTYPE_IQ4_XS) return decode_s<GM_QTYPE_IQ3_XXS, GM_QTYPE_IQ4_XS>(P, x, y, T, flags, ws, lay, s, stage);
  if (qg == GM_QTYPE_IQ4_XS && qd == GM_QTYPE_IQ4_XS) return decode_s<GM_QTYPE_IQ4_XS, GM_QTYPE_IQ4_XS>(P, x, y, T, flags, ws, lay, s, stage);
  if (qg == GM_QTYPE_IQ3_XXS && qd == GM_QTYPE_IQ3_XXS) return decode_s<GM_QTYPE_IQ3_XXS, GM_QTYPE_IQ3_XXS>(P, x, y, T, flags, ws, lay, s, stage);
  return gm_fail_arg("gm_moe_forward: unsupported routed formats gate/up %d down %d", qg, qd);
}
