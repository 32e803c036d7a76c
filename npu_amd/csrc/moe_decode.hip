// MoE block, decode path (T <= 8 tokens): three kernels per block.
//
//   K1 k_moe_router   router logits (bf16 W, fp32 xn) + shared scalar gate, and the
//                     shared expert's gate/up + SwiGLU (independent of routing).
//                     The last router block to finish (atomic ticket) computes
//                     top-k, the renormalised weights and the per-expert grouping
//                     of (token, slot) pairs, and publishes them for K2/K3.
//   K2 k_moe_gateup   per (unique expert, row chunk): silu(G x) * (U x)
//   K3 k_moe_down     per output-row tile: sum over unique experts in ascending
//                     id of w * (Down_e . h), then + sigmoid-gated shared expert
//                     (+ residual x); fixed order, no atomics -> bit-reproducible
//
// Kernel boundaries are the grid-wide synchronisation points.  Inside a kernel
// every lane issues its weight loads before x is staged, activations are read
// from bank-conflict-free LDS layouts and row reductions use DPP.
// Reference semantics: qwen/forward.py:563-665 (moe_forward).
#include "moe_common.h"

using namespace gm_moe;

namespace {

constexpr int kBatch = 8;     // experts whose down rows are in flight at once in K3

template <int QT, int MS>
struct Fetch {
  typename RawSub<QT>::T r[MS];
};

// Sub-blocks lir + LR*(c0 + i), i < MS, of one row.
template <int QT, int LR, int MS>
__device__ __forceinline__ void fetch_row(Fetch<QT, MS>& f, const uint8_t* __restrict__ row, int lir, int c0, int nsub) {
#pragma unroll
  for (int i = 0; i < MS; ++i) {
    const int sub = lir + LR * (c0 + i);
    if (sub < nsub) f.r[i] = gm_load_sub<QT>(row, sub);
  }
}

// acc[m] += W_row . act[idx[m]] over the fetched sub-blocks.  IL: activations
// are interleaved LDS rows (stride K floats); otherwise contiguous rows.
template <int QT, int LR, int MS, int NT, bool IL>
__device__ __forceinline__ void dot_row(const Fetch<QT, MS>& f, int lir, int c0, int nsub, const float* __restrict__ act,
                                        int K, const int (&idx)[NT], int nt, const uint32_t* __restrict__ grid,
                                        float (&acc)[NT]) {
#pragma unroll
  for (int i = 0; i < MS; ++i) {
    const int sub = lir + LR * (c0 + i);
    if (sub < nsub) {
      float wv[32];
      const float sc = gm_decode_sub<QT>(f.r[i], sub, grid, wv);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (t < nt) {
          const float d = IL ? gm_dot32_il(wv, act + idx[t] * K, sub, nsub) : gm_dot32(wv, act + (int64_t)idx[t] * K + sub * GM_SUB);
          acc[t] = fmaf(sc, d, acc[t]);
        }
      }
    }
  }
}

template <int LR>
__device__ __forceinline__ float row_sum(float v) {
  v = gm_row_sum16(v);
  if constexpr (LR == 32) v += __shfl_xor(v, 16, 64);
  return v;
}

// SwiGLU rows (LR lanes per row, 64/LR rows per wave): hv[m] = silu(G.x) * (U.x)
// for the tokens idx[m], valid in every lane of the row.  The first pass's
// weight loads are issued before x is staged.  All threads of the block call.
template <int QT, int NT, int LR, int MS>
__device__ __forceinline__ void gateup_rows(const uint8_t* __restrict__ g_row, const uint8_t* __restrict__ u_row,
                                            bool live, int nsub, const float* __restrict__ x, int T, int D,
                                            const float* __restrict__ norm_w, float eps, const int (&idx)[NT],
                                            int nt, const uint32_t* __restrict__ grid, float* __restrict__ xs,
                                            float* __restrict__ red, float (&hv)[NT]) {
  const int lir = (threadIdx.x & 63) % LR;
  float ag[NT], au[NT];
#pragma unroll
  for (int m = 0; m < NT; ++m) { ag[m] = 0.f; au[m] = 0.f; }
  for (int c0 = 0; c0 * LR < nsub; c0 += MS) {
    Fetch<QT, MS> fg, fu;
    if (live) {
      fetch_row<QT, LR, MS>(fg, g_row, lir, c0, nsub);
      fetch_row<QT, LR, MS>(fu, u_row, lir, c0, nsub);
    }
    if (c0 == 0) stage_xn<NT>(x, 0, T, D, norm_w, eps, xs, red);
    if (live) {
      dot_row<QT, LR, MS, NT, true>(fg, lir, c0, nsub, xs, D, idx, nt, grid, ag);
      dot_row<QT, LR, MS, NT, true>(fu, lir, c0, nsub, xs, D, idx, nt, grid, au);
    }
  }
#pragma unroll
  for (int m = 0; m < NT; ++m) hv[m] = gm_silu(row_sum<LR>(ag[m])) * row_sum<LR>(au[m]);
}

// ------------------------------------------------------------------- K1
// Blocks [0, n_router_blocks): one router row per wave (bf16, 64 lanes per row);
// row E is the shared scalar gate.  Remaining blocks: 16 shared SwiGLU rows each.
template <int QTS, int NT, int MAXV>
__global__ void __launch_bounds__(256) k_moe_router(gm_moe_layer P, const float* __restrict__ x, int T,
                                                    float* __restrict__ logits, float* __restrict__ shg,
                                                    float* __restrict__ hsh, int32_t* __restrict__ g_ids,
                                                    float* __restrict__ g_wts, int32_t* __restrict__ g_grp,
                                                    uint32_t* __restrict__ ticket, int n_router_blocks) {
  extern __shared__ float smem[];
  float* xs = smem;                                     // [NT * D], 16-byte aligned for float4
  uint32_t* grid = reinterpret_cast<uint32_t*>(smem + NT * P.D);
  float* red = reinterpret_cast<float*>(grid + 256);    // [32]
  int32_t* ids = reinterpret_cast<int32_t*>(red + 32);  // [64]
  float* wts = reinterpret_cast<float*>(ids + 64);      // [64]
  int32_t* grp = reinterpret_cast<int32_t*>(wts + 64);  // [GM_GRP_WORDS]
  uint32_t* bits = reinterpret_cast<uint32_t*>(grp + GM_GRP_WORDS);  // [16]
  __shared__ uint32_t is_last;
  const int D = P.D, E = P.E, k = P.k;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nsub = D / GM_SUB;
  if ((int)blockIdx.x < n_router_blocks) {
    const int nrows = E + (P.sh_gate_inp != nullptr ? 1 : 0);
    const int row = blockIdx.x * 4 + wave;
    const bool live = row < nrows;
    const uint8_t* wr = row < E ? reinterpret_cast<const uint8_t*>(P.router) + (int64_t)row * D * 2
                                : reinterpret_cast<const uint8_t*>(P.sh_gate_inp);
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.f;
    for (int c0 = 0; c0 * 64 < nsub; ++c0) {     // one pass for D <= 2048
      const int sub = lane + 64 * c0;
      RawBf16 rr;
      if (live && sub < nsub) rr = gm_load_bf16(wr, sub);
      if (c0 == 0) stage_xn<NT>(x, 0, T, D, P.norm_w, P.norm_eps, xs, red);
      if (live && sub < nsub) {
        float wv[32];
        gm_decode_bf16(rr, wv);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] += gm_dot32_il(wv, xs + t * D, sub, nsub);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = gm_wave_sum64(acc[t]);
    if (live && lane == 0) {
      for (int t = 0; t < T && t < NT; ++t) {
        if (row < E) logits[t * E + row] = acc[t] + (P.router_bias ? P.router_bias[row] : 0.f);
        else shg[t] = gm_sigmoid(acc[t]);
      }
    }
    // last router block: routing for all tokens (publish-then-ticket pattern)
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      is_last = prev == (uint32_t)(n_router_blocks - 1);
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int t = wave; t < T; t += 4) wave_topk<MAXV>(logits + t * E, E, k, ids + t * k, wts + t * k);
    __syncthreads();
    block_group(ids, T * k, E, grp, bits);
    for (int i = threadIdx.x; i < T * k; i += blockDim.x) { g_ids[i] = ids[i]; g_wts[i] = wts[i]; }
    for (int i = threadIdx.x; i < GM_GRP_WORDS; i += blockDim.x) g_grp[i] = grp[i];
    if (threadIdx.x == 0) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if constexpr (QTS == GM_QTYPE_IQ3_XXS) gm_stage_grid(grid);   // visible after stage_xn's barrier
  const int FF = P.FF_sh;
  const int64_t rb = gm_row_bytes(QTS, D);
  const int row = ((blockIdx.x - n_router_blocks) * 4 + wave) * 4 + lane / 16;
  const bool live = row < FF;
  const int r = live ? row : 0;
  int idx[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) idx[t] = t;
  float hv[NT];
  gateup_rows<QTS, NT, 16, 4>(static_cast<const uint8_t*>(P.gate_sh) + r * rb,
                              static_cast<const uint8_t*>(P.up_sh) + r * rb, live, nsub, x, T, D, P.norm_w,
                              P.norm_eps, idx, T, grid, xs, red, hv);
  if (live && (lane % 16) == 0) {
    for (int t = 0; t < T && t < NT; ++t) hsh[t * FF + row] = hv[t];
  }
}

// ------------------------------------------------------------------- K2
// Block = (unique expert u, chunk of 4 * (64 / LR) SwiGLU rows).
template <int QT, int NT, int LR, int MS>
__global__ void __launch_bounds__(256) k_moe_gateup(gm_moe_layer P, const float* __restrict__ x, int T,
                                                    const int32_t* __restrict__ g_grp, float* __restrict__ h) {
  extern __shared__ float smem[];
  uint32_t* grid = reinterpret_cast<uint32_t*>(smem);
  float* red = smem + 256;                              // [32]
  float* xs = red + 32;
  __shared__ int32_t gs[2 + GM_GRP_MAXM];
  constexpr int RPS = 64 / LR;
  constexpr int RPB = 4 * RPS;
  const int D = P.D, k = P.k, FF = P.FF;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n_chunks = (FF + RPB - 1) / RPB;
  const int u = blockIdx.x / n_chunks, chunk = blockIdx.x - u * n_chunks;
  if (threadIdx.x == 0) {
    const int nu = g_grp[0];
    gs[0] = u < nu ? g_grp[1 + u] : -1;
    gs[1] = u < nu ? g_grp[1 + GM_GRP_MAXU + u] : 0;
  }
  if (threadIdx.x < GM_GRP_MAXM) gs[2 + threadIdx.x] = g_grp[1 + 2 * GM_GRP_MAXU + u * GM_GRP_MAXM + threadIdx.x];
  if constexpr (QT == GM_QTYPE_IQ3_XXS) gm_stage_grid(grid);
  __syncthreads();
  const int e = gs[0];
  if (e < 0) return;                                    // uniform per block
  const int nm = gs[1];
  int idx[NT], pair[NT];
#pragma unroll
  for (int m = 0; m < NT; ++m) {
    const int p = m < nm ? gs[2 + m] : 0;
    pair[m] = p;
    idx[m] = p / k;
  }
  const int nsub = D / GM_SUB;
  const int64_t rb = gm_row_bytes(QT, D);
  const int row = chunk * RPB + wave * RPS + lane / LR;
  const bool live = row < FF;
  const int r = live ? row : 0;
  const uint8_t* wg = static_cast<const uint8_t*>(P.gate_exps) + ((int64_t)e * FF + r) * rb;
  const uint8_t* wu = static_cast<const uint8_t*>(P.up_exps) + ((int64_t)e * FF + r) * rb;
  float hv[NT];
  gateup_rows<QT, NT, LR, MS>(wg, wu, live, nsub, x, T, D, P.norm_w, P.norm_eps, idx, nm, grid, xs, red, hv);
  if (live && (lane % LR) == 0) {
#pragma unroll
    for (int m = 0; m < NT; ++m)
      if (m < nm) h[(int64_t)pair[m] * FF + row] = hv[m];
  }
}

// ------------------------------------------------------------------- K3
// Block = 8 output rows (2 waves x 4 rows, 16 lanes per row).  Down rows of
// kBatch experts are in flight at once.  For NT == 1 the SwiGLU activations
// are staged in LDS (interleaved layout).
template <int QTD, int QTS, int NT>
__global__ void __launch_bounds__(128) k_moe_down(gm_moe_layer P, const float* __restrict__ x, int T, int flags,
                                                  const float* __restrict__ g_wts, const int32_t* __restrict__ g_grp,
                                                  const float* __restrict__ h, const float* __restrict__ shg,
                                                  const float* __restrict__ hsh, float* __restrict__ y) {
  extern __shared__ float hs[];                 // NT == 1: h [k][FF] then h_sh [FF], interleaved rows
  __shared__ uint32_t grid[256];
  __shared__ int32_t grp[GM_GRP_WORDS];
  __shared__ float wts[64];
  __shared__ float sg[GM_DECODE_MAX_T];
  constexpr bool IL = NT == 1;
  const int D = P.D, FF = P.FF, k = P.k;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lir = lane % 16;
  const int nsub = FF / GM_SUB;
  const int64_t rbd = gm_row_bytes(QTD, FF);
  const int64_t rbs = gm_row_bytes(QTS, FF);
  const int row = (blockIdx.x * 2 + wave) * 4 + lane / 16;
  const bool live = row < D;
  const int r = live ? row : 0;
  const bool has_sh = P.down_sh != nullptr;
  if constexpr (QTD == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS) gm_stage_grid(grid);
  for (int i = threadIdx.x; i < GM_GRP_WORDS; i += blockDim.x) grp[i] = g_grp[i];
  for (int i = threadIdx.x; i < T * k; i += blockDim.x) wts[i] = g_wts[i];
  if ((int)threadIdx.x < T) sg[threadIdx.x] = has_sh ? shg[threadIdx.x] : 0.f;
  if constexpr (IL) {
    stage_rows_il(h, k, FF, hs);
    if (has_sh) stage_rows_il(hsh, 1, FF, hs + k * FF);
  }
  __syncthreads();
  const float* hsrc = IL ? hs : h;
  const float* hshsrc = IL ? hs + k * FF : hsh;
  const int nu = grp[0];
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.f;
  for (int c0 = 0; c0 * 16 < nsub; ++c0) {    // one pass for FF <= 512
    for (int u0 = 0; u0 < nu; u0 += kBatch) {
      Fetch<QTD, 1> fd[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int u = u0 + j;
        if (u < nu) {
          const int e = grp[1 + u];
          fetch_row<QTD, 16, 1>(fd[j], static_cast<const uint8_t*>(P.down_exps) + ((int64_t)e * D + r) * rbd, lir, c0,
                                nsub);
        }
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int u = u0 + j;
        if (u < nu) {
          const int nm = grp[1 + GM_GRP_MAXU + u];
          float part[NT];
          int pr[NT];
#pragma unroll
          for (int m = 0; m < NT; ++m) {
            pr[m] = m < nm ? grp[1 + 2 * GM_GRP_MAXU + u * GM_GRP_MAXM + m] : 0;   // h rows are pairs
            part[m] = 0.f;
          }
          dot_row<QTD, 16, 1, NT, IL>(fd[j], lir, c0, nsub, hsrc, FF, pr, nm, grid, part);
#pragma unroll
          for (int m = 0; m < NT; ++m) {
            const float s = gm_row_sum16(part[m]);
            if (m < nm) {
              const int t = pr[m] / k;
#pragma unroll
              for (int tt = 0; tt < NT; ++tt)
                if (tt == t) acc[tt] = fmaf(wts[pr[m]], s, acc[tt]);
            }
          }
        }
      }
    }
  }
  if (has_sh) {
    float part[NT];
    int tk[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) { part[t] = 0.f; tk[t] = t; }
    for (int c0 = 0; c0 * 16 < nsub; ++c0) {
      Fetch<QTS, 1> fs;
      fetch_row<QTS, 16, 1>(fs, static_cast<const uint8_t*>(P.down_sh) + (int64_t)r * rbs, lir, c0, nsub);
      dot_row<QTS, 16, 1, NT, IL>(fs, lir, c0, nsub, hshsrc, FF, tk, T, grid, part);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float s = gm_row_sum16(part[t]);
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

// ------------------------------------------------------------- decode driver
template <int QTG, int QTD, int QTSG, int QTSD, int NT, int MAXV>
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
  uint32_t* ticket = reinterpret_cast<uint32_t*>(ws + lay.counters);
  if (stage == 0 || stage == 1) {          // K1: router rows (+ shared gate) and shared gate/up rows
    const int nrows = E + (P->sh_gate_inp ? 1 : 0);
    const int nrb = (nrows + 3) / 4;
    const int nsb = P->gate_sh ? (P->FF_sh + 15) / 16 : 0;
    const size_t smem = (256 + 32 + 64 + 64 + GM_GRP_WORDS + 16 + (size_t)NT * D) * 4;
    if (int rc = gm_set_smem(k_moe_router<QTSG, NT, MAXV>, smem)) return rc;
    hipLaunchKernelGGL((k_moe_router<QTSG, NT, MAXV>), dim3(nrb + nsb), dim3(256), smem, s, *P, x, T, logits, shg, hsh,
                       ids, wts, grp, ticket, nrb);
    GM_TRY(hipGetLastError());
  }
  if (stage == 0 || stage == 2) {          // K2: routed gate/up
    constexpr int LR = NT == 1 ? 32 : 16;
    constexpr int MS = NT == 1 ? 2 : 4;
    const int max_u = T * k < E ? T * k : E;
    const int rpb = 4 * (64 / LR);
    const int n_chunks = (FF + rpb - 1) / rpb;
    const size_t smem = (256 + 32 + (size_t)NT * D) * 4;
    if (int rc = gm_set_smem(k_moe_gateup<QTG, NT, LR, MS>, smem)) return rc;
    hipLaunchKernelGGL((k_moe_gateup<QTG, NT, LR, MS>), dim3(max_u * n_chunks), dim3(256), smem, s, *P, x, T, grp, h);
    GM_TRY(hipGetLastError());
  }
  if (stage == 0 || stage == 3) {          // K3: down + combine (+ residual)
    const int nb = (D + 7) / 8;
    const size_t smem = NT == 1 ? (size_t)(k + 1) * FF * 4 : 0;
    if (int rc = gm_set_smem(k_moe_down<QTD, QTSD, NT>, smem)) return rc;
    hipLaunchKernelGGL((k_moe_down<QTD, QTSD, NT>), dim3(nb), dim3(128), smem, s, *P, x, T, flags, wts, grp, h, shg,
                       hsh, y);
    GM_TRY(hipGetLastError());
  }
  return GM_OK;
}

template <int QTG, int QTD, int QTSG, int QTSD>
int decode_q(const gm_moe_layer* P, const float* x, float* y, int T, int flags, uint8_t* ws, const GmMoeWs& lay,
             hipStream_t s, int stage) {
  const bool small_e = P->E <= 256;
  if (T == 1) return small_e ? decode_t<QTG, QTD, QTSG, QTSD, 1, 4>(P, x, y, T, flags, ws, lay, s, stage)
                             : decode_t<QTG, QTD, QTSG, QTSD, 1, 8>(P, x, y, T, flags, ws, lay, s, stage);
  return small_e ? decode_t<QTG, QTD, QTSG, QTSD, 8, 4>(P, x, y, T, flags, ws, lay, s, stage)
                 : decode_t<QTG, QTD, QTSG, QTSD, 8, 8>(P, x, y, T, flags, ws, lay, s, stage);
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
  if (P->D / GM_SUB < 16 || P->FF / GM_SUB < 8)
    return gm_fail_arg("gm_moe_forward: decode kernels need D >= 512 and FF >= 256");
  if (P->D % 256 || P->FF % 256) return gm_fail_arg("gm_moe_forward: D and FF must be multiples of 256");
  if (T == 1 && (size_t)(P->k + 1) * P->FF * 4 > 65536)
    return gm_fail_arg("gm_moe_forward: decode stages (k + 1) x FF activations in LDS (FF=%d too large)", P->FF);
  const int qg = P->q_gate, qd = P->q_down;
  if (qg == GM_QTYPE_IQ4_XS && qd == GM_QTYPE_IQ3_XXS) return decode_s<GM_QTYPE_IQ4_XS, GM_QTYPE_IQ3_XXS>(P, x, y, T, flags, ws, lay, s, stage);
  if (qg == GM_QTYPE_IQ3_XXS && qd == GM_QTYPE_IQ4_XS) return decode_s<GM_QTYPE_IQ3_XXS, GM_QTYPE_IQ4_XS>(P, x, y, T, flags, ws, lay, s, stage);
  if (qg == GM_QTYPE_IQ4_XS && qd == GM_QTYPE_IQ4_XS) return decode_s<GM_QTYPE_IQ4_XS, GM_QTYPE_IQ4_XS>(P, x, y, T, flags, ws, lay, s, stage);
  if (qg == GM_QTYPE_IQ3_XXS && qd == GM_QTYPE_IQ3_XXS) return decode_s<GM_QTYPE_IQ3_XXS, GM_QTYPE_IQ3_XXS>(P, x, y, T, flags, ws, lay, s, stage);
  return gm_fail_arg("gm_moe_forward: unsupported routed formats gate/up %d down %d", qg, qd);
}
