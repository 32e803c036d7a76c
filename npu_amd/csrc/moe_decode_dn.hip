// MoE decode, stage 3: down projections and the weighted combine
// (qwen/forward.py:659-665: routed experts accumulated in ascending expert id,
// then + sigmoid(gate) * shared expert; the residual add of :880-884 fused).
//
// T = 1 (k_dec_down1): block = 8 output rows; every lane loads its sub-block
// of all k routed down rows and the shared down row up front, the k + 1 SwiGLU
// rows are staged in LDS meanwhile, and the rows are reduced in a fixed order.
//
// T > 1: k_dec_down8 (unique expert or shared expert, 64-row tile) writes one
// partial output row per member token, k_dec_combine sums each token's
// partials in ascending expert order.  Fixed order, no atomics.
#include "moe_common.h"
#include "moe_decode.h"

using namespace gm_moe;

namespace {

// Sum over aligned groups of n lanes (n = 8, 16 or 32), result in every lane.
__device__ __forceinline__ float group_sum(float v, int n) {
  if (n == 8) {
    v += GM_DPP_F(v, 0x141);               // row_half_mirror: lane i <-> 7 - i
    v += GM_DPP_F(v, GM_QPERM_2301);
    v += GM_DPP_F(v, GM_QPERM_1032);
    return v;
  }
  v = gm_row_sum16(v);
  if (n == 32) v += __shfl_xor(v, 16, 64);
  return v;
}

// Block = 8 output rows, 9 waves: wave w reduces routed down matrix w (w < k,
// in ascending expert order) or, for w == k, the shared one.  Lane (rg, sub)
// takes sub-block sub of rows rg R .. rg R + R - 1 (R = nsub / 8), so every
// lane decodes 32 R weights and reads its 32 SwiGLU values once for them.
// The 8-row slices of the k + 1 down matrices are contiguous, 16-byte aligned
// runs of raw superblocks: they are copied to LDS with 16-byte loads and
// decoded from there.  The 9 x 8 partial sums are added in a fixed order.
// One sub-block of a staged down row (LDS) against the limbs of the SwiGLU
// sub-block: bf16 rows in fp32 (activations rebuilt from the limbs), I8 rows
// with their half scales and offset, IQ rows on v_dot4 with one scale.
template <int Q>
__device__ __forceinline__ float down_sub_dot(const uint8_t* __restrict__ rowp, int sub, const Iq3Tab* __restrict__ tab,
                                              const uint32_t (&l0)[8], const uint32_t (&l1)[8],
                                              const uint32_t (&l2)[8], float2 hsa) {
  const typename RawSub<Q>::T raw = gm_load_sub<Q>(rowp, sub);
  if constexpr (Q == GM_QTYPE_BF16) {
    float wv[32];
    const float sc = gm_decode_sub_t<Q>(raw, sub, tab, wv);
    float a = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        a = fmaf(wv[4 * c + b], fmaf(gm_sbyte(l2[c], b), 65536.f, fmaf(gm_sbyte(l1[c], b), 256.f, gm_sbyte(l0[c], b))), a);
    return sc * hsa.x * a;
  } else if constexpr (Q == GM_QTYPE_I8) {
    return gm_i8_limb_dot(raw, l0, l1, l2, hsa.x, hsa.y);
  } else {
    uint32_t w[8];
    const float sc = gm_decode_i8<Q>(raw, sub, tab, w);
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      s0 = __builtin_amdgcn_sdot4((int)w[c], (int)l0[c], s0, false);
      s1 = __builtin_amdgcn_sdot4((int)w[c], (int)l1[c], s1, false);
      s2 = __builtin_amdgcn_sdot4((int)w[c], (int)l2[c], s2, false);
    }
    return sc * hsa.x * fmaf((float)s2, 65536.f, fmaf((float)s1, 256.f, (float)s0));
  }
}

// With NXT (a chain's next layer, nx): thread t <= E of the next layer also
// loads its router row t (row E: the shared gate vector) at columns r0 .. r0+7
// from the grouped transpose router_t (one contiguous run per block) and,
// once the block's 8 outputs y are final, adds
// sum_i W[t][r0 + i] (y[r0 + i] w_norm[r0 + i]) and (thread E + 1) the sum of
// y^2 over the 8 rows to copy blockIdx % 8 of the next layer's router
// accumulators with fp64 atomics.  That replaces the next layer's router
// launch (qwen/forward.py:608 on rms_norm of this block's output).
template <int QTD, int QTS, int FC, bool NXT>
__global__ void __launch_bounds__(576) k_dec_down1(gm_moe_layer P, const float* __restrict__ x, int flags,
                                                   const int32_t* __restrict__ g_grp, const float* __restrict__ h,
                                                   const float* __restrict__ shg, float* __restrict__ y,
                                                   GmNextRouter nx GM_TL_PARAM) {
  constexpr int NTH = 576;
  GM_TL_BEGIN();
  constexpr bool IQ3 = QTD == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS;
  constexpr int RMAX = 2 * FC;                                 // rows per lane, FF <= 512 FC
  constexpr int HPT = (9 * 128 * FC + NTH - 1) / NTH;          // float4 of the k + 1 SwiGLU rows per thread
  constexpr int RB_MAX = QTD == GM_QTYPE_BF16 ? 1024 * FC : QTD == GM_QTYPE_I8 ? 768 * FC
                                                          : 2 * FC * GM_IQ4XS_BYTES;   // widest routed row
  constexpr int CR = (8 * 8 * RB_MAX / 16 + NTH - 1) / NTH;    // routed 16-byte chunks per thread
  constexpr int RBS_MAX = QTS == GM_QTYPE_BF16 ? 1024 * FC : QTS == GM_QTYPE_I8 ? 768 * FC : RB_MAX;
  constexpr int CS = (8 * RBS_MAX / 16 + NTH - 1) / NTH;       // shared 16-byte chunks per thread
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ float s_wj[8];        // routing weight and h row of routed matrix m
  __shared__ int32_t s_pr[8];
  __shared__ float s_part[9][8];
  __shared__ float s_y[8];
  const int D = P.D, FF = P.FF, k = P.k, nsub = FF / GM_SUB;
  const int rbd = (int)gm_row_bytes(QTD, FF), rbs = (int)gm_row_bytes(QTS, FF);
  const int nqr = FF >> 2;
  const int wbytes = k * 8 * rbd + 8 * rbs;
  const int hbytes = gm_limb_row_bytes(FF);
  uint8_t* hs = smem;                                                  // (k + 1) limb rows of FF (+ spare)
  uint8_t* wr = smem + (k + 2) * hbytes;                               // [k][8][rbd], [8][rbs], 16 spare
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(wr + ((wbytes + 16 + 15) & ~15));
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r0 = blockIdx.x * 8;
  const bool has_sh = P.down_sh != nullptr;
  const int trash = wbytes;                                            // spare 16 bytes
  // --- A: the ids, then the loads that do not depend on the routing
  int ex[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) ex[j] = g_grp[1 + (j < k ? j : k - 1)];
  const int jj = (tid & 7) < k ? (tid & 7) : k - 1;               // every thread loads, threads < 8 store
  const int my_pr = g_grp[1 + 2 * GM_GRP_MAXU + GM_GRP_MAXM * jj];
  const float my_wj = __int_as_float(g_grp[GM_GRP_WORDS + jj]);
  const float sg = has_sh ? shg[0] : 0.f;
  const float xres = (flags & GM_MOE_RESIDUAL) ? x[r0 + (tid & 7)] : 0.f;
  uint32_t gw = 0;
  if constexpr (IQ3) gw = gm_iq3_tab_load();
  const int nq_rows = (k + (has_sh ? 1 : 0)) * nqr;             // h [k][FF] directly followed by h_sh [FF]
  const gm_f32x4* h4 = reinterpret_cast<const gm_f32x4*>(h);
  gm_f32x4 hr[HPT];
#pragma unroll
  for (int i = 0; i < HPT; ++i) {
    const int c = tid + NTH * i;
    hr[i] = h4[c < nq_rows ? c : nq_rows - 1];
  }
  const int n16s = has_sh ? 8 * rbs / 16 : 1;
  const uint8_t* sbase = has_sh ? static_cast<const uint8_t*>(P.down_sh) + (int64_t)r0 * rbs
                                : static_cast<const uint8_t*>(P.down_exps);
  gm_u32x4 sr[CS];
#pragma unroll
  for (int i = 0; i < CS; ++i) {
    const int c = tid + NTH * i;
    sr[i] = gm_ld<true>(reinterpret_cast<const gm_u32x4*>(sbase + 16 * (c < n16s ? c : n16s - 1)));
  }
  // --- B: routed rows, addresses from the routing: issued as soon as the ids
  // are in, before anything else is waited for
  const int n16 = 8 * rbd / 16, total = k * n16;
  gm_u32x4 rr[CR];
  int dst[CR];
  {
    const uint32_t magic = 0xffffffffu / (uint32_t)n16 + 1u;
#pragma unroll
    for (int i = 0; i < CR; ++i) {
      const int c = tid + NTH * i;
      const int cc = c < total ? c : total - 1;
      const int m = (int)__umulhi((uint32_t)cc, magic), j = cc - m * n16;
      int e = ex[0];
#pragma unroll
      for (int q = 1; q < 8; ++q) e = m == q ? ex[q] : e;
      rr[i] = gm_ld<true>(reinterpret_cast<const gm_u32x4*>(static_cast<const uint8_t*>(P.down_exps) +
                                                           ((int64_t)e * D + r0) * rbd + 16 * j));
      dst[i] = c < total ? m * 8 * rbd + 16 * j : trash;
    }
  }
  // the next layer's router columns r0 .. r0 + 7 (needed only at the end)
  gm_u32x4 nr0{}, nr1{};
  gm_f32x4 nwa{}, nwb{};
  // thread tid adds the accumulator word at position tid (gm_acc_pos), so that a
  // wave's atomics fall on consecutive words: word nw_e = 64 (tid % MV) + tid / MV
  // below 64 MV, then E (shared gate row) and E + 1 (sum of squares)
  const int mvn = gm_acc_mv(nx.E);
  const int nw_e = tid < 64 * mvn ? 64 * (tid % mvn) + tid / mvn : nx.E + (tid - 64 * mvn);
  const bool nw_live = tid < 64 * mvn ? nw_e < nx.E : nw_e <= nx.E + 1;
  if constexpr (NXT) {
    const int t = nw_e <= nx.E ? nw_e : 0;
    const int es = nx.f32 ? 4 : 2;
    const uint8_t* p = static_cast<const uint8_t*>(nx.w) + ((int64_t)blockIdx.x * (nx.E + 1) + t) * 8 * es;
    nr0 = gm_ld<true>(reinterpret_cast<const gm_u32x4*>(p));
    nr1 = gm_ld<true>(reinterpret_cast<const gm_u32x4*>(p + (nx.f32 ? 16 : 0)));
    // without a norm weight the loads read the router's first 32 bytes and are replaced by ones
    const bool hn = nx.nw != nullptr;
    const float* nwp = hn ? nx.nw + r0 : static_cast<const float*>(nx.w);
    const gm_f32x4 la = *reinterpret_cast<const gm_f32x4*>(nwp), lb = *reinterpret_cast<const gm_f32x4*>(nwp + 4);
    const gm_f32x4 one{1.f, 1.f, 1.f, 1.f};
    nwa = hn ? la : one;
    nwb = hn ? lb : one;
  }
  GM_TL_MARK1(ex[0]);
  issue_fence();
  // --- C: stage the SwiGLU rows and the shared rows, then the routed rows
  if (tid < 8) { s_pr[tid] = my_pr; s_wj[tid] = my_wj; }
  if constexpr (IQ3) gm_iq3_tab_store(gw, tab);
  {
    const uint32_t magic = 0xffffffffu / (uint32_t)nqr + 1u;     // c / nqr == umulhi(c, magic) for c < 2^16
#pragma unroll
    for (int i = 0; i < HPT; ++i) {
      const int c = tid + NTH * i;                               // 8-lane groups never straddle a row
      const int rr = (int)__umulhi((uint32_t)c, magic), cc = c - rr * nqr;
      gm_put_limbs4(hr[i], c < nq_rows ? cc : (c & 7), hs + (c < nq_rows ? rr : k + 1) * hbytes);
    }
  }
#pragma unroll
  for (int i = 0; i < CS; ++i) {
    const int c = tid + NTH * i;
    *reinterpret_cast<gm_u32x4*>(wr + (c < n16s && has_sh ? k * 8 * rbd + 16 * c : trash)) = sr[i];
  }
#pragma unroll
  for (int i = 0; i < CR; ++i) *reinterpret_cast<gm_u32x4*>(wr + dst[i]) = rr[i];
  __syncthreads();
  GM_TL_MARK2(s_pr[0]);
  // --- D: decode from LDS; wave w -> matrix w
  const bool routed = wave < k, shared = has_sh && wave == k;
  if (routed || shared) {
    const int lg = nsub == 8 ? 3 : nsub == 16 ? 4 : 5;
    const int R = nsub >> 3, rg = lane >> lg, sub = lane & (nsub - 1);
    const int hrow = routed ? s_pr[wave] : k;                   // h row of rank w (the gate/up kernel's order)
    // limbs and scale of this sub-block of the SwiGLU row
    const uint8_t* hsub = hs + hrow * hbytes + sub * GM_LSUB;
    const gm_u32x4* hp = reinterpret_cast<const gm_u32x4*>(hsub);
    const gm_u32x4 l0a = hp[0], l0b = hp[1], l1a = hp[2], l1b = hp[3], l2a = hp[4], l2b = hp[5];
    const uint32_t l0[8] = {l0a.x, l0a.y, l0a.z, l0a.w, l0b.x, l0b.y, l0b.z, l0b.w};
    const uint32_t l1[8] = {l1a.x, l1a.y, l1a.z, l1a.w, l1b.x, l1b.y, l1b.z, l1b.w};
    const uint32_t l2[8] = {l2a.x, l2a.y, l2a.z, l2a.w, l2b.x, l2b.y, l2b.z, l2b.w};
    const float2 hsa = *reinterpret_cast<const float2*>(hsub + 96);   // limb scale, activation sum
    float part[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      part[r] = 0.f;
      if (r < R) {
        part[r] = routed ? down_sub_dot<QTD>(wr + (wave * 8 + rg * R + r) * rbd, sub, tab, l0, l1, l2, hsa)
                         : down_sub_dot<QTS>(wr + k * 8 * rbd + (rg * R + r) * rbs, sub, tab, l0, l1, l2, hsa);
      }
    }
    GM_TL_MARK3(part[0]);
    const float wgt = routed ? s_wj[wave] : sg;
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      if (r < R) {
        const float v = group_sum(part[r], nsub);
        if (sub == 0) s_part[wave][rg * R + r] = wgt * v;
      }
    }
  }
  __syncthreads();
  if (tid < 8) {
    float acc = 0.f;
    for (int w = 0; w < k; ++w) acc += s_part[w][tid];
    if (has_sh) acc += s_part[k][tid];
    const float yv = (flags & GM_MOE_RESIDUAL) ? xres + acc : acc;
    if (r0 + tid < D) y[r0 + tid] = yv;
    if constexpr (NXT) s_y[tid] = yv;
  }
  if constexpr (NXT) {
    __syncthreads();
    if (nw_live) {
      const float yv[8] = {s_y[0], s_y[1], s_y[2], s_y[3], s_y[4], s_y[5], s_y[6], s_y[7]};
      const float nv[8] = {nwa.x, nwa.y, nwa.z, nwa.w, nwb.x, nwb.y, nwb.z, nwb.w};
      float wv[8];
      if (nx.f32) {
        const uint32_t q[8] = {nr0.x, nr0.y, nr0.z, nr0.w, nr1.x, nr1.y, nr1.z, nr1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) wv[i] = __uint_as_float(q[i]);
      } else {
        const uint32_t q[4] = {nr0.x, nr0.y, nr0.z, nr0.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          wv[2 * i] = __uint_as_float(q[i] << 16);
          wv[2 * i + 1] = __uint_as_float(q[i] & 0xffff0000u);
        }
      }
      float p = 0.f;
      if (nw_e <= nx.E) {
#pragma unroll
        for (int i = 0; i < 8; ++i) p = fmaf(wv[i], yv[i] * nv[i], p);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) p = fmaf(yv[i], yv[i], p);
      }
      // copy = this block's XCD: all adds into one copy meet in one L2, so a
      // workgroup-scope atomic (performed in that L2, not at device scope) is
      // enough; the kernel boundary writes the L2 back for the next launch
      int xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      __hip_atomic_fetch_add(nx.acc + (xcc & (GM_ACC_COPIES - 1)) * nx.ld + tid, (double)p, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  GM_TL_END(2);
}

// 64 rows of one down matrix for nm <= 8 member rows of hsrc (global rows
// src[m] of h, where h_sh follows h), written to yp rows dst[m].
// Rows [row0, row0 + kDnRows NTILE) of one down matrix for nm member rows of h
// (h rows src[m] -> yp rows dst[m]): the members' h rows are loaded, then
// every tile's raw rows (wave w, pass q < kDnPasses of tile t -> row row0 +
// kDnRows t + 4 kDnPasses w + 4q + (lane >> 4), 16 lanes per row); the members
// are staged in LDS as limb rows while the weights are in flight, then the
// tiles are decoded as they land.
// Four passes (64-row tiles, 78 VGPRs, 6 waves per SIMD): 2.04 ms per B = 8 step,
// against 2.15 ms with two and 2.51 ms with one (more blocks, each staging the
// members' limb rows again), and 2.16 ms with eight (136 VGPRs, 3 waves per SIMD).
constexpr int kDnPasses = 4;
constexpr int kDnRows = 16 * kDnPasses;                      // rows per tile (4 waves)

template <int QTW, int FC, int NTILE>
__device__ __forceinline__ void down_rows(const uint8_t* __restrict__ wbase, int D, int FF, int row0, int nm,
                                          const int (&src)[8], const int (&dst)[8], const float* __restrict__ h,
                                          uint8_t* __restrict__ hs, uint32_t gw, Iq3Tab* __restrict__ tab,
                                          float* __restrict__ yp) {
  constexpr int HPT = 4 * FC;     // float4 per thread: 8 * FF <= 8 * 512 * FC floats over 256 threads
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lir = lane & 15, nsub = FF >> 5;
  const int64_t rb = gm_row_bytes(QTW, FF);
  // the member rows first: vmcnt retires in issue order, so the wait for
  // them before the limb staging does not wait for the weights
  const int nqr = FF >> 2, nq = nm * nqr;
  const gm_f32x4* h4 = reinterpret_cast<const gm_f32x4*>(h);
  gm_f32x4 hr[HPT];
#pragma unroll
  for (int i = 0; i < HPT; ++i) {
    const int c = threadIdx.x + 256 * i;
    const int m = c < nq ? c / nqr : 0;
    int s = src[0];
#pragma unroll
    for (int mm = 1; mm < 8; ++mm) s = m == mm ? src[mm] : s;
    hr[i] = h4[(int64_t)s * nqr + (c < nq ? c - m * nqr : 0)];
  }
  issue_fence();
  RowFetch<QTW, FC> f[NTILE][kDnPasses];
#pragma unroll
  for (int t = 0; t < NTILE; ++t)
#pragma unroll
    for (int q = 0; q < kDnPasses; ++q) {
      const int row = row0 + kDnRows * t + wave * 4 * kDnPasses + q * 4 + (lane >> 4);
      fetch_subs<QTW, 16, FC, true>(f[t][q], wbase + (int64_t)(row < D ? row : 0) * rb, lir, nsub);
    }
  issue_fence();
  if constexpr (QTW == GM_QTYPE_IQ3_XXS) gm_iq3_tab_store(gw, tab);
  const int rbytes = gm_limb_row_bytes(FF);
#pragma unroll
  for (int i = 0; i < HPT; ++i) {
    const int c = threadIdx.x + 256 * i;
    const int m = c / nqr, cc = c - m * nqr;
    gm_put_limbs4(hr[i], c < nq ? cc : (c & 7), hs + (c < nq ? m : 8) * rbytes);   // unconditional (DPP inside)
  }
  __syncthreads();
  int idx[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) idx[m] = m;
#pragma unroll
  for (int t = 0; t < NTILE; ++t) {
#pragma unroll
    for (int q = 0; q < kDnPasses; ++q) {
      opaque(f[t][q]);
      float part[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) part[m] = 0.f;
      dot_subs_i8<QTW, 16, FC, 8>(f[t][q], lir, nsub, hs, rbytes, idx, nm, tab, part);
      const int row = row0 + kDnRows * t + wave * 4 * kDnPasses + q * 4 + (lane >> 4);
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        if (m < nm) {
          const float sm = row_sum<16>(part[m]);
          if (lir == 0 && row < D) yp[(int64_t)dst[m] * D + row] = sm;
        }
      }
      issue_fence();                                          // one pass's decoded row live at a time
    }
  }
}

// Blocks [0, n_sh): the shared expert (all T tokens), dn_tiles(FC) kDnRows-row
// tiles each; blocks [n_sh, ...): unit (b - n_sh) / n_tg of the unique routed
// experts.
constexpr int dn_tiles(int fc) { return 1; }

template <int QTD, int QTS, int FC>
__global__ void __launch_bounds__(256) k_dec_down8(gm_moe_layer P, int T, const int32_t* __restrict__ g_grp,
                                                   const float* __restrict__ h, float* __restrict__ yp,
                                                   int n_sh, int n_tg GM_TL_PARAM) {
  GM_TL_BEGIN();
  extern __shared__ __attribute__((aligned(16))) uint8_t hs[];   // 8 limb rows of FF (+ a spare sub-block)
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(hs + 8 * gm_limb_row_bytes(P.FF) + GM_LSUB);
  const int D = P.D, FF = P.FF, k = P.k, Ptot = T * k;
  const int nu = g_grp[0];
  const bool shared = (int)blockIdx.x < n_sh;
  const int u = shared ? nu : ((int)blockIdx.x - n_sh) / n_tg;
  const int tg = shared ? (int)blockIdx.x : (int)blockIdx.x - n_sh - u * n_tg;
  if (u > nu || (!shared && u == nu)) return;   // uniform per block
  constexpr int NT = dn_tiles(FC);
  const int row0 = tg * kDnRows * NT;
  uint32_t gw = 0;
  if constexpr (QTD == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS) gw = gm_iq3_tab_load();
  int src[8], dst[8];
  if (shared) {
#pragma unroll
    for (int m = 0; m < 8; ++m) { src[m] = Ptot + (m < T ? m : 0); dst[m] = src[m]; }
    down_rows<QTS, FC, NT>(static_cast<const uint8_t*>(P.down_sh), D, FF, row0, T, src, dst, h, hs, gw, tab, yp);
  } else {
    const int e = g_grp[1 + u];
    const int nm = g_grp[1 + GM_GRP_MAXU + u];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      src[m] = g_grp[1 + 2 * GM_GRP_MAXU + GM_GRP_MAXM * u + (m < nm ? m : 0)];
      dst[m] = src[m];
    }
    down_rows<QTD, FC, NT>(static_cast<const uint8_t*>(P.down_exps) + (int64_t)e * D * gm_row_bytes(QTD, FF), D, FF,
                           row0, nm, src, dst, h, hs, gw, tab, yp);
  }
  GM_TL_END(7);
}

// y[t] = sum over t's top-k slots in ascending expert id of w * yp[t*k + j]
//        + sigmoid gate * yp[T*k + t]  (+ x[t]).  Every slot's partial row (and
// the shared one and x) is loaded before the slots are sorted by expert id, so
// the block waits on one round of loads; the sort then reorders the loaded
// values with the ids and weights.
__global__ void __launch_bounds__(256) k_dec_combine(const float* __restrict__ x, int T, int k, int D, int flags,
                                                     const int32_t* __restrict__ g_ids,
                                                     const float* __restrict__ g_wts, const float* __restrict__ shg,
                                                     int has_sh, const float* __restrict__ yp,
                                                     float* __restrict__ y GM_TL_PARAM) {
  GM_TL_BEGIN();
  const int t = blockIdx.y;
  const int d = blockIdx.x * 256 + threadIdx.x;
  const int dc = d < D ? d : D - 1;
  int id[8];
  float w[8], v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int jj = j < k ? j : k - 1;
    id[j] = g_ids[t * k + jj];
    w[j] = g_wts[t * k + jj];
    v[j] = yp[(int64_t)(t * k + jj) * D + dc];
  }
  const float vs = has_sh ? yp[(int64_t)(T * k + t) * D + dc] : 0.f;
  const float gs = has_sh ? shg[t] : 0.f;
  const float xr = (flags & GM_MOE_RESIDUAL) ? x[(int64_t)t * D + dc] : 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) id[j] = j < k ? id[j] : 0x7fffffff;
#pragma unroll
  for (int i = 1; i < 8; ++i)
#pragma unroll
    for (int j = i; j > 0; --j)
      if (id[j] < id[j - 1]) {
        const int ti = id[j]; id[j] = id[j - 1]; id[j - 1] = ti;
        const float tw = w[j]; w[j] = w[j - 1]; w[j - 1] = tw;
        const float tv = v[j]; v[j] = v[j - 1]; v[j - 1] = tv;
      }
  if (d >= D) return;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (j < k) acc = fmaf(w[j], v[j], acc);
  if (has_sh) acc = fmaf(gs, vs, acc);
  if (flags & GM_MOE_RESIDUAL) acc = xr + acc;
  y[(int64_t)t * D + d] = acc;
  GM_TL_END(3);
}

// T > 1 chain: the combine of k_dec_combine over the 256-column slice c =
// blockIdx.x for every token, plus the next layer's router inputs over that
// slice for its router rows 16 blockIdx.y .. +15 (row E: the shared gate
// vector), so that the next layer starts with its routing kernel:
//   part[c][t][r] = sum_{d in slice} (y[t][d] w_norm[d]) Wn[r][d]
// and, from the blocks with blockIdx.y == 0, y itself, ssq[c][t] =
// sum_{d in slice} y[t][d]^2 and the limb rows of y w_norm over the slice (the
// outputs k_dec_router_ks has for its K ranges).  Combine: thread 64 t + q
// holds columns 4q .. 4q+3 of token t; the slots are added in ascending
// expert id, in the order and with the roundings of k_dec_combine (the lanes
// rank their token's slots, every slot value goes to LDS, and each lane reads
// them back in rank order).  Router: the block's rows come from router_t (8
// columns of E + 1 rows per 16-byte group, so the block's 16 rows of a group
// are one contiguous 256-byte run), loaded behind the combine's loads and
// staged in LDS; thread 64 t + 16 h + r then forms row r's dot product for
// token t over the quarter h of the slice in four interleaved partial sums,
// and the quarters are added across lanes (h = 0 + 1, 2 + 3, then both).
constexpr int kNxRows = 16;                                      // router rows per block

template <bool RF32>
__global__ void __launch_bounds__(512) k_dec_combine_nx(const float* __restrict__ x, int T, int k, int D, int flags,
                                                        const int32_t* __restrict__ g_ids,
                                                        const float* __restrict__ g_wts,
                                                        const float* __restrict__ shg, int has_sh,
                                                        const float* __restrict__ yp, float* __restrict__ y,
                                                        GmNextB8 nx GM_TL_PARAM) {
  GM_TL_BEGIN();
  constexpr int NG = GM_DEC_LINK_KR / 8;                         // 8-column groups of the slice
  constexpr int CW = RF32 ? 2 : 1;                               // 16-byte chunks per group row
  constexpr int NRC = (NG * kNxRows * CW + 511) / 512;           // router chunks per thread
  __shared__ gm_f32x4 vbuf[8][8][64];                            // [token][slot][column quad]
  __shared__ gm_f32x4 ys[8][64];                                 // y w_norm of the slice
  __shared__ gm_u32x4 rsl[NRC * 512];                            // router rows [group][row][chunk]
  __shared__ int pslot[8][8];
  __shared__ float pw[8][8];
  const int tid = threadIdx.x, t = tid >> 6, q = tid & 63;
  const int tc = t < T ? t : T - 1;
  const int c = blockIdx.x, d = GM_DEC_LINK_KR * c + 4 * q;
  int id[8];
  float w[8];
  gm_f32x4 v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int jj = j < k ? j : k - 1;
    id[j] = g_ids[tc * k + jj];
    w[j] = g_wts[tc * k + jj];
    v[j] = *reinterpret_cast<const gm_f32x4*>(yp + (int64_t)(tc * k + jj) * D + d);
  }
  const gm_f32x4 zero4 = {0.f, 0.f, 0.f, 0.f}, one4 = {1.f, 1.f, 1.f, 1.f};
  const gm_f32x4 vs = has_sh ? *reinterpret_cast<const gm_f32x4*>(yp + (int64_t)(T * k + tc) * D + d) : zero4;
  const gm_f32x4 xr = (flags & GM_MOE_RESIDUAL) ? *reinterpret_cast<const gm_f32x4*>(x + (int64_t)tc * D + d) : zero4;
  const gm_f32x4 nw4 = nx.nw ? *reinterpret_cast<const gm_f32x4*>(nx.nw + d) : one4;
  const float gs = has_sh ? shg[tc] : 0.f;
  // the block's router rows (rows past E: row E again, never stored)
  const int es = RF32 ? 4 : 2;
  const int64_t gstride = (int64_t)(nx.E + 1) * 8 * es;           // bytes per 8-column group
  const uint8_t* rbase = static_cast<const uint8_t*>(nx.w) + (int64_t)(NG * c) * gstride;
  gm_u32x4 rc[NRC];
#pragma unroll
  for (int i = 0; i < NRC; ++i) {
    const int ch0 = tid + 512 * i, ch = ch0 < NG * kNxRows * CW ? ch0 : 0;
    const int g = ch / (kNxRows * CW), rr = (ch / CW) % kNxRows, h = ch % CW;
    const int R = kNxRows * (int)blockIdx.y + rr;
    rc[i] = gm_ld<true>(reinterpret_cast<const gm_u32x4*>(rbase + g * gstride + (int64_t)(R <= nx.E ? R : nx.E) * 8 * es) + h);
  }
  issue_fence();
  // rank of slot q % 8 among the token's slots (ascending id; slots past k after
  // every real one, in slot order)
  int key[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) key[j] = j < k ? id[j] : 0x7ffffff0 + j;
  const int j0 = q & 7;
  int mk = key[0];
  float mw = w[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) {
    mk = j0 == j ? key[j] : mk;
    mw = j0 == j ? w[j] : mw;
  }
  int rank = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) rank += key[j] < mk ? 1 : 0;
  if (q < 8) {
    pslot[t][rank] = j0;
    pw[t][rank] = mw;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) vbuf[t][j][q] = v[j];
  __syncthreads();
  GM_TL_MARK1(vbuf[t][0][q].x);
  gm_f32x4 acc = zero4;
  for (int i = 0; i < k; ++i) {
    const float wi = pw[t][i];
    const gm_f32x4 vi = vbuf[t][pslot[t][i]][q];
    acc.x = fmaf(wi, vi.x, acc.x);
    acc.y = fmaf(wi, vi.y, acc.y);
    acc.z = fmaf(wi, vi.z, acc.z);
    acc.w = fmaf(wi, vi.w, acc.w);
  }
  if (has_sh) {
    acc.x = fmaf(gs, vs.x, acc.x);
    acc.y = fmaf(gs, vs.y, acc.y);
    acc.z = fmaf(gs, vs.z, acc.z);
    acc.w = fmaf(gs, vs.w, acc.w);
  }
  if (flags & GM_MOE_RESIDUAL) acc = xr + acc;
  const gm_f32x4 yn = {acc.x * nw4.x, acc.y * nw4.y, acc.z * nw4.z, acc.w * nw4.w};
  ys[t][q] = yn;
  if (blockIdx.y == 0) {                                         // uniform per block
    if (t < T) *reinterpret_cast<gm_f32x4*>(y + (int64_t)t * D + d) = acc;
    const float s2 = gm_wave_sum64(fmaf(acc.x, acc.x, fmaf(acc.y, acc.y, fmaf(acc.z, acc.z, acc.w * acc.w))));
    if (q == 0 && t < T) nx.ssq[c * T + t] = s2;
    // the 8 lanes of a sub-block are lanes 8j .. 8j+7; tokens past T: spare row T
    gm_put_limbs4(yn, d >> 2, nx.xl + (int64_t)(t < T ? t : T) * gm_limb_row_bytes(D));
  }
#pragma unroll
  for (int i = 0; i < NRC; ++i)
    if (tid + 512 * i < NG * kNxRows * CW) rsl[tid + 512 * i] = rc[i];
  __syncthreads();
  GM_TL_MARK2(ys[0][q].x);
  const int r = q & 15, hq = q >> 4;                             // row, quarter of the slice
  float da[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int gi = 0; gi < NG / 4; ++gi) {
    const int g = (NG / 4) * hq + gi;
    RouterChunk<RF32> wc;
#pragma unroll
    for (int h = 0; h < CW; ++h) wc[h] = rsl[(g * kNxRows + r) * CW + h];
    float wv[8];
    router_unpack8<RF32>(wc, wv);
    const gm_f32x4 a0 = ys[t][2 * g], b0 = ys[t][2 * g + 1];
    const float xv[8] = {a0.x, a0.y, a0.z, a0.w, b0.x, b0.y, b0.z, b0.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) da[gi & 3] = fmaf(xv[i], wv[i], da[gi & 3]);
  }
  float dsum = (da[0] + da[1]) + (da[2] + da[3]);
  dsum += __shfl_xor(dsum, 16, 64);
  dsum += __shfl_xor(dsum, 32, 64);
  GM_TL_MARK3(dsum);
  const int R = kNxRows * (int)blockIdx.y + r;
  if (hq == 0 && R <= nx.E && t < T) nx.part[((int64_t)c * T + t) * nx.ldp + R] = dsum;
  GM_TL_END(3);
}

template <int QTD, int QTS, int FC>
int launch_dn(const gm_moe_layer* P, const float* x, float* y, int T, int flags, bool fast1, const GmDecArgs& a,
              hipStream_t s, const GmNextRouter* next, const GmNextB8* next8) {
  const int D = P->D, FF = P->FF, k = P->k;
  if (fast1) {
    if constexpr (FC <= (QTD == GM_QTYPE_BF16 || QTD == GM_QTYPE_I8 ? 1 : 2)) {   // bf16 / I8 rows: 8 / 6 KB per slice
      const size_t wbytes = (size_t)k * 8 * gm_row_bytes(QTD, FF) + 8 * (size_t)gm_row_bytes(QTS, FF);
      const size_t smem = (size_t)(k + 2) * gm_limb_row_bytes(FF) + ((wbytes + 16 + 15) & ~(size_t)15) +
                          (QTD == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
      if (next != nullptr) {
        if (int rc = gm_set_smem(k_dec_down1<QTD, QTS, FC, true>, smem)) return rc;
        hipLaunchKernelGGL((k_dec_down1<QTD, QTS, FC, true>), dim3((D + 7) / 8), dim3(576), smem, s, *P, x, flags,
                           a.grp, a.h, a.shg, y, *next GM_TL_ARG(a.tl));
      } else {
        if (int rc = gm_set_smem(k_dec_down1<QTD, QTS, FC, false>, smem)) return rc;
        hipLaunchKernelGGL((k_dec_down1<QTD, QTS, FC, false>), dim3((D + 7) / 8), dim3(576), smem, s, *P, x, flags,
                           a.grp, a.h, a.shg, y, GmNextRouter{} GM_TL_ARG(a.tl));
      }
      GM_TRY(hipGetLastError());
      return GM_OK;
    }
  }
  const int n_tg = (D + kDnRows * dn_tiles(FC) - 1) / (kDnRows * dn_tiles(FC));
  const int n_sh = P->down_sh ? n_tg : 0;
  const int max_u = T * k < P->E ? T * k : P->E;
  const size_t smem = 8 * (size_t)gm_limb_row_bytes(FF) + GM_LSUB +
                      (QTD == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
  if (int rc = gm_set_smem(k_dec_down8<QTD, QTS, FC>, smem)) return rc;
  hipLaunchKernelGGL((k_dec_down8<QTD, QTS, FC>), dim3(n_sh + max_u * n_tg), dim3(256), smem, s, *P, T, a.grp, a.h,
                     a.yp, n_sh, n_tg GM_TL_ARG(a.tl));
  GM_TRY(hipGetLastError());
  if (next8 != nullptr) {
    const dim3 grid((unsigned)(D / GM_DEC_LINK_KR), (unsigned)((next8->E + kNxRows) / kNxRows));
    if (next8->f32)
      hipLaunchKernelGGL(k_dec_combine_nx<true>, grid, dim3(512), 0, s, x, T, k, D, flags, a.ids, a.wts, a.shg,
                         P->down_sh ? 1 : 0, a.yp, y, *next8 GM_TL_ARG(a.tl));
    else
      hipLaunchKernelGGL(k_dec_combine_nx<false>, grid, dim3(512), 0, s, x, T, k, D, flags, a.ids, a.wts, a.shg,
                         P->down_sh ? 1 : 0, a.yp, y, *next8 GM_TL_ARG(a.tl));
  } else {
    hipLaunchKernelGGL(k_dec_combine, dim3((D + 255) / 256, T), dim3(256), 0, s, x, T, k, D, flags, a.ids, a.wts,
                       a.shg, P->down_sh ? 1 : 0, a.yp, y GM_TL_ARG(a.tl));
  }
  GM_TRY(hipGetLastError());
  return GM_OK;
}

template <int QTD, int QTS>
int launch_dn_f(const gm_moe_layer* P, const float* x, float* y, int T, int flags, bool fast1, const GmDecArgs& a,
                hipStream_t s, const GmNextRouter* next, const GmNextB8* next8) {
  switch (gm_dec_fc(P->FF)) {
    case 1: return launch_dn<QTD, QTS, 1>(P, x, y, T, flags, fast1, a, s, next, next8);
    case 2: return launch_dn<QTD, QTS, 2>(P, x, y, T, flags, fast1, a, s, next, next8);
    default: return launch_dn<QTD, QTS, 4>(P, x, y, T, flags, fast1, a, s, next, next8);
  }
}

template <int QTD>
int launch_dn_s(const gm_moe_layer* P, const float* x, float* y, int T, int flags, bool fast1, const GmDecArgs& a,
                hipStream_t s, const GmNextRouter* next, const GmNextB8* next8) {
  if (!P->down_sh) return launch_dn_f<QTD, QTD>(P, x, y, T, flags, fast1, a, s, next, next8);
  switch (P->q_down_sh) {
    case GM_QTYPE_IQ4_XS: return launch_dn_f<QTD, GM_QTYPE_IQ4_XS>(P, x, y, T, flags, fast1, a, s, next, next8);
    case GM_QTYPE_IQ3_XXS: return launch_dn_f<QTD, GM_QTYPE_IQ3_XXS>(P, x, y, T, flags, fast1, a, s, next, next8);
    case GM_QTYPE_BF16: return launch_dn_f<QTD, GM_QTYPE_BF16>(P, x, y, T, flags, fast1, a, s, next, next8);
    case GM_QTYPE_I8: return launch_dn_f<QTD, GM_QTYPE_I8>(P, x, y, T, flags, fast1, a, s, next, next8);
    default: return gm_fail_arg("gm_moe_forward: shared down format %d unsupported", P->q_down_sh);
  }
}

}  // namespace

int gm_dec_down(const gm_moe_layer* P, const float* x, float* y, int T, int flags, bool fast1, const GmDecArgs& a,
                hipStream_t s, const GmNextRouter* next, const GmNextB8* next8) {
  if (next != nullptr && !(fast1 && T == 1)) return gm_fail_arg("gm_moe_chain: internal error (next router off T = 1)");
  if (next8 != nullptr && (fast1 || P->D % GM_DEC_LINK_KR || gm_dec_link_nz(P->D) > GM_DEC_MAX_NZ))
    return gm_fail_arg("gm_moe_chain: internal error (linked combine)");
  switch (P->q_down) {
    case GM_QTYPE_IQ4_XS: return launch_dn_s<GM_QTYPE_IQ4_XS>(P, x, y, T, flags, fast1, a, s, next, next8);
    case GM_QTYPE_IQ3_XXS: return launch_dn_s<GM_QTYPE_IQ3_XXS>(P, x, y, T, flags, fast1, a, s, next, next8);
    case GM_QTYPE_BF16: return launch_dn_s<GM_QTYPE_BF16>(P, x, y, T, flags, fast1, a, s, next, next8);
    case GM_QTYPE_I8: return launch_dn_s<GM_QTYPE_I8>(P, x, y, T, flags, fast1, a, s, next, next8);
    default: return gm_fail_arg("gm_moe_forward: routed down format %d unsupported", P->q_down);
  }
}
