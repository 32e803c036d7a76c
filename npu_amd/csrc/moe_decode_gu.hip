// MoE decode, stage 2: top-k routing, expert grouping, routed gate/up + SwiGLU.
//
// T = 1 (k_dec_gateup1): every wave of every routed block recomputes the
// token's top-k selection from the router logits instead of waiting for a
// separate routing kernel, picks the expert of rank `u` among the k picks
// (ascending id, the order of torch.unique in qwen/forward.py:612) and runs 8
// SwiGLU rows of it; the shared expert's rows run in blocks of their own.
// The first routed block also computes the routing weights, once its weight
// rows are in flight, and publishes ids, weights and the grouping table for
// stage 3.
//
// T > 1: k_dec_route (one block) runs the per-token top-k and groups the
// (token, slot) pairs by expert; k_dec_gateup8 then runs (unit, 8-row chunk)
// blocks, a unit being a unique routed expert over its member tokens only or
// the shared expert over all T tokens, reading the limb rows of x that stage 1
// wrote and the RMSNorm factors of the routing kernel.
#include "moe_common.h"
#include "moe_decode.h"

using namespace gm_moe;

namespace {

// Blocks [0, n_sh): 8 rows of the shared expert's gate/up pair (format QTS),
// which do not depend on the routing.  Blocks [n_sh, ...): unit u = (b - n_sh)
// / n_chunks, the pick of rank u in ascending expert id (the order of
// torch.unique, qwen/forward.py:612), rows 8 c .. 8 c + 7 of its gate/up pair
// (c = chunk).  In a routed block wave 0 runs the top-k of the logits
// (topk_masks, wave-uniform) while every thread loads its chunks of the limb
// row of xn that the router kernel wrote; the expert id reaches the other
// waves through LDS at the block's one barrier, after which every wave issues
// its weight loads.  Shared blocks issue theirs before the barrier.  The first
// routed block also publishes the ids and renormalised weights (in
// descending order) and the grouping table (ascending id; the SwiGLU row of
// rank u is h row u) once its weight loads are in flight.
template <int QT, int QTS, int DC, int MAXV>
__global__ void __launch_bounds__(256) k_dec_gateup1(gm_moe_layer P, const float* __restrict__ logits,
                                                     int32_t* __restrict__ g_ids, float* __restrict__ g_wts,
                                                     int32_t* __restrict__ g_grp, float* __restrict__ h,
                                                     float* __restrict__ hsh, int n_chunks, int n_sh,
                                                     const uint8_t* __restrict__ xl GM_TL_PARAM) {
  GM_TL_BEGIN();
  constexpr bool IQ3 = QT == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS;
  constexpr int CPT = (32 * DC * GM_LSUB / 16 + 255) / 256;     // 16-byte limb chunks per thread
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int32_t s_e;
  const int D = P.D, E = P.E, k = P.k, FF = P.FF, nsub = D / GM_SUB, rbytes = gm_limb_row_bytes(D);
  uint8_t* xs = smem;                                           // limb row of xn (+ a spare chunk)
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(smem + rbytes + GM_LSUB);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lir = lane & 31;
  const bool shared = (int)blockIdx.x < n_sh;                   // uniform per block
  const int rch = rbytes >> 4;
  gm_u32x4 cp[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + 256 * i;
    cp[i] = reinterpret_cast<const gm_u32x4*>(xl)[c < rch ? c : rch - 1];
  }
  uint32_t gw = 0;
  if constexpr (IQ3) gw = gm_iq3_tab_load();
  const int b = (int)blockIdx.x - n_sh;
  const int u = shared ? 0 : b / n_chunks, chunk = shared ? (int)blockIdx.x : b - u * n_chunks;
  const int row = chunk * 8 + wave * 2 + (lane >> 5);
  const bool live = row < FF;
  const int r = live ? row : 0;
  RowFetch<QT, DC> fg, fu;
  RowFetch<QTS, DC> sg, su;
  uint32_t uk[MAXV];
  uint64_t sel[MAXV];
  if (shared) {
    const int64_t rbs = gm_row_bytes(QTS, D);
    fetch_subs<QTS, 32, DC, true>(sg, static_cast<const uint8_t*>(P.gate_sh) + r * rbs, lir, nsub);
    fetch_subs<QTS, 32, DC, true>(su, static_cast<const uint8_t*>(P.up_sh) + r * rbs, lir, nsub);
  } else if (wave == 0) {
    // The selection is a dependent chain of one wave that every wave of the
    // block waits for: it issues ahead of the co-resident blocks' decode.
    __builtin_amdgcn_s_setprio(3);
    float v[MAXV];
    int ix[MAXV];
    topk_load<MAXV>(logits, E, v, ix);
    GM_TL_MARK3(v[0]);
    topk_keys<MAXV>(v, ix, E, uk);
    topk_masks<MAXV>(uk, k, sel);
    if (lane == 0) s_e = topk_rank_id<MAXV>(sel, u);
    __builtin_amdgcn_s_setprio(0);
  }
  issue_fence();
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + 256 * i;
    reinterpret_cast<gm_u32x4*>(xs)[c < rch ? c : rch] = cp[i];   // past the row: the spare chunk
  }
  if constexpr (IQ3) gm_iq3_tab_store(gw, tab);
  __syncthreads();
  if (!shared) {
    const int e = s_e;
    GM_TL_MARK1(e);
    const int64_t rb = gm_row_bytes(QT, D);
    fetch_subs<QT, 32, DC, true>(fg, static_cast<const uint8_t*>(P.gate_exps) + ((int64_t)e * FF + r) * rb, lir,
                                 nsub);
    fetch_subs<QT, 32, DC, true>(fu, static_cast<const uint8_t*>(P.up_exps) + ((int64_t)e * FF + r) * rb, lir,
                                 nsub);
    if (b == 0 && wave == 0) {
      // publish for stage 3 and the caller while this block's rows are in flight
      int rid;
      uint32_t rkey;
      topk_compact<MAXV>(sel, uk, k, rkey, rid);               // lane r: pick of rank r (ascending id)
      const float w = topk_weight<MAXV>(uk, rkey, k);
      uint32_t sk = rkey;
      int sid = rid;
      float sw = w;
      topk_sort8(sk, sid, sw);                                  // lane s: pick s in descending order
      if (lane < k) {
        g_ids[lane] = sid;
        g_wts[lane] = sw;
        g_grp[1 + lane] = rid;
        g_grp[1 + GM_GRP_MAXU + lane] = 1;
        g_grp[1 + 2 * GM_GRP_MAXU + GM_GRP_MAXM * lane] = lane;
        g_grp[GM_GRP_WORDS + lane] = __float_as_int(w);
      }
      if (lane == 0) g_grp[0] = k;
    }
  }
  const int tok[1] = {0};
  float ag[1] = {0.f}, au[1] = {0.f};
  if (shared) {
    dot_subs_i8<QTS, 32, DC, 1>(sg, lir, nsub, xs, rbytes, tok, 1, tab, ag);
    dot_subs_i8<QTS, 32, DC, 1>(su, lir, nsub, xs, rbytes, tok, 1, tab, au);
  } else {
    dot_subs_i8<QT, 32, DC, 1>(fg, lir, nsub, xs, rbytes, tok, 1, tab, ag);
    dot_subs_i8<QT, 32, DC, 1>(fu, lir, nsub, xs, rbytes, tok, 1, tab, au);
  }
  GM_TL_MARK2(au[0]);
  const float hv = gm_silu(row_sum<32>(ag[0])) * row_sum<32>(au[0]);
  if (live && lir == 0) {
    if (shared) hsh[row] = hv;
    else h[(int64_t)u * FF + row] = hv;
  }
  GM_TL_END(1);
}

// T = 1, one block per CU: block b runs rows 16c .. 16c + 15 (c = b % n_chunks)
// of the pick of rank u = b / n_chunks on waves 0-7 (two rows per wave, 32
// lanes per row) and, on wave 8, shared rows 2b and 2b + 1, whose loads are in
// flight from the block's start while wave 0 runs the top-k.  With k n_chunks
// = 256 blocks every block starts at once: in the 8-row layout above, 576
// blocks made 2-3 per CU, and the last ones dispatched ended up to 1.5 us after
// the median.
// Routing input: the router accumulators (raw dot products W . (x w_norm) of
// the E rows and the shared gate row, and the sum of x^2, each the fp64 sum of
// GM_ACC_COPIES copies, written by the router kernel or by the previous
// layer's down kernel).  Wave 0 adds the copies in copy order, forms the
// logits rms * S_e + bias (rms = 1 / sqrt(mean(x^2) + eps), qwen/forward.py:
// 58-61) and selects, while waves 1-7 build the limb row of x * w_norm in LDS
// (the gate and up sums are scaled by rms instead).  A variant where waves
// 1-7 added the copies into LDS ahead of a second barrier took 0.45 us longer
// to the top-k.  Block 0
// publishes the ids, weights, grouping table, logits and shared gate once its
// rows are in flight; every block clears its share of the next layer's
// accumulators (acc_zero) for the down kernel that follows.
template <int QT, int QTS, int DC, int MAXV>
__global__ void __launch_bounds__(576) k_dec_gateup1w(gm_moe_layer P, const float* __restrict__ x,
                                                      const double* __restrict__ acc, double* __restrict__ acc_zero,
                                                      int acc_ld, float* __restrict__ logits,
                                                      float* __restrict__ shg, int32_t* __restrict__ g_ids,
                                                      float* __restrict__ g_wts, int32_t* __restrict__ g_grp,
                                                      float* __restrict__ h, float* __restrict__ hsh,
                                                      int n_chunks GM_TL_PARAM) {
  GM_TL_BEGIN();
  constexpr int NTH = 576;
  constexpr bool IQ3 = QT == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int32_t s_e;
  __shared__ float s_rms;
  const int D = P.D, E = P.E, k = P.k, FF = P.FF, nsub = D / GM_SUB, rbytes = gm_limb_row_bytes(D);
  uint8_t* xs = smem;                                           // limb row of x w_norm (+ a spare chunk)
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(smem + rbytes + GM_LSUB);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lir = lane & 31;
  const int b = blockIdx.x, u = b / n_chunks, chunk = b - u * n_chunks;
  const bool shw = wave == 8;                                   // uniform per wave
  if (acc_zero != nullptr) {                                    // this block's share of the next layer's accumulators
    const int n16 = GM_ACC_COPIES * acc_ld / 2, per = (n16 + (int)gridDim.x - 1) / (int)gridDim.x;
    const int c = b * per + (int)threadIdx.x;
    if ((int)threadIdx.x < per && c < n16) reinterpret_cast<gm_u32x4*>(acc_zero)[c] = gm_u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t gw = 0;
  if constexpr (IQ3) gw = gm_iq3_tab_load();
  const int srow = 2 * b + (lane >> 5);                         // wave 8: shared row
  const bool slive = P.gate_sh != nullptr && srow < P.FF_sh;
  const int row = shw ? srow : chunk * 16 + wave * 2 + (lane >> 5);
  const bool live = shw ? slive : row < FF;
  const int r = live ? row : 0;
  RowFetch<QT, DC> fg, fu;
  RowFetch<QTS, DC> sg, su;
  uint32_t uk[MAXV];
  uint64_t sel[MAXV];
  if (shw) {
    if (P.gate_sh != nullptr) {
      const int64_t rbs = gm_row_bytes(QTS, D);
      fetch_subs<QTS, 32, DC, true>(sg, static_cast<const uint8_t*>(P.gate_sh) + r * rbs, lir, nsub);
      fetch_subs<QTS, 32, DC, true>(su, static_cast<const uint8_t*>(P.up_sh) + r * rbs, lir, nsub);
    }
  } else if (wave == 0) {
    __builtin_amdgcn_s_setprio(3);
    // the copies of the lane's words lane + 64 i (MAXV consecutive doubles, see
    // gm_acc_pos), of the shared gate word and of the sum of squares, loaded a
    // batch of CB copies at a time (all 8 at E <= 256) before any is added; the
    // copies are added in copy order
    static_assert(MAXV == 4 || MAXV == 8, "accumulator layout: MAXV = gm_acc_mv(E)");
    constexpr int CB = MAXV > 4 ? 4 : GM_ACC_COPIES;
    double sd[MAXV], ssd = 0.0, sgd = 0.0;
#pragma unroll
    for (int c0 = 0; c0 < GM_ACC_COPIES; c0 += CB) {
      gm_f64x2 a[CB][MAXV / 2], gq[CB];
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        const gm_f64x2* cp = reinterpret_cast<const gm_f64x2*>(acc + (c0 + c) * acc_ld);
#pragma unroll
        for (int i = 0; i < MAXV / 2; ++i) a[c][i] = cp[(MAXV / 2) * lane + i];
        gq[c] = cp[32 * MAXV];                                    // words E, E + 1
      }
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        sgd = c0 + c == 0 ? gq[c].x : sgd + gq[c].x;
        ssd = c0 + c == 0 ? gq[c].y : ssd + gq[c].y;
#pragma unroll
        for (int i = 0; i < MAXV / 2; ++i) {
          sd[2 * i] = c0 + c == 0 ? a[c][i].x : sd[2 * i] + a[c][i].x;
          sd[2 * i + 1] = c0 + c == 0 ? a[c][i].y : sd[2 * i + 1] + a[c][i].y;
        }
      }
      issue_fence();
    }
    const float rms = P.norm_w != nullptr ? 1.0f / sqrtf((float)ssd / (float)D + P.norm_eps) : 1.0f;
    float v[MAXV];
    int ix[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      ix[i] = lane + 64 * i;
      const float bias = P.router_bias != nullptr ? P.router_bias[ix[i] < E ? ix[i] : E - 1] : 0.f;
      v[i] = rms * (float)sd[i] + bias;
    }
    GM_TL_MARK3(v[0]);
    topk_keys<MAXV>(v, ix, E, uk);
    topk_masks<MAXV>(uk, k, sel);
    if (lane == 0) {
      s_e = topk_rank_id<MAXV>(sel, u);
      s_rms = rms;
    }
    __builtin_amdgcn_s_setprio(0);
    if (b == 0) {                                               // logits and shared gate, for stage 3 and the caller
#pragma unroll
      for (int i = 0; i < MAXV; ++i)
        if (ix[i] < E) logits[ix[i]] = v[i];
      if (lane == 0) shg[0] = P.sh_gate_inp != nullptr ? gm_sigmoid(rms * (float)sgd) : 1.f;
    }
  } else if (512 * (wave - 1) < D) {
    // waves 1-7: chunks of 512 values (wave - 1 + 7 j) of the limb row of x w_norm;
    // lanes past D write the spare sub-block after the row
    const gm_f32x4* x4 = reinterpret_cast<const gm_f32x4*>(x);
    const gm_f32x4* w4 = reinterpret_cast<const gm_f32x4*>(P.norm_w);
    for (int i = wave - 1; 512 * i < D; i += 7) {
      const int kk = 512 * i + 8 * lane, c = kk >> 2;             // float4 index, even
      const int cl = kk < D ? c : (D >> 2) - 2;                   // lanes past D re-read the end
      gm_f32x4 va = x4[cl], vb = x4[cl + 1];
      if (P.norm_w != nullptr) {
        const gm_f32x4 wa = w4[cl], wb = w4[cl + 1];
        va.x *= wa.x; va.y *= wa.y; va.z *= wa.z; va.w *= wa.w;
        vb.x *= wb.x; vb.y *= wb.y; vb.z *= wb.z; vb.w *= wb.w;
      }
      gm_put_limbs8(va, vb, kk < D ? c : (D >> 2) + (c & 7), xs);
    }
  }
  issue_fence();
  if constexpr (IQ3) gm_iq3_tab_store(gw, tab);
  __syncthreads();
  const float rms = s_rms;
  const int tok[1] = {0};
  float ag[1] = {0.f}, au[1] = {0.f};
  if (!shw) {
    const int e = s_e;
    GM_TL_MARK1(e);
    const int64_t rb = gm_row_bytes(QT, D);
    fetch_subs<QT, 32, DC, true>(fg, static_cast<const uint8_t*>(P.gate_exps) + ((int64_t)e * FF + r) * rb, lir,
                                 nsub);
    fetch_subs<QT, 32, DC, true>(fu, static_cast<const uint8_t*>(P.up_exps) + ((int64_t)e * FF + r) * rb, lir,
                                 nsub);
    if (b == 0 && wave == 0) {
      // publish for stage 3 and the caller while this block's rows are in flight
      int rid;
      uint32_t rkey;
      topk_compact<MAXV>(sel, uk, k, rkey, rid);               // lane r: pick of rank r (ascending id)
      const float w = topk_weight<MAXV>(uk, rkey, k);
      uint32_t sk = rkey;
      int sid = rid;
      float sw = w;
      topk_sort8(sk, sid, sw);                                  // lane s: pick s in descending order
      if (lane < k) {
        g_ids[lane] = sid;
        g_wts[lane] = sw;
        g_grp[1 + lane] = rid;
        g_grp[1 + GM_GRP_MAXU + lane] = 1;
        g_grp[1 + 2 * GM_GRP_MAXU + GM_GRP_MAXM * lane] = lane;
        g_grp[GM_GRP_WORDS + lane] = __float_as_int(w);
      }
      if (lane == 0) g_grp[0] = k;
    }
    dot_subs_i8<QT, 32, DC, 1>(fg, lir, nsub, xs, rbytes, tok, 1, tab, ag);
    dot_subs_i8<QT, 32, DC, 1>(fu, lir, nsub, xs, rbytes, tok, 1, tab, au);
  } else if (P.gate_sh != nullptr) {
    dot_subs_i8<QTS, 32, DC, 1>(sg, lir, nsub, xs, rbytes, tok, 1, tab, ag);
    dot_subs_i8<QTS, 32, DC, 1>(su, lir, nsub, xs, rbytes, tok, 1, tab, au);
  }
  GM_TL_MARK2(au[0]);
  const float hv = gm_silu(rms * row_sum<32>(ag[0])) * (rms * row_sum<32>(au[0]));
  if (live && lir == 0) {
    if (shw) hsh[row] = hv;
    else h[(int64_t)u * FF + row] = hv;
  }
  GM_TL_END(1);
}

// One block: the router logits of every token from the partial sums of
// k_dec_router_ks (fixed order), times the token's RMSNorm factor
// 1 / sqrt(mean(x^2) + eps) (qwen/forward.py:58-61), + bias; the shared gate
// sigmoid; the top-k (wave t -> token t) and the grouping table.
template <int MAXV, int NZ>
__global__ void __launch_bounds__(512) k_dec_route(gm_moe_layer P, const float* __restrict__ part,
                                                   const float* __restrict__ ssq, int nz, int ldp, int T,
                                                   float* __restrict__ rmsv, float* __restrict__ logits,
                                                   float* __restrict__ shg,
                                                   int32_t* __restrict__ g_ids, float* __restrict__ g_wts,
                                                   int32_t* __restrict__ g_grp GM_TL_PARAM) {
  GM_TL_BEGIN();
  __shared__ int32_t ids[64];
  __shared__ float wts[64];
  __shared__ int32_t grp[GM_GRP_WORDS];
  __shared__ uint32_t bits[32];                                 // expert bitmap, then its prefix counts
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int E = P.E, k = P.k;
  if (wave < T) {
    // every partial is loaded before any is summed (nz <= NZ; a load in a
    // runtime loop would wait before the next one is issued)
    float pv[MAXV][NZ], ps[NZ], pg[NZ];
#pragma unroll
    for (int z = 0; z < NZ; ++z) {
      const int zz = z < nz ? z : nz - 1;
      const float* pz = part + ((int64_t)zz * T + wave) * ldp;
#pragma unroll
      for (int i = 0; i < MAXV; ++i) {
        const int r = lane + 64 * i;
        pv[i][z] = pz[r < E ? r : E - 1];
      }
      ps[z] = ssq[zz * T + wave];
      pg[z] = pz[E];
    }
    float rms = 1.f;
    if (P.norm_w) {
      float q = 0.f;
#pragma unroll
      for (int z = 0; z < NZ; ++z) q += z < nz ? ps[z] : 0.f;
      rms = 1.0f / sqrtf(q / (float)P.D + P.norm_eps);
    }
    if (lane == 0) rmsv[wave] = rms;
    float v[MAXV];
    int ix[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      ix[i] = lane + 64 * i;
      const int r = ix[i] < E ? ix[i] : E - 1;
      float a = 0.f;
#pragma unroll
      for (int z = 0; z < NZ; ++z) a += z < nz ? pv[i][z] : 0.f;
      v[i] = rms * a + (P.router_bias ? P.router_bias[r] : 0.f);
      if (ix[i] < E) logits[(int64_t)wave * E + ix[i]] = v[i];
    }
    GM_TL_MARK3(v[0]);
    if (lane == 0) {                                            // no gate row: the shared expert is ungated
      float a = 0.f;
#pragma unroll
      for (int z = 0; z < NZ; ++z) a += z < nz ? pg[z] : 0.f;
      shg[wave] = P.sh_gate_inp ? gm_sigmoid(rms * a) : 1.f;
    }
    int id;
    float w;
    topk_finish<MAXV>(v, ix, E, k, id, w);
    if (lane < k) { ids[wave * k + lane] = id; wts[wave * k + lane] = w; }
  }
  __syncthreads();
  GM_TL_MARK1(ids[0]);
  block_group(ids, T * k, E, grp, bits);
  for (int i = threadIdx.x; i < T * k; i += blockDim.x) { g_ids[i] = ids[i]; g_wts[i] = wts[i]; }
  for (int i = threadIdx.x; i < GM_GRP_WORDS; i += blockDim.x) g_grp[i] = grp[i];
  GM_TL_END(5);
}

// Member tokens whose limb rows a gate/up block holds in LDS at once.
constexpr int kGuMembers = 2;

// Rows r0 .. r0 + 8 NP - 1 of one gate/up pair for nm member tokens (limb
// rows tok[m] of x w_norm in xl, RMSNorm factors rmsv; h rows dst[m]): all NP
// passes' raw rows are fetched first (wave w, pass p -> rows r0 + 8p + 2w +
// (lane >> 5), 32 lanes per row), then the members' limb rows are copied to
// LDS MG = kGuMembers at a time (most routed units have one member; a shared
// block has one token pair) and every pass is decoded.
template <int QT, int DC, int NP>
__device__ __forceinline__ void gateup_rows(const uint8_t* __restrict__ gbase, const uint8_t* __restrict__ ubase,
                                            int FF, int D, int r0, int nm, const int (&tok)[8], const int (&dst)[8],
                                            const uint8_t* __restrict__ xl, const float* __restrict__ rmsv,
                                            uint8_t* __restrict__ xs, uint32_t gw, Iq3Tab* __restrict__ tab,
                                            float* __restrict__ h) {
  constexpr int MG = kGuMembers;
  constexpr int CPT = (MG * 32 * DC * GM_LSUB / 16 + 255) / 256;   // 16-byte chunks per thread (D <= 1024 DC)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lir = lane & 31, nsub = D / GM_SUB;
  const int64_t rb = gm_row_bytes(QT, D);
  const int rbytes = gm_limb_row_bytes(D), rch = rbytes >> 4;
  RowFetch<QT, DC> fg[NP], fu[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int row = r0 + 8 * p + 2 * wave + (lane >> 5);
    const int r = row < FF ? row : 0;
    fetch_subs<QT, 32, DC, true>(fg[p], gbase + r * rb, lir, nsub);
    fetch_subs<QT, 32, DC, true>(fu[p], ubase + r * rb, lir, nsub);
  }
  for (int g0 = 0; g0 < nm; g0 += MG) {                      // usually one group
    int gt[MG], idx[MG];
    float rs[MG];
#pragma unroll
    for (int m = 0; m < MG; ++m) {
      int t = tok[0];
#pragma unroll
      for (int q = 1; q < 8; ++q) t = g0 + m == q ? tok[q] : t;
      gt[m] = t;
      idx[m] = m;
      rs[m] = rmsv[t];
    }
    const int ng = nm - g0 < MG ? nm - g0 : MG;
    gm_u32x4 cp[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = threadIdx.x + 256 * i;                   // chunk c of the ng rows
      const int m = c < ng * rch ? c / rch : 0, cc = c < ng * rch ? c - m * rch : 0;
      cp[i] = reinterpret_cast<const gm_u32x4*>(xl + (int64_t)(m == 0 ? gt[0] : gt[1]) * rbytes)[cc];
    }
    if (g0 > 0) __syncthreads();                             // previous group's reads are done
    else if constexpr (QT == GM_QTYPE_IQ3_XXS) gm_iq3_tab_store(gw, tab);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = threadIdx.x + 256 * i;
      reinterpret_cast<gm_u32x4*>(xs)[c < ng * rch ? c : MG * rch] = cp[i];   // past the rows: spare chunk
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      opaque(fg[p]);
      opaque(fu[p]);
      float ag[MG], au[MG];
#pragma unroll
      for (int m = 0; m < MG; ++m) { ag[m] = 0.f; au[m] = 0.f; }
      dot_subs_i8<QT, 32, DC, MG>(fg[p], lir, nsub, xs, rbytes, idx, ng, tab, ag);
      dot_subs_i8<QT, 32, DC, MG>(fu[p], lir, nsub, xs, rbytes, idx, ng, tab, au);
      const int row = r0 + 8 * p + 2 * wave + (lane >> 5);
#pragma unroll
      for (int m = 0; m < MG; ++m) {
        if (m < ng) {
          const float hv = gm_silu(rs[m] * row_sum<32>(ag[m])) * (rs[m] * row_sum<32>(au[m]));
          int d = dst[0];
#pragma unroll
          for (int q = 1; q < 8; ++q) d = g0 + m == q ? dst[q] : d;
          if (row < FF && lir == 0) h[(int64_t)d * FF + row] = hv;
        }
      }
      issue_fence();                                           // one pass's decoded rows live at a time
    }
  }
}

// Blocks [0, n_sh): the shared expert, token pair b / n_rg (h rows after the
// routed ones; one block per pair and row chunk, so that no block decodes its
// rows for all T tokens: 2.034 -> 2.021 ms per B = 8 step); blocks
// [n_sh, ...): unit (b - n_sh) / n_rg of the unique routed experts (members
// from the grouping table); 8 kGuPasses rows per block.  The
// launcher sets n_sh = 0 when the shared expert is in another format, and
// launches its blocks separately with that format.  One pass (8 rows) per
// block: 84 VGPRs, 5 waves per SIMD, and twice the blocks of two passes, whose
// last ones (the launch's tail, where few blocks still run) end sooner:
// 2.07 -> 2.03 ms per B = 8 step.
constexpr int kGuPasses = 1;

template <int QT, int DC>
__global__ void __launch_bounds__(256) k_dec_gateup8(gm_moe_layer P, const uint8_t* __restrict__ xl,
                                                     const float* __restrict__ rmsv, int T,
                                                     const int32_t* __restrict__ g_grp, float* __restrict__ h,
                                                     int n_sh, int n_rg GM_TL_PARAM) {
  GM_TL_BEGIN();
  constexpr bool IQ3 = QT == GM_QTYPE_IQ3_XXS;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* xs = smem;                                          // 2 limb rows (+ a spare sub-block)
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(smem + 2 * gm_limb_row_bytes(P.D) + GM_LSUB);   // IQ3 only
  const int D = P.D, k = P.k, FF = P.FF, Ptot = T * k;
  const int nu = g_grp[0];
  const bool shared = (int)blockIdx.x < n_sh;
  const int u = shared ? nu : ((int)blockIdx.x - n_sh) / n_rg;
  const int sgi = shared ? (int)blockIdx.x / n_rg : 0;              // shared blocks: token pair sgi
  const int chunk = shared ? (int)blockIdx.x - sgi * n_rg : (int)blockIdx.x - n_sh - u * n_rg;
  if (u > nu || (!shared && u == nu)) return;                  // uniform per block
  uint32_t gw = 0;
  if constexpr (IQ3) gw = gm_iq3_tab_load();
  const int64_t rb = gm_row_bytes(QT, D);
  const uint8_t* gbase;
  const uint8_t* ubase;
  int nm, tok[8], dst[8];
  if (shared) {
    gbase = static_cast<const uint8_t*>(P.gate_sh);
    ubase = static_cast<const uint8_t*>(P.up_sh);
    const int t0 = kGuMembers * sgi;
    nm = T - t0 < kGuMembers ? T - t0 : kGuMembers;
#pragma unroll
    for (int m = 0; m < 8; ++m) { tok[m] = t0 + (m < nm ? m : 0); dst[m] = Ptot + tok[m]; }
  } else {
    const int e = g_grp[1 + u];
    gbase = static_cast<const uint8_t*>(P.gate_exps) + (int64_t)e * FF * rb;
    ubase = static_cast<const uint8_t*>(P.up_exps) + (int64_t)e * FF * rb;
    nm = g_grp[1 + GM_GRP_MAXU + u];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      dst[m] = g_grp[1 + 2 * GM_GRP_MAXU + GM_GRP_MAXM * u + (m < nm ? m : 0)];
      tok[m] = dst[m] / k;
    }
  }
  gateup_rows<QT, DC, kGuPasses>(gbase, ubase, FF, D, chunk * 8 * kGuPasses, nm, tok, dst, xl, rmsv, xs, gw, tab, h);
  GM_TL_END(6);
}

template <int QT, int QTS, int DC>
int launch_gu(const gm_moe_layer* P, const float* x, int T, bool fast1, const GmDecArgs& a, hipStream_t s) {
  if (fast1) {
    if (a.acc != nullptr) {
      // one block per CU: 16 routed rows per block, two shared rows on a ninth wave
      // (gm_dec_chain_ok checked the shape)
      const int n16 = P->FF / 16, nblk = P->k * n16;
      const size_t smem = (size_t)gm_limb_row_bytes(P->D) + GM_LSUB +
                          (QT == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
      auto kern = P->E <= 256 ? k_dec_gateup1w<QT, QTS, DC, 4> : k_dec_gateup1w<QT, QTS, DC, 8>;
      if (int rc = gm_set_smem(kern, smem)) return rc;
      hipLaunchKernelGGL(kern, dim3(nblk), dim3(576), smem, s, *P, x, a.acc, a.acc_zero, gm_acc_ld(P->E), a.logits,
                         a.shg, a.ids, a.wts, a.grp, a.h, a.hsh, n16 GM_TL_ARG(a.tl));
      GM_TRY(hipGetLastError());
      return GM_OK;
    }
    const int n_chunks = (P->FF + 7) / 8;
    const int n_sh = P->gate_sh ? (P->FF_sh + 7) / 8 : 0;
    const size_t smem = (size_t)gm_limb_row_bytes(P->D) + GM_LSUB +
                        (QT == GM_QTYPE_IQ3_XXS || QTS == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
    auto kern = P->E <= 256 ? k_dec_gateup1<QT, QTS, DC, 4> : k_dec_gateup1<QT, QTS, DC, 8>;
    if (int rc = gm_set_smem(kern, smem)) return rc;
    hipLaunchKernelGGL(kern, dim3(n_sh + P->k * n_chunks), dim3(256), smem, s, *P, a.logits, a.ids, a.wts, a.grp,
                       a.h, a.hsh, n_chunks, n_sh, a.xl GM_TL_ARG(a.tl));
    GM_TRY(hipGetLastError());
    return GM_OK;
  }
  const int nz = a.nz;                                             // <= GM_DEC_MAX_NZ (checked below)
  if (nz > GM_DEC_MAX_NZ) return gm_fail_arg("gm_moe_forward: D=%d needs more than %d router ranges", P->D, GM_DEC_MAX_NZ);
  auto route = nz <= 8 ? (P->E <= 256 ? k_dec_route<4, 8> : k_dec_route<8, 8>)
                       : (P->E <= 256 ? k_dec_route<4, 16> : k_dec_route<8, 16>);
  hipLaunchKernelGGL(route, dim3(1), dim3(512), 0, s, *P, a.part, a.ssq, nz, gm_dec_part_ld(P), T, a.rms, a.logits,
                     a.shg, a.ids, a.wts, a.grp GM_TL_ARG(a.tl));
  GM_TRY(hipGetLastError());
  const int n_rg = (P->FF + 8 * kGuPasses - 1) / (8 * kGuPasses);  // blocks per unit
  // the shared expert's blocks: (token pair, row chunk), so that none decodes
  // its rows for more than one pair
  const int n_sh = P->gate_sh ? n_rg * ((T + kGuMembers - 1) / kGuMembers) : 0;
  const int max_u = T * P->k < P->E ? T * P->k : P->E;
  const bool sh_own = P->gate_sh && P->q_gate_sh != QT;            // shared expert in its own format
  {
    const size_t smem = 2 * (size_t)gm_limb_row_bytes(P->D) + GM_LSUB + (QT == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
    const int nsh = sh_own ? 0 : n_sh;
    if (int rc = gm_set_smem(k_dec_gateup8<QT, DC>, smem)) return rc;
    hipLaunchKernelGGL((k_dec_gateup8<QT, DC>), dim3(nsh + max_u * n_rg), dim3(256), smem, s, *P, a.xl, a.rms, T,
                       a.grp, a.h, nsh, n_rg GM_TL_ARG(a.tl));
    GM_TRY(hipGetLastError());
  }
  if (sh_own) {
    const size_t smem = 2 * (size_t)gm_limb_row_bytes(P->D) + GM_LSUB + (QTS == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
    if (int rc = gm_set_smem(k_dec_gateup8<QTS, DC>, smem)) return rc;
    hipLaunchKernelGGL((k_dec_gateup8<QTS, DC>), dim3(n_sh), dim3(256), smem, s, *P, a.xl, a.rms, T, a.grp, a.h,
                       n_sh, n_rg GM_TL_ARG(a.tl));
  }
  GM_TRY(hipGetLastError());
  return GM_OK;
}

template <int QT, int QTS>
int launch_gu_q(const gm_moe_layer* P, const float* x, int T, bool fast1, const GmDecArgs& a, hipStream_t s) {
  switch (gm_dec_dc(P->D)) {
    case 1: return launch_gu<QT, QTS, 1>(P, x, T, fast1, a, s);
    case 2: return launch_gu<QT, QTS, 2>(P, x, T, fast1, a, s);
    default: return launch_gu<QT, QTS, 4>(P, x, T, fast1, a, s);
  }
}

template <int QT>
int launch_gu_s(const gm_moe_layer* P, const float* x, int T, bool fast1, const GmDecArgs& a, hipStream_t s) {
  if (!P->gate_sh) return launch_gu_q<QT, QT>(P, x, T, fast1, a, s);
  switch (P->q_gate_sh) {
    case GM_QTYPE_IQ4_XS: return launch_gu_q<QT, GM_QTYPE_IQ4_XS>(P, x, T, fast1, a, s);
    case GM_QTYPE_IQ3_XXS: return launch_gu_q<QT, GM_QTYPE_IQ3_XXS>(P, x, T, fast1, a, s);
    case GM_QTYPE_BF16: return launch_gu_q<QT, GM_QTYPE_BF16>(P, x, T, fast1, a, s);
    case GM_QTYPE_I8: return launch_gu_q<QT, GM_QTYPE_I8>(P, x, T, fast1, a, s);
    default: return gm_fail_arg("gm_moe_forward: shared gate/up format %d unsupported", P->q_gate_sh);
  }
}

}  // namespace

int gm_dec_gateup(const gm_moe_layer* P, const float* x, int T, bool fast1, const GmDecArgs& a, hipStream_t s) {
  switch (P->q_gate) {
    case GM_QTYPE_IQ4_XS: return launch_gu_s<GM_QTYPE_IQ4_XS>(P, x, T, fast1, a, s);
    case GM_QTYPE_IQ3_XXS: return launch_gu_s<GM_QTYPE_IQ3_XXS>(P, x, T, fast1, a, s);
    case GM_QTYPE_BF16: return launch_gu_s<GM_QTYPE_BF16>(P, x, T, fast1, a, s);
    case GM_QTYPE_I8: return launch_gu_s<GM_QTYPE_I8>(P, x, T, fast1, a, s);
    default: return gm_fail_arg("gm_moe_forward: routed gate/up format %d unsupported", P->q_gate);
  }
}
