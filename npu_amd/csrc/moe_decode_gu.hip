// MoE decode, stage 2: top-k routing, expert grouping, routed gate/up + SwiGLU.
//
// T = 1 (k_dec_gateup1): every block recomputes the token's top-k from the
// router logits (wave 0, while wave 1 stages x) instead of waiting for a
// separate routing kernel, picks the expert of rank `u` among the k picks
// (ascending id, the order of torch.unique in qwen/forward.py:612) and runs 8
// SwiGLU rows of it.  Block 0 publishes ids, weights and the grouping table
// for stage 3.
//
// T > 1: k_dec_route (one block) runs the per-token top-k and groups the
// (token, slot) pairs by expert; k_dec_gateup8 then runs (unique expert, 8-row
// chunk) blocks over the expert's member tokens only.
#include "moe_common.h"
#include "moe_decode.h"

using namespace gm_moe;

namespace {

template <int QT, int DC, int MAXV>
__global__ void __launch_bounds__(256) k_dec_gateup1(gm_moe_layer P, const float* __restrict__ x,
                                                     const float* __restrict__ logits, int32_t* __restrict__ g_ids,
                                                     float* __restrict__ g_wts, int32_t* __restrict__ g_grp,
                                                     float* __restrict__ h, int n_chunks) {
  constexpr bool IQ3 = QT == GM_QTYPE_IQ3_XXS;
  extern __shared__ float smem[];
  float* xs = smem;                                            // [D + 4] interleaved
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(smem + P.D + 4);     // IQ3 only
  __shared__ int32_t s_sid[8], s_slot[8];                      // picks in ascending expert order
  const int D = P.D, E = P.E, k = P.k, FF = P.FF, nsub = D / GM_SUB;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int u = blockIdx.x / n_chunks, chunk = blockIdx.x - u * n_chunks;
  uint32_t gw = 0;
  if constexpr (IQ3) gw = gm_iq3_tab_load();
  if (wave == 0) {
    // top-k of the router logits; lane j < k holds pick j
    float v[MAXV];
    int ix[MAXV];
    topk_load<MAXV>(logits, E, v, ix);
    int myid;
    float myw;
    topk_finish<MAXV>(v, ix, E, k, myid, myw);
    int rk = 0;                                                // rank of the pick among the k (distinct) ids
#pragma unroll
    for (int i = 0; i < 8; ++i) rk += __builtin_amdgcn_readlane(myid, i) < myid ? 1 : 0;
    if (lane < k) { s_sid[rk] = myid; s_slot[rk] = lane; }
    if (blockIdx.x == 0) {                                     // publish for stage 3 and the caller
      if (lane < k) {
        g_ids[lane] = myid;
        g_wts[lane] = myw;
        g_grp[1 + rk] = myid;
        g_grp[1 + GM_GRP_MAXU + rk] = 1;
        g_grp[1 + 2 * GM_GRP_MAXU + GM_GRP_MAXM * rk] = lane;
        g_grp[GM_GRP_WORDS + rk] = __float_as_int(myw);
      }
      if (lane == 0) g_grp[0] = k;
    }
  } else if (wave == 1) {
    stage_x_wave<4 * DC>(x, D, P.norm_w, P.norm_eps, xs);     // concurrently with the top-k
  }
  if constexpr (IQ3) gm_iq3_tab_store(gw, tab);
  __syncthreads();
  const int e = s_sid[u], pair = s_slot[u];
  const int64_t rb = gm_row_bytes(QT, D);
  const int row = chunk * 8 + wave * 2 + (lane >> 5);
  const bool live = row < FF;
  const int r = live ? row : 0;
  RowFetch<QT, DC> fg, fu;
  fetch_subs<QT, 32, DC>(fg, static_cast<const uint8_t*>(P.gate_exps) + ((int64_t)e * FF + r) * rb, lane & 31, nsub);
  fetch_subs<QT, 32, DC>(fu, static_cast<const uint8_t*>(P.up_exps) + ((int64_t)e * FF + r) * rb, lane & 31, nsub);
  const int tok[1] = {0};
  float ag[1] = {0.f}, au[1] = {0.f};
  dot_subs<QT, 32, DC, 1>(fg, lane & 31, nsub, xs, D, tok, 1, tab, ag);
  dot_subs<QT, 32, DC, 1>(fu, lane & 31, nsub, xs, D, tok, 1, tab, au);
  const float hv = gm_silu(row_sum<32>(ag[0])) * row_sum<32>(au[0]);
  if (live && (lane & 31) == 0) h[(int64_t)pair * FF + row] = hv;
}

// One block: top-k of every token (wave t -> token t) and the grouping table.
template <int MAXV>
__global__ void __launch_bounds__(512) k_dec_route(const float* __restrict__ logits, int T, int E, int k,
                                                   int32_t* __restrict__ g_ids, float* __restrict__ g_wts,
                                                   int32_t* __restrict__ g_grp) {
  __shared__ int32_t ids[64];
  __shared__ float wts[64];
  __shared__ int32_t grp[GM_GRP_WORDS];
  __shared__ uint32_t bits[16];
  const int wave = threadIdx.x >> 6;
  if (wave < T) wave_topk<MAXV>(logits + (int64_t)wave * E, E, k, ids + wave * k, wts + wave * k);
  __syncthreads();
  block_group(ids, T * k, E, grp, bits);
  for (int i = threadIdx.x; i < T * k; i += blockDim.x) { g_ids[i] = ids[i]; g_wts[i] = wts[i]; }
  for (int i = threadIdx.x; i < GM_GRP_WORDS; i += blockDim.x) g_grp[i] = grp[i];
}

// Block = (unique expert u, 8 rows); x rows of the expert's member tokens only.
template <int QT, int DC>
__global__ void __launch_bounds__(256) k_dec_gateup8(gm_moe_layer P, const float* __restrict__ x,
                                                     const int32_t* __restrict__ g_grp, float* __restrict__ h,
                                                     int n_chunks) {
  constexpr bool IQ3 = QT == GM_QTYPE_IQ3_XXS;
  extern __shared__ float smem[];
  float* xs = smem;                                            // [8][D] interleaved (+ 4)
  float* red = smem + 8 * P.D + 4;                             // [32]
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(red + 32);           // IQ3 only
  const int D = P.D, k = P.k, FF = P.FF, nsub = D / GM_SUB;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int u = blockIdx.x / n_chunks, chunk = blockIdx.x - u * n_chunks;
  const int nu = g_grp[0];
  if (u >= nu) return;                                         // uniform per block
  const int e = g_grp[1 + u];
  const int nm = g_grp[1 + GM_GRP_MAXU + u];
  int pair[8], tok[8], idx[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    pair[m] = g_grp[1 + 2 * GM_GRP_MAXU + GM_GRP_MAXM * u + (m < nm ? m : 0)];
    tok[m] = pair[m] / k;
    idx[m] = m;
  }
  uint32_t gw = 0;
  if constexpr (IQ3) gw = gm_iq3_tab_load();
  const int64_t rb = gm_row_bytes(QT, D);
  const int row = chunk * 8 + wave * 2 + (lane >> 5);
  const bool live = row < FF;
  const int r = live ? row : 0;
  RowFetch<QT, DC> fg, fu;
  fetch_subs<QT, 32, DC>(fg, static_cast<const uint8_t*>(P.gate_exps) + ((int64_t)e * FF + r) * rb, lane & 31, nsub);
  fetch_subs<QT, 32, DC>(fu, static_cast<const uint8_t*>(P.up_exps) + ((int64_t)e * FF + r) * rb, lane & 31, nsub);
  XRegs<8, DC> xr;
  load_x<8, DC>(xr, x, tok, nm, D, P.norm_w);
  if constexpr (IQ3) gm_iq3_tab_store(gw, tab);
  stage_x_regs<8, DC>(xr, nm, D, P.norm_w, P.norm_eps, xs, red);
  float ag[8], au[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) { ag[m] = 0.f; au[m] = 0.f; }
  dot_subs<QT, 32, DC, 8>(fg, lane & 31, nsub, xs, D, idx, nm, tab, ag);
  dot_subs<QT, 32, DC, 8>(fu, lane & 31, nsub, xs, D, idx, nm, tab, au);
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    if (m < nm) {
      const float hv = gm_silu(row_sum<32>(ag[m])) * row_sum<32>(au[m]);
      if (live && (lane & 31) == 0) h[(int64_t)pair[m] * FF + row] = hv;
    }
  }
}

template <int QT, int DC>
int launch_gu(const gm_moe_layer* P, const float* x, int T, bool fast1, const GmDecArgs& a, hipStream_t s) {
  const int n_chunks = (P->FF + 7) / 8;
  if (fast1) {
    const size_t smem = ((size_t)P->D + 4) * 4 + (QT == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
    if (int rc = gm_set_smem(k_dec_gateup1<QT, DC, 4>, smem)) return rc;
    if (int rc = gm_set_smem(k_dec_gateup1<QT, DC, 8>, smem)) return rc;
    if (P->E <= 256)
      hipLaunchKernelGGL((k_dec_gateup1<QT, DC, 4>), dim3(P->k * n_chunks), dim3(256), smem, s, *P, x, a.logits,
                         a.ids, a.wts, a.grp, a.h, n_chunks);
    else
      hipLaunchKernelGGL((k_dec_gateup1<QT, DC, 8>), dim3(P->k * n_chunks), dim3(256), smem, s, *P, x, a.logits,
                         a.ids, a.wts, a.grp, a.h, n_chunks);
    GM_TRY(hipGetLastError());
    return GM_OK;
  }
  if (P->E <= 256)
    hipLaunchKernelGGL(k_dec_route<4>, dim3(1), dim3(512), 0, s, a.logits, T, P->E, P->k, a.ids, a.wts, a.grp);
  else
    hipLaunchKernelGGL(k_dec_route<8>, dim3(1), dim3(512), 0, s, a.logits, T, P->E, P->k, a.ids, a.wts, a.grp);
  GM_TRY(hipGetLastError());
  const int max_u = T * P->k < P->E ? T * P->k : P->E;
  const size_t smem = (8 * (size_t)P->D + 4 + 32) * 4 + (QT == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
  if (int rc = gm_set_smem(k_dec_gateup8<QT, DC>, smem)) return rc;
  hipLaunchKernelGGL((k_dec_gateup8<QT, DC>), dim3(max_u * n_chunks), dim3(256), smem, s, *P, x, a.grp, a.h,
                     n_chunks);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

template <int QT>
int launch_gu_q(const gm_moe_layer* P, const float* x, int T, bool fast1, const GmDecArgs& a, hipStream_t s) {
  switch (gm_dec_dc(P->D)) {
    case 1: return launch_gu<QT, 1>(P, x, T, fast1, a, s);
    case 2: return launch_gu<QT, 2>(P, x, T, fast1, a, s);
    default: return launch_gu<QT, 4>(P, x, T, fast1, a, s);
  }
}

}  // namespace

int gm_dec_gateup(const gm_moe_layer* P, const float* x, int T, bool fast1, const GmDecArgs& a, hipStream_t s) {
  switch (P->q_gate) {
    case GM_QTYPE_IQ4_XS: return launch_gu_q<GM_QTYPE_IQ4_XS>(P, x, T, fast1, a, s);
    case GM_QTYPE_IQ3_XXS: return launch_gu_q<GM_QTYPE_IQ3_XXS>(P, x, T, fast1, a, s);
    default: return gm_fail_arg("gm_moe_forward: routed gate/up format %d unsupported", P->q_gate);
  }
}
