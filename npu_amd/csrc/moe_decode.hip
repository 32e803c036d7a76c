// MoE block, decode path (T <= 8 tokens).  Reference semantics:
// qwen/forward.py:563-665 (moe_forward).
//
// Stage 1  k_dec_router   router logits (bf16 W, fp32 RMSNorm'd x), the shared
//                         scalar gate, and (T = 1 kernels) the shared expert's
//                         gate/up + SwiGLU; none of it depends on the routing.
//                         For the grouped T > 1 kernels it publishes xn instead
//                         and the shared expert runs with the routed ones.
// Stage 2  (moe_decode_gu.hip) top-k, expert grouping, routed gate/up + SwiGLU.
// Stage 3  (moe_decode_dn.hip) down projections, weighted combine in ascending
//                         expert order, + sigmoid-gated shared expert (+ x).
//
// Kernel boundaries are the only grid-wide synchronisation.  Every kernel
// issues all the weight loads of a lane before it waits on anything (see
// fetch_subs), so one HBM round trip covers a block's whole weight tile.
#include "moe_common.h"
#include "moe_decode.h"

using namespace gm_moe;

namespace {

// Blocks [0, n_rb): one router row per wave (64 lanes; row E is the shared
// scalar gate).  Blocks [n_rb, ...): two shared gate/up rows per wave (32 lanes
// per row).  DC = ceil(D / 1024).
template <int QTS, int NT, int DC>
__global__ void __launch_bounds__(256) k_dec_router(gm_moe_layer P, const float* __restrict__ x, int T,
                                                    float* __restrict__ logits, float* __restrict__ shg,
                                                    float* __restrict__ hsh, float* __restrict__ xn, int n_rb) {
  constexpr int SPLR = DC > 1 ? DC / 2 : 1;
  constexpr bool IQ3 = QTS == GM_QTYPE_IQ3_XXS;
  extern __shared__ float smem[];
  float* xs = smem;                                            // NT interleaved rows of D (+ 4)
  float* red = smem + NT * P.D + 4;                            // [4 * NT]
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(red + 4 * NT);       // IQ3 shared expert only
  const int D = P.D, E = P.E, nsub = D / GM_SUB;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int tok[NT];
#pragma unroll
  for (int m = 0; m < NT; ++m) tok[m] = m;
  XRegs<NT, DC> xr;
  load_x<NT, DC>(xr, x, tok, T, D, P.norm_w);
  uint32_t gw = 0;
  if constexpr (IQ3) gw = gm_iq3_tab_load();
  if ((int)blockIdx.x < n_rb) {
    const int row = blockIdx.x * 4 + wave;
    const int nrows = E + (P.sh_gate_inp != nullptr ? 1 : 0);
    const uint8_t* wr = row < E ? reinterpret_cast<const uint8_t*>(P.router) + (int64_t)row * D * 2
                                : reinterpret_cast<const uint8_t*>(row < nrows ? P.sh_gate_inp : P.router);
    RowFetch<GM_QTYPE_BF16, SPLR> f;
    fetch_subs<GM_QTYPE_BF16, 64, SPLR>(f, wr, lane, nsub);
    issue_fence();
    stage_x_regs<NT, DC>(xr, T, D, P.norm_w, P.norm_eps, xs, red);
    if (xn != nullptr && blockIdx.x == 0) {                    // publish xn [T][D] for the grouped kernels
      const int nq = D >> 2;
      const gm_f32x4* xs4 = reinterpret_cast<const gm_f32x4*>(xs);
      gm_f32x4* xn4 = reinterpret_cast<gm_f32x4*>(xn);
      for (int i = threadIdx.x; i < T * nq; i += 256) {
        const int t = i / nq, c = i - t * nq;
        xn4[i] = xs4[t * nq + il_index4(c & 7, c >> 3, nsub)];
      }
    }
    float acc[NT];
#pragma unroll
    for (int m = 0; m < NT; ++m) acc[m] = 0.f;
    dot_subs<GM_QTYPE_BF16, 64, SPLR, NT>(f, lane, nsub, xs, D, tok, T, nullptr, acc);
#pragma unroll
    for (int m = 0; m < NT; ++m) acc[m] = gm_wave_sum64(acc[m]);
    if (row < nrows && lane == 0) {
#pragma unroll
      for (int m = 0; m < NT; ++m) {
        if (m < T) {
          if (row < E) logits[m * E + row] = acc[m] + (P.router_bias ? P.router_bias[row] : 0.f);
          else shg[m] = gm_sigmoid(acc[m]);
        }
      }
    }
    return;
  }
  if constexpr (IQ3) gm_iq3_tab_store(gw, tab);                // visible after stage_x_regs' barrier
  const int FFs = P.FF_sh;
  const int64_t rb = gm_row_bytes(QTS, D);
  const int row = ((blockIdx.x - n_rb) * 4 + wave) * 2 + (lane >> 5);
  const bool live = row < FFs;
  const int r = live ? row : 0;
  RowFetch<QTS, DC> fg, fu;
  fetch_subs<QTS, 32, DC>(fg, static_cast<const uint8_t*>(P.gate_sh) + r * rb, lane & 31, nsub);
  fetch_subs<QTS, 32, DC>(fu, static_cast<const uint8_t*>(P.up_sh) + r * rb, lane & 31, nsub);
  issue_fence();
  uint8_t* xl = reinterpret_cast<uint8_t*>(xs);                // limb rows (fit in the fp32 rows' space)
  stage_limbs_regs<NT, DC>(xr, T, D, P.norm_w, P.norm_eps, xl, red);
  float ag[NT], au[NT];
#pragma unroll
  for (int m = 0; m < NT; ++m) { ag[m] = 0.f; au[m] = 0.f; }
  const int rbytes = gm_limb_row_bytes(D);
  dot_subs_i8<QTS, 32, DC, NT>(fg, lane & 31, nsub, xl, rbytes, tok, T, tab, ag);
  dot_subs_i8<QTS, 32, DC, NT>(fu, lane & 31, nsub, xl, rbytes, tok, T, tab, au);
#pragma unroll
  for (int m = 0; m < NT; ++m) {
    const float hv = gm_silu(row_sum<32>(ag[m])) * row_sum<32>(au[m]);
    if (live && (lane & 31) == 0 && m < T) hsh[m * FFs + row] = hv;
  }
}

// with_shared: the shared expert's gate/up run here (T = 1 kernels); otherwise
// they run with the routed experts in k_dec_gateup8 and this kernel publishes xn.
template <int QTS, int NT, int DC>
int launch_router_t(const gm_moe_layer* P, const float* x, int T, const GmDecArgs& a, hipStream_t s,
                    bool with_shared) {
  const int nrows = P->E + (P->sh_gate_inp ? 1 : 0);
  const int n_rb = (nrows + 3) / 4;
  const int n_sb = P->gate_sh && with_shared ? (P->FF_sh + 7) / 8 : 0;
  const size_t smem = ((size_t)NT * P->D + 4 + 4 * NT) * 4 + (QTS == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
  if (int rc = gm_set_smem(k_dec_router<QTS, NT, DC>, smem)) return rc;
  hipLaunchKernelGGL((k_dec_router<QTS, NT, DC>), dim3(n_rb + n_sb), dim3(256), smem, s, *P, x, T, a.logits, a.shg,
                     a.hsh, with_shared ? nullptr : a.xn, n_rb);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

template <int QTS, int NT>
int launch_router_n(const gm_moe_layer* P, const float* x, int T, const GmDecArgs& a, hipStream_t s, bool ws) {
  switch (gm_dec_dc(P->D)) {
    case 1: return launch_router_t<QTS, NT, 1>(P, x, T, a, s, ws);
    case 2: return launch_router_t<QTS, NT, 2>(P, x, T, a, s, ws);
    default: return launch_router_t<QTS, NT, 4>(P, x, T, a, s, ws);
  }
}

int launch_router(const gm_moe_layer* P, const float* x, int T, const GmDecArgs& a, hipStream_t s, bool fast1) {
  if (!fast1) return launch_router_n<GM_QTYPE_IQ4_XS, 8>(P, x, T, a, s, false);   // router rows only
  if (!P->gate_sh) return launch_router_n<GM_QTYPE_IQ4_XS, 1>(P, x, T, a, s, true);
  switch (P->q_gate_sh) {
    case GM_QTYPE_IQ4_XS: return launch_router_n<GM_QTYPE_IQ4_XS, 1>(P, x, T, a, s, true);
    case GM_QTYPE_IQ3_XXS: return launch_router_n<GM_QTYPE_IQ3_XXS, 1>(P, x, T, a, s, true);
    case GM_QTYPE_BF16: return launch_router_n<GM_QTYPE_BF16, 1>(P, x, T, a, s, true);
    default: return gm_fail_arg("gm_moe_forward: shared gate/up format %d unsupported", P->q_gate_sh);
  }
}

}  // namespace

int gm_dec_run(const gm_moe_layer* P, const float* x, float* y, int T, int flags, uint8_t* ws,
                  const GmMoeWs& lay, hipStream_t s, int stage) {
  if (T < 1 || T > GM_DECODE_MAX_T) return gm_fail_arg("gm_moe_forward: decode path needs 1 <= T <= 8 (T=%d)", T);
  if (P->D % 256 || P->FF % 256) return gm_fail_arg("gm_moe_forward: D and FF must be multiples of 256");
  if (P->D > 4096 || P->FF > 2048)
    return gm_fail_arg("gm_moe_forward: decode kernels support D <= 4096 and FF <= 2048 (D=%d FF=%d)", P->D, P->FF);
  if (P->k > 8) return gm_fail_arg("gm_moe_forward: k=%d > 8", P->k);
  GmDecArgs a;
  a.logits = reinterpret_cast<float*>(ws + lay.logits);
  a.shg = reinterpret_cast<float*>(ws + lay.shg);
  a.ids = reinterpret_cast<int32_t*>(ws + lay.ids);
  a.wts = reinterpret_cast<float*>(ws + lay.wts);
  a.grp = reinterpret_cast<int32_t*>(ws + lay.grp);
  a.h = reinterpret_cast<float*>(ws + lay.h);
  a.hsh = reinterpret_cast<float*>(ws + lay.hsh);
  a.yp = reinterpret_cast<float*>(ws + lay.yp);
  a.xn = reinterpret_cast<float*>(ws + lay.xn);
  if (a.hsh != a.h + (size_t)T * P->k * P->FF) return gm_fail_arg("gm_moe_forward: internal workspace layout error");
  // The T = 1 down kernel stages (k + 1) rows of FF activations per block and
  // maps a wave's lanes onto 8 rows x FF/32 sub-blocks (FF/32 in {8, 16, 32}).
  const bool fast1 = T == 1 && (P->FF == 256 || P->FF == 512 || P->FF == 1024);
  if (stage == 0 || stage == 1)
    if (int rc = launch_router(P, x, T, a, s, fast1)) return rc;
  if (stage == 0 || stage == 2)
    if (int rc = gm_dec_gateup(P, x, T, fast1, a, s)) return rc;
  if (stage == 0 || stage == 3)
    if (int rc = gm_dec_down(P, x, y, T, flags, fast1, a, s)) return rc;
  return GM_OK;
}
