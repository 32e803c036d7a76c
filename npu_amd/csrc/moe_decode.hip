// MoE block, decode path (T <= 8 tokens).  Reference semantics:
// qwen/forward.py:563-665 (moe_forward).
//
// Stage 1  T = 1: k_dec_router: router logits (bf16 W, fp32 RMSNorm'd x), the
//                         shared scalar gate, and the shared expert's gate/up +
//                         SwiGLU; none of it depends on the routing.
//          T > 1: k_dec_router_ks: partial router dot products over K ranges
//                         (the routing kernel of stage 2 sums them and applies
//                         the RMSNorm factor); the shared expert runs with the
//                         routed ones.
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
// per row); block n_rb also writes its limb rows of the RMSNorm'd x to xl_out
// (when set) for the gate/up kernel.  DC = ceil(D / 1024).
template <int QTS, int NT, int DC>
__global__ void __launch_bounds__(256) k_dec_router(gm_moe_layer P, const float* __restrict__ x, int T,
                                                    float* __restrict__ logits, float* __restrict__ shg,
                                                    float* __restrict__ hsh, int n_rb, uint8_t* __restrict__ xl_out GM_TL_PARAM) {
  constexpr int SPLR = DC > 1 ? DC / 2 : 1;
  constexpr bool IQ3 = QTS == GM_QTYPE_IQ3_XXS;
  extern __shared__ float smem[];
  float* xs = smem;                                            // NT interleaved rows of D (+ 4)
  float* red = smem + NT * P.D + 4;                            // [4 * NT]
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(red + 4 * NT);       // IQ3 shared expert only
  const int D = P.D, E = P.E, nsub = D / GM_SUB;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  GM_TL_BEGIN();
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
    fetch_subs<GM_QTYPE_BF16, 64, SPLR, true>(f, wr, lane, nsub);
    issue_fence();
    stage_x_regs<NT, DC>(xr, T, D, P.norm_w, P.norm_eps, xs, red);
    GM_TL_MARK1(xs[0]);
    float acc[NT];
#pragma unroll
    for (int m = 0; m < NT; ++m) acc[m] = 0.f;
    dot_subs<GM_QTYPE_BF16, 64, SPLR, NT>(f, lane, nsub, xs, D, tok, T, nullptr, acc);
    GM_TL_MARK2(acc[0]);
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
    GM_TL_END(0);
    return;
  }
  if constexpr (IQ3) gm_iq3_tab_store(gw, tab);                // visible after stage_x_regs' barrier
  const int FFs = P.FF_sh;
  const int64_t rb = gm_row_bytes(QTS, D);
  const int row = ((blockIdx.x - n_rb) * 4 + wave) * 2 + (lane >> 5);
  const bool live = row < FFs;
  const int r = live ? row : 0;
  RowFetch<QTS, DC> fg, fu;
  fetch_subs<QTS, 32, DC, true>(fg, static_cast<const uint8_t*>(P.gate_sh) + r * rb, lane & 31, nsub);
  fetch_subs<QTS, 32, DC, true>(fu, static_cast<const uint8_t*>(P.up_sh) + r * rb, lane & 31, nsub);
  issue_fence();
  uint8_t* xl = reinterpret_cast<uint8_t*>(xs);                // limb rows (fit in the fp32 rows' space)
  stage_limbs_regs<NT, DC>(xr, T, D, P.norm_w, P.norm_eps, xl, red);
  GM_TL_MARK1(xl[0]);
  float ag[NT], au[NT];
#pragma unroll
  for (int m = 0; m < NT; ++m) { ag[m] = 0.f; au[m] = 0.f; }
  const int rbytes = gm_limb_row_bytes(D);
  dot_subs_i8<QTS, 32, DC, NT>(fg, lane & 31, nsub, xl, rbytes, tok, T, tab, ag);
  dot_subs_i8<QTS, 32, DC, NT>(fu, lane & 31, nsub, xl, rbytes, tok, T, tab, au);
  GM_TL_MARK2(au[0]);
#pragma unroll
  for (int m = 0; m < NT; ++m) {
    const float hv = gm_silu(row_sum<32>(ag[m])) * row_sum<32>(au[m]);
    if (live && (lane & 31) == 0 && m < T) hsh[m * FFs + row] = hv;
  }
  if (xl_out != nullptr && (int)blockIdx.x == n_rb) {         // the limb rows for the gate/up kernel
    const gm_u32x4* src = reinterpret_cast<const gm_u32x4*>(xl);
    gm_u32x4* dst = reinterpret_cast<gm_u32x4*>(xl_out);
    for (int c = threadIdx.x; c < NT * (rbytes >> 4); c += 256) dst[c] = src[c];
  }
  GM_TL_END(0);
}

// T > 1: partial router dot products over K ranges, part[z][t][r] =
// sum_{k in range z} (x[t][k] w_norm[k]) W[r][k] (row E: the shared gate
// vector) and ssq[z][t] = sum_{k in range z} x[t][k]^2, so that no block loads
// more than its range of the T input rows; k_dec_route applies the RMSNorm
// factor (qwen/forward.py:58-61) to the summed partials.  Block = 4 rows (one
// per wave) x one range of kr = gm_dec_kr(D) values (512, or 256 when 512 does
// not divide D); lane l takes k = 8l .. 8l+7.
// Wave 0 of the first row block of each range also writes the limb rows of
// x w_norm for the range (the RMSNorm factor is applied to the dot products
// instead), so the grouped gate/up kernel only copies them.
template <int NT>
__global__ void __launch_bounds__(256) k_dec_router_ks(gm_moe_layer P, const float* __restrict__ x, int T,
                                                       float* __restrict__ part, float* __restrict__ ssq, int ldp,
                                                       int kr, uint8_t* __restrict__ xl) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int D = P.D, E = P.E, nrows = E + (P.sh_gate_inp != nullptr ? 1 : 0);
  const int z = blockIdx.y, k0 = z * kr + 8 * lane;
  const bool lv = 8 * lane < kr;
  const int kk = lv ? k0 : z * kr;                              // lanes past the range re-read its start
  const int row = blockIdx.x * 4 + wave;
  const uint16_t* wr = row < E ? P.router + (int64_t)row * D : (row < nrows ? P.sh_gate_inp : P.router);
  const gm_u32x4 wb = *reinterpret_cast<const gm_u32x4*>(wr + kk);        // 8 bf16
  gm_f32x4 nw0 = {1.f, 1.f, 1.f, 1.f}, nw1 = nw0;
  if (P.norm_w) {
    nw0 = *reinterpret_cast<const gm_f32x4*>(P.norm_w + kk);
    nw1 = *reinterpret_cast<const gm_f32x4*>(P.norm_w + kk + 4);
  }
  gm_f32x4 xa[NT], xb[NT];
#pragma unroll
  for (int m = 0; m < NT; ++m) {
    const int t = m < T ? m : 0;
    xa[m] = *reinterpret_cast<const gm_f32x4*>(x + (int64_t)t * D + kk);
    xb[m] = *reinterpret_cast<const gm_f32x4*>(x + (int64_t)t * D + kk + 4);
  }
  const float w[8] = {gm_bf2f(wb.x & 0xffffu), gm_bf2f(wb.x >> 16), gm_bf2f(wb.y & 0xffffu), gm_bf2f(wb.y >> 16),
                      gm_bf2f(wb.z & 0xffffu), gm_bf2f(wb.z >> 16), gm_bf2f(wb.w & 0xffffu), gm_bf2f(wb.w >> 16)};
  if (blockIdx.x == 0 && wave == 0) {                           // uniform per wave
    const int rbytes = gm_limb_row_bytes(D);
#pragma unroll
    for (int m = 0; m < NT; ++m) {
      if (m < T) {
        gm_f32x4 a = xa[m], b = xb[m];
        a.x *= nw0.x; a.y *= nw0.y; a.z *= nw0.z; a.w *= nw0.w;
        b.x *= nw1.x; b.y *= nw1.y; b.z *= nw1.z; b.w *= nw1.w;
        // lanes past the range write a spare row (row T), quads stay whole
        gm_put_limbs8(a, b, lv ? kk >> 2 : (kk >> 2) & 7, xl + (lv ? m : T) * rbytes);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < NT; ++m) {
    if (m < T) {                                                // uniform
      const float xv[8] = {xa[m].x, xa[m].y, xa[m].z, xa[m].w, xb[m].x, xb[m].y, xb[m].z, xb[m].w};
      const float nv[8] = {nw0.x, nw0.y, nw0.z, nw0.w, nw1.x, nw1.y, nw1.z, nw1.w};
      float d = 0.f, q = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) { d = fmaf(xv[i] * nv[i], w[i], d); q = fmaf(xv[i], xv[i], q); }
      d = gm_wave_sum64(lv ? d : 0.f);
      if (lane == 0 && row < nrows) part[((int64_t)z * T + m) * ldp + row] = d;
      if (blockIdx.x == 0 && wave == 0) {
        q = gm_wave_sum64(lv ? q : 0.f);
        if (lane == 0) ssq[z * T + m] = q;
      }
    }
  }
}

// with_shared: the shared expert's gate/up run here as well.
template <int QTS, int NT, int DC>
int launch_router_t(const gm_moe_layer* P, const float* x, int T, const GmDecArgs& a, hipStream_t s,
                    bool with_shared) {
  const int nrows = P->E + (P->sh_gate_inp ? 1 : 0);
  const int n_rb = (nrows + 3) / 4;
  const int n_sb = P->gate_sh && with_shared ? (P->FF_sh + 7) / 8 : 0;
  const size_t smem = ((size_t)NT * P->D + 4 + 4 * NT) * 4 + (QTS == GM_QTYPE_IQ3_XXS ? sizeof(Iq3Tab) : 0);
  if (int rc = gm_set_smem(k_dec_router<QTS, NT, DC>, smem)) return rc;
  hipLaunchKernelGGL((k_dec_router<QTS, NT, DC>), dim3(n_rb + n_sb), dim3(256), smem, s, *P, x, T, a.logits, a.shg,
                     a.hsh, n_rb, n_sb > 0 ? a.xl : nullptr GM_TL_ARG(a.tl));
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
  if (!fast1) {                                                      // router partials only
    const int nrows = P->E + (P->sh_gate_inp ? 1 : 0);
    const int kr = gm_dec_kr(P->D);
    hipLaunchKernelGGL(k_dec_router_ks<8>, dim3((nrows + 3) / 4, P->D / kr), dim3(256), 0, s, *P, x, T, a.part,
                       a.ssq, gm_dec_part_ld(P), kr, a.xl);
    GM_TRY(hipGetLastError());
    return GM_OK;
  }
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
  a.tl = reinterpret_cast<uint64_t*>(ws + lay.tl);
  // general path: router partials, x^2 partials, RMSNorm factors and the limb
  // rows of x w_norm live in yp, which stage 3 overwrites only after stage 2
  a.part = a.yp;
  a.ssq = a.part + (size_t)gm_dec_nz(P->D) * T * gm_dec_part_ld(P);
  a.rms = a.ssq + GM_DEC_MAX_NZ * T;
  a.xl = reinterpret_cast<uint8_t*>(a.rms + 16);
  if (a.xl + (size_t)(T + 1) * gm_limb_row_bytes(P->D) > reinterpret_cast<uint8_t*>(a.yp + (size_t)(T * P->k + T) * P->D))
    return gm_fail_arg("gm_moe_forward: internal workspace layout error (yp)");
  if (a.hsh != a.h + (size_t)T * P->k * P->FF) return gm_fail_arg("gm_moe_forward: internal workspace layout error");
  // The T = 1 down kernel stages (k + 1) rows of FF activations per block and
  // maps a wave's lanes onto 8 rows x FF/32 sub-blocks (FF/32 in {8, 16, 32}).
  // (bf16 routed down rows fit the down kernel's LDS slices up to FF = 512)
  const bool fast1 = T == 1 && (P->FF == 256 || P->FF == 512 || (P->FF == 1024 && P->q_down != GM_QTYPE_BF16));
  if (stage == 0 || stage == 1)
    if (int rc = launch_router(P, x, T, a, s, fast1)) return rc;
  if (stage == 0 || stage == 2)
    if (int rc = gm_dec_gateup(P, x, T, fast1, a, s)) return rc;
  if (stage == 0 || stage == 3)
    if (int rc = gm_dec_down(P, x, y, T, flags, fast1, a, s)) return rc;
  return GM_OK;
}
