// MoE block, decode path (T <= 8 tokens).  Reference semantics:
// qwen/forward.py:563-665 (moe_forward).
//
// Stage 1  T = 1: k_dec_router1: router logits (bf16 or fp32 W, fp32 RMSNorm'd x), the
//                         shared scalar gate and the limb row of the RMSNorm'd
//                         x for the gate/up kernel.
//          T > 1: k_dec_router_ks: partial router dot products over K ranges
//                         (the routing kernel of stage 2 sums them and applies
//                         the RMSNorm factor); the shared expert runs with the
//                         routed ones.
// Stage 2  (moe_decode_gu.hip) top-k, expert grouping, routed gate/up + SwiGLU
//                         (T = 1: also the shared expert's gate/up).
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

// T = 1: one router row per wave (row E: the shared scalar gate), two waves per
// block, no LDS and no barrier.  Lane l of a wave holds x, the RMSNorm weight
// and the row at k = 512 i + 8 l .. +7 for the NCH = ceil(D / 512) chunks i;
// all of them are loaded before anything waits, so the row costs one round
// trip.  Every wave sums x^2 over its own copy of x, so the RMSNorm factor
// rms = 1 / sqrt(mean(x^2) + eps) (qwen/forward.py:58-61) needs no block
// reduction; it scales the finished dot product W . (x * w_norm).  The first
// NL = NCH global waves (when xl_out is set) load no router row: wave i writes
// chunk i of the limb row of xn = (x * rms) * w_norm that the gate/up kernel
// multiplies with, a dependent chain of about 0.35 us that a row wave would
// otherwise add to its dot product.
// With acc set (the accumulator kernels of the T = 1 gate/up launch that
// k_dec_gateup1w runs) the raw dot products W . (x * w_norm) go to copy 0 of
// the accumulators instead (word E: the shared gate row, word E + 1: the sum of
// x^2), lanes 1-7 clear the other copies, and no limb row is written: the
// gate/up kernel applies the RMSNorm factor and the bias itself.
template <int NCH, bool RF32>
__global__ void __launch_bounds__(128) k_dec_router1(gm_moe_layer P, const float* __restrict__ x,
                                                     float* __restrict__ logits, float* __restrict__ shg,
                                                     uint8_t* __restrict__ xl_out, double* __restrict__ acc,
                                                     int acc_ld GM_TL_PARAM) {
  GM_TL_BEGIN();
  const int lane = threadIdx.x & 63, gw = blockIdx.x * 2 + (threadIdx.x >> 6);
  const int D = P.D, E = P.E, nrows = E + (P.sh_gate_inp != nullptr ? 1 : 0);
  const int nl = xl_out != nullptr ? NCH : 0;
  const bool limb_wave = gw < nl;                               // uniform per wave
  const int r = gw - nl;
  const int row = r < nrows ? (r < 0 ? 0 : r) : nrows - 1;    // spare waves redo the last row
  if (gw == 0 && lane == 0 && P.sh_gate_inp == nullptr && acc == nullptr) shg[0] = 1.f;   // ungated shared expert
  const void* wr = row < E ? router_row<RF32>(P.router, row, D) : P.sh_gate_inp;
  RouterChunk<RF32> wb[NCH];
  gm_f32x4 xa[NCH], xb[NCH], na[NCH], nb[NCH];
  // x and the RMSNorm weight first: the wait for them (vmcnt retires in issue
  // order) then never waits for the router row
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int kk = 512 * i + 8 * lane < D ? 512 * i + 8 * lane : D - 8;   // lanes past D re-read the end
    xa[i] = *reinterpret_cast<const gm_f32x4*>(x + kk);
    xb[i] = *reinterpret_cast<const gm_f32x4*>(x + kk + 4);
    if (P.norm_w) {
      na[i] = *reinterpret_cast<const gm_f32x4*>(P.norm_w + kk);
      nb[i] = *reinterpret_cast<const gm_f32x4*>(P.norm_w + kk + 4);
    } else {
      na[i] = gm_f32x4{1.f, 1.f, 1.f, 1.f};
      nb[i] = na[i];
    }
  }
  if (!limb_wave) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int kk = 512 * i + 8 * lane < D ? 512 * i + 8 * lane : D - 8;
      router_load8<RF32, true>(wr, kk, wb[i]);
    }
  }
  const float bias = P.router_bias != nullptr && row < E ? P.router_bias[row] : 0.f;
  issue_fence();
  // branch-free sums (lanes past D select 0): a branch per chunk made the
  // compiler wait for every outstanding memory operation
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const float xv[8] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w, xb[i].x, xb[i].y, xb[i].z, xb[i].w};
    float p = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) p = fmaf(xv[j], xv[j], p);
    ss += 512 * i + 8 * lane < D ? p : 0.f;
  }
  ss = gm_wave_sum64(ss);
  const float rms = P.norm_w != nullptr ? 1.0f / sqrtf(ss / (float)D + P.norm_eps) : 1.0f;
  GM_TL_MARK1(rms);
  if (limb_wave) {
    if (512 * gw < D) {
      const int i = gw;
      gm_f32x4 a = xa[0], b = xb[0], wa = na[0], wb2 = nb[0];
#pragma unroll
      for (int q = 1; q < NCH; ++q)
        if (q == i) { a = xa[q]; b = xb[q]; wa = na[q]; wb2 = nb[q]; }
      a.x = (a.x * rms) * wa.x; a.y = (a.y * rms) * wa.y; a.z = (a.z * rms) * wa.z; a.w = (a.w * rms) * wa.w;
      b.x = (b.x * rms) * wb2.x; b.y = (b.y * rms) * wb2.y; b.z = (b.z * rms) * wb2.z; b.w = (b.w * rms) * wb2.w;
      const int c = (512 * i + 8 * lane) >> 2;                   // float4 index, even
      // lanes past D write the spare sub-block after the row
      gm_put_limbs8(a, b, 512 * i + 8 * lane < D ? c : (D >> 2) + (c & 7), xl_out);
    }
    GM_TL_END(0);
    return;
  }
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const float xv[8] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w, xb[i].x, xb[i].y, xb[i].z, xb[i].w};
    const float nv[8] = {na[i].x, na[i].y, na[i].z, na[i].w, nb[i].x, nb[i].y, nb[i].z, nb[i].w};
    float w[8];
    router_unpack8<RF32>(wb[i], w);
    float p = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) p = fmaf(w[j], xv[j] * nv[j], p);
    dot += 512 * i + 8 * lane < D ? p : 0.f;
  }
  dot = gm_wave_sum64(dot);
  GM_TL_MARK2(dot);
  if (acc != nullptr) {
    if (lane < GM_ACC_COPIES) {
      if (r < nrows) acc[lane * acc_ld + gm_acc_pos(row, E)] = lane == 0 ? (double)dot : 0.0;
      if (r == 0) acc[lane * acc_ld + gm_acc_pos(E + 1, E)] = lane == 0 ? (double)ss : 0.0;
    }
  } else if (r < nrows && lane == 0) {
    if (row < E) logits[row] = rms * dot + bias;
    else shg[0] = gm_sigmoid(rms * dot);
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
// Wave 0 of row block b of each range also writes, for the tokens t with
// t % gridDim.x == b (one token per block when there are at least T row
// blocks), the limb row of x w_norm over the range (the RMSNorm factor is
// applied to the dot products instead), so that the grouped gate/up kernel
// only copies them, and the range's sum of x^2.  With all T tokens on one
// block that block ended 3 us after the others.
template <int NT, bool RF32>
__global__ void __launch_bounds__(256) k_dec_router_ks(gm_moe_layer P, const float* __restrict__ x, int T,
                                                       float* __restrict__ part, float* __restrict__ ssq, int ldp,
                                                       int kr, uint8_t* __restrict__ xl GM_TL_PARAM) {
  GM_TL_BEGIN();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int D = P.D, E = P.E, nrows = E + (P.sh_gate_inp != nullptr ? 1 : 0);
  const int z = blockIdx.y, k0 = z * kr + 8 * lane;
  const bool lv = 8 * lane < kr;
  const int kk = lv ? k0 : z * kr;                              // lanes past the range re-read its start
  const int row = blockIdx.x * 4 + wave;
  const void* wr = row < E ? router_row<RF32>(P.router, row, D) : (row < nrows ? P.sh_gate_inp : P.router);
  RouterChunk<RF32> wb;
  router_load8<RF32, false>(wr, kk, wb);
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
  float w[8];
  router_unpack8<RF32>(wb, w);
  const int nb = gridDim.x, b0 = blockIdx.x;
  if (wave == 0) {                                              // uniform per wave
    const int rbytes = gm_limb_row_bytes(D);
#pragma unroll
    for (int m = 0; m < NT; ++m) {
      if (m < T && m % nb == b0) {
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
      if (m % nb == b0 && wave == 0) {
        q = gm_wave_sum64(lv ? q : 0.f);
        if (lane == 0) ssq[z * T + m] = q;
      }
    }
  }
  GM_TL_END(4);
}

template <bool RF32>
int launch_router_t(const gm_moe_layer* P, const float* x, int T, const GmDecArgs& a, hipStream_t s, bool fast1) {
  const int nrows = P->E + (P->sh_gate_inp ? 1 : 0);
  if (!fast1) {                                                      // router partials only
    const int kr = gm_dec_kr(P->D);
    hipLaunchKernelGGL((k_dec_router_ks<8, RF32>), dim3((nrows + 3) / 4, P->D / kr), dim3(256), 0, s, *P, x, T,
                       a.part, a.ssq, gm_dec_part_ld(P), kr, a.xl GM_TL_ARG(a.tl));
    GM_TRY(hipGetLastError());
    return GM_OK;
  }
  // limb waves (not with the accumulators), then one wave per row
  const int nl = a.acc != nullptr ? 0 : (P->D + 511) / 512;
  const dim3 grid((nrows + nl + 1) / 2);
  uint8_t* xl = a.acc != nullptr ? nullptr : a.xl;
  const int ld = gm_acc_ld(P->E);
#define GM_R1(n) hipLaunchKernelGGL((k_dec_router1<n, RF32>), grid, dim3(128), 0, s, *P, x, a.logits, a.shg, xl, \
                                    a.acc, ld GM_TL_ARG(a.tl))
  switch ((P->D + 511) / 512) {
    case 1: GM_R1(1); break;
    case 2: GM_R1(2); break;
    case 3: GM_R1(3); break;
    case 4: GM_R1(4); break;
    case 5: GM_R1(5); break;
    case 6: GM_R1(6); break;
    case 7: GM_R1(7); break;
    default: GM_R1(8); break;
  }
#undef GM_R1
  GM_TRY(hipGetLastError());
  return GM_OK;
}

int launch_router(const gm_moe_layer* P, const float* x, int T, const GmDecArgs& a, hipStream_t s, bool fast1) {
  return P->q_router == GM_QTYPE_F32 ? launch_router_t<true>(P, x, T, a, s, fast1)
                                     : launch_router_t<false>(P, x, T, a, s, fast1);
}

}  // namespace

bool gm_dec_chain_ok(const gm_moe_layer* P) {
  const bool fast1 = P->FF == 256 || P->FF == 512 ||
                     (P->FF == 1024 && P->q_down != GM_QTYPE_BF16 && P->q_down != GM_QTYPE_I8);
  const int nblk = P->k * (P->FF / 16);
  return fast1 && P->FF % 16 == 0 && nblk >= 192 && nblk <= 1024 && (!P->gate_sh || P->FF_sh <= 2 * nblk);
}

int gm_dec_run(const gm_moe_layer* P, const float* x, float* y, int T, int flags, uint8_t* ws,
                  const GmMoeWs& lay, hipStream_t s, int stage, const GmChainStep* cs) {
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
  // rows of x w_norm live in yp, which stage 3 overwrites only after stage 2;
  // in a T > 1 chain the previous layer's combine kernel wrote them (256-column
  // ranges) unless this is the chain's first layer
  const bool linked_in = cs != nullptr && T > 1 && !cs->router;
  a.nz = linked_in ? gm_dec_link_nz(P->D) : gm_dec_nz(P->D);
  if (!gm_dec_part_ptrs(P, T, a.nz, ws, lay, &a.part, &a.ssq, &a.rms, &a.xl))
    return gm_fail_arg("gm_moe_forward: internal workspace layout error (yp)");
  if (a.hsh != a.h + (size_t)T * P->k * P->FF) return gm_fail_arg("gm_moe_forward: internal workspace layout error");
  // The T = 1 down kernel stages (k + 1) rows of FF activations per block and
  // maps a wave's lanes onto 8 rows x FF/32 sub-blocks (FF/32 in {8, 16, 32}).
  // (bf16 and I8 routed down rows fit the down kernel's LDS slices up to FF = 512)
  const bool fast1 = T == 1 && (P->FF == 256 || P->FF == 512 ||
                                (P->FF == 1024 && P->q_down != GM_QTYPE_BF16 && P->q_down != GM_QTYPE_I8));
  // T = 1 shapes of k_dec_gateup1w: the router kernel writes raw dot products
  // into the accumulators of buffer 0 (in a chain: the buffers cs names)
  a.acc = nullptr;
  a.acc_zero = nullptr;
  const GmNextRouter* next = nullptr;
  const GmNextB8* next8 = nullptr;
  bool run_router = stage == 0 || stage == 1;
  if (cs != nullptr && T > 1) {
    if (stage != 0 || (a.nz > GM_DEC_MAX_NZ)) return gm_fail_arg("gm_moe_chain: internal error (linked step)");
    next8 = cs->next8;
    run_router = cs->router;
  } else if (cs != nullptr) {
    if (!(fast1 && gm_dec_chain_ok(P)) || stage != 0) return gm_fail_arg("gm_moe_chain: internal error (chain step)");
    a.acc = cs->acc;
    a.acc_zero = cs->acc_zero;
    next = cs->next;
    run_router = cs->router;
  } else if (fast1 && gm_dec_chain_ok(P)) {
    a.acc = reinterpret_cast<double*>(ws + lay.acc);
  }
  if (run_router)
    if (int rc = launch_router(P, x, T, a, s, fast1)) return rc;
  if (stage == 0 || stage == 2)
    if (int rc = gm_dec_gateup(P, x, T, fast1, a, s)) return rc;
  if (stage == 0 || stage == 3)
    if (int rc = gm_dec_down(P, x, y, T, flags, fast1, a, s, next, next8)) return rc;
  return GM_OK;
}

bool gm_dec_part_fits(const gm_moe_layer* P, int T, int nz) {
  const size_t words = (size_t)nz * T * gm_dec_part_ld(P) + (size_t)GM_DEC_MAX_NZ * T + 16;
  return words * sizeof(float) + (size_t)(T + 1) * gm_limb_row_bytes(P->D) <= (size_t)(T * P->k + T) * P->D * sizeof(float);
}

bool gm_dec_part_ptrs(const gm_moe_layer* P, int T, int nz, uint8_t* ws, const GmMoeWs& lay, float** part,
                      float** ssq, float** rms, uint8_t** xl) {
  float* yp = reinterpret_cast<float*>(ws + lay.yp);
  *part = yp;
  *ssq = *part + (size_t)nz * T * gm_dec_part_ld(P);
  *rms = *ssq + GM_DEC_MAX_NZ * T;
  *xl = reinterpret_cast<uint8_t*>(*rms + 16);
  return gm_dec_part_fits(P, T, nz);
}
