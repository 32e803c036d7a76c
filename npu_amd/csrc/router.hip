// Router logits (bf16 W, fp32 x, optional RMSNorm and bias) for any number of
// tokens, and the stand-alone top-k kernel behind gm_router_topk.
#include "moe_common.h"

using namespace gm_moe;

namespace {

// ---------------------------------------------------------- stand-alone top-k
template <int MAXV>
__global__ void __launch_bounds__(256) k_topk(const float* __restrict__ logits, int T, int E, int k,
                                              int32_t* __restrict__ ids, float* __restrict__ wts) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  wave_topk<MAXV>(logits + (int64_t)t * E, E, k, ids + (int64_t)t * k, wts + (int64_t)t * k);
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
  constexpr int RPS = 64 / L;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nsub = D / GM_SUB;
  const int nrows = E + (w_sh != nullptr ? 1 : 0);
  const int row = (blockIdx.x * 4 + wave) * RPS + lane / L;
  const bool live = row < nrows;
  const uint8_t* wr = row < E ? reinterpret_cast<const uint8_t*>(w_router) + (int64_t)row * D * 2
                              : reinterpret_cast<const uint8_t*>(w_sh);
  // first sub-block's weights in flight while x is staged
  const int sub0 = lane % L;
  RawBf16 r0;
  if (live && sub0 < nsub) r0 = gm_load_bf16(wr, sub0);
  stage_xn<NT>(x, t0, nt, D, norm_w, eps, xs, red);
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.f;
  if (live) {
    for (int sub = sub0; sub < nsub; sub += L) {
      const RawBf16 r = sub == sub0 ? r0 : gm_load_bf16(wr, sub);
      float wv[32];
      gm_decode_bf16(r, wv);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] += gm_dot32_il(wv, xs + t * D, sub, nsub);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = gm_lane_group_sum<L>(acc[t]);
  if (live && (lane % L) == 0) {
    for (int t = 0; t < nt; ++t) {
      if (row < E) logits[(int64_t)(t0 + t) * E + row] = acc[t] + (bias ? bias[row] : 0.f);
      else shg[t0 + t] = gm_sigmoid(acc[t]);
    }
  }
}

constexpr size_t kMaxLds = 160 * 1024;    // LDS per workgroup on gfx950

template <int L>
int launch_router_l(const uint16_t* w, const float* bias, const float* x, int T, int D, int E,
                    const uint16_t* wsh, const float* nw, float eps, float* logits, float* shg,
                    hipStream_t s) {
  constexpr int RPS = 64 / L;
  const int nrows = E + (wsh ? 1 : 0);
  const int nb = (nrows + 4 * RPS - 1) / (4 * RPS);
  const size_t smem1 = (16 + (size_t)D) * 4, smem8 = (16 + 8 * (size_t)D) * 4;
  if (T == 1 || smem8 > kMaxLds) {
    // one token per launch: x staged once (D <= 16384: at most 64 KiB + 64 B);
    // T > 1 with D > 5088, where 8 staged rows of x exceed the LDS, loops over
    // the tokens
    if (int rc = gm_set_smem(k_router_only<L, 1>, smem1)) return rc;
    for (int t = 0; t < T; ++t)
      hipLaunchKernelGGL((k_router_only<L, 1>), dim3(nb, 1), dim3(256), smem1, s, w, bias, x + (int64_t)t * D, 1, D,
                         E, wsh, nw, eps, logits + (int64_t)t * E, shg ? shg + t : nullptr);
  } else {
    if (int rc = gm_set_smem(k_router_only<L, 8>, smem8)) return rc;
    hipLaunchKernelGGL((k_router_only<L, 8>), dim3(nb, (T + 7) / 8), dim3(256), smem8, s, w, bias, x, T, D, E,
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
  if (E <= 256) hipLaunchKernelGGL(k_topk<4>, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E, k, ids, wts);
  else hipLaunchKernelGGL(k_topk<8>, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E, k, ids, wts);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

