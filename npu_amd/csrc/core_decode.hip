// One decode token through the Qwen3-Next core layers that sit beside the MoE
// block in every decoder layer (qwen/forward.py:834-893): gated attention
// (:133-239) and the Gated DeltaNet SSM (:292-431).  fp32 state and
// activations; the large projections are bf16 weights (the reference's NPU
// operators for these sites stage bf16, qwen/forward.py:813-831) on the bf16
// matvec kernels of mv_bf16.hip, the small alpha / beta projections fp32.
//
// Attention, one token at position pos (gm_attn_decode):
//   mv_bf16 (+norm)  qkv = Wqkv rmsnorm(x, attn_norm) ([q_h | gate_h] per head,
//                    then k, then v); the norm is formed while x is staged
//   k_attn_prep      per head: RMSNorm of q / k over head_dim, partial RoPE at
//                    pos; k and v written to the caches at row pos
//   k_attn_part      per (q head, chunk of cached positions): online softmax
//                    partials (max, sum, weighted v) of q . k / sqrt(Dh); for
//                    rope_dim <= 64 (a power of two) it also does k_attn_prep's
//                    work and k_attn_prep is not launched
//   k_attn_combine   per q head: the partials merged, times sigmoid(gate)
//   mv_bf16 (+ x)    y = Wo out (+ x)
// Gated DeltaNet, one token (gm_ssm_decode):
//   mv_bf16 (+norm)  mixed = W_in h and z = W_gate h in one launch, h =
//                    rmsnorm(x, attn_norm) formed while x is staged
//   k_ssm_conv_ab    the depthwise causal conv (kernel conv_k) over [state,
//                    mixed], SiLU, the state shifted, q and k heads
//                    L2-normalised, q times 1/sqrt(Sk); beside it (other
//                    blocks of the launch) g = softplus(alpha h + dt_bias) a
//                    and beta = sigmoid(beta h)
//   k_ssm_rec        per (V head, 32 state columns): S = S exp(g),
//                    d = (v - S^T k) beta, S += k d^T, o = S^T q; the state
//                    [Hv][Sk][Sv] (the reference's layout) updated in place
//   k_ssm_gnorm      rmsnorm(o_head, ssm_norm) * silu(z)
//   (k_ssm_rec_gn    both in one launch, one block per V head, for d_state
//                    64 and 128)
//   mv_bf16 (+ x)    y = W_out o (+ x)
// Linked to the following MoE block (gm_attn_decode_moe / gm_ssm_decode_moe):
// the first launch also clears that block's T = 1 router accumulators, and the
// output projection adds the router dot products and the sum of squares of its
// rows of y into them (as a chain's down kernel does for the next layer), so
// the MoE block runs without its router launch.
// No kernel holds a scratch buffer of its own: intermediates live in the
// caller's workspace (gm_attn_ws_layout / gm_ssm_ws_layout).
#include "common.h"
#include "kernels.h"
#include "moe_decode.h"

namespace {

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

constexpr int kAttnChunk = 64;     // cached positions per attention partial
constexpr int kAttnNB = 8;         // positions per wave and load round (4 waves: 32 per round)

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = gm_wave_sum64(v);
  const int wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  __syncthreads();                                            // red reused across calls
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
  for (int w = 0; w < nw; ++w) s += red[w];
  return s;
}

// ------------------------------------------------------------ RMSNorm row
// y = (x * rsqrt(mean(x^2) + eps)) * w (qwen/forward.py:58-61); one block per row.
__global__ void __launch_bounds__(256) k_rms_row(const float* __restrict__ x, const float* __restrict__ w, int D,
                                                 float eps, float* __restrict__ y) {
  __shared__ float red[4];
  x += (size_t)blockIdx.x * D;
  y += (size_t)blockIdx.x * D;
  float ss = 0.f;
#pragma unroll 8
  for (int i = threadIdx.x; i < D; i += 256) ss = fmaf(x[i], x[i], ss);
  const float r = 1.0f / sqrtf(block_sum(ss, red) / (float)D + eps);
#pragma unroll 8
  for (int i = threadIdx.x; i < D; i += 256) y[i] = (x[i] * r) * w[i];
}

// ------------------------------------------------------------ attention
// One block per head, blockDim = Dh (one value per thread).  Blocks 0..Hq-1:
// q head b = qkv[2 Dh b ..] (its gate follows at + Dh), RMSNorm with q_norm,
// RoPE -> qr[b]; blocks Hq..Hq+Hkv-1: k / v head j -> the caches' row pos.
// RoPE (qwen/forward.py:81-97): lane i < rd/2 pairs with i + rd/2:
// out_i = x_i cos_i - x_{i+h} sin_i, out_{i+h} = x_{i+h} cos_{i+h} + x_i sin_{i+h}.
__global__ void k_attn_prep(const float* __restrict__ qkv, const float* __restrict__ q_norm,
                            const float* __restrict__ k_norm, float eps, int Hq, int Hkv, int Dh, int rd,
                            const float* __restrict__ cosr, const float* __restrict__ sinr,
                            float* __restrict__ qr, float* __restrict__ kc, float* __restrict__ vc) {
  extern __shared__ float sm[];                                 // [Dh] normalised row + [16] reduction
  float* row = sm;
  float* red = sm + Dh;
  const int b = blockIdx.x, i = threadIdx.x;
  const bool isq = b < Hq;
  const float* src = isq ? qkv + (size_t)2 * Dh * b : qkv + (size_t)2 * Dh * Hq + (size_t)Dh * (b - Hq);
  const float v = src[i];
  const float r = 1.0f / sqrtf(block_sum(v * v, red) / (float)Dh + eps);
  const float n = (v * r) * (isq ? q_norm[i] : k_norm[i]);
  row[i] = n;
  __syncthreads();
  float o = n;
  const int h = rd >> 1;
  if (i < rd) {
    const float other = i < h ? -row[i + h] : row[i - h];
    o = n * cosr[i] + other * sinr[i];
  }
  if (isq) {
    qr[(size_t)Dh * b + i] = o;
  } else {
    const int j = b - Hq;
    kc[(size_t)Dh * j + i] = o;
    vc[(size_t)Dh * j + i] = qkv[(size_t)2 * Dh * Hq + (size_t)Dh * Hkv + (size_t)Dh * j + i];
  }
}

// Partial attention of q head hq over cached positions [c0, c0 + kAttnChunk)
// (clipped to n = pos + 1): 4 waves, each lane holding DV = Dh / 64 dims; wave
// w takes positions c0 + w, c0 + w + 4, ...  Per position the score
// s = (q . k) / sqrt(Dh) (a wave sum), then the online softmax update
// m' = max(m, s), l = l e^(m - m') + e^(s - m'), acc = acc e^(m - m') + e^(s - m') v.
// The 4 waves' states are merged in LDS; part[hq][chunk] = {m, l, acc[Dh]}.
//
// With ROPE the launch also does k_attn_prep's work (rope_dim rd <= 64, rd / 2
// a power of two): every wave forms its head's q from qkv itself, the blocks
// of the last chunk form the new k and v row at pos = n - 1 and use it for
// that position instead of the cache, and the first q head of each kv group
// writes it to the caches.
struct AttnRope {
  const float* qkv;
  const float* q_norm;
  const float* k_norm;
  float eps;
  int rd;
  const float* cosr;   // at pos
  const float* sinr;
};

// One head row of qkv (DV values per lane), RMSNorm'd with nw over 64 DV
// values, then the partial RoPE on dims i < rd (partner i ^ (rd / 2), in the
// same wave); as k_attn_prep forms it.
template <int DV>
__device__ __forceinline__ void rope_head(const float* __restrict__ src, const float* __restrict__ nw,
                                          const AttnRope& rp, float (&out)[DV]) {
  const int lane = threadIdx.x & 63;
  float v[DV];
#pragma unroll
  for (int d = 0; d < DV; ++d) v[d] = src[lane + 64 * d];
  float ss = 0.f;
#pragma unroll
  for (int d = 0; d < DV; ++d) ss = fmaf(v[d], v[d], ss);
  const float r = 1.0f / sqrtf(gm_wave_sum64(ss) / (float)(64 * DV) + rp.eps);
#pragma unroll
  for (int d = 0; d < DV; ++d) out[d] = (v[d] * r) * nw[lane + 64 * d];
  const int h = rp.rd >> 1;
  const float other = __shfl_xor(out[0], h, 64);
  if (lane < rp.rd) out[0] = out[0] * rp.cosr[lane] + (lane < h ? -other : other) * rp.sinr[lane];
}

template <int DV, bool ROPE>
__global__ void __launch_bounds__(256) k_attn_part(const float* __restrict__ qr, float* __restrict__ kc,
                                                   float* __restrict__ vc, int Hq, int Hkv, int n,
                                                   float scale, float* __restrict__ part, int ld, AttnRope rp) {
  __shared__ float ms[4], ls[4];
  __shared__ float accs[4][64 * DV];
  const int hq = blockIdx.x, chunk = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int Dh = 64 * DV, hk = hq / (Hq / Hkv), c0 = chunk * kAttnChunk;
  const int c1 = min(c0 + kAttnChunk, n);
  float q[DV], acc[DV], kp[DV], vp[DV];
#pragma unroll
  for (int d = 0; d < DV; ++d) { acc[d] = 0.f; kp[d] = 0.f; vp[d] = 0.f; }
  const bool last = c1 == n;                                     // this chunk holds pos = n - 1
  if constexpr (ROPE) {
    rope_head<DV>(rp.qkv + (size_t)2 * Dh * hq, rp.q_norm, rp, q);
    if (last) {
      const float* kv0 = rp.qkv + (size_t)2 * Dh * Hq;
      rope_head<DV>(kv0 + (size_t)Dh * hk, rp.k_norm, rp, kp);
#pragma unroll
      for (int d = 0; d < DV; ++d) vp[d] = kv0[(size_t)Dh * Hkv + (size_t)Dh * hk + lane + 64 * d];
      if (hq % (Hq / Hkv) == 0 && wave == 0) {
        float* kr = kc + ((size_t)(n - 1) * Hkv + hk) * Dh;
        float* vr = vc + ((size_t)(n - 1) * Hkv + hk) * Dh;
#pragma unroll
        for (int d = 0; d < DV; ++d) { kr[lane + 64 * d] = kp[d]; vr[lane + 64 * d] = vp[d]; }
      }
    }
  } else {
#pragma unroll
    for (int d = 0; d < DV; ++d) q[d] = qr[(size_t)Dh * hq + lane + 64 * d];
  }
  float m = -__builtin_inff(), l = 0.f;
  // kAttnNB positions per round, every k / v load of the round issued before
  // the first use; positions past c1 reload the last one and leave the state
  // unchanged (selects, so no branch separates a load from its use)
  for (int t0 = c0 + wave; t0 < c1; t0 += 4 * kAttnNB) {
    float kv[kAttnNB][DV], vv[kAttnNB][DV];
#pragma unroll
    for (int j = 0; j < kAttnNB; ++j) {
      const int t = t0 + 4 * j, tc = t < c1 ? t : c1 - 1;
      const float* kt = kc + ((size_t)tc * Hkv + hk) * Dh;
      const float* vt = vc + ((size_t)tc * Hkv + hk) * Dh;
#pragma unroll
      for (int d = 0; d < DV; ++d) { kv[j][d] = kt[lane + 64 * d]; vv[j][d] = vt[lane + 64 * d]; }
    }
#pragma unroll
    for (int j = 0; j < kAttnNB; ++j) {
      const bool live = t0 + 4 * j < c1;                         // wave-uniform
      if (ROPE && t0 + 4 * j == n - 1) {                        // the new row, formed above
#pragma unroll
        for (int d = 0; d < DV; ++d) { kv[j][d] = kp[d]; vv[j][d] = vp[d]; }
      }
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < DV; ++d) s = fmaf(q[d], kv[j][d], s);
      s = gm_wave_sum64(s) * scale;
      const float mn = fmaxf(m, s);
      const float a = expf(m - mn), p = expf(s - mn);
      l = live ? l * a + p : l;
#pragma unroll
      for (int d = 0; d < DV; ++d) acc[d] = live ? fmaf(acc[d], a, p * vv[j][d]) : acc[d];
      m = live ? mn : m;
    }
  }
  if (lane == 0) { ms[wave] = m; ls[wave] = l; }
#pragma unroll
  for (int d = 0; d < DV; ++d) accs[wave][lane + 64 * d] = acc[d];
  __syncthreads();
  if (wave == 0) {
    const float M = fmaxf(fmaxf(ms[0], ms[1]), fmaxf(ms[2], ms[3]));
    float f[4], L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) { f[w] = ms[w] == -__builtin_inff() ? 0.f : expf(ms[w] - M); L = fmaf(ls[w], f[w], L); }
    float* out = part + ((size_t)hq * ld + chunk) * (Dh + 2);
#pragma unroll
    for (int d = 0; d < DV; ++d) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) o = fmaf(accs[w][lane + 64 * d], f[w], o);
      out[2 + lane + 64 * d] = o;
    }
    if (lane == 0) { out[0] = M; out[1] = L; }
  }
}

// out[hq][i] = (sum_c acc_c[i] e^(m_c - M)) / (sum_c l_c e^(m_c - M)) * sigmoid(gate);
// one block per q head, blockDim = Dh.  Both loops over the chunks run unrolled
// (8 chunks' loads issued before their first use; a rolled loop waited one
// round trip per chunk: 265-268 against 245-246 us per eager attention step at
// position 4096, unchanged at 64).
__global__ void k_attn_combine(const float* __restrict__ part, int ld, int nch, const float* __restrict__ qkv,
                               int Dh, float* __restrict__ out) {
  const int hq = blockIdx.x, i = threadIdx.x;
  const float* p = part + (size_t)hq * ld * (Dh + 2);
  float M = -__builtin_inff();
#pragma unroll 8
  for (int c = 0; c < nch; ++c) M = fmaxf(M, p[(size_t)c * (Dh + 2)]);
  float L = 0.f, o = 0.f;
#pragma unroll 8
  for (int c = 0; c < nch; ++c) {
    const float* pc = p + (size_t)c * (Dh + 2);
    const float f = expf(pc[0] - M);
    L = fmaf(pc[1], f, L);
    o = fmaf(pc[2 + i], f, o);
  }
  const float g = qkv[(size_t)2 * Dh * hq + Dh + i];
  out[(size_t)Dh * hq + i] = (o / L) * (1.0f / (1.0f + expf(-g)));
}

// ------------------------------------------------------------ Gated DeltaNet
// One launch, two kinds of block (blockDim = Sk; block-uniform roles):
// blocks [0, C / Sk), one per group of Sk channels: the depthwise causal conv
// out_c = sum_j w[c][j] in_c[j] over in_c = [state_c[0 .. ck-2], mixed_c],
// SiLU; the state shifted by one (mixed_c last).  Groups 0..Hk-1 (q heads) and
// Hk..2Hk-1 (k heads) are L2-normalised (x / sqrt(max(sum x^2, eps))), q then
// times 1/sqrt(Sk).
// Blocks [C / Sk, ...): one wave per alpha / beta row (rows 0..Hv-1 alpha,
// Hv..2Hv-1 beta, fp32 weights [Hv][D]) on h = (x * rsqrt(mean(x^2) + eps)) *
// attn_norm, which each wave forms from x itself: g = softplus(alpha . h +
// dt_bias) * a (torch's softplus: x above 20 passes through, else
// log1p(exp(x))), beta = sigmoid(beta . h).
__global__ void __launch_bounds__(256) k_ssm_conv_ab(const float* __restrict__ mixed, const float* __restrict__ w, float* __restrict__ state,
                              int ck, int Hk, int Sk, float eps, float* __restrict__ conv, int nconv,
                              const float* __restrict__ alpha, const float* __restrict__ beta,
                              const float* __restrict__ dt_bias, const float* __restrict__ a,
                              const float* __restrict__ x, const float* __restrict__ norm_w, int D, int Hv,
                              float* __restrict__ gb) {
  __shared__ float red[16];
  if ((int)blockIdx.x < nconv) {
    const int c = blockIdx.x * Sk + threadIdx.x, g = blockIdx.x;
    float* st = state + (size_t)c * (ck - 1);
    const float* wc = w + (size_t)c * ck;
    // the channel's weights and state in registers, every load issued before the
    // first use (ck <= 8; indices past the kernel reload the last entry)
    constexpr int KMAX = 8;
    const float xin = mixed[c];
    float wv[KMAX], sv[KMAX - 1];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) wv[j] = wc[j < ck ? j : ck - 1];
#pragma unroll
    for (int j = 0; j < KMAX - 1; ++j) sv[j] = ck > 1 ? st[j < ck - 1 ? j : ck - 2] : 0.f;
    float acc = 0.f, wl = wv[0];
#pragma unroll
    for (int j = 0; j < KMAX - 1; ++j)
      if (j < ck - 1) acc = fmaf(wv[j], sv[j], acc);
#pragma unroll
    for (int j = 1; j < KMAX; ++j) wl = j == ck - 1 ? wv[j] : wl;
    acc = fmaf(wl, xin, acc);
#pragma unroll
    for (int j = 0; j < KMAX - 1; ++j)
      if (j < ck - 1) st[j] = j + 1 < ck - 1 ? sv[j + 1] : xin;
    float v = acc / (1.0f + expf(-acc));
    if (g < 2 * Hk) {                                            // block-uniform
      const float ss = block_sum(v * v, red);
      v = v / sqrtf(fmaxf(ss, eps));
      if (g < Hk) v = v * (1.0f / sqrtf((float)Sk));
    }
    conv[c] = v;
    return;
  }
  const int lane = threadIdx.x & 63;
  const int r = ((int)blockIdx.x - nconv) * ((int)blockDim.x >> 6) + (int)(threadIdx.x >> 6);
  if (r >= 2 * Hv) return;
  // alpha . h = rs (alpha . (x * norm_w)): one pass over x, the row and the norm
  // weight in float4s, every load of a round (8 per lane and array) issued
  // before the first use (D % 32 == 0; lanes past D reload the last float4
  // and add nothing)
  const gm_f32x4* x4 = reinterpret_cast<const gm_f32x4*>(x);
  const gm_f32x4* n4 = reinterpret_cast<const gm_f32x4*>(norm_w);
  const gm_f32x4* w4 = reinterpret_cast<const gm_f32x4*>(r < Hv ? alpha + (size_t)r * D : beta + (size_t)(r - Hv) * D);
  const int d4 = D >> 2;
  float ss = 0.f, sd = 0.f;
  for (int i0 = 0; i0 < d4; i0 += 64 * 8) {
    gm_f32x4 xv[8], wv[8], nv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + lane + 64 * u, ic = i < d4 ? i : d4 - 1;
      xv[u] = x4[ic];
      wv[u] = w4[ic];
      nv[u] = n4[ic];
    }
    __builtin_amdgcn_sched_barrier(0);                           // all 24 loads before the first use
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const bool live = i0 + lane + 64 * u < d4;
      const gm_f32x4 xn = xv[u] * nv[u];
      const float q = fmaf(xv[u].x, xv[u].x, fmaf(xv[u].y, xv[u].y, fmaf(xv[u].z, xv[u].z, xv[u].w * xv[u].w)));
      const float t = fmaf(wv[u].x, xn.x, fmaf(wv[u].y, xn.y, fmaf(wv[u].z, xn.z, wv[u].w * xn.w)));
      ss += live ? q : 0.f;
      sd += live ? t : 0.f;
    }
  }
  const float rs = 1.0f / sqrtf(gm_wave_sum64(ss) / (float)D + eps);
  sd = rs * gm_wave_sum64(sd);
  if (lane == 0) {
    if (r < Hv) {
      const float u = sd + dt_bias[r];
      gb[r] = (u > 20.f ? u : log1pf(expf(u))) * a[r];
    } else {
      gb[r] = 1.0f / (1.0f + expf(-sd));
    }
  }
}

// Delta rule for V head hv, state columns v0 .. v0 + 31 (blockDim = 32 x KG):
// thread (kg, col) holds rows kg SPT .. + SPT - 1 of column col of
// S[hv][k][v] (row-major [Sk][Sv], the reference's layout).  K / Q head
// hv % Hk (the reference tiles the Hk heads over the Hv heads).
template <int SPT>
__global__ void __launch_bounds__(256) k_ssm_rec(float* __restrict__ S, const float* __restrict__ conv,
                                                 const float* __restrict__ gb, int Hk, int Hv, int Sk, int Sv,
                                                 float* __restrict__ o) {
  __shared__ float red[8][33];
  __shared__ float dsh[32];
  const int hv = blockIdx.x, col = threadIdx.x & 31, kg = threadIdx.x >> 5, v = blockIdx.y * 32 + col;
  const int hk = hv % Hk, Ck = Hk * Sk;
  const float* q = conv + (size_t)hk * Sk;
  const float* k = conv + (size_t)Ck + (size_t)hk * Sk;
  const float vv = conv[(size_t)2 * Ck + (size_t)hv * Sv + v];
  const float decay = expf(gb[hv]), bt = gb[Hv + hv];
  float* Sc = S + (size_t)hv * Sk * Sv + v;
  float s[SPT], kk[SPT], qq[SPT];
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    const int r = kg * SPT + j;
    s[j] = Sc[(size_t)r * Sv] * decay;
    kk[j] = k[r];
    qq[j] = q[r];
  }
  float p = 0.f;
#pragma unroll
  for (int j = 0; j < SPT; ++j) p = fmaf(s[j], kk[j], p);
  red[kg][col] = p;
  __syncthreads();
  if (kg == 0) {
    float sk = 0.f;
    for (int g = 0; g < 8; ++g) sk += red[g][col];
    dsh[col] = (vv - sk) * bt;
  }
  __syncthreads();
  const float d = dsh[col];
  p = 0.f;
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    s[j] = fmaf(kk[j], d, s[j]);
    Sc[(size_t)(kg * SPT + j) * Sv] = s[j];
    p = fmaf(s[j], qq[j], p);
  }
  __syncthreads();
  red[kg][col] = p;
  __syncthreads();
  if (kg == 0) {
    float ov = 0.f;
    for (int g = 0; g < 8; ++g) ov += red[g][col];
    o[(size_t)hv * Sv + v] = ov;
  }
}

// The delta rule of k_ssm_rec and the gated norm of k_ssm_gnorm for a whole V
// head in one block (Sk == Sv == SV, blockDim = 1024 = SV columns x KG row
// groups of SPT state rows): the head's SV outputs o end up in the first SV
// threads, which form rmsnorm(o, ssm_norm) * silu(z) directly.
template <int SV>
__global__ void __launch_bounds__(1024) k_ssm_rec_gn(float* __restrict__ S, const float* __restrict__ conv,
                                                     const float* __restrict__ gb, int Hk, int Hv,
                                                     const float* __restrict__ nw, const float* __restrict__ z,
                                                     float eps, float* __restrict__ out) {
  constexpr int KG = 1024 / SV, SPT = SV / KG;
  __shared__ float red[KG][SV + 1];
  __shared__ float dsh[SV];
  __shared__ float wred[SV / 64];
  const int hv = blockIdx.x, col = threadIdx.x % SV, kg = threadIdx.x / SV;
  const int hk = hv % Hk, Ck = Hk * SV;
  const float* q = conv + (size_t)hk * SV;
  const float* k = conv + (size_t)Ck + (size_t)hk * SV;
  const float vv = conv[(size_t)2 * Ck + (size_t)hv * SV + col];
  const float decay = expf(gb[hv]), bt = gb[Hv + hv];
  const size_t oi = (size_t)hv * SV + col;
  const float zi = kg == 0 ? z[oi] : 0.f, nwc = kg == 0 ? nw[col] : 0.f;
  float* Sc = S + (size_t)hv * SV * SV + col;
  float s[SPT], kk[SPT], qq[SPT];
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    const int r = kg * SPT + j;
    s[j] = Sc[(size_t)r * SV] * decay;
    kk[j] = k[r];
    qq[j] = q[r];
  }
  float p = 0.f;
#pragma unroll
  for (int j = 0; j < SPT; ++j) p = fmaf(s[j], kk[j], p);
  red[kg][col] = p;
  __syncthreads();
  if (kg == 0) {
    float sk = 0.f;
    for (int g = 0; g < KG; ++g) sk += red[g][col];
    dsh[col] = (vv - sk) * bt;
  }
  __syncthreads();
  const float d = dsh[col];
  p = 0.f;
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    s[j] = fmaf(kk[j], d, s[j]);
    Sc[(size_t)(kg * SPT + j) * SV] = s[j];
    p = fmaf(s[j], qq[j], p);
  }
  __syncthreads();
  red[kg][col] = p;
  __syncthreads();
  float ov = 0.f;
  if (kg == 0)
    for (int g = 0; g < KG; ++g) ov += red[g][col];
  // the first SV threads (SV / 64 whole waves) hold the head's outputs
  const float sq = gm_wave_sum64(kg == 0 ? ov * ov : 0.f);
  if ((threadIdx.x & 63) == 0 && (int)threadIdx.x < SV) wred[threadIdx.x >> 6] = sq;
  __syncthreads();
  if (kg == 0) {
    float ss = 0.f;
#pragma unroll
    for (int w = 0; w < SV / 64; ++w) ss += wred[w];
    const float r = 1.0f / sqrtf(ss / (float)SV + eps);
    out[oi] = ((ov * r) * nwc) * (zi / (1.0f + expf(-zi)));
  }
}

// rmsnorm(o_head, ssm_norm) * silu(z) per V head (blockDim = Sv).
__global__ void k_ssm_gnorm(const float* __restrict__ o, const float* __restrict__ nw, const float* __restrict__ z,
                            int Sv, float eps, float* __restrict__ out) {
  __shared__ float red[16];
  const size_t i = (size_t)blockIdx.x * Sv + threadIdx.x;
  const float v = o[i];
  const float r = 1.0f / sqrtf(block_sum(v * v, red) / (float)Sv + eps);
  const float zi = z[i];
  out[i] = ((v * r) * nw[threadIdx.x]) * (zi / (1.0f + expf(-zi)));
}

}  // namespace

// ------------------------------------------------------------ host side
GmAttnWs gm_attn_ws_layout(const gm_attn_layer* L, int max_pos) {
  GmAttnWs w{};
  size_t o = 0;
  const size_t Dh = (size_t)L->head_dim, Hq = (size_t)L->n_head, Hkv = (size_t)L->n_head_kv;
  const size_t nch = ((size_t)max_pos + kAttnChunk - 1) / kAttnChunk;
  w.h = o; o = align256(o + (size_t)L->D * 4);
  w.qkv = o; o = align256(o + (2 * Hq + 2 * Hkv) * Dh * 4);
  w.qr = o; o = align256(o + Hq * Dh * 4);
  w.part = o; o = align256(o + Hq * nch * (Dh + 2) * 4);
  w.out = o; o = align256(o + Hq * Dh * 4);
  w.nch = (int)nch;
  w.total = o;
  return w;
}

int gm_attn_run(const gm_attn_layer* L, const float* x, float* y, float* kc, float* vc, int pos, int max_pos,
                const float* cosr, const float* sinr, int flags, uint8_t* ws, hipStream_t s, const GmNextRouter* moe) {
  const GmAttnWs lay = gm_attn_ws_layout(L, max_pos);
  const int D = L->D, Hq = L->n_head, Hkv = L->n_head_kv, Dh = L->head_dim, rd = L->rope_dim;
  float* qkv = reinterpret_cast<float*>(ws + lay.qkv);
  float* qr = reinterpret_cast<float*>(ws + lay.qr);
  float* part = reinterpret_cast<float*>(ws + lay.part);
  float* out = reinterpret_cast<float*>(ws + lay.out);
  const int Mqkv = (2 * Hq + 2 * Hkv) * Dh;
  if (int rc = gm_launch_mv_bf16_norm2(static_cast<const uint16_t*>(L->wqkv), Mqkv, nullptr, 0, D, x, L->attn_norm,
                                       L->eps, qkv, nullptr, s, moe ? moe->acc : nullptr,
                                       moe ? GM_ACC_COPIES * moe->ld : 0))
    return rc;
  const int n = pos + 1, nch = (n + kAttnChunk - 1) / kAttnChunk;
  const float scale = 1.0f / sqrtf((float)Dh);
  const dim3 g(Hq, nch);
  float* kpos = kc + (size_t)pos * Hkv * Dh;
  float* vpos = vc + (size_t)pos * Hkv * Dh;
  const float* cp = cosr + (size_t)pos * rd;
  const float* sp = sinr + (size_t)pos * rd;
  // q / k norm and RoPE inside the partial launch when the rotated pairs sit in one wave
  const bool fused = rd >= 2 && rd <= 64 && ((rd >> 1) & ((rd >> 1) - 1)) == 0;
  const AttnRope rp{qkv, L->q_norm, L->k_norm, L->eps, rd, cp, sp};
  if (!fused) {
    hipLaunchKernelGGL(k_attn_prep, dim3(Hq + Hkv), dim3(Dh), (Dh + 16) * sizeof(float), s, qkv, L->q_norm,
                       L->k_norm, L->eps, Hq, Hkv, Dh, rd, cp, sp, qr, kpos, vpos);
    GM_TRY(hipGetLastError());
  }
#define GM_AP(DV)                                                                                              \
  if (fused) hipLaunchKernelGGL((k_attn_part<DV, true>), g, dim3(256), 0, s, qr, kc, vc, Hq, Hkv, n, scale, part, \
                                lay.nch, rp);                                                                  \
  else hipLaunchKernelGGL((k_attn_part<DV, false>), g, dim3(256), 0, s, qr, kc, vc, Hq, Hkv, n, scale, part,    \
                          lay.nch, rp);                                                                        \
  break;
  switch (Dh / 64) {
    case 1: GM_AP(1)
    case 2: GM_AP(2)
    case 4: GM_AP(4)
    default: GM_AP(8)
  }
#undef GM_AP
  GM_TRY(hipGetLastError());
  hipLaunchKernelGGL(k_attn_combine, dim3(Hq), dim3(Dh), 0, s, part, lay.nch, nch, qkv, Dh, out);
  GM_TRY(hipGetLastError());
  return gm_launch_mv_bf16_add(static_cast<const uint16_t*>(L->wo), D, Hq * Dh, out, y,
                               (flags & GM_MOE_RESIDUAL) ? x : nullptr, s, moe);
}

GmSsmWs gm_ssm_ws_layout(const gm_ssm_layer* L) {
  GmSsmWs w{};
  size_t o = 0;
  const size_t Ck = (size_t)L->n_k_heads * L->d_state, di = (size_t)L->n_v_heads * L->d_state;
  const size_t C = 2 * Ck + di;
  w.h = o; o = align256(o + (size_t)L->D * 4);
  w.mixed = o; o = align256(o + C * 4);
  w.z = o; o = align256(o + di * 4);
  w.gb = o; o = align256(o + 2 * (size_t)L->n_v_heads * 4);
  w.conv = o; o = align256(o + C * 4);
  w.o = o; o = align256(o + di * 4);
  w.o2 = o; o = align256(o + di * 4);
  w.total = o;
  return w;
}

int gm_ssm_run(const gm_ssm_layer* L, const float* x, float* y, float* conv_state, float* rec_state, int flags,
               uint8_t* ws, hipStream_t s, const GmNextRouter* moe) {
  const GmSsmWs lay = gm_ssm_ws_layout(L);
  const int D = L->D, Hk = L->n_k_heads, Hv = L->n_v_heads, Sk = L->d_state, Sv = L->d_state;
  const int Ck = Hk * Sk, di = Hv * Sv, C = 2 * Ck + di;
  float* mixed = reinterpret_cast<float*>(ws + lay.mixed);
  float* z = reinterpret_cast<float*>(ws + lay.z);
  float* gb = reinterpret_cast<float*>(ws + lay.gb);
  float* conv = reinterpret_cast<float*>(ws + lay.conv);
  float* o = reinterpret_cast<float*>(ws + lay.o);
  float* o2 = reinterpret_cast<float*>(ws + lay.o2);
  if (int rc = gm_launch_mv_bf16_norm2(static_cast<const uint16_t*>(L->w_in), C,
                                       static_cast<const uint16_t*>(L->w_gate), di, D, x, L->attn_norm, L->eps, mixed,
                                       z, s, moe ? moe->acc : nullptr, moe ? GM_ACC_COPIES * moe->ld : 0))
    return rc;
  const int nconv = C / Sk, nab = (2 * Hv + Sk / 64 - 1) / (Sk / 64);
  hipLaunchKernelGGL(k_ssm_conv_ab, dim3(nconv + nab), dim3(Sk), 0, s, mixed, L->conv1d, conv_state, L->conv_k, Hk,
                     Sk, L->eps, conv, nconv, L->alpha, L->beta, L->dt_bias, L->a, x, L->attn_norm, D, Hv, gb);
  GM_TRY(hipGetLastError());
  if (Sk == Sv && (Sv == 64 || Sv == 128)) {         // delta rule and gated norm in one launch
    if (Sv == 128)
      hipLaunchKernelGGL(k_ssm_rec_gn<128>, dim3(Hv), dim3(1024), 0, s, rec_state, conv, gb, Hk, Hv, L->ssm_norm, z,
                         L->eps, o2);
    else
      hipLaunchKernelGGL(k_ssm_rec_gn<64>, dim3(Hv), dim3(1024), 0, s, rec_state, conv, gb, Hk, Hv, L->ssm_norm, z,
                         L->eps, o2);
    GM_TRY(hipGetLastError());
    return gm_launch_mv_bf16_add(static_cast<const uint16_t*>(L->w_out), D, di, o2, y,
                                 (flags & GM_MOE_RESIDUAL) ? x : nullptr, s, moe);
  }
  const dim3 g(Hv, Sv / 32);
  switch (Sk / 8) {
    case 8: hipLaunchKernelGGL(k_ssm_rec<8>, g, dim3(256), 0, s, rec_state, conv, gb, Hk, Hv, Sk, Sv, o); break;
    case 16: hipLaunchKernelGGL(k_ssm_rec<16>, g, dim3(256), 0, s, rec_state, conv, gb, Hk, Hv, Sk, Sv, o); break;
    case 32: hipLaunchKernelGGL(k_ssm_rec<32>, g, dim3(256), 0, s, rec_state, conv, gb, Hk, Hv, Sk, Sv, o); break;
    default: return gm_fail_arg("gm_ssm_decode: d_state=%d must be 64, 128 or 256", Sk);
  }
  GM_TRY(hipGetLastError());
  hipLaunchKernelGGL(k_ssm_gnorm, dim3(Hv), dim3(Sv), 0, s, o, L->ssm_norm, z, Sv, L->eps, o2);
  GM_TRY(hipGetLastError());
  return gm_launch_mv_bf16_add(static_cast<const uint16_t*>(L->w_out), D, di, o2, y,
                               (flags & GM_MOE_RESIDUAL) ? x : nullptr, s, moe);
}

int gm_launch_rms_row(const float* x, const float* w, int D, int n_rows, float eps, float* y, hipStream_t s) {
  hipLaunchKernelGGL(k_rms_row, dim3(n_rows), dim3(256), 0, s, x, w, D, eps, y);
  GM_TRY(hipGetLastError());
  return GM_OK;
}
