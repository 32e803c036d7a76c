// Dequant (parity/debug) and dequant-matvec kernels for raw GGUF weights.
//
// Matvec lane mapping: one 64-lane wave works on RPS = 64/L rows at a time;
// each row is covered by L lanes, lane l taking sub-blocks l, l+L, l+2L, ...
// (L = min(64, K/32)).  Consecutive lanes read consecutive sub-blocks, so a
// wave's loads cover whole rows contiguously.  x (fp32, up to NT tokens) is
// staged in LDS; weights are decoded in registers and never written back.
#include "iq_decode.h"
#include "kernels.h"
#include "moe_common.h"

// ------------------------------------------------------------- dequant
template <int QT>
__global__ void __launch_bounds__(256) k_dequant(const uint8_t* __restrict__ raw, int64_t n_sub,
                                                 float* __restrict__ out) {
  __shared__ uint32_t grid[256];
  if constexpr (QT == GM_QTYPE_IQ3_XXS) {
    gm_stage_grid(grid);
    __syncthreads();
  }
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_sub) return;
  // Treat the buffer as one row of n_sub/8 superblocks.
  const int64_t sb = i >> 3;
  const int sub = (int)(i & 7);
  const uint8_t* blk = raw + sb * gm_block_bytes(QT);
  float wv[32];
  const auto r = gm_load_sub<QT>(blk, sub);
  const float sc = gm_decode_sub<QT>(r, sub, grid, wv);
  float4* o = reinterpret_cast<float4*>(out + i * 32);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    o[j] = make_float4(sc * wv[4 * j], sc * wv[4 * j + 1], sc * wv[4 * j + 2], sc * wv[4 * j + 3]);
}

int gm_launch_dequant(int qtype, const void* raw, int64_t n_sb, float* out, hipStream_t s) {
  const int64_t n_sub = n_sb * 8;
  const dim3 grid((unsigned)((n_sub + 255) / 256)), block(256);
  const uint8_t* p = static_cast<const uint8_t*>(raw);
  if (qtype == GM_QTYPE_IQ4_XS) hipLaunchKernelGGL(k_dequant<GM_QTYPE_IQ4_XS>, grid, block, 0, s, p, n_sub, out);
  else if (qtype == GM_QTYPE_IQ3_XXS) hipLaunchKernelGGL(k_dequant<GM_QTYPE_IQ3_XXS>, grid, block, 0, s, p, n_sub, out);
  else return gm_fail_arg("gm_dequant_f32: unsupported qtype %d", qtype);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

// ggml K-quant / Q8_0 blocks (loader path; the MoE kernels take IQ4_XS / IQ3_XXS).
// One thread per 32 outputs (one Q8_0 block, or one sub-block of a 256-weight
// K-quant block); bytes are read one at a time, so no alignment is assumed.
// Layouts (little-endian, fp16 d / dmin):
//   Q8_0  d, int8 q[32]                                 y = d q
//   Q4_K  d, dmin, scales[12], qs[128]                  y = (d sc_s) q - dmin m_s
//   Q5_K  d, dmin, scales[12], qh[32], qs[128]          q += 16 bit s of qh[l]
//   Q6_K  ql[128], qh[64], int8 sc[16], d               y = (d sc[e / 16]) (q - 32)
// Sub-block s of Q4_K / Q5_K: weights 32s .. 32s + 31 are the low (s even) or
// high (s odd) nibbles of qs[32 (s / 2) .. + 31]; its 6-bit scale and min come
// from scales[12] (s < 4: bytes s and s + 4; s >= 4: byte s + 4 plus the top
// two bits of bytes s - 4 and s).  Q6_K weight e = 128 n + 32 c + l: low four
// bits from ql[64 n + 32 (c & 1) + l] (low nibble for c < 2), high two from
// bits 2c .. 2c + 1 of qh[32 n + l].
__device__ __forceinline__ float kq_h2f(const uint8_t* p) { return gm_h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

template <int QT>
__global__ void __launch_bounds__(256) k_dequant_k(const uint8_t* __restrict__ raw, int64_t n_units,
                                                   float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_units) return;
  float* y = out + i * 32;
  if constexpr (QT == GM_QTYPE_Q8_0) {
    const uint8_t* b = raw + i * 34;
    const float d = kq_h2f(b);
#pragma unroll
    for (int l = 0; l < 32; ++l) y[l] = d * (float)(int8_t)b[2 + l];
  } else if constexpr (QT == GM_QTYPE_Q6_K) {
    const int s = (int)(i & 7);
    const uint8_t* b = raw + (i >> 3) * 210;
    const float d = kq_h2f(b + 208);
    const int n = s >> 2, c = s & 3;
    const uint8_t* ql = b + 64 * n + 32 * (c & 1);
    const uint8_t* qh = b + 128 + 32 * n;
    const float d0 = d * (float)(int8_t)b[192 + 2 * s], d1 = d * (float)(int8_t)b[193 + 2 * s];
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      const int lo = c < 2 ? (ql[l] & 15) : (ql[l] >> 4);
      const int q = (lo | (((qh[l] >> (2 * c)) & 3) << 4)) - 32;
      y[l] = (l < 16 ? d0 : d1) * (float)q;
    }
  } else {
    constexpr bool five = QT == GM_QTYPE_Q5_K;
    constexpr int NB = five ? 176 : 144;
    const int s = (int)(i & 7);
    const uint8_t* b = raw + (i >> 3) * NB;
    const float d = kq_h2f(b), dmin = kq_h2f(b + 2);
    const uint8_t* sc = b + 4;
    int scv, mv;
    if (s < 4) { scv = sc[s] & 63; mv = sc[s + 4] & 63; }
    else { scv = (sc[s + 4] & 15) | ((sc[s - 4] >> 6) << 4); mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4); }
    const float dsc = d * (float)scv, dm = dmin * (float)mv;
    const uint8_t* qs = b + (five ? 48 : 16) + 32 * (s >> 1);
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      int q = (s & 1) ? (qs[l] >> 4) : (qs[l] & 15);
      if constexpr (five) q += ((b[16 + l] >> s) & 1) << 4;
      y[l] = dsc * (float)q - dm;
    }
  }
}

int gm_launch_dequant_k(int qtype, const void* raw, int64_t n_blocks, float* out, hipStream_t s) {
  const GmKBlock kb = gm_kquant_block(qtype);
  const int64_t n_units = n_blocks * (kb.weights / 32);
  if (n_units == 0) return GM_OK;
  if (reinterpret_cast<uintptr_t>(out) % 4) return gm_fail_arg("gm_dequant_f32: out must be 4-byte aligned");
  const dim3 grid((unsigned)((n_units + 255) / 256)), block(256);
  const uint8_t* p = static_cast<const uint8_t*>(raw);
  switch (qtype) {
    case GM_QTYPE_Q8_0: hipLaunchKernelGGL(k_dequant_k<GM_QTYPE_Q8_0>, grid, block, 0, s, p, n_units, out); break;
    case GM_QTYPE_Q4_K: hipLaunchKernelGGL(k_dequant_k<GM_QTYPE_Q4_K>, grid, block, 0, s, p, n_units, out); break;
    case GM_QTYPE_Q5_K: hipLaunchKernelGGL(k_dequant_k<GM_QTYPE_Q5_K>, grid, block, 0, s, p, n_units, out); break;
    case GM_QTYPE_Q6_K: hipLaunchKernelGGL(k_dequant_k<GM_QTYPE_Q6_K>, grid, block, 0, s, p, n_units, out); break;
    default: return gm_fail_arg("gm_dequant_f32: unsupported qtype %d", qtype);
  }
  GM_TRY(hipGetLastError());
  return GM_OK;
}

// K-quant / Q8_0 rows -> I8 rows (GM_QTYPE_I8), one thread per 32-weight
// sub-block: int8 quants in weight order, fp32 scales of weights 0-15 and
// 16-31, fp32 offset, 4 zero bytes (48 bytes):
//   Q8_0  q,                s0 = s1 = d,                 off = 0
//   Q4_K  q (0..15),        s0 = s1 = d sc_s,            off = -(dmin m_s)
//   Q5_K  q (0..31),        s0 = s1 = d sc_s,            off = -(dmin m_s)
//   Q6_K  value - 32,       s0 = d sc[2s], s1 = d sc[2s+1], off = 0
// The products d sc are exact in fp32, so s q + off is the dequantised weight
// of k_dequant_k bit for bit (Q4_K / Q5_K: the same single rounding).
template <int QT>
__global__ void __launch_bounds__(256) k_transcode_i8(const uint8_t* __restrict__ raw, int64_t n_units,
                                                      uint8_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_units) return;
  int q[32];
  float s0, s1, off = 0.f;
  if constexpr (QT == GM_QTYPE_Q8_0) {
    const uint8_t* b = raw + i * 34;
    s0 = s1 = kq_h2f(b);
#pragma unroll
    for (int l = 0; l < 32; ++l) q[l] = (int8_t)b[2 + l];
  } else if constexpr (QT == GM_QTYPE_Q6_K) {
    const int s = (int)(i & 7);
    const uint8_t* b = raw + (i >> 3) * 210;
    const float d = kq_h2f(b + 208);
    const int n = s >> 2, c = s & 3;
    const uint8_t* ql = b + 64 * n + 32 * (c & 1);
    const uint8_t* qh = b + 128 + 32 * n;
    s0 = d * (float)(int8_t)b[192 + 2 * s];
    s1 = d * (float)(int8_t)b[193 + 2 * s];
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      const int lo = c < 2 ? (ql[l] & 15) : (ql[l] >> 4);
      q[l] = (lo | (((qh[l] >> (2 * c)) & 3) << 4)) - 32;
    }
  } else {
    constexpr bool five = QT == GM_QTYPE_Q5_K;
    constexpr int NB = five ? 176 : 144;
    const int s = (int)(i & 7);
    const uint8_t* b = raw + (i >> 3) * NB;
    const float d = kq_h2f(b), dmin = kq_h2f(b + 2);
    const uint8_t* sc = b + 4;
    int scv, mv;
    if (s < 4) { scv = sc[s] & 63; mv = sc[s + 4] & 63; }
    else { scv = (sc[s + 4] & 15) | ((sc[s - 4] >> 6) << 4); mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4); }
    s0 = s1 = d * (float)scv;
    off = -(dmin * (float)mv);
    const uint8_t* qs = b + (five ? 48 : 16) + 32 * (s >> 1);
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      q[l] = (s & 1) ? (qs[l] >> 4) : (qs[l] & 15);
      if constexpr (five) q[l] += ((b[16 + l] >> s) & 1) << 4;
    }
  }
  uint32_t w[8];
#pragma unroll
  for (int c = 0; c < 8; ++c)
    w[c] = (uint32_t)(q[4 * c] & 255) | ((uint32_t)(q[4 * c + 1] & 255) << 8) | ((uint32_t)(q[4 * c + 2] & 255) << 16) |
           ((uint32_t)(q[4 * c + 3] & 255) << 24);
  gm_u32x4* o = reinterpret_cast<gm_u32x4*>(out + i * 48);
  o[0] = gm_u32x4{w[0], w[1], w[2], w[3]};
  o[1] = gm_u32x4{w[4], w[5], w[6], w[7]};
  o[2] = gm_u32x4{__float_as_uint(s0), __float_as_uint(s1), __float_as_uint(off), 0u};
}

int gm_launch_transcode_i8(int qtype, const void* raw, int64_t n_blocks, void* out, hipStream_t s) {
  const GmKBlock kb = gm_kquant_block(qtype);
  const int64_t n_units = n_blocks * (kb.weights / 32);
  if (n_units == 0) return GM_OK;
  const dim3 grid((unsigned)((n_units + 255) / 256)), block(256);
  const uint8_t* p = static_cast<const uint8_t*>(raw);
  uint8_t* o = static_cast<uint8_t*>(out);
  switch (qtype) {
    case GM_QTYPE_Q8_0: hipLaunchKernelGGL(k_transcode_i8<GM_QTYPE_Q8_0>, grid, block, 0, s, p, n_units, o); break;
    case GM_QTYPE_Q4_K: hipLaunchKernelGGL(k_transcode_i8<GM_QTYPE_Q4_K>, grid, block, 0, s, p, n_units, o); break;
    case GM_QTYPE_Q5_K: hipLaunchKernelGGL(k_transcode_i8<GM_QTYPE_Q5_K>, grid, block, 0, s, p, n_units, o); break;
    case GM_QTYPE_Q6_K: hipLaunchKernelGGL(k_transcode_i8<GM_QTYPE_Q6_K>, grid, block, 0, s, p, n_units, o); break;
    default: return gm_fail_arg("gm_transcode_i8: unsupported qtype %d", qtype);
  }
  GM_TRY(hipGetLastError());
  return GM_OK;
}

// --------------------------------------------------------------- matvec
// Partial dot products of one lane for one row over its sub-blocks.
template <int QT, int L, int NT>
__device__ __forceinline__ void gm_row_partial(const uint8_t* __restrict__ row, int nsub, int lane_in_row,
                                               const float* __restrict__ xs, int xstride, int nt,
                                               const uint32_t* __restrict__ grid, float (&acc)[NT]) {
  for (int sub = lane_in_row; sub < nsub; sub += L) {
    const auto r = gm_load_sub<QT, true>(row, sub);
    float wv[32];
    const float sc = gm_decode_sub<QT>(r, sub, grid, wv);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < nt) acc[t] = fmaf(sc, gm_dot32(wv, xs + t * xstride + sub * GM_SUB), acc[t]);
    }
  }
}

// y[t][row] for the rows of this block; x staged as [NT][K] in LDS.
template <int QT, int L, int NT>
__global__ void __launch_bounds__(256) k_matvec(const uint8_t* __restrict__ w, int M, int K,
                                                int64_t row_bytes, const float* __restrict__ x,
                                                int n_tok, float* __restrict__ y, int rows_per_wave) {
  extern __shared__ float smem[];
  uint32_t* grid = reinterpret_cast<uint32_t*>(smem);
  float* xs = smem + 256;
  const int t0 = blockIdx.y * NT;
  const int nt = min(NT, n_tok - t0);
  for (int i = threadIdx.x; i < NT * K; i += 256) {
    const int t = i / K;
    xs[i] = t < nt ? x[(int64_t)(t0 + t) * K + (i - t * K)] : 0.f;
  }
  if constexpr (QT == GM_QTYPE_IQ3_XXS) gm_stage_grid(grid);
  __syncthreads();

  constexpr int RPS = 64 / L;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nsub = K / GM_SUB;
  const int rbase = (blockIdx.x * 4 + wave) * rows_per_wave;
  for (int r0 = 0; r0 < rows_per_wave; r0 += RPS) {
    const int row = rbase + r0 + lane / L;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.f;
    if (row < M) gm_row_partial<QT, L, NT>(w + row * row_bytes, nsub, lane % L, xs, K, nt, grid, acc);
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = gm_group_sum<L>(acc[t]);
    if (row < M && (lane % L) == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (t < nt) y[(int64_t)(t0 + t) * M + row] = acc[t];
    }
  }
}

template <int QT, int L, int NT>
static int launch_matvec_t(const uint8_t* w, int M, int K, const float* x, int n_tok, float* y,
                           hipStream_t s) {
  constexpr int RPS = 64 / L;
  const int rows_per_wave = 2 * RPS;
  const int rows_per_block = 4 * rows_per_wave;
  const dim3 grid((unsigned)((M + rows_per_block - 1) / rows_per_block), (unsigned)((n_tok + NT - 1) / NT));
  const size_t smem = (256 + (size_t)NT * K) * sizeof(float);
  if (int rc = gm_set_smem(k_matvec<QT, L, NT>, smem)) return rc;
  hipLaunchKernelGGL((k_matvec<QT, L, NT>), grid, dim3(256), smem, s, w, M, K, gm_row_bytes(QT, K), x,
                     n_tok, y, rows_per_wave);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

template <int QT, int L>
static int launch_matvec_l(const uint8_t* w, int M, int K, const float* x, int n_tok, float* y,
                           hipStream_t s) {
  if (n_tok == 1) return launch_matvec_t<QT, L, 1>(w, M, K, x, n_tok, y, s);
  if (n_tok <= 4 && 4 * K <= 16384) return launch_matvec_t<QT, L, 4>(w, M, K, x, n_tok, y, s);
  if (8 * K <= 16384) return launch_matvec_t<QT, L, 8>(w, M, K, x, n_tok, y, s);
  if (4 * K <= 16384) return launch_matvec_t<QT, L, 4>(w, M, K, x, n_tok, y, s);
  return launch_matvec_t<QT, L, 1>(w, M, K, x, n_tok, y, s);
}

// One token (BASELINE configs 1 and 2, the reference's NpuQuantMatVec /
// NpuIQ4MatVec call, npu/quant_mv.py:419-463).  LR lanes per row, so a wave
// covers G = 64 / LR rows per row group, and each wave takes RPW row groups:
// a block of 4 waves computes 4 RPW G rows.  Every thread first loads its 8
// values of x per 2048-wide pass, then every lane issues the loads of all
// RPW x SPL sub-blocks it multiplies (sub-blocks lir + LR i of each of its
// RPW rows), so the wait for x (vmcnt retires in issue order) never waits
// for weights and every row's bytes are in flight at once.  While they
// arrive the block converts x into the int8-limb row in LDS; then each lane
// reads the limbs of a sub-block once and multiplies them with that
// sub-block of all RPW rows on v_dot4_i32_i8 (the MoE decode kernels'
// arithmetic), row by row, so that each row waits only for its own loads.
// RPW > 1 amortises the x load and its conversion over RPW times the weight
// bytes (a batched launch of many matrices has thousands of blocks, each of
// which used to convert x for 4 rows).  Issue order, waits and the absence
// of branches around the loads' uses were checked in the kernel's gfx950
// assembly: x's loads first, then every weight load, one wait for x before
// the limbs and one per row after the barrier.
constexpr int kMv1MaxK = 8192;

// The three limb planes and the scale of one activation sub-block (LDS).
struct GmLimbSub {
  uint32_t l0[8], l1[8], l2[8];
  float scale;
};

__device__ __forceinline__ void gm_read_limb_sub(const uint8_t* __restrict__ s, GmLimbSub& a) {
  const gm_u32x4* p = reinterpret_cast<const gm_u32x4*>(s);
  const gm_u32x4 v[6] = {p[0], p[1], p[2], p[3], p[4], p[5]};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    a.l0[4 * h] = v[h].x; a.l0[4 * h + 1] = v[h].y; a.l0[4 * h + 2] = v[h].z; a.l0[4 * h + 3] = v[h].w;
    a.l1[4 * h] = v[2 + h].x; a.l1[4 * h + 1] = v[2 + h].y; a.l1[4 * h + 2] = v[2 + h].z; a.l1[4 * h + 3] = v[2 + h].w;
    a.l2[4 * h] = v[4 + h].x; a.l2[4 * h + 1] = v[4 + h].y; a.l2[4 * h + 2] = v[4 + h].z; a.l2[4 * h + 3] = v[4 + h].w;
  }
  a.scale = *reinterpret_cast<const float*>(s + 96);
}

// sum_k w_k a_k of 32 int8 weights against one limb sub-block, before scales.
__device__ __forceinline__ float gm_dot_limb_sub(const uint32_t (&w)[8], const GmLimbSub& a) {
  int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    s0 = __builtin_amdgcn_sdot4((int)w[c], (int)a.l0[c], s0, false);
    s1 = __builtin_amdgcn_sdot4((int)w[c], (int)a.l1[c], s1, false);
    s2 = __builtin_amdgcn_sdot4((int)w[c], (int)a.l2[c], s2, false);
  }
  return fmaf((float)s2, 65536.f, fmaf((float)s1, 256.f, (float)s0));
}

template <int QT, int LR, int SPL, int RPW>
__global__ void __launch_bounds__(256) k_mv1q(const uint8_t* __restrict__ w, int M, int K, int64_t rb,
                                              const float* __restrict__ x, float* __restrict__ y) {
  using namespace gm_moe;
  constexpr int NXP = SPL;                      // passes of 8 values per thread: K <= 2048 SPL (LR = 64 for SPL > 1)
  constexpr int G = 64 / LR;                                     // rows per row group of a wave
  constexpr bool IQ3 = QT == GM_QTYPE_IQ3_XXS;
  extern __shared__ float smem[];              // the limb row of NXP 2048-wide passes, then the IQ3 tables
  const int nsub = K / GM_SUB;
  uint8_t* xs = reinterpret_cast<uint8_t*>(smem);
  Iq3Tab* tab = reinterpret_cast<Iq3Tab*>(xs + gm_limb_row_bytes(2048 * NXP));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lir = lane % LR;
  const int row0 = (blockIdx.x * 4 + wave) * (RPW * G) + lane / LR;  // row of group j: row0 + G j
  typename FetchRaw<QT>::T f[RPW][SPL];
  auto fetch_rows = [&]() {
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int row = row0 + G * j;
      const uint8_t* wr = w + (int64_t)(row < M ? row : M - 1) * rb;
#pragma unroll
      for (int i = 0; i < SPL; ++i) {
        const int sub = lir + LR * i;
        f[j][i] = gm_fetch_sub<QT, true>(wr, sub < nsub ? sub : nsub - 1);
      }
    }
    issue_fence();
  };
  gm_f32x4 xa[NXP], xb[NXP];
#pragma unroll
  for (int p = 0; p < NXP; ++p) {
    const int k0 = 2048 * p + 8 * (int)threadIdx.x;
    const int kc = k0 < K ? k0 : K - 8;                          // past K: a duplicate load, not stored
    xa[p] = *reinterpret_cast<const gm_f32x4*>(x + kc);
    xb[p] = *reinterpret_cast<const gm_f32x4*>(x + kc + 4);
  }
  uint32_t gw = 0;
  if constexpr (IQ3) gw = gm_iq3_tab_load();
  issue_fence();                                                 // x and the table ahead of the weights
  fetch_rows();
  // Unconditional stores (threads past K fill the row's unused tail, one
  // slot each): a store under `if (k0 < K)` let the compiler sink the x loads
  // into the branch, behind every weight load, and wait for all of them
  // before the limbs.
#pragma unroll
  for (int p = 0; p < NXP; ++p)
    gm_put_limbs8(xa[p], xb[p], (2048 * p + 8 * (int)threadIdx.x) >> 2, xs);   // uniform per quad
  if constexpr (IQ3) gm_iq3_tab_store(gw, tab);
  __syncthreads();
  float acc[RPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) acc[j] = 0.f;
  // Branch-free over the sub-blocks (a sub-block past K repeats the last one
  // with a zero factor): under `if (sub < nsub)` the compiler sank the weight
  // loads into the branch, behind the block barrier.
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    const int sub = lir + LR * i, subc = sub < nsub ? sub : nsub - 1;
    GmLimbSub a;
    gm_read_limb_sub(xs + subc * GM_LSUB, a);
    const float live = sub < nsub ? a.scale : 0.f;
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      uint32_t wq[8];
      const float ws = gm_decode_i8<QT>(gm_fetched<QT>(f[j][i]), subc, tab, wq);
      acc[j] = fmaf(ws * live, gm_dot_limb_sub(wq, a), acc[j]);
      issue_fence();                              // row by row, so each waits only for its own loads
    }
  }
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const float v = row_sum<LR>(acc[j]);
    const int row = row0 + G * j;
    if (row < M && lir == 0) y[row] = v;
  }
}

template <int QT, int LR, int SPL, int RPW>
static int launch_mv1q_t(const uint8_t* w, int M, int K, const float* x, float* y, hipStream_t s) {
  const int rows_per_block = 4 * RPW * (64 / LR);
  const size_t smem = (size_t)gm_moe::gm_limb_row_bytes(2048 * SPL) + sizeof(Iq3Tab);   // NXP = SPL passes
  if (int rc = gm_set_smem(k_mv1q<QT, LR, SPL, RPW>, smem)) return rc;
  hipLaunchKernelGGL((k_mv1q<QT, LR, SPL, RPW>), dim3((unsigned)((M + rows_per_block - 1) / rows_per_block)),
                     dim3(256), smem, s, w, M, K, gm_row_bytes(QT, K), x, y);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

// Row groups per wave: as many as keep at least kMv1Blocks blocks in the grid
// (4 per CU), up to 8 sub-block loads in flight per lane.
#ifndef GM_MV1_BLOCKS
#define GM_MV1_BLOCKS 1024
#endif
#ifndef GM_MV1_IQ3_RPW
#define GM_MV1_IQ3_RPW 4
#endif
constexpr int kMv1Blocks = GM_MV1_BLOCKS;

template <int QT, int LR, int SPL>
static int launch_mv1q_r(const uint8_t* w, int M, int K, const float* x, float* y, hipStream_t s) {
  const int64_t groups = (int64_t)(M + 64 / LR - 1) / (64 / LR);        // row groups over the matrix
  // IQ3_XXS (6 narrow loads per sub-block against IQ4_XS's 2): 4 row groups
  // per wave measured 13.4 us for 64 config-2 matrices against 15.7 at 8
  const int max_rpw = QT == GM_QTYPE_IQ3_XXS ? GM_MV1_IQ3_RPW : 8;
  auto fits = [&](int rpw) {
    return SPL * rpw <= 8 && rpw <= max_rpw && groups >= (int64_t)4 * rpw * kMv1Blocks;
  };
  if (fits(8)) return launch_mv1q_t<QT, LR, SPL, 8>(w, M, K, x, y, s);
  if (fits(4)) return launch_mv1q_t<QT, LR, SPL, 4>(w, M, K, x, y, s);
  if (fits(2)) return launch_mv1q_t<QT, LR, SPL, 2>(w, M, K, x, y, s);
  return launch_mv1q_t<QT, LR, SPL, 1>(w, M, K, x, y, s);
}

template <int QT>
static int launch_mv1q(const uint8_t* w, int M, int K, const float* x, float* y, hipStream_t s) {
  const int nsub = K / GM_SUB;                                   // 8 .. 256
  if (nsub <= 16) return launch_mv1q_r<QT, 16, 1>(w, M, K, x, y, s);
  if (nsub <= 32) return launch_mv1q_r<QT, 32, 1>(w, M, K, x, y, s);
  if (nsub <= 64) return launch_mv1q_r<QT, 64, 1>(w, M, K, x, y, s);
  if (nsub <= 128) return launch_mv1q_r<QT, 64, 2>(w, M, K, x, y, s);
  return launch_mv1q_r<QT, 64, 4>(w, M, K, x, y, s);
}

template <int QT>
static int launch_matvec_q(const uint8_t* w, int M, int K, const float* x, int n_tok, float* y,
                           hipStream_t s) {
  if constexpr (QT != GM_QTYPE_I8)
    if (n_tok == 1 && K <= kMv1MaxK) return launch_mv1q<QT>(w, M, K, x, y, s);
  const int nsub = K / GM_SUB;
  if (nsub >= 64) return launch_matvec_l<QT, 64>(w, M, K, x, n_tok, y, s);
  if (nsub >= 32) return launch_matvec_l<QT, 32>(w, M, K, x, n_tok, y, s);
  if (nsub >= 16) return launch_matvec_l<QT, 16>(w, M, K, x, n_tok, y, s);
  if (nsub >= 8) return launch_matvec_l<QT, 8>(w, M, K, x, n_tok, y, s);
  if (nsub >= 4) return launch_matvec_l<QT, 4>(w, M, K, x, n_tok, y, s);
  if (nsub >= 2) return launch_matvec_l<QT, 2>(w, M, K, x, n_tok, y, s);
  return launch_matvec_l<QT, 1>(w, M, K, x, n_tok, y, s);
}

int gm_launch_matvec(int qtype, const void* w, int M, int K, const float* x, int n_tok, float* y,
                     hipStream_t s) {
  const uint8_t* p = static_cast<const uint8_t*>(w);
  switch (qtype) {
    case GM_QTYPE_IQ4_XS: return launch_matvec_q<GM_QTYPE_IQ4_XS>(p, M, K, x, n_tok, y, s);
    case GM_QTYPE_IQ3_XXS: return launch_matvec_q<GM_QTYPE_IQ3_XXS>(p, M, K, x, n_tok, y, s);
    case GM_QTYPE_BF16: return gm_launch_mv_bf16(static_cast<const uint16_t*>(w), M, K, x, n_tok, y, s);
    case GM_QTYPE_I8: return launch_matvec_q<GM_QTYPE_I8>(p, M, K, x, n_tok, y, s);   // prefill's shared expert
    default: return gm_fail_arg("gm_matvec: unsupported qtype %d", qtype);
  }
}

// ------------------------------------------------------ SwiGLU gate/up
// h[t][r] = silu(G[r] . x[t]) * (U[r] . x[t]); one wave per RPS rows.
template <int QT, int L, int NT>
__global__ void __launch_bounds__(256) k_gateup(const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu,
                                                int FF, int D, int64_t row_bytes,
                                                const float* __restrict__ x, int n_tok,
                                                float* __restrict__ h, int rows_per_wave) {
  extern __shared__ float smem[];
  uint32_t* grid = reinterpret_cast<uint32_t*>(smem);
  float* xs = smem + 256;
  const int t0 = blockIdx.y * NT;
  const int nt = min(NT, n_tok - t0);
  for (int i = threadIdx.x; i < NT * D; i += 256) {
    const int t = i / D;
    xs[i] = t < nt ? x[(int64_t)(t0 + t) * D + (i - t * D)] : 0.f;
  }
  if constexpr (QT == GM_QTYPE_IQ3_XXS) gm_stage_grid(grid);
  __syncthreads();
  constexpr int RPS = 64 / L;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nsub = D / GM_SUB;
  const int rbase = (blockIdx.x * 4 + wave) * rows_per_wave;
  for (int r0 = 0; r0 < rows_per_wave; r0 += RPS) {
    const int row = rbase + r0 + lane / L;
    float ag[NT], au[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) { ag[t] = 0.f; au[t] = 0.f; }
    if (row < FF) {
      gm_row_partial<QT, L, NT>(wg + row * row_bytes, nsub, lane % L, xs, D, nt, grid, ag);
      gm_row_partial<QT, L, NT>(wu + row * row_bytes, nsub, lane % L, xs, D, nt, grid, au);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) { ag[t] = gm_group_sum<L>(ag[t]); au[t] = gm_group_sum<L>(au[t]); }
    if (row < FF && (lane % L) == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (t < nt) h[(int64_t)(t0 + t) * FF + row] = gm_silu(ag[t]) * au[t];
    }
  }
}

template <int QT, int L, int NT>
static int launch_gateup_t(const uint8_t* wg, const uint8_t* wu, int FF, int D, const float* x, int n_tok,
                           float* h, hipStream_t s) {
  constexpr int RPS = 64 / L;
  const int rows_per_wave = 2 * RPS;
  const int rows_per_block = 4 * rows_per_wave;
  const dim3 grid((unsigned)((FF + rows_per_block - 1) / rows_per_block), (unsigned)((n_tok + NT - 1) / NT));
  const size_t smem = (256 + (size_t)NT * D) * sizeof(float);
  if (int rc = gm_set_smem(k_gateup<QT, L, NT>, smem)) return rc;
  hipLaunchKernelGGL((k_gateup<QT, L, NT>), grid, dim3(256), smem, s, wg, wu, FF, D, gm_row_bytes(QT, D), x,
                     n_tok, h, rows_per_wave);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

template <int QT>
static int launch_gateup_q(const uint8_t* wg, const uint8_t* wu, int FF, int D, const float* x, int n_tok,
                           float* h, hipStream_t s) {
  const int nsub = D / GM_SUB;
  const bool one = n_tok == 1;
#define GM_GU(LL)                                                                     \
  return one ? launch_gateup_t<QT, LL, 1>(wg, wu, FF, D, x, n_tok, h, s)              \
             : (8 * D <= 16384 ? launch_gateup_t<QT, LL, 8>(wg, wu, FF, D, x, n_tok, h, s) \
                               : launch_gateup_t<QT, LL, 1>(wg, wu, FF, D, x, n_tok, h, s))
  if (nsub >= 64) GM_GU(64);
  if (nsub >= 32) GM_GU(32);
  if (nsub >= 16) GM_GU(16);
  GM_GU(8);
#undef GM_GU
}

int gm_launch_gateup(int qtype, const void* wg, const void* wu, int FF, int D, const float* x, int n_tok,
                     float* h, hipStream_t s) {
  const uint8_t* g = static_cast<const uint8_t*>(wg);
  const uint8_t* u = static_cast<const uint8_t*>(wu);
  switch (qtype) {
    case GM_QTYPE_IQ4_XS: return launch_gateup_q<GM_QTYPE_IQ4_XS>(g, u, FF, D, x, n_tok, h, s);
    case GM_QTYPE_IQ3_XXS: return launch_gateup_q<GM_QTYPE_IQ3_XXS>(g, u, FF, D, x, n_tok, h, s);
    case GM_QTYPE_BF16: return launch_gateup_q<GM_QTYPE_BF16>(g, u, FF, D, x, n_tok, h, s);
    case GM_QTYPE_I8: return launch_gateup_q<GM_QTYPE_I8>(g, u, FF, D, x, n_tok, h, s);
    default: return gm_fail_arg("gm_swiglu_mlp: unsupported gate/up qtype %d", qtype);
  }
}
