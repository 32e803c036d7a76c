// Dense bf16 matvec for the projection sites NpuMatVec / NpuConcatMatVec
// serve (npu/mv.py:222-265, 292-347; qwen/forward.py:813-831):
//   y[t][m] = sum_k W[m][k] * x[t][k],  W bf16 [M x K] row-major, x / y fp32.
//
// HBM-streaming layout: a wave owns R consecutive rows; in slot s lane l
// covers k = 512 s + 8 l .. +7, i.e. 16 contiguous bytes of every row, so one
// slot of one row is one fully coalesced 1 KB wave load.  A pass issues all
// R x S nontemporal loads of its k range (up to 16 x 16 B per lane) before
// the first FMA; with one row per wave and many waves per CU the chip keeps
// the whole matrix (or most of it) in flight at once.  The token tile x[NT][K]
// is staged in LDS once per block (after the weight loads are issued) and
// read per slot, shared by the R rows.  Every product is an fp32 FMA of the
// exact bf16 weight and the fp32 activation; each lane's partial sum is
// reduced over the wave with DPP.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int kSlotK = 512;                   // k values per slot (64 lanes x 8)

template <int NT, int R, int S>
__global__ void __launch_bounds__(256) k_mv_bf16(const uint16_t* __restrict__ w, int M, int K,
                                                 const float* __restrict__ x, int n_tok, float* __restrict__ y) {
  extern __shared__ gm_f32x4 xs4[];                               // [NT][K / 4]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const int t0 = blockIdx.y * NT;
  const int nt = min(NT, n_tok - t0);
  const int npass = (K + S * kSlotK - 1) / (S * kSlotK);
  const float* xs = reinterpret_cast<const float*>(xs4);

  const gm_u32x4* rp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, M - 1);                        // rows past M: loaded, never stored
    rp[r] = reinterpret_cast<const gm_u32x4*>(w + (int64_t)row * K);
  }

  float acc[R][NT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[r][t] = 0.f;

  for (int p = 0; p < npass; ++p) {
    gm_u32x4 wv[R][S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int gb = (p * S + s) * 64;                           // first 16-byte granule of the slot
      if (8 * gb < K) {                                          // wave-uniform
        const int g = min(gb + lane, (K >> 3) - 1);              // lanes past K reload the last granule
#pragma unroll
        for (int r = 0; r < R; ++r) wv[r][s] = gm_ld<true>(rp[r] + g);
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) wv[r][s] = gm_u32x4{0u, 0u, 0u, 0u};
      }
    }
    if (p == 0) {
      const int kq = K >> 2;
      for (int i = threadIdx.x; i < NT * kq; i += 256) {
        const int t = i / kq;
        xs4[i] = t < nt ? reinterpret_cast<const gm_f32x4*>(x + (int64_t)(t0 + t) * K)[i - t * kq]
                        : gm_f32x4{0.f, 0.f, 0.f, 0.f};
      }
      __syncthreads();
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int k0 = 8 * ((p * S + s) * 64 + lane);
      if (k0 >= K) continue;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const gm_f32x4 xa = *reinterpret_cast<const gm_f32x4*>(xs + t * K + k0);
        const gm_f32x4 xb = *reinterpret_cast<const gm_f32x4*>(xs + t * K + k0 + 4);
        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t u[4] = {wv[r][s].x, wv[r][s].y, wv[r][s].z, wv[r][s].w};
          float a = acc[r][t];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            a = fmaf(__uint_as_float(u[j] << 16), xv[2 * j], a);
            a = fmaf(__uint_as_float(u[j] & 0xffff0000u), xv[2 * j + 1], a);
          }
          acc[r][t] = a;
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float v = gm_wave_sum64(acc[r][t]);
      if (lane == 0 && row0 + r < M && t < nt) y[(int64_t)(t0 + t) * M + row0 + r] = v;
    }
  }
}

template <int NT, int R, int S>
int launch_mv(const uint16_t* w, int M, int K, const float* x, int n_tok, float* y, hipStream_t s) {
  const size_t smem = (size_t)NT * K * sizeof(float);
  if (int rc = gm_set_smem(k_mv_bf16<NT, R, S>, smem)) return rc;
  const dim3 grid((unsigned)((M + 4 * R - 1) / (4 * R)), (unsigned)((n_tok + NT - 1) / NT));
  hipLaunchKernelGGL((k_mv_bf16<NT, R, S>), grid, dim3(256), smem, s, w, M, K, x, n_tok, y);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

// S = the row's slots (at most 16 per pass).  One row per wave for one token
// (the most waves, each with the whole row in flight, was the fastest launch
// shape on MI355X); two rows per wave for a token tile, whose LDS copy of x
// is then shared by 8 rows per block.
template <int NT, int R>
int launch_mv_r(const uint16_t* w, int M, int K, const float* x, int n_tok, float* y, hipStream_t s) {
  const int slots = (K + kSlotK - 1) / kSlotK;
  if (slots <= 1) return launch_mv<NT, R, 1>(w, M, K, x, n_tok, y, s);
  if (slots <= 2) return launch_mv<NT, R, 2>(w, M, K, x, n_tok, y, s);
  if (slots <= 4) return launch_mv<NT, R, 4>(w, M, K, x, n_tok, y, s);
  if (slots <= 8) return launch_mv<NT, R, 8>(w, M, K, x, n_tok, y, s);
  return launch_mv<NT, R, 16>(w, M, K, x, n_tok, y, s);
}

}  // namespace

// K a multiple of 256 and <= 16384, w and x 16-byte aligned (checked by the
// caller).  The token tile is sized so that NT x K fp32 values fit 64 KB of LDS.
int gm_launch_mv_bf16(const uint16_t* w, int M, int K, const float* x, int n_tok, float* y, hipStream_t s) {
  const int nt_lds = 16384 / K;                                   // 1 .. 64
  if (n_tok == 1) return launch_mv_r<1, 1>(w, M, K, x, n_tok, y, s);
  if (n_tok == 2 || nt_lds < 4) return launch_mv_r<2, 2>(w, M, K, x, n_tok, y, s);
  if (n_tok <= 4 || nt_lds < 8) return launch_mv_r<4, 2>(w, M, K, x, n_tok, y, s);
  return launch_mv_r<8, 2>(w, M, K, x, n_tok, y, s);
}
