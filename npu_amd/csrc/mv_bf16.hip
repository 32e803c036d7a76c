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
// reduced over the wave with DPP.  This path serves one token.
//
// Two or more tokens (k_mv_bf16_mfma): v_mfma_f32_16x16x32_bf16 with the
// weight rows as A (lane l: row l % 16, k = 8 (l / 16) .. +7 of each 32-wide
// k-step, one 16-byte nontemporal load) and the token columns as B.  Every
// lane splits its column's 8 fp32 activations into three bf16 planes,
// x = h + m + l exactly (h = x truncated to bf16, m = (x - h) truncated,
// l = x - h - m, which has at most 8 significant bits), so the three MFMAs
// per A operand add exact bf16 x bf16 products in fp32 and x loses nothing.
// A block holds 16 RT rows; its WPB waves split K, each issuing NC k-steps'
// loads at a time, and their tiles are summed in LDS in wave order.
#include "common.h"
#include "kernels.h"
#include "moe_decode.h"

namespace {

constexpr int kSlotK = 512;                   // k values per slot (64 lanes x 8)

// One-token extras of k_mv_bf16: a second matrix w2 [M2 x K] whose rows follow
// w's in the launch (its products go to y2), and an RMSNorm weight: with
// norm_w, x is staged as (x * rsqrt(mean(x^2) + eps)) * norm_w.  zacc: zn
// doubles the last block clears (a MoE block's router accumulators, which a
// later launch of the same core layer adds into).
struct MvEx {
  const uint16_t* w2;
  int M2;
  float* y2;
  const float* norm_w;
  float eps;
  double* zacc;
  int zn;
};

// Accumulator positions per thread of the next-router epilogue (512 threads;
// E <= 512: 8 x 64 + 2 positions).
constexpr int kNxSlots = 2;

// The router epilogue's loads: thread t takes accumulator positions t + NT j
// (gm_acc_pos order, so a wave's atomics fall on consecutive words) and loads
// the 8 router values of its word at columns r0 .. r0+7 (one 8-column group of
// router_t: 16 bytes of bf16 or 32 of fp32; positions without a router row load
// row 0), and every thread the 8 norm weights (ones without a norm weight).
template <int NT>
__device__ __forceinline__ void nx_load(const GmNextRouter& nx, int r0, gm_u32x4 (&wv)[kNxSlots][2],
                                        gm_f32x4 (&nw)[2]) {
  const int mvn = gm_acc_mv(nx.E), es = nx.f32 ? 4 : 2;
#pragma unroll
  for (int j = 0; j < kNxSlots; ++j) {
    const int pos = threadIdx.x + NT * j;
    const int e = pos < 64 * mvn ? 64 * (pos % mvn) + pos / mvn : nx.E + (pos - 64 * mvn);
    const int er = e <= nx.E ? e : 0;
    const gm_u32x4* q = reinterpret_cast<const gm_u32x4*>(static_cast<const uint8_t*>(nx.w) +
                                                          ((int64_t)(r0 >> 3) * (nx.E + 1) + er) * 8 * es);
    wv[j][0] = gm_ld<true>(q);
    wv[j][1] = gm_ld<true>(q + (nx.f32 ? 1 : 0));
  }
  const gm_f32x4 one = {1.f, 1.f, 1.f, 1.f};
  nw[0] = nx.nw ? *reinterpret_cast<const gm_f32x4*>(nx.nw + r0) : one;
  nw[1] = nx.nw ? *reinterpret_cast<const gm_f32x4*>(nx.nw + r0 + 4) : one;
}

template <int NT>
__device__ __forceinline__ void nx_add(const GmNextRouter& nx, const float* s_y, const gm_u32x4 (&wv)[kNxSlots][2],
                                       const gm_f32x4 (&nw)[2]) {
  const int mvn = gm_acc_mv(nx.E);
  float yv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) yv[i] = s_y[i];
  const float nv[8] = {nw[0].x, nw[0].y, nw[0].z, nw[0].w, nw[1].x, nw[1].y, nw[1].z, nw[1].w};
  int xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  double* copy = nx.acc + (xcc & (GM_ACC_COPIES - 1)) * nx.ld;
#pragma unroll
  for (int j = 0; j < kNxSlots; ++j) {
    const int pos = threadIdx.x + NT * j;
    const int e = pos < 64 * mvn ? 64 * (pos % mvn) + pos / mvn : nx.E + (pos - 64 * mvn);
    const bool live = pos < 64 * mvn ? e < nx.E : e <= nx.E + 1;
    if (!live) continue;
    float wf[8];
    if (nx.f32) {
      const uint32_t u[8] = {wv[j][0].x, wv[j][0].y, wv[j][0].z, wv[j][0].w,
                             wv[j][1].x, wv[j][1].y, wv[j][1].z, wv[j][1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) wf[i] = __uint_as_float(u[i]);
    } else {
      const uint32_t u[4] = {wv[j][0].x, wv[j][0].y, wv[j][0].z, wv[j][0].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wf[2 * i] = __uint_as_float(u[i] << 16);
        wf[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
      }
    }
    float p = 0.f;
    if (e <= nx.E) {
#pragma unroll
      for (int i = 0; i < 8; ++i) p = fmaf(wf[i], yv[i] * nv[i], p);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) p = fmaf(yv[i], yv[i], p);
    }
    // all adds into one copy come from one XCD and meet in its L2: workgroup scope
    // is enough, and the kernel boundary writes the L2 back for the MoE launch
    __hip_atomic_fetch_add(copy + pos, (double)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// One token.  Per pass of S slots: the pass's x values are loaded into
// registers first (their loads retire before the weights', vmcnt being in
// issue order), then every weight load of the pass, all unconditional (lanes
// and slots past K reload the last granule and are zeroed by a select, so no
// branch separates a load from its use); x goes to LDS while the weights are
// in flight (normalised first with ex.norm_w), and each slot is multiplied as
// it lands.
//
// NW waves per block.  NXT (8 waves, one row each): the block's 8 outputs y
// (rows r0 .. r0+7) also feed a MoE block's router (nx, its T = 1 accumulators,
// as the chain's down kernel feeds the next layer's): every accumulator
// position gets sum_i Wn[e][r0 + i] (y[r0 + i] w_norm[r0 + i]) (router row e,
// row E the shared gate vector, from router_t) or, at word E + 1,
// sum_i y[r0 + i]^2, added with fp64 atomics into the copy of the block's XCD.
// The router values and norm weights are loaded behind the matrix rows.
template <int R, int S, int NW, bool NXT>
__global__ void __launch_bounds__(64 * NW) k_mv_bf16(const uint16_t* __restrict__ w, int M, int K,
                                                     const float* __restrict__ x, float* __restrict__ y,
                                                     const float* __restrict__ add, MvEx ex, GmNextRouter nx) {
  static_assert(!NXT || (R == 1 && NW == 8), "the router epilogue takes 8 waves of one row");
  constexpr int NT = 64 * NW;
  extern __shared__ gm_f32x4 xs4[];                               // [XQ x NT]: one pass of x
  __shared__ float red[NW];
  __shared__ float s_y[NW];
  constexpr int XQ = (S * kSlotK / 4 + NT - 1) / NT;              // x float4 per thread and pass
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * NW + wave) * R;
  const int npass = (K + S * kSlotK - 1) / (S * kSlotK);
  const int kq = K >> 2, ng = K >> 3;
  const float* xs = reinterpret_cast<const float*>(xs4);
  const gm_f32x4* x4 = reinterpret_cast<const gm_f32x4*>(x);
  const int Mt = M + ex.M2;

  gm_u32x4 nxw[kNxSlots][2];                                      // router values of the epilogue (NXT)
  gm_f32x4 nxn[2];
  const gm_u32x4* rp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, Mt - 1);                       // rows past Mt: loaded, never stored
    rp[r] = reinterpret_cast<const gm_u32x4*>(row < M ? w + (int64_t)row * K : ex.w2 + (int64_t)(row - M) * K);
  }

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  if (ex.zacc != nullptr && blockIdx.x == gridDim.x - 1)          // uniform per block
    for (int i = threadIdx.x; i < ex.zn; i += NT) ex.zacc[i] = 0.0;

  for (int p = 0; p < npass; ++p) {
    const int q0 = p * (S * kSlotK / 4);                          // first float4 of the pass
    // x and the norm weights (x again without a norm: a harmless duplicate)
    const gm_f32x4* n4 = ex.norm_w ? reinterpret_cast<const gm_f32x4*>(ex.norm_w) : x4;
    gm_f32x4 xr[XQ], nr[XQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      const int i = q0 + (int)threadIdx.x + NT * q, ic = i < kq ? i : kq - 1;    // past K: zeroed below
      xr[q] = x4[ic];
      nr[q] = n4[ic];
    }
    __builtin_amdgcn_sched_barrier(0);
    gm_u32x4 wv[R][S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int g = min((p * S + s) * 64 + lane, ng - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) wv[r][s] = gm_ld<true>(rp[r] + g);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NXT) {
      if (p == 0) nx_load<NT>(nx, blockIdx.x * 8, nxw, nxn);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (p > 0) __syncthreads();                                   // the previous pass's x reads are done
#pragma unroll
    for (int q = 0; q < XQ; ++q)
      if (q0 + (int)threadIdx.x + NT * q >= kq) xr[q] = gm_f32x4{0.f, 0.f, 0.f, 0.f};
    if (ex.norm_w) {                                              // one pass (the launcher checks)
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < XQ; ++q)
        ss = fmaf(xr[q].x, xr[q].x, fmaf(xr[q].y, xr[q].y, fmaf(xr[q].z, xr[q].z, fmaf(xr[q].w, xr[q].w, ss))));
      ss = gm_wave_sum64(ss);
      if (lane == 0) red[wave] = ss;
      __syncthreads();
      float rsum = 0.f;
#pragma unroll
      for (int i = 0; i < NW; ++i) rsum += red[i];
      const float rs = 1.0f / sqrtf(rsum / (float)K + ex.eps);
#pragma unroll
      for (int q = 0; q < XQ; ++q) xr[q] = (xr[q] * rs) * nr[q];
    }
#pragma unroll
    for (int q = 0; q < XQ; ++q) xs4[threadIdx.x + NT * q] = xr[q];    // unconditional: XQ x NT slots
    __syncthreads();
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int k0 = 8 * ((p * S + s) * 64 + lane);
      const bool live = k0 < K;
      const int kl = 8 * (s * 64 + lane);                         // offset in the pass's x
      const gm_f32x4 xa = *reinterpret_cast<const gm_f32x4*>(xs + kl);
      const gm_f32x4 xb = *reinterpret_cast<const gm_f32x4*>(xs + kl + 4);
      const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t u[4] = {live ? wv[r][s].x : 0u, live ? wv[r][s].y : 0u, live ? wv[r][s].z : 0u,
                               live ? wv[r][s].w : 0u};
        float a = acc[r];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a = fmaf(__uint_as_float(u[j] << 16), xv[2 * j], a);
          a = fmaf(__uint_as_float(u[j] & 0xffff0000u), xv[2 * j + 1], a);
        }
        acc[r] = a;
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = gm_wave_sum64(acc[r]);
    if (lane == 0 && row0 + r < M) {
      const float yv = add ? add[row0 + r] + v : v;               // y = add + W x (a residual), or W x
      y[row0 + r] = yv;
      if constexpr (NXT) s_y[wave] = yv;
    } else if (lane == 0 && row0 + r >= M && row0 + r < Mt) {
      ex.y2[row0 + r - M] = v;
    }
    if constexpr (NXT)
      if (lane == 0 && row0 + r >= M) s_y[wave] = 0.f;
  }
  if constexpr (NXT) {
    __syncthreads();
    nx_add<NT>(nx, s_y, nxw, nxn);
  }
}

typedef __bf16 gm_bf16x8 __attribute__((ext_vector_type(8)));

// x = h + m + l over 8 fp32 values -> three bf16x8 planes (exact split, see above).
__device__ __forceinline__ void split3(const gm_f32x4& xa, const gm_f32x4& xb, gm_u32x4 (&pl)[3]) {
  const float v[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  uint32_t hb[8], mb[8], lb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    hb[i] = __float_as_uint(v[i]) & 0xffff0000u;
    const float r = v[i] - __uint_as_float(hb[i]);
    mb[i] = __float_as_uint(r) & 0xffff0000u;
    lb[i] = __float_as_uint(r - __uint_as_float(mb[i]));     // low 16 bits are zero
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    pl[0][d] = __builtin_amdgcn_perm(hb[2 * d + 1], hb[2 * d], 0x07060302u);
    pl[1][d] = __builtin_amdgcn_perm(mb[2 * d + 1], mb[2 * d], 0x07060302u);
    pl[2][d] = __builtin_amdgcn_perm(lb[2 * d + 1], lb[2 * d], 0x07060302u);
  }
}

template <int RT, int WPB, int NC>
__global__ void __launch_bounds__(64 * WPB) k_mv_bf16_mfma(const uint16_t* __restrict__ w, int M, int K,
                                                        const float* __restrict__ x, int n_tok,
                                                        float* __restrict__ y) {
  __shared__ gm_f32x4 red[WPB > 1 ? WPB - 1 : 1][RT][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, q = lane >> 4;
  const int row0 = blockIdx.x * 16 * RT;
  const int tok = blockIdx.y * 16 + l16;
  const int kw = K / WPB, kbeg = wave * kw;                      // this wave's K range (K % (32 WPB) == 0)
  const gm_u32x4* ar[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = min(row0 + rt * 16 + l16, M - 1);           // rows past M: loaded, never stored
    ar[rt] = reinterpret_cast<const gm_u32x4*>(w + (int64_t)row * K + kbeg + 8 * q);
  }
  const gm_f32x4* xr = reinterpret_cast<const gm_f32x4*>(x + (int64_t)min(tok, n_tok - 1) * K + kbeg + 8 * q);
  gm_f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) acc[rt] = gm_f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < kw; c0 += 32 * NC) {
    gm_u32x4 a[RT][NC];
    gm_f32x4 xa[NC], xb[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) a[rt][c] = gm_ld<true>(ar[rt] + (c0 + 32 * c) / 8);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      xa[c] = xr[(c0 + 32 * c) / 4];
      xb[c] = xr[(c0 + 32 * c) / 4 + 1];
    }
    __builtin_amdgcn_sched_barrier(0);                          // every load of the chunk before the first use
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      gm_u32x4 pl[3];
      split3(xa[c], xb[c], pl);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int p = 0; p < 3; ++p)
          acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gm_bf16x8, a[rt][c]),
                                                            __builtin_bit_cast(gm_bf16x8, pl[p]), acc[rt], 0, 0, 0);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) red[wave - 1][rt][lane] = acc[rt];
  }
  __syncthreads();
  if (wave > 0 || tok >= n_tok) return;
#pragma unroll
  for (int v = 0; v < WPB - 1; ++v)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] += red[v][rt][lane];
  // C layout: lane l holds rows 4 (l / 16) + i of the tile, column (token) l % 16
  float* out = y + (int64_t)tok * M;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = row0 + rt * 16 + 4 * q;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (row + i < M) out[row + i] = acc[rt][i];
  }
}

template <int RT, int WPB>
int launch_mfma_w(const uint16_t* w, int M, int K, const float* x, int n_tok, float* y, hipStream_t s) {
  const dim3 grid((unsigned)((M + 16 * RT - 1) / (16 * RT)), (unsigned)((n_tok + 15) / 16));
  const int steps = K / (32 * WPB);                              // k-steps per wave (exact: WPB divides K / 32)
#define GM_MV_GO(NC)                                                                               \
  hipLaunchKernelGGL((k_mv_bf16_mfma<RT, WPB, NC>), grid, dim3(64 * WPB), 0, s, w, M, K, x, n_tok, y); \
  break;
  switch (steps % 8 == 0 ? 8 : steps % 4 == 0 ? 4 : steps % 2 == 0 ? 2 : 1) {
    case 8: GM_MV_GO(8)
    case 4: GM_MV_GO(4)
    case 2: GM_MV_GO(2)
    default: GM_MV_GO(1)
  }
#undef GM_MV_GO
  GM_TRY(hipGetLastError());
  return GM_OK;
}

// Two row tiles per block for tall matrices, else one; waves per block so that
// the grid holds about 1024 waves, each wave taking an equal number of 32-wide
// k-steps: the largest of 8 (4 for grids of >= 256 blocks), 4, 2, 1 that divides
// K / 32 (K = 576: 2 waves of 9 steps).
int launch_mfma(const uint16_t* w, int M, int K, const float* x, int n_tok, float* y, hipStream_t s) {
  const int rt = M >= 8192 ? 2 : 1;
  const int blocks = (M + 16 * rt - 1) / (16 * rt);
  int wpb = blocks < 256 ? 8 : 4;
  while ((K / 32) % wpb) wpb >>= 1;
#define GM_MV_W(R)                                              \
  switch (wpb) {                                                \
    case 8: return launch_mfma_w<R, 8>(w, M, K, x, n_tok, y, s); \
    case 4: return launch_mfma_w<R, 4>(w, M, K, x, n_tok, y, s); \
    case 2: return launch_mfma_w<R, 2>(w, M, K, x, n_tok, y, s); \
    default: return launch_mfma_w<R, 1>(w, M, K, x, n_tok, y, s); \
  }
  if (rt == 2) GM_MV_W(2)
  GM_MV_W(1)
#undef GM_MV_W
}

template <int R, int S, int NW, bool NXT>
int launch_mv(const uint16_t* w, int M, int K, const float* x, float* y, const float* add, const MvEx& ex,
              const GmNextRouter& nx, hipStream_t s) {
  constexpr int NT = 64 * NW;
  const size_t smem = (size_t)((S * kSlotK / 4 + NT - 1) / NT) * NT * sizeof(gm_f32x4);   // XQ x NT float4
  if (int rc = gm_set_smem(k_mv_bf16<R, S, NW, NXT>, smem)) return rc;
  const dim3 grid((unsigned)((M + ex.M2 + NW * R - 1) / (NW * R)));
  hipLaunchKernelGGL((k_mv_bf16<R, S, NW, NXT>), grid, dim3(NT), smem, s, w, M, K, x, y, add, ex, nx);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

// 4 waves per block, or 8 with the router epilogue (one 8-column router group per block).
template <bool NXT>
int launch_mv1_t(const uint16_t* w, int M, int K, const float* x, float* y, const float* add, const MvEx& ex,
                 const GmNextRouter& nx, hipStream_t s) {
  constexpr int NW = NXT ? 8 : 4;
  const int slots = (K + kSlotK - 1) / kSlotK;
  if (slots <= 1) return launch_mv<1, 1, NW, NXT>(w, M, K, x, y, add, ex, nx, s);
  if (slots <= 2) return launch_mv<1, 2, NW, NXT>(w, M, K, x, y, add, ex, nx, s);
  if (slots <= 4) return launch_mv<1, 4, NW, NXT>(w, M, K, x, y, add, ex, nx, s);
  if (slots <= 8) return launch_mv<1, 8, NW, NXT>(w, M, K, x, y, add, ex, nx, s);
  return launch_mv<1, 16, NW, NXT>(w, M, K, x, y, add, ex, nx, s);
}

// S = the row's slots (at most 16 per pass), one row per wave (the most
// waves, each with its whole row in flight, was the fastest launch shape).
// The RMSNorm of ex.norm_w needs the whole row in one pass (K <= 8192).  With
// nx, the launch also adds the MoE router inputs of its rows (M % 8 == 0, M
// the router's D, E <= 512).
int launch_mv1(const uint16_t* w, int M, int K, const float* x, float* y, const float* add, hipStream_t s,
               const MvEx& ex = MvEx{nullptr, 0, nullptr, nullptr, 0.f, nullptr, 0},
               const GmNextRouter* nx = nullptr) {
  const int slots = (K + kSlotK - 1) / kSlotK;
  if (ex.norm_w && slots > 16) return gm_fail_arg("mv_bf16: a fused RMSNorm needs K <= %d", 16 * kSlotK);
  if (nx != nullptr) {
    if (M % 8 || ex.M2 || nx->E > 512 || 64 * gm_acc_mv(nx->E) + 2 > 512 * kNxSlots)
      return gm_fail_arg("mv_bf16: router epilogue needs M %% 8 == 0, one matrix and E <= 512");
    return launch_mv1_t<true>(w, M, K, x, y, add, ex, *nx, s);
  }
  return launch_mv1_t<false>(w, M, K, x, y, add, ex, GmNextRouter{}, s);
}

}  // namespace

// K a multiple of 32 and <= 16384, w and x 16-byte aligned (checked by the
// caller).  One token: the streaming FMA kernel; more: the MFMA kernel, 16
// tokens per column tile.
int gm_launch_mv_bf16(const uint16_t* w, int M, int K, const float* x, int n_tok, float* y, hipStream_t s) {
  if (n_tok == 1) return launch_mv1(w, M, K, x, y, nullptr, s);
  return launch_mfma(w, M, K, x, n_tok, y, s);
}

// One token, y = add + W x (the residual of the core layers' output projections);
// with nx, y also feeds the MoE router accumulators nx->acc (cleared beforehand).
int gm_launch_mv_bf16_add(const uint16_t* w, int M, int K, const float* x, float* y, const float* add,
                          hipStream_t s, const GmNextRouter* nx) {
  return launch_mv1(w, M, K, x, y, add, s, MvEx{nullptr, 0, nullptr, nullptr, 0.f, nullptr, 0}, nx);
}

// One token, the core layers' input projections in one launch: h = RMSNorm(x)
// (norm_w, eps; skipped when norm_w is null), y = W h and, when w2 is given,
// y2 = W2 h (its M2 rows follow W's in the launch); zacc: zn doubles to clear.
int gm_launch_mv_bf16_norm2(const uint16_t* w, int M, const uint16_t* w2, int M2, int K, const float* x,
                            const float* norm_w, float eps, float* y, float* y2, hipStream_t s, double* zacc,
                            int zn) {
  return launch_mv1(w, M, K, x, y, nullptr, s, MvEx{w2, w2 ? M2 : 0, y2, norm_w, eps, zacc, zn});
}
