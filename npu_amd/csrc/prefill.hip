// MoE block, prefill path (T > 8 tokens): grouped dequant-GEMMs on MFMA.
//
//   1. k_pf_prep_router, two roles in one launch:
//      prep blocks:   xn = rmsnorm(x) (or x) -> an f16 copy (gate/up operand),
//                     and each token's RMSNorm factor
//      router blocks: partial router dot products of x w_norm over K ranges and
//                     the shared scalar gate's on v_mfma_f32_16x16x32_bf16, x w_norm
//                     split in registers into three bf16 planes whose sum is it
//                     to ~2^-27, one MFMA per plane: every product of a bf16
//                     weight and a bf16 plane is exact in fp32; the RMSNorm
//                     factor multiplies the summed partials in step 3
//   3. k_pf_topk sums the router partials (times the RMSNorm factor, + bias),
//      then dispatch (dispatch.hip):
//      histogram -> exclusive scan -> stable scatter of (token, slot) pairs by
//      expert, the inverse permutation, and every expert's token list (and the
//      shared expert's, which takes all T tokens) cut into segments of <= kSegTok
//   4. k_pf_gateup:   per (segment, 64 weight rows): h = silu(G x) * (U x).  The raw
//                     superblocks are fetched one superblock ahead into registers
//                     and decoded to f16 integers (kvalue or grid magnitude times
//                     the integer part of the sub-block scale) straight into
//                     v_mfma_f32_16x16x32_f16 operands; the superblock's fp16 d
//                     multiplies the fp32 partial sum of each superblock.  The
//                     segment's activation tile is double-buffered in LDS.  h is
//                     stored as bf16 in expert-sorted row order.
//   5. k_pf_h16:      every h row scaled by a power of two into f16's range and
//                     converted exactly (the scale is kept per row)
//   6. k_pf_down:     per (segment, 2 x 128 weight rows): y_pair = Down_e h on
//                     v_mfma_f32_16x16x32_f16 with f16 integer weight operands as in
//                     4, fp32 out times the row's h scale; the segment's h tile is
//                     staged in LDS once per block
//   7. k_pf_combine:  y[t] = sum over t's experts in ascending id of w * y_pair
//                     + sigmoid gate * y_shared (+ x); fixed order, no atomics
//
// Reference semantics: the CPU loop of qwen/forward.py:563-665 (prefill takes
// that path in the reference; its NPU kernels are T = 1 only).
#include <type_traits>

#include "moe_common.h"

using namespace gm_moe;

typedef __bf16 gm_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 gm_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 gm_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 gm_f16x2 __attribute__((ext_vector_type(2)));
typedef float gm_f32x2 __attribute__((ext_vector_type(2)));
typedef float gm_f32x8 __attribute__((ext_vector_type(8)));

namespace {

// Tokens per segment.  32 (two MFMA column tiles) leaves the GEMM kernels at
// 168 VGPRs, three waves per SIMD: config 4 227 -> 219 us per block against 64
// tokens (four tiles, 2 waves per SIMD), although the 512-token shared unit
// then decodes its weights for 16 segments instead of 8.
constexpr int kSegTok = 32;
constexpr int kNT = kSegTok / 16;   // MFMA column tiles per segment
constexpr int kChunk = 256;         // K elements per pipeline step (one superblock column)
constexpr int kRowB = 2 * kChunk;          // bytes per gate/up LDS activation row (f16, swizzled)
constexpr int kTileG = kSegTok * kRowB;    // one gate/up activation buffer
constexpr int kGran = kSegTok * (2 * kChunk / 16) / 256;  // 16-byte granules per thread of one chunk

// f(integral_constant<int, n>) for the segment's tile count n = ntiles in
// [1, NT], as a chain of uniform branches (one instantiation per count).
template <int NT, class F>
__device__ __forceinline__ void nt_dispatch(int ntiles, F&& f) {
  if constexpr (NT > 1) {
    if (ntiles < NT) { nt_dispatch<NT - 1>(ntiles, f); return; }
  }
  f(std::integral_constant<int, NT>{});
}

struct PfWs {
  int32_t* counts;    // [E]
  int32_t* offsets;   // [E + 1]
  int32_t* sorted;    // [P]
  int32_t* inv;       // [P]   position of pair p in sorted order
  int32_t* segs;      // [1 + 4 * max_seg]  n_seg, then (expert, start, n, unused)
  float* rmsv;        // [T]        RMSNorm factor per token (1 without a norm), for k_pf_topk
  uint16_t* xh;       // [T][D]     f16 xn 2^s (gate/up operand)
  float* xsc;         // [T]        2^-s per token
  float* part;        // [kRouterSplit][T][ldp]  partial router dot products
  uint16_t* hb;       // [P + T][FF]  bf16 SwiGLU rows (sorted pairs, then shared per token)
  uint16_t* hh;       // [P + T][FF]  the same rows as scaled f16
  float* hsc;         // [P + T]      their scales
  float* yp;          // [P + T][D]   fp32 per-pair / shared outputs
  float* xn;          // [T][D]  fp32 xn, for a shared expert in other formats than the routed ones
  float* hsh;         // [T][FF] its fp32 SwiGLU rows
};

// A shared expert stored in other formats than the routed experts (the real
// model's K-quant shared experts, held as I8 rows, beside IQ routed experts; or
// a dense bf16 one) does not run as the GEMMs' ninth unit.  In I8 rows it runs
// as two dense f16 MFMA GEMMs of its own (k_pfs_gateup_i8 into the shared
// SwiGLU rows hb[P + t], k_pf_h16, k_pfs_down_i8 into yp[P + t]); in bf16 its T
// tokens run as one fp32 pass of the multi-token gate/up and down matvec
// kernels over xn.  Either way it writes the rows yp[P + t] the combine reads,
// and the routed experts keep the grouped GEMMs.
inline bool pf_shared_apart(const gm_moe_layer* L) {
  return L->gate_sh && (L->q_gate_sh != L->q_gate || L->q_down_sh != L->q_down);
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

constexpr int kRouterSplit = 16;  // most K ranges of the router GEMM (partials summed in k_pf_topk)

// K ranges actually used: 256 wide (2 k-steps per wave; twice the blocks of
// 512-wide ranges, measured 11.0 against 12.4 us at D = 2048) up to D = 2048,
// then 512 wide when D allows.  At most kRouterSplit ranges (checked at entry).
int router_krange(int D) { return D <= 2048 || D % 512 ? 256 : 512; }
int router_split(int D) { return D / router_krange(D); }

// Row stride of the router partials: E rows + the shared gate row, padded to 4.
int router_ld(const gm_moe_layer* L) { return (L->E + 1 + 3) & ~3; }

int max_segments(int T, int k, int E) { return (T * k) / kSegTok + E + (T + kSegTok - 1) / kSegTok + 1; }

PfWs pf_layout(const gm_moe_layer* L, int T, uint8_t* base, size_t* total) {
  const size_t P = (size_t)T * L->k, E = L->E;
  size_t o = 0;
  PfWs w{};
  auto take = [&](size_t bytes) { uint8_t* p = base ? base + o : nullptr; o = align256(o + bytes); return p; };
  w.counts = reinterpret_cast<int32_t*>(take(E * 4));
  w.offsets = reinterpret_cast<int32_t*>(take((E + 1) * 4));
  w.sorted = reinterpret_cast<int32_t*>(take(P * 4));
  w.inv = reinterpret_cast<int32_t*>(take(P * 4));
  w.segs = reinterpret_cast<int32_t*>(take((1 + 4 * (size_t)max_segments(T, L->k, L->E)) * 4));
  w.rmsv = reinterpret_cast<float*>(take((size_t)T * 4));
  w.xh = reinterpret_cast<uint16_t*>(take((size_t)T * L->D * 2));
  w.xsc = reinterpret_cast<float*>(take((size_t)T * 4));
  w.part = reinterpret_cast<float*>(take((size_t)kRouterSplit * T * router_ld(L) * 4));
  w.hb = reinterpret_cast<uint16_t*>(take((P + T) * (size_t)L->FF * 2));
  w.hh = reinterpret_cast<uint16_t*>(take((P + T) * (size_t)L->FF * 2));
  w.hsc = reinterpret_cast<float*>(take((P + T) * 4));
  w.yp = reinterpret_cast<float*>(take((P + T) * (size_t)L->D * 4));
  if (pf_shared_apart(L)) {
    w.xn = reinterpret_cast<float*>(take((size_t)T * L->D * 4));
    w.hsh = reinterpret_cast<float*>(take((size_t)T * L->FF * 4));
  }
  if (total) *total = o;
  return w;
}

// Blocks run on the 8 XCDs round-robin (block b on XCD b % 8).  Segment
// seg goes to XCD seg % 8 and its nrt row tiles to consecutive slots there,
// so they share the segment's activation tile in one L2, and the grid's
// unused tail (it is sized for the most segments the routing can produce)
// is spread over all XCDs.  Grid size: a multiple of 8 * nrt.
__device__ __forceinline__ void xcd_tile(int b, int nrt, int& seg, int& rt) {
  const int slot = b >> 3;
  seg = (slot / nrt) * 8 + (b & 7);
  rt = slot - (slot / nrt) * nrt;
}

// ---------------------------------------------------------------- prep x
// xn = (x * rms) * w (qwen/forward.py:58-61) or x; xh = f16(xn 2^s) with the
// per-token power of two that puts max |xn| in [2^14, 2^15) (no f16 overflow
// whatever the input scale, and f16's 11 bits for every value down to 2^-10 of
// the token's maximum; rows below 2^-100 are scaled as if their maximum were
// 2^-100), xsc[t] = 2^-s, which the gate/up kernel multiplies into its sums,
// and rmsv[t] = rms (1 without a norm).  One block per token.
__device__ __forceinline__ float pf_block_max(float m, float* red4) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = m;
  __syncthreads();
  return fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
}

// 2^s for a row whose largest magnitude is m (m >= 0): m 2^s in [2^14, 2^15).
__device__ __forceinline__ int pf_f16_shift(float m) {
  const int E = m > 0.f && m <= 3.4e38f ? max(__builtin_amdgcn_frexp_expf(m), -100) : 0;
  return 15 - E;
}

__device__ __forceinline__ uint32_t pf_f16x2(gm_f32x2 v, int sh) {
  const gm_f32x2 vs = {__builtin_ldexpf(v.x, sh), __builtin_ldexpf(v.y, sh)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(vs, gm_f16x2));
}

__device__ __forceinline__ void pf_prep_token(int t, const float* __restrict__ x, int D,
                                              const float* __restrict__ norm_w, float eps,
                                              uint16_t* __restrict__ xh, float* __restrict__ xsc,
                                              float* __restrict__ xn32, float* __restrict__ rmsv, float* red,
                                              float* redm) {
  const gm_f32x2* x2 = reinterpret_cast<const gm_f32x2*>(x + (int64_t)t * D);
  const int n2 = D >> 1;
  int sh;
  if (D <= 4096) {                                             // uniform: the row held in registers
    constexpr int NQ = 4;                                      // 16-byte granules per thread
    const int n4 = D >> 2;
    const gm_f32x4* x4 = reinterpret_cast<const gm_f32x4*>(x + (int64_t)t * D);
    gm_f32x4 v[NQ], wv[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {                             // every load before the first use
      const int c = min((int)threadIdx.x + 256 * i, n4 - 1);   // past the row: a duplicate, not used
      v[i] = x4[c];
      wv[i] = norm_w ? reinterpret_cast<const gm_f32x4*>(norm_w)[c] : gm_f32x4{1.f, 1.f, 1.f, 1.f};
    }
    float rms = 1.f;
    if (norm_w) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < NQ; ++i)
        if ((int)threadIdx.x + 256 * i < n4)
          ss = fmaf(v[i].x, v[i].x, fmaf(v[i].y, v[i].y, fmaf(v[i].z, v[i].z, fmaf(v[i].w, v[i].w, ss))));
      ss = gm_wave_sum64(ss);
      if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
      __syncthreads();
      rms = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)D + eps);
    }
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      if (norm_w) {
        v[i].x = (v[i].x * rms) * wv[i].x; v[i].y = (v[i].y * rms) * wv[i].y;
        v[i].z = (v[i].z * rms) * wv[i].z; v[i].w = (v[i].w * rms) * wv[i].w;
      }
      if ((int)threadIdx.x + 256 * i < n4)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    sh = pf_f16_shift(pf_block_max(m, redm));
    if (threadIdx.x == 0) rmsv[t] = rms;
    uint2* qh = reinterpret_cast<uint2*>(xh) + (int64_t)t * n4;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int c = (int)threadIdx.x + 256 * i;
      if (c >= n4) break;
      qh[c] = make_uint2(pf_f16x2(gm_f32x2{v[i].x, v[i].y}, sh), pf_f16x2(gm_f32x2{v[i].z, v[i].w}, sh));
      if (xn32) reinterpret_cast<gm_f32x4*>(xn32 + (int64_t)t * D)[c] = v[i];
    }
  } else {
    // two passes over the row: x^2 and max |x w| (rms > 0 scales the maximum
    // exactly up to rounding, and the target range leaves a factor 2 of f16 room)
    const gm_f32x2* w2 = reinterpret_cast<const gm_f32x2*>(norm_w);
    float ss = 0.f, m = 0.f;
    for (int i = threadIdx.x; i < n2; i += 256) {
      const gm_f32x2 v = x2[i];
      const gm_f32x2 w = norm_w ? w2[i] : gm_f32x2{1.f, 1.f};
      ss = fmaf(v.x, v.x, fmaf(v.y, v.y, ss));
      m = fmaxf(m, fmaxf(fabsf(v.x * w.x), fabsf(v.y * w.y)));
    }
    float rms = 1.f;
    if (norm_w) {
      ss = gm_wave_sum64(ss);
      if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
      __syncthreads();
      rms = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)D + eps);
    }
    sh = pf_f16_shift(pf_block_max(m, redm) * rms);
    if (threadIdx.x == 0) rmsv[t] = rms;
    uint32_t* ph = reinterpret_cast<uint32_t*>(xh) + (int64_t)t * n2;
    for (int i = threadIdx.x; i < n2; i += 256) {
      gm_f32x2 v = x2[i];
      if (norm_w) { const gm_f32x2 w = w2[i]; v.x = (v.x * rms) * w.x; v.y = (v.y * rms) * w.y; }
      ph[i] = pf_f16x2(v, sh);
      if (xn32) reinterpret_cast<gm_f32x2*>(xn32 + (int64_t)t * D)[i] = v;
    }
  }
  if (threadIdx.x == 0) xsc[t] = __builtin_ldexpf(1.0f, -sh);
}

// ---------------------------------------------------------------- router
// Partial router dot products part[z][t][r] = (x[t] w_norm) . W[r] over the z-th
// K range of kr = 128 NK values (rows r < E of W and row E = the shared gate
// vector, qwen/forward.py:599-600, 608; the token's RMSNorm factor is applied to
// the summed partials by k_pf_topk, so no block needs a whole row of x).  Block:
// 64 rows x 16 tokens x one K range; wave w takes the w-th quarter of the range
// for all four 16-row tiles, and issues every operand load of its NK k-steps (x,
// the norm weights and the router rows) before its first MFMA (one memory round
// trip); x w_norm is formed in fp32 and split into three bf16 planes in
// registers.  The four waves' tiles are added in LDS in wave order.
// MFMA operand layout (16x16x32): lane l holds row / column l % 16 at
// k = 8 (l / 16) .. +7.

// An fp32 router (RF32) is split in registers into three bf16 pieces,
// w = w0 + w1 + w2 exactly (each piece holds the next 8 significant bits of
// the 24; exact unless |w| < 2^-100, where bf16 subnormals cut the last
// piece), and all nine piece products are accumulated.
__device__ __forceinline__ void split3_bf16(const gm_u32x4 (&r)[2], gm_bf16x8 (&o)[3]) {
  gm_f32x8 v;
  v[0] = __uint_as_float(r[0].x); v[1] = __uint_as_float(r[0].y);
  v[2] = __uint_as_float(r[0].z); v[3] = __uint_as_float(r[0].w);
  v[4] = __uint_as_float(r[1].x); v[5] = __uint_as_float(r[1].y);
  v[6] = __uint_as_float(r[1].z); v[7] = __uint_as_float(r[1].w);
  o[0] = __builtin_convertvector(v, gm_bf16x8);
  const gm_f32x8 r0 = v - __builtin_convertvector(o[0], gm_f32x8);
  o[1] = __builtin_convertvector(r0, gm_bf16x8);
  const gm_f32x8 r1 = r0 - __builtin_convertvector(o[1], gm_f32x8);
  o[2] = __builtin_convertvector(r1, gm_bf16x8);
}

template <bool RF32>
__device__ __forceinline__ void router_step(const gm_u32x4 (&a)[4][RF32 ? 2 : 1], const gm_u32x4 (&b)[3],
                                            gm_f32x4 (&acc)[4]) {
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    if constexpr (RF32) {
      gm_bf16x8 ap[3];
      split3_bf16(a[rt], ap);
#pragma unroll
      for (int pa = 0; pa < 3; ++pa)
#pragma unroll
        for (int p = 0; p < 3; ++p)
          acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[pa], __builtin_bit_cast(gm_bf16x8, b[p]), acc[rt], 0,
                                                            0, 0);
    } else {
#pragma unroll
      for (int p = 0; p < 3; ++p)
        acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gm_bf16x8, a[rt][0]),
                                                          __builtin_bit_cast(gm_bf16x8, b[p]), acc[rt], 0, 0, 0);
    }
  }
}

template <int NK, bool RF32>
__device__ __forceinline__ void pf_router_block(int rb, int tb, int z, const void* __restrict__ w,
                                                const void* __restrict__ wsh, const float* __restrict__ x,
                                                const float* __restrict__ norm_w, int T, int D, int E, int ldp,
                                                float* __restrict__ part, gm_f32x4 (*red)[4][64]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, q = lane >> 4;
  const int nrows = E + (wsh ? 1 : 0);
  const int r0 = rb * 64;
  const int tok = tb * 16 + l16;
  const int tokc = tok < T ? tok : T - 1;
  const int k0 = (z * 4 + wave) * (32 * NK);
  const gm_f32x4* xrow = reinterpret_cast<const gm_f32x4*>(x + (int64_t)tokc * D + k0 + 8 * q);
  const gm_f32x4* nrow = reinterpret_cast<const gm_f32x4*>((norm_w ? norm_w : x) + k0 + 8 * q);
  constexpr int RW = RF32 ? 2 : 1;                              // 16-byte loads per 8 weights
  gm_u32x4 a[NK][4][RW];
  gm_f32x4 xv[NK][2], nv[NK][2];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const int row = r0 + rt * 16 + l16;
    const void* pr = row < E ? router_row<RF32>(w, row, D) : (row == E && wsh ? wsh : w);
    const gm_u32x4* ar = reinterpret_cast<const gm_u32x4*>(static_cast<const char*>(pr) + (k0 + 8 * q) * 2 * RW);
#pragma unroll
    for (int ks = 0; ks < NK; ++ks)
#pragma unroll
      for (int h = 0; h < RW; ++h) a[ks][rt][h] = ar[4 * RW * ks + h];
  }
#pragma unroll
  for (int ks = 0; ks < NK; ++ks)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      xv[ks][h] = xrow[8 * ks + h];
      nv[ks][h] = nrow[8 * ks + h];                             // x again without a norm: not used
    }
  gm_f32x4 acc[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) acc[rt] = gm_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < NK; ++ks) {
    gm_u32x4 xw[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const gm_f32x4 v = norm_w ? xv[ks][h] * nv[ks][h] : xv[ks][h];
      xw[h] = __builtin_bit_cast(gm_u32x4, v);
    }
    gm_bf16x8 pl[3];
    split3_bf16(xw, pl);
    const gm_u32x4 b[3] = {__builtin_bit_cast(gm_u32x4, pl[0]), __builtin_bit_cast(gm_u32x4, pl[1]),
                           __builtin_bit_cast(gm_u32x4, pl[2])};
    router_step<RF32>(a[ks], b, acc);
  }
  if (wave > 0) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) red[wave - 1][rt][lane] = acc[rt];
  }
  __syncthreads();
  if (wave > 0 || tok >= T) return;
#pragma unroll
  for (int v = 0; v < 3; ++v)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[rt] += red[v][rt][lane];
  float* out = part + ((int64_t)z * T + tok) * ldp;
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const int row = r0 + rt * 16 + 4 * q;
    if (row + 3 < nrows) *reinterpret_cast<gm_f32x4*>(out + row) = acc[rt];
    else
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (row + i < nrows) out[row + i] = acc[rt][i];
  }
}

// Blocks [0, n_rt): the router blocks (row block, token tile, K range) = (b %
// nrb, b / nrb % ntb, b / (nrb ntb)); blocks [n_rt, n_rt + T): the prep of
// token b - n_rt.  The two roles share nothing: the launch replaces a prep
// launch followed by a router launch.
template <int NK, bool RF32>
__global__ void __launch_bounds__(256) k_pf_prep_router(const void* __restrict__ w, const void* __restrict__ wsh,
                                                        const float* __restrict__ x, const float* __restrict__ norm_w,
                                                        float eps, int T, int D, int E, int ldp,
                                                        float* __restrict__ part, int nrb, int ntb, int n_rt,
                                                        uint16_t* __restrict__ xh, float* __restrict__ xsc,
                                                        float* __restrict__ xn32, float* __restrict__ rmsv) {
  __shared__ gm_f32x4 red[3][4][64];
  __shared__ float pred[4], predm[4];
  const int b = blockIdx.x;
  if (b >= n_rt) {                                              // uniform per block
    pf_prep_token(b - n_rt, x, D, norm_w, eps, xh, xsc, xn32, rmsv, pred, predm);
    return;
  }
  pf_router_block<NK, RF32>(b % nrb, (b / nrb) % ntb, b / (nrb * ntb), w, wsh, x, norm_w, T, D, E, ldp, part, red);
}

// One wave per token: logits = the token's RMSNorm factor x the sum of the
// nsplit <= NZ partials (fixed order) + bias, the shared gate sigmoid, and the top-k (ties -> lower id) with
// renormalised softmax weights (qwen/forward.py:609-611).  Every partial is
// loaded (clamped index) before any is summed.
template <int MAXV, int NZ>
__global__ void __launch_bounds__(256) k_pf_topk(const float* __restrict__ part, int ldp, int nsplit, int T, int E, int k,
                                                 int has_gate, const float* __restrict__ bias,
                                                 const float* __restrict__ rmsv,
                                                 float* __restrict__ logits, float* __restrict__ shg,
                                                 int32_t* __restrict__ ids, float* __restrict__ wts) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  const int64_t zs = (int64_t)T * ldp;
  const float* pt = part + (int64_t)t * ldp;
  const float rms = rmsv[t];
  float v[MAXV], pv[MAXV][NZ], pg[NZ];
  int ix[MAXV];
#pragma unroll
  for (int z = 0; z < NZ; ++z) {
    const int64_t zo = (int64_t)(z < nsplit ? z : nsplit - 1) * zs;
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      const int r = lane + 64 * i;
      pv[i][z] = pt[zo + (r < E ? r : E - 1)];
    }
    pg[z] = pt[zo + E];
  }
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    ix[i] = lane + 64 * i;
    const int r = ix[i] < E ? ix[i] : E - 1;
    float acc = 0.f;
#pragma unroll
    for (int z = 0; z < NZ; ++z) acc += z < nsplit ? pv[i][z] : 0.f;
    v[i] = rms * acc + (bias ? bias[r] : 0.f);
    if (ix[i] < E) logits[(int64_t)t * E + ix[i]] = v[i];
  }
  if (lane == 0) {                                          // no gate row: the shared expert is ungated
    float g = 0.f;
#pragma unroll
    for (int z = 0; z < NZ; ++z) g += z < nsplit ? pg[z] : 0.f;
    shg[t] = has_gate ? gm_sigmoid(rms * g) : 1.f;
  }
  int id;
  float wt;
  topk_finish<MAXV>(v, ix, E, k, id, wt);
  if (lane < k) {
    ids[(int64_t)t * k + lane] = id;
    wts[(int64_t)t * k + lane] = wt;
  }
}

// ------------------------------------------------------- raw superblocks
// The bytes of one superblock of one weight row that lane quarter q needs.
// Lane quarter q covers sub-blocks 2q and 2q+1 of every superblock; k-step j
// (0..7) of the superblock uses sub-block 2q + (j >> 2).
template <int QT> struct PfRaw;
template <> struct PfRaw<GM_QTYPE_IQ4_XS> {
  uint32_t h0, h1;      // d | scales_h, scales_l[0..3]
  uint32_t q[8];        // qs bytes 32q .. 32q+31 (sub-blocks 2q, 2q+1)
};
template <> struct PfRaw<GM_QTYPE_IQ3_XXS> {
  uint32_t d;           // fp16 bits
  uint32_t q[4];        // qs bytes 16q .. 16q+15 (sub-blocks 2q, 2q+1)
  uint32_t w0, w1;      // scale/sign words 2q, 2q+1
};

// IQ4_XS superblocks are 8-byte aligned (136 = 8 * 17, rows of whole superblocks).
__device__ __forceinline__ PfRaw<GM_QTYPE_IQ4_XS> pf_load_iq4(const uint8_t* __restrict__ sb, int q) {
  PfRaw<GM_QTYPE_IQ4_XS> r;
  const uint2 h = *reinterpret_cast<const uint2*>(sb);
  const uint2* p = reinterpret_cast<const uint2*>(sb + 8 + 32 * q);
  r.h0 = h.x; r.h1 = h.y;
#pragma unroll
  for (int i = 0; i < 4; ++i) { const uint2 v = p[i]; r.q[2 * i] = v.x; r.q[2 * i + 1] = v.y; }
  return r;
}

// IQ3_XXS superblocks are 2-byte aligned (98 B): dword loads re-aligned with
// v_alignbyte_b32.  Every dword read holds at least one byte of this
// superblock, so no read leaves the superblock's 4 KB page.
__device__ __forceinline__ PfRaw<GM_QTYPE_IQ3_XXS> pf_load_iq3(const uint8_t* __restrict__ sb, int q) {
  PfRaw<GM_QTYPE_IQ3_XXS> r;
  const int odd = (int)((reinterpret_cast<uintptr_t>(sb) >> 1) & 1);     // sb % 4 == 2 * odd
  const int rq = odd ? 0 : 2;                                           // (sb + 2) % 4
  const uint32_t* dp = reinterpret_cast<const uint32_t*>(sb - 2 * odd);
  const uint32_t dw = dp[0];
  r.d = odd ? (dw >> 16) : (dw & 0xffffu);
  const uint32_t* qp = reinterpret_cast<const uint32_t*>(sb + 2 + 16 * q - rq);
  uint32_t v[5];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = qp[i];
  v[4] = qp[rq ? 4 : 3];
#pragma unroll
  for (int i = 0; i < 4; ++i) r.q[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], rq);
  const uint32_t* wp = reinterpret_cast<const uint32_t*>(sb + 66 + 8 * q - rq);
  const uint32_t w0 = wp[0], w1 = wp[1], w2 = wp[rq ? 2 : 1];
  r.w0 = __builtin_amdgcn_alignbyte(w1, w0, rq);
  r.w1 = __builtin_amdgcn_alignbyte(w2, w1, rq);
  return r;
}

template <int QT>
__device__ __forceinline__ PfRaw<QT> pf_load(const uint8_t* __restrict__ sb, int q) {
  if constexpr (QT == GM_QTYPE_IQ4_XS) return pf_load_iq4(sb, q);
  else return pf_load_iq3(sb, q);
}

// Sub-block scales of the lane's two sub-blocks (2q, 2q+1): the full scale
// (bf16 path) or, for the f16 path, only its integer factor, with the
// superblock factor pf_dscale applied to the fp32 accumulator instead:
//   IQ4_XS: d * (ls - 32)            -> integer ls - 32 in [-32, 31], factor d
//   IQ3_XXS: d * (0.5 + s4) * 0.5    -> integer 2 s4 + 1 in [1, 31], factor d / 4
// so every f16 weight is an integer product, exact up to 2048 in magnitude:
// |(2 s4 + 1) g| <= 1922 is always exact, |kv (ls - 32)| <= 4064 is rounded
// once to f16's 11 significant bits when odd and above 2048; f16's small
// exponent range never meets a tiny d.
template <int QT>
__device__ __forceinline__ gm_f32x2 pf_scales(const PfRaw<QT>& r, int q) {
  if constexpr (QT == GM_QTYPE_IQ4_XS) {
    const float d = gm_h2f(r.h0 & 0xffffu);
    const uint32_t sh = r.h0 >> 16, sl = (r.h1 >> (8 * q)) & 0xffu;
    const int ls0 = (int)((sl & 15u) | (((sh >> (4 * q)) & 3u) << 4));
    const int ls1 = (int)((sl >> 4) | (((sh >> (4 * q + 2)) & 3u) << 4));
    return gm_f32x2{d * (float)(ls0 - 32), d * (float)(ls1 - 32)};
  } else {
    const float d = gm_h2f(r.d);
    return gm_f32x2{d * (0.5f + (float)(r.w0 >> 28)) * 0.5f, d * (0.5f + (float)(r.w1 >> 28)) * 0.5f};
  }
}

template <int QT>
__device__ __forceinline__ gm_f32x2 pf_int_scales(const PfRaw<QT>& r, int q) {
  if constexpr (QT == GM_QTYPE_IQ4_XS) {
    const uint32_t sh = r.h0 >> 16, sl = (r.h1 >> (8 * q)) & 0xffu;
    const int ls0 = (int)((sl & 15u) | (((sh >> (4 * q)) & 3u) << 4));
    const int ls1 = (int)((sl >> 4) | (((sh >> (4 * q + 2)) & 3u) << 4));
    return gm_f32x2{(float)(ls0 - 32), (float)(ls1 - 32)};
  } else {
    return gm_f32x2{(float)(2 * (r.w0 >> 28) + 1), (float)(2 * (r.w1 >> 28) + 1)};
  }
}

template <int QT>
__device__ __forceinline__ float pf_dscale(const PfRaw<QT>& r) {
  if constexpr (QT == GM_QTYPE_IQ4_XS) return gm_h2f(r.h0 & 0xffffu);
  else return gm_h2f(r.d) * 0.25f;
}

// kvalues_iq4nl + 128 as unsigned bytes (entry n in byte n % 4 of word n / 4).
constexpr uint32_t kKvU[4] = {kGmKv[0] ^ 0x80808080u, kGmKv[1] ^ 0x80808080u, kGmKv[2] ^ 0x80808080u,
                              kGmKv[3] ^ 0x80808080u};

// Two-lookup XOR form of the table (see gm_lut16_xor), checked at compile time.
constexpr gm_iq4_xor::Tabs kKvUx = gm_iq4_xor::solve(kKvU);
static_assert(gm_iq4_xor::check(kKvU, kKvUx), "XOR lookup of kvalues + 128");

__device__ __forceinline__ uint32_t lut_kvu(uint32_t nib) { return gm_lut16_xor(kKvUx, nib); }

// Four unsigned bytes u -> two f16x2 holding (u - 128) * s, rounded once:
// 0x6400 | u is the f16 1024 + u, and fma(1024 + u, s, c) with c = -1152 s
// (exact in f16 for |s| <= 32: 9 s 2^7) is (u - 128) s in one rounding.
__device__ __forceinline__ void u8x4_to_f16(uint32_t u, gm_f16x2 s, gm_f16x2 c, uint32_t& o0, uint32_t& o1) {
  const gm_f16x2 a = __builtin_bit_cast(gm_f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
  const gm_f16x2 b = __builtin_bit_cast(gm_f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
  o0 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(a, s, c));
  o1 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(b, s, c));
}

// IQ3_XXS sign table for k-step decode: entry i (7-bit ksigns index) holds
// byte masks (0x00 / 0xff) for the 8 signs of ksigns(i) and the same masks
// & 0x01 per byte: {signs 0-3, signs 4-7, low bits 0-3, low bits 4-7}.
__device__ __forceinline__ void pf_stage_signs_u8(gm_u32x4* tab) {
  for (int i = threadIdx.x; i < 128; i += blockDim.x) {
    const uint32_t s = gm_ksigns((uint32_t)i);
    uint32_t m0 = 0, m1 = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      m0 |= ((s >> b) & 1u) ? 0xffu << (8 * b) : 0u;
      m1 |= ((s >> (b + 4)) & 1u) ? 0xffu << (8 * b) : 0u;
    }
    tab[i] = gm_u32x4{m0, m1, m0 & 0x01010101u, m1 & 0x01010101u};
  }
}

// f16 A operand of k-step j: 8 weights (scale folded in) at the lane's k-slots
// k = 32s + 8c + i (i < 8), s = 2q + (j >> 2), c = j & 3, so that the matching
// activations are 8 consecutive values:
//   IQ4_XS: the low (c < 2) or high (c >= 2) nibbles of qs bytes 8 (c & 1) .. + 7
//   IQ3_XXS: grid points 2c, 2c + 1 of the sub-block
template <int QT>
__device__ __forceinline__ gm_f16x8 a_f16(const PfRaw<QT>& r, int j, gm_f16x2 sc, gm_f16x2 cc,
                                          const uint32_t* __restrict__ grid,
                                          const gm_u32x4* __restrict__ sgn) {
  uint32_t o[4];
  if constexpr (QT == GM_QTYPE_IQ4_XS) {
    const int sl = j >> 2, c = j & 3, sh = 4 * (c >> 1);
    const uint32_t w0 = r.q[4 * sl + 2 * (c & 1)], w1 = r.q[4 * sl + 2 * (c & 1) + 1];
    u8x4_to_f16(lut_kvu((w0 >> sh) & 0x0f0f0f0fu), sc, cc, o[0], o[1]);
    u8x4_to_f16(lut_kvu((w1 >> sh) & 0x0f0f0f0fu), sc, cc, o[2], o[3]);
  } else {
    const int sl = j >> 2, g = j & 3;
    const uint32_t qw = r.q[2 * sl + (g >> 1)] >> (16 * (g & 1));
    const uint32_t ga = grid[qw & 0xffu], gb = grid[(qw >> 8) & 0xffu];
    const uint32_t w = sl ? r.w1 : r.w0;
    const gm_u32x4 m = sgn[(w >> (7 * g)) & 127u];
    // signed magnitude + 128 per byte: |v| <= 62, so no byte carries into the next
    const uint32_t ua = ((ga ^ m.x) + m.z) ^ 0x80808080u;
    const uint32_t ub = ((gb ^ m.y) + m.w) ^ 0x80808080u;
    u8x4_to_f16(ua, sc, cc, o[0], o[1]);
    u8x4_to_f16(ub, sc, cc, o[2], o[3]);
  }
  return __builtin_bit_cast(gm_f16x8, gm_u32x4{o[0], o[1], o[2], o[3]});
}

// B operand of k-step j from an LDS activation row: the 8 activations of the
// lane's k-slots are contiguous, so one 16-byte read.
__device__ __forceinline__ gm_u32x4 b_lds(const uint8_t* __restrict__ row, int q, int j) {
  return *reinterpret_cast<const gm_u32x4*>(row + 2 * (32 * (2 * q + (j >> 2)) + 8 * (j & 3)));
}

// The same from row r of a gate/up activation tile, whose granule g (8 values)
// of row r sits at slot g ^ (r & 15): the 16 rows a wave reads at once then hit
// 16 different 16-byte bank groups without padding the 512-byte rows.
__device__ __forceinline__ gm_u32x4 b_lds_swz(const uint8_t* __restrict__ tile, int r, int q, int j) {
  const int g = 4 * (2 * q + (j >> 2)) + (j & 3);
  return *reinterpret_cast<const gm_u32x4*>(tile + r * kRowB + 16 * (g ^ (r & 15)));
}

// Half H (k-steps 4H .. 4H+3) of one superblock column of the gate and up
// rows against NT token tiles: f16 integer operands into the superblock's
// partial sums pg / pu.
template <int QT, int NT, int H>
__device__ __forceinline__ void gu_half(const PfRaw<QT>& wg, const PfRaw<QT>& wu, int q, int l16,
                                        const uint8_t* __restrict__ xb, const uint32_t* __restrict__ grid,
                                        const gm_u32x4* __restrict__ sgn, gm_f32x4 (&pg)[kNT], gm_f32x4 (&pu)[kNT]) {
  const gm_f32x2 sg2 = pf_int_scales<QT>(wg, q), su2 = pf_int_scales<QT>(wu, q);
  const float sgf = H ? sg2.y : sg2.x, suf = H ? su2.y : su2.x;
  const gm_f16x2 sgh = {(_Float16)sgf, (_Float16)sgf}, suh = {(_Float16)suf, (_Float16)suf};
  const gm_f16x2 cgh = {(_Float16)(-1152.f * sgf), (_Float16)(-1152.f * sgf)};
  const gm_f16x2 cuh = {(_Float16)(-1152.f * suf), (_Float16)(-1152.f * suf)};
#pragma unroll
  for (int j = 4 * H; j < 4 * H + 4; ++j) {
    const gm_f16x8 A = a_f16<QT>(wg, j, sgh, cgh, grid, sgn);
    const gm_f16x8 U = a_f16<QT>(wu, j, suh, cuh, grid, sgn);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const gm_f16x8 B = __builtin_bit_cast(gm_f16x8, b_lds_swz(xb, t * 16 + l16, q, j));
      pg[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, pg[t], 0, 0, 0);
      pu[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(U, B, pu[t], 0, 0, 0);
    }
    if (j & 1) issue_fence();                          // two k-steps' operands live at a time
  }
}

// The superblock's partial sums times the superblock factor of each
// accumulator row (rows 4q + i, whose factors lanes 4q + i hold) into ag / au.
template <int QT, int NT>
__device__ __forceinline__ void gu_fold(const PfRaw<QT>& wg, const PfRaw<QT>& wu, int q, const gm_f32x4 (&pg)[kNT],
                                        const gm_f32x4 (&pu)[kNT], gm_f32x4 (&ag)[kNT], gm_f32x4 (&au)[kNT]) {
  const float dgl = pf_dscale<QT>(wg), dul = pf_dscale<QT>(wu);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float dg = __shfl(dgl, 4 * q + i, 64), du = __shfl(dul, 4 * q + i, 64);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      ag[t][i] = fmaf(dg, pg[t][i], ag[t][i]);
      au[t][i] = fmaf(du, pu[t][i], au[t][i]);
    }
  }
}

// One superblock column of two down row tiles against NT token tiles: f16
// integer operands into the superblock's partial sums, then the partial sums
// times the superblock factor of each accumulator row into acc.
template <int QT, int NT>
__device__ __forceinline__ void dn_superblock(const PfRaw<QT>& w0, const PfRaw<QT>& w1, int q, int l16,
                                              const uint8_t* __restrict__ hbuf, int pitch,
                                              const uint32_t* __restrict__ grid, const gm_u32x4* __restrict__ sgn,
                                              gm_f32x4 (&acc)[2][kNT]) {
  const gm_f32x2 s0 = pf_int_scales<QT>(w0, q), s1 = pf_int_scales<QT>(w1, q);
  gm_f32x4 p0[NT], p1[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) { p0[t] = gm_f32x4{0.f, 0.f, 0.f, 0.f}; p1[t] = p0[t]; }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float f0 = j < 4 ? s0.x : s0.y, f1 = j < 4 ? s1.x : s1.y;
    const gm_f16x2 h0 = {(_Float16)f0, (_Float16)f0}, h1 = {(_Float16)f1, (_Float16)f1};
    const gm_f16x2 c0 = {(_Float16)(-1152.f * f0), (_Float16)(-1152.f * f0)};
    const gm_f16x2 c1 = {(_Float16)(-1152.f * f1), (_Float16)(-1152.f * f1)};
    const gm_f16x8 A0 = a_f16<QT>(w0, j, h0, c0, grid, sgn);
    const gm_f16x8 A1 = a_f16<QT>(w1, j, h1, c1, grid, sgn);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const gm_f16x8 B = __builtin_bit_cast(gm_f16x8, b_lds(hbuf + (t * 16 + l16) * pitch, q, j));
      p0[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B, p0[t], 0, 0, 0);
      p1[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B, p1[t], 0, 0, 0);
    }
    if (j & 1) issue_fence();
  }
  const float d0l = pf_dscale<QT>(w0), d1l = pf_dscale<QT>(w1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float d0 = __shfl(d0l, 4 * q + i, 64), d1 = __shfl(d1l, 4 * q + i, 64);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      acc[0][t][i] = fmaf(d0, p0[t][i], acc[0][t][i]);
      acc[1][t][i] = fmaf(d1, p1[t][i], acc[1][t][i]);
    }
  }
}

// ------------------------------------------------------------- h to f16
// One wave per SwiGLU row (FF <= 2048: 4 granules of 8 values per lane): the
// bf16 row scaled by 2^-e, e chosen so that its largest |value| lands in
// [2^14, 2^15), is exact in f16 (11 significand bits >= bf16's 8) for every
// value above 2^-29 of the largest; hsc[row] = 2^e, which the down kernel
// multiplies into its outputs.
__global__ void __launch_bounds__(256) k_pf_h16(const uint16_t* __restrict__ hb, int rows, int FF,
                                                uint16_t* __restrict__ hh, float* __restrict__ hsc) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const gm_u32x4* src = reinterpret_cast<const gm_u32x4*>(hb + (int64_t)r * FF);
  gm_u32x4* dst = reinterpret_cast<gm_u32x4*>(hh + (int64_t)r * FF);
  const int ng = FF >> 3;                                      // 16-byte granules per row
  constexpr int G = 4;                                         // FF <= 2048
  gm_u32x4 v[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + 64 * i;
    v[i] = src[g < ng ? g : ng - 1];
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      m = fmaxf(m, fmaxf(fabsf(gm_bf2f(w[c] & 0xffffu)), fabsf(gm_bf2f(w[c] >> 16))));
  }
  m = fmaxf(m, GM_DPP_F(m, GM_ROW_ROR8));
  m = fmaxf(m, GM_DPP_F(m, GM_ROW_ROR4));
  m = fmaxf(m, GM_DPP_F(m, GM_QPERM_2301));
  m = fmaxf(m, GM_DPP_F(m, GM_QPERM_1032));
  m = fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 0)),
                  __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 16))),
            fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 32)),
                  __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 48))));
  // m in [2^(E-1), 2^E): scale so that the largest value lands in [2^14, 2^15)
  const int e = m > 0.f && m <= 3.4e38f ? __builtin_amdgcn_frexp_expf(m) - 15 : 0;
  const float down = __builtin_ldexpf(1.0f, -e);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + 64 * i;
    const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
    uint32_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const gm_f32x2 f = {gm_bf2f(w[c] & 0xffffu) * down, gm_bf2f(w[c] >> 16) * down};
      o[c] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, gm_f16x2));
    }
    if (g < ng) dst[g] = gm_u32x4{o[0], o[1], o[2], o[3]};
  }
  if (lane == 0) hsc[r] = m <= 3.4e38f ? __builtin_ldexpf(1.0f, e) : __builtin_nanf("");
}

// Activation chunk [c0, c0 + 256) of the segment's rows <-> registers: kSegTok rows
// x 32 granules of 16 B, granule g = threadIdx + 256 i for i in [I0, I0 + N)
// (rows past n repeat a valid row; their output columns are never stored).
template <int N>
struct ActRegs { gm_u32x4 v[N]; };

template <int N>
__device__ __forceinline__ void act_load(ActRegs<N>& a, const uint16_t* __restrict__ src, int K,
                                         const int32_t* __restrict__ rows, int c0, int i0 = 0) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int g = threadIdx.x + 256 * (i0 + i), r = g >> 5, c = g & 31;
    a.v[i] = *reinterpret_cast<const gm_u32x4*>(src + (int64_t)rows[r] * K + c0 + 8 * c);
  }
}

template <int N>
__device__ __forceinline__ void act_store(const ActRegs<N>& a, uint8_t* __restrict__ buf, int pitch, int i0 = 0) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int g = threadIdx.x + 256 * (i0 + i), r = g >> 5, c = g & 31;
    *reinterpret_cast<gm_u32x4*>(buf + r * pitch + 16 * c) = a.v[i];
  }
}

// Chunk [c0, c0 + kChunk) of the segment's kSegTok f16 activation rows into the
// swizzled tile with global -> LDS loads (no registers, no wait here): wave
// instruction m of wave w writes 1 KB, rows 2 mi and 2 mi + 1 (mi = NI w + m);
// lane i lands at slot i & 31 of row 2 mi + (i >> 5) and so loads granule
// (i & 31) ^ (row & 15) of that row.
__device__ __forceinline__ void act_lds_load(const uint16_t* __restrict__ src, int K,
                                             const int32_t* __restrict__ rows, int c0, uint8_t* __restrict__ tile) {
  constexpr int NI = kSegTok * (kRowB / 16) / 256;                     // 1 KB loads per wave
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < NI; ++m) {
    const int mi = wave * NI + m, r = 2 * mi + (lane >> 5), c = (lane & 31) ^ (r & 15);
    __builtin_amdgcn_global_load_lds(src + (int64_t)rows[r] * K + c0 + 8 * c, tile + mi * 1024, 16, 0, 0);
  }
}

// -------------------------------------------------------------- gate/up
// Block = (segment, 64 rows of FF); wave w -> rows 16w .. 16w+15 of both the
// gate and the up matrix, all of the segment's token tiles.
template <int QT>
__global__ void __launch_bounds__(256, kSegTok == 64 ? 2 : 3) k_pf_gateup(gm_moe_layer P, const int32_t* __restrict__ segs,
                                                      const int32_t* __restrict__ offsets,
                                                      const int32_t* __restrict__ sorted,
                                                      const uint16_t* __restrict__ xh,
                                                      const float* __restrict__ xsc, uint16_t* __restrict__ hb,
                                                      int T, int n_row_tiles) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* xl = smem;                                                   // [2][kSegTok][kRowB]
  uint32_t* grid = reinterpret_cast<uint32_t*>(smem + 2 * kTileG);      // [256] (IQ3)
  gm_u32x4* sgn = reinterpret_cast<gm_u32x4*>(grid + 256);              // [128] (IQ3)
  int32_t* tok_row = reinterpret_cast<int32_t*>(sgn + 128);             // [64]
  int32_t* out_row = tok_row + kSegTok;                                 // [kSegTok]
  int seg, rt;
  xcd_tile(blockIdx.x, n_row_tiles, seg, rt);
  if (seg >= segs[0]) return;
  const int e = segs[1 + 4 * seg], start = segs[2 + 4 * seg], n = segs[3 + 4 * seg];
  const int D = P.D, FF = P.FF, k = P.k, E = P.E;
  const bool shared = e == E;
  if constexpr (QT == GM_QTYPE_IQ3_XXS) {
    gm_stage_grid(grid);
    pf_stage_signs_u8(sgn);
  }
  if (threadIdx.x < kSegTok) {
    const int c = threadIdx.x;
    int tr = 0, orow = 0;
    if (c < n) {
      if (shared) { tr = start + c; orow = T * k + start + c; }
      else { const int pos = offsets[e] + start + c; tr = sorted[pos] / k; orow = pos; }
    } else {
      tr = shared ? start : sorted[offsets[e] + start] / k;     // a valid row of the segment
    }
    tok_row[c] = tr;
    out_row[c] = orow;
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, l16 = lane & 15;
  const int row = rt * 64 + wave * 16 + l16;
  const int64_t rb = gm_row_bytes(QT, D);
  const uint8_t* gbase = shared ? static_cast<const uint8_t*>(P.gate_sh)
                                : static_cast<const uint8_t*>(P.gate_exps) + (int64_t)e * FF * rb;
  const uint8_t* ubase = shared ? static_cast<const uint8_t*>(P.up_sh)
                                : static_cast<const uint8_t*>(P.up_exps) + (int64_t)e * FF * rb;
  const uint8_t* grow = gbase + (int64_t)(row < FF ? row : 0) * rb;
  const uint8_t* urow = ubase + (int64_t)(row < FF ? row : 0) * rb;
  constexpr int SBB = QT == GM_QTYPE_IQ4_XS ? GM_IQ4XS_BYTES : GM_IQ3XXS_BYTES;
  const int nsb = D / kChunk, ntiles = (n + 15) >> 4;
  gm_f32x4 ag[kNT], au[kNT];
#pragma unroll
  for (int t = 0; t < kNT; ++t) { ag[t] = gm_f32x4{0.f, 0.f, 0.f, 0.f}; au[t] = ag[t]; }
  act_lds_load(xh, D, tok_row, 0, xl);
  PfRaw<QT> wg = pf_load<QT>(grow, q), wu = pf_load<QT>(urow, q);
  __builtin_amdgcn_s_waitcnt(0);                                        // the first chunk is in LDS
  __syncthreads();
  for (int sb = 0; sb < nsb; ++sb) {
    // next superblock's raw rows and, straight into the other LDS buffer, its
    // activation chunk (that buffer's last reader finished before the barrier)
    const int sn = sb + 1 < nsb ? sb + 1 : sb;                   // the last step re-reads itself
    const PfRaw<QT> wgn = pf_load<QT>(grow + sn * SBB, q), wun = pf_load<QT>(urow + sn * SBB, q);
    const uint8_t* xb = xl + (sb & 1) * kTileG;
    if (sb + 1 < nsb) act_lds_load(xh, D, tok_row, (sb + 1) * kChunk, xl + ((sb + 1) & 1) * kTileG);
    gm_f32x4 pg[kNT], pu[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) { pg[t] = gm_f32x4{0.f, 0.f, 0.f, 0.f}; pu[t] = pg[t]; }
    nt_dispatch<kNT>(ntiles, [&](auto nt) { gu_half<QT, decltype(nt)::value, 0>(wg, wu, q, l16, xb, grid, sgn, pg, pu); });
    nt_dispatch<kNT>(ntiles, [&](auto nt) {
      gu_half<QT, decltype(nt)::value, 1>(wg, wu, q, l16, xb, grid, sgn, pg, pu);
      gu_fold<QT, decltype(nt)::value>(wg, wu, q, pg, pu, ag, au);
    });
    wg = wgn;
    wu = wun;
    __builtin_amdgcn_s_waitcnt(0);                                      // the next chunk is in LDS
    __syncthreads();
  }
  // C layout: lane l holds rows 4 (l / 16) + i of the 16-row tile, column l % 16
  const int r0 = rt * 64 + wave * 16 + 4 * q;
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int col = t * 16 + l16;
    if (t < ntiles && col < n && r0 < FF) {
      const float ds = xsc[tok_row[col]];                        // the token's f16 scale, undone exactly
      const gm_f32x4 g = ag[t] * ds, u = au[t] * ds;
      gm_f32x2 h01 = {gm_silu(g[0]) * u[0], gm_silu(g[1]) * u[1]};
      gm_f32x2 h23 = {gm_silu(g[2]) * u[2], gm_silu(g[3]) * u[3]};
      *reinterpret_cast<uint2*>(hb + (int64_t)out_row[col] * FF + r0) =
          make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(h01, gm_bf16x2)),
                     __builtin_bit_cast(uint32_t, __builtin_convertvector(h23, gm_bf16x2)));
    }
  }
}

// ------------------------------------------------------------------ down
// Block = (segment, rg_per_blk groups of 128 rows of D).  The segment's whole
// h tile (kSegTok rows x FF, FF = 256 NSB) is staged in LDS once; the block then
// walks its row groups with the next group's raw superblocks in flight.
// Wave w -> row tiles 2w, 2w+1 (16 rows each) of a group.
template <int QT, int NSB>
__global__ void __launch_bounds__(256, NSB == 4 ? 1 : (kSegTok == 64 || QT == GM_QTYPE_IQ4_XS ? 2 : 3)) k_pf_down(gm_moe_layer P, const int32_t* __restrict__ segs,
                                                    const int32_t* __restrict__ offsets,
                                                    const uint16_t* __restrict__ hh, const float* __restrict__ hsc,
                                                    float* __restrict__ yp, int T, int n_blk, int rg_per_blk) {
  constexpr int PITCH = NSB * 2 * kChunk + 16;                          // bytes per LDS h row
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* hl = smem;                                                   // [64][PITCH]
  uint32_t* grid = reinterpret_cast<uint32_t*>(smem + kSegTok * PITCH);
  gm_u32x4* sgn = reinterpret_cast<gm_u32x4*>(grid + 256);
  int32_t* in_row = reinterpret_cast<int32_t*>(sgn + 128);
  int seg, bi;
  xcd_tile(blockIdx.x, n_blk, seg, bi);
  if (seg >= segs[0]) return;
  const int e = segs[1 + 4 * seg], start = segs[2 + 4 * seg], n = segs[3 + 4 * seg];
  const int D = P.D, FF = P.FF, k = P.k, E = P.E;
  const bool shared = e == E;
  const int row0 = shared ? T * k + start : offsets[e] + start;        // rows of hb / yp
  if constexpr (QT == GM_QTYPE_IQ3_XXS) {
    gm_stage_grid(grid);
    pf_stage_signs_u8(sgn);
  }
  if (threadIdx.x < kSegTok) in_row[threadIdx.x] = row0 + (threadIdx.x < n ? threadIdx.x : 0);
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, l16 = lane & 15;
  const int64_t rb = gm_row_bytes(QT, FF);
  const uint8_t* base = shared ? static_cast<const uint8_t*>(P.down_sh)
                               : static_cast<const uint8_t*>(P.down_exps) + (int64_t)e * D * rb;
  constexpr int SBB = QT == GM_QTYPE_IQ4_XS ? GM_IQ4XS_BYTES : GM_IQ3XXS_BYTES;
  const int n_groups = (D + 127) / 128, g0 = bi * rg_per_blk;
  const int g1 = g0 + rg_per_blk < n_groups ? g0 + rg_per_blk : n_groups;
  auto row_ptr = [&](int g, int m) {
    const int row = g * 128 + wave * 32 + m * 16 + l16;
    return base + (int64_t)(row < D ? row : 0) * rb;
  };
  PfRaw<QT> wc[2][NSB];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) wc[m][sb] = pf_load<QT>(row_ptr(g0, m) + sb * SBB, q);
#pragma unroll
  for (int sb = 0; sb < NSB; ++sb) {
    ActRegs<kGran> ha;
    act_load<kGran>(ha, hh, FF, in_row, sb * kChunk);
    act_store<kGran>(ha, hl + sb * 2 * kChunk, PITCH);
  }
  __syncthreads();
  const int ntiles = (n + 15) >> 4;
  float cs[kNT];                                                        // h scale of each output column
#pragma unroll
  for (int t = 0; t < kNT; ++t) cs[t] = hsc[in_row[t * 16 + l16]];
  for (int g = g0; g < g1; ++g) {
    const int gn = g + 1 < g1 ? g + 1 : g;
    PfRaw<QT> wn[2][NSB];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) wn[m][sb] = pf_load<QT>(row_ptr(gn, m) + sb * SBB, q);
    gm_f32x4 acc[2][kNT];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < kNT; ++t) acc[m][t] = gm_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      const uint8_t* hbuf = hl + sb * 2 * kChunk;
      nt_dispatch<kNT>(ntiles, [&](auto nt) {
        dn_superblock<QT, decltype(nt)::value>(wc[0][sb], wc[1][sb], q, l16, hbuf, PITCH, grid, sgn, acc);
      });
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int r0 = g * 128 + wave * 32 + m * 16 + 4 * q;
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        const int col = t * 16 + l16;
        if (t < ntiles && col < n && r0 < D)
          *reinterpret_cast<gm_f32x4*>(yp + (int64_t)(row0 + col) * D + r0) =
              gm_f32x4{acc[m][t][0] * cs[t], acc[m][t][1] * cs[t], acc[m][t][2] * cs[t], acc[m][t][3] * cs[t]};
      }
    }
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) wc[m][sb] = wn[m][sb];
  }
}

// --------------------------------------------------------------- combine
// One block per token: y = sum_j w_j * yp[pos_j] over the token's experts in
// ascending id (= ascending sorted position), + shared gate * yp[P + t] (+ x).
__global__ void __launch_bounds__(256) k_pf_combine(const float* __restrict__ x, const float* __restrict__ yp,
                                                    const int32_t* __restrict__ inv, const float* __restrict__ wts,
                                                    const float* __restrict__ shg, int T, int k, int D, int has_sh,
                                                    int flags, float* __restrict__ y) {
  const int t = blockIdx.x;
  int pos[8];
  float w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pos[j] = j < k ? inv[t * k + j] : 0x7fffffff;
    w[j] = j < k ? wts[t * k + j] : 0.f;
  }
  // insertion sort by position (k <= 8)
#pragma unroll
  for (int i = 1; i < 8; ++i) {
#pragma unroll
    for (int j = i; j > 0; --j) {
      if (pos[j] < pos[j - 1]) {
        const int tp = pos[j]; pos[j] = pos[j - 1]; pos[j - 1] = tp;
        const float tw = w[j]; w[j] = w[j - 1]; w[j - 1] = tw;
      }
    }
  }
  const float sg = has_sh ? shg[t] : 0.f;
  const int Ptot = T * k, nq = D >> 2;
  const gm_f32x4* yp4 = reinterpret_cast<const gm_f32x4*>(yp);
  const gm_f32x4* x4 = reinterpret_cast<const gm_f32x4*>(x + (int64_t)t * D);
  constexpr int CS = 2;                      // column steps whose loads are issued together
  for (int c0 = threadIdx.x; c0 < nq; c0 += 256 * CS) {
    gm_f32x4 v[CS][9], xv[CS];
#pragma unroll
    for (int u = 0; u < CS; ++u) {
      const int c = min(c0 + 256 * u, nq - 1);                   // past the row: a duplicate, not stored
#pragma unroll
      for (int j = 0; j < 8; ++j) v[u][j] = yp4[(int64_t)(j < k ? pos[j] : pos[0]) * nq + c];
      v[u][8] = yp4[(int64_t)(has_sh ? Ptot + t : pos[0]) * nq + c];
      xv[u] = (flags & GM_MOE_RESIDUAL) ? x4[c] : gm_f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < CS; ++u) {
      const int c = c0 + 256 * u;
      if (c >= nq) break;
      gm_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < k) {
          acc.x = fmaf(w[j], v[u][j].x, acc.x); acc.y = fmaf(w[j], v[u][j].y, acc.y);
          acc.z = fmaf(w[j], v[u][j].z, acc.z); acc.w = fmaf(w[j], v[u][j].w, acc.w);
        }
      if (has_sh) {
        acc.x += sg * v[u][8].x; acc.y += sg * v[u][8].y; acc.z += sg * v[u][8].z; acc.w += sg * v[u][8].w;
      }
      if (flags & GM_MOE_RESIDUAL) {
        acc.x = xv[u].x + acc.x; acc.y = xv[u].y + acc.y; acc.z = xv[u].z + acc.z; acc.w = xv[u].w + acc.w;
      }
      reinterpret_cast<gm_f32x4*>(y + (int64_t)t * D)[c] = acc;
    }
  }
}

// ------------------------------------------------- shared expert in I8 rows
// A shared expert held as I8 rows (the reference model's K-quant shared
// experts, transcoded) beside IQ routed experts runs as two dense GEMMs of its
// own over all T tokens, on the routed experts' f16 MFMA: A = the I8 weights
// decoded to f16 (s q + off, rounded once), B = the tokens' f16 rows (xh for
// gate/up, the scaled SwiGLU rows hh for down).  Wave tile: 16 weight rows x
// 16 kShTiles tokens over a K part, one I8 sub-block (32 k) per step, one
// decoded A operand for kShTiles MFMAs: lane l holds row l % 16 and k-octet
// o = l / 16 of A (8 quants, 8 bytes, and the sub-block's {s0, s1, off}),
// token l % 16 of each token tile and the same octet of B (16 bytes).
// Sub-blocks are loaded kShStep at a time into two register sets used in turn
// (no register copy at the loop latch), so one set's loads are in flight
// while the other is multiplied.
constexpr int kShStep = 2;
constexpr int kShTiles = 4;           // 16-token tiles per wave: one decoded A operand, 4 MFMAs

typedef uint32_t gm_u32x3 __attribute__((ext_vector_type(3)));

struct I8Oct {
  uint2 q;       // quants 8o .. 8o + 7 of the sub-block
  gm_u32x3 m;    // s0 (quants 0-15), s1 (16-31), off
};

__device__ __forceinline__ I8Oct i8_oct_load(const uint8_t* __restrict__ row, int sub, int o) {
  const uint8_t* sb = row + sub * 48;
  return I8Oct{*reinterpret_cast<const uint2*>(sb + 8 * o), *reinterpret_cast<const gm_u32x3*>(sb + 32)};
}

// The octet's 8 weights s q + off as f16 (each rounded once from fp32, where
// s q + off is the transcoded row's exact weight).
__device__ __forceinline__ gm_f16x8 i8_oct_f16(const I8Oct& r, int o) {
  const float sc = __uint_as_float(o < 2 ? r.m.x : r.m.y), off = __uint_as_float(r.m.z);
  gm_f16x8 a;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    a[b] = (_Float16)fmaf(sc, gm_sbyte(r.q.x, b), off);
    a[4 + b] = (_Float16)fmaf(sc, gm_sbyte(r.q.y, b), off);
  }
  return a;
}

// One pipeline stage: kShStep sub-blocks of NW weight rows and of the
// kShTiles token rows.
template <int NW>
struct ShStage {
  I8Oct w[NW][kShStep];
  gm_u32x4 b[kShStep][kShTiles];
};

template <int NW>
__device__ __forceinline__ void sh_stage_load(ShStage<NW>& st, const uint8_t* const (&wrow)[NW],
                                              const uint16_t* const (&brow)[kShTiles], int s0, int o) {
#pragma unroll
  for (int i = 0; i < kShStep; ++i) {
#pragma unroll
    for (int n = 0; n < NW; ++n) st.w[n][i] = i8_oct_load(wrow[n], s0 + i, o);
#pragma unroll
    for (int j = 0; j < kShTiles; ++j) st.b[i][j] = *reinterpret_cast<const gm_u32x4*>(brow[j] + 32 * (s0 + i));
  }
  issue_fence();
}

template <int NW>
__device__ __forceinline__ void sh_stage_mfma(const ShStage<NW>& st, int o, gm_f32x4 (&acc)[NW][kShTiles]) {
#pragma unroll
  for (int i = 0; i < kShStep; ++i) {
#pragma unroll
    for (int n = 0; n < NW; ++n) {
      const gm_f16x8 A = i8_oct_f16(st.w[n][i], o);
#pragma unroll
      for (int j = 0; j < kShTiles; ++j)
        acc[n][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(gm_f16x8, st.b[i][j]), acc[n][j],
                                                           0, 0, 0);
    }
  }
  issue_fence();
}

// acc[n][j] = W_n[rows r0 .. r0 + 15] . brow[j] over sub-blocks [sb, sb + ns) (ns
// a multiple of 2 kShStep) for the lane's token of tile j.
template <int NW>
__device__ __forceinline__ void sh_gemm_tile(const uint8_t* const (&wrow)[NW], const uint16_t* const (&brow)[kShTiles],
                                             int sb, int ns, int o, gm_f32x4 (&acc)[NW][kShTiles]) {
#pragma unroll
  for (int n = 0; n < NW; ++n)
#pragma unroll
    for (int j = 0; j < kShTiles; ++j) acc[n][j] = gm_f32x4{0.f, 0.f, 0.f, 0.f};
  ShStage<NW> sa, sb2;
  const int se = sb + ns;
  sh_stage_load<NW>(sa, wrow, brow, sb, o);
  for (int s0 = sb; s0 < se; s0 += 2 * kShStep) {
    sh_stage_load<NW>(sb2, wrow, brow, s0 + kShStep, o);
    sh_stage_mfma<NW>(sa, o, acc);
    const int s2 = s0 + 2 * kShStep < se ? s0 + 2 * kShStep : s0;      // the last round reloads, unused
    sh_stage_load<NW>(sa, wrow, brow, s2, o);
    sh_stage_mfma<NW>(sb2, o, acc);
  }
}

// K parts: the block's 4 waves split K into nkw parts (4, 2 or 1) of whole
// pipeline rounds and cover 4 / nkw token groups; the parts are added in LDS
// in part order by the group's part-0 wave.
inline int sh_kparts(int nsub) {
  return nsub % (8 * kShStep) == 0 ? 4 : nsub % (4 * kShStep) == 0 ? 2 : 1;
}

// Sums the block's K parts of acc (LDS red: 4 waves x NW x kShTiles x 256
// floats) into the part-0 wave of each token group; true on those waves.
template <int NW>
__device__ __forceinline__ bool sh_reduce(gm_f32x4 (&acc)[NW][kShTiles], int nkw, float* __restrict__ red) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, part = wave % nkw;
  gm_f32x4* r4 = reinterpret_cast<gm_f32x4*>(red);
  if (nkw > 1 && part != 0) {
#pragma unroll
    for (int n = 0; n < NW; ++n)
#pragma unroll
      for (int j = 0; j < kShTiles; ++j) r4[((wave * NW + n) * kShTiles + j) * 64 + lane] = acc[n][j];
  }
  __syncthreads();
  if (part != 0) return false;
  for (int p = 1; p < nkw; ++p)
#pragma unroll
    for (int n = 0; n < NW; ++n)
#pragma unroll
      for (int j = 0; j < kShTiles; ++j) acc[n][j] += r4[(((wave + p) * NW + n) * kShTiles + j) * 64 + lane];
  return true;
}

// h[P + t] = silu(g) u for the shared expert, t < T: block (row tile of 16 FF
// rows, 4 / nkw token groups of 16 kShTiles tokens, nkw K parts each); bf16
// rows as k_pf_gateup writes them.
__global__ void __launch_bounds__(256) k_pfs_gateup_i8(const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu,
                                                       int FF, int D, const uint16_t* __restrict__ xh,
                                                       const float* __restrict__ xsc, int T, int nkw,
                                                       uint16_t* __restrict__ hsh) {
  __shared__ float red[4 * 2 * kShTiles * 256];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, o = lane >> 4;
  const int gpb = 4 / nkw, part = wave % nkw, ns = D / 32 / nkw;
  const int r0 = blockIdx.x * 16, t0 = (blockIdx.y * gpb + wave / nkw) * 16 * kShTiles;
  const int64_t rb = (int64_t)(D / 32) * 48;
  const uint8_t* const wrow[2] = {wg + (r0 + l16) * rb, wu + (r0 + l16) * rb};
  const uint16_t* brow[kShTiles];
#pragma unroll
  for (int j = 0; j < kShTiles; ++j) {                         // tokens past T read a valid row, unstored
    const int t = t0 + 16 * j + l16;
    brow[j] = xh + (int64_t)(t < T ? t : T - 1) * D + 8 * o;
  }
  gm_f32x4 acc[2][kShTiles];
  sh_gemm_tile<2>(wrow, brow, part * ns, ns, o, acc);
  if (!sh_reduce<2>(acc, nkw, red)) return;
#pragma unroll
  for (int j = 0; j < kShTiles; ++j) {                         // C: rows r0 + 4 o + i, token column l16
    const int t = t0 + 16 * j + l16;
    if (t < T) {
      const float ds = xsc[t];
      const gm_f32x4 g = acc[0][j] * ds, u = acc[1][j] * ds;
      const gm_f32x2 h01 = {gm_silu(g[0]) * u[0], gm_silu(g[1]) * u[1]};
      const gm_f32x2 h23 = {gm_silu(g[2]) * u[2], gm_silu(g[3]) * u[3]};
      *reinterpret_cast<uint2*>(hsh + (int64_t)t * FF + r0 + 4 * o) =
          make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(h01, gm_bf16x2)),
                     __builtin_bit_cast(uint32_t, __builtin_convertvector(h23, gm_bf16x2)));
    }
  }
}

// y[t] = W_down h[t] for the shared expert from its scaled f16 rows (hh, scales
// hsc, as k_pf_h16 writes them): block (row tile of 16 D rows, 4 / nkw token
// groups, nkw K parts), fp32 rows y[t] that k_pf_combine adds last.
__global__ void __launch_bounds__(256) k_pfs_down_i8(const uint8_t* __restrict__ wd, int D, int FF,
                                                     const uint16_t* __restrict__ hh, const float* __restrict__ hsc,
                                                     int T, int nkw, float* __restrict__ y) {
  __shared__ float red[4 * kShTiles * 256];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, o = lane >> 4;
  const int gpb = 4 / nkw, part = wave % nkw, ns = FF / 32 / nkw;
  const int r0 = blockIdx.x * 16, t0 = (blockIdx.y * gpb + wave / nkw) * 16 * kShTiles;
  const int64_t rb = (int64_t)(FF / 32) * 48;
  const uint8_t* const wrow[1] = {wd + (r0 + l16) * rb};
  const uint16_t* brow[kShTiles];
#pragma unroll
  for (int j = 0; j < kShTiles; ++j) {
    const int t = t0 + 16 * j + l16;
    brow[j] = hh + (int64_t)(t < T ? t : T - 1) * FF + 8 * o;
  }
  gm_f32x4 acc[1][kShTiles];
  sh_gemm_tile<1>(wrow, brow, part * ns, ns, o, acc);
  if (!sh_reduce<1>(acc, nkw, red)) return;
#pragma unroll
  for (int j = 0; j < kShTiles; ++j) {
    const int t = t0 + 16 * j + l16;
    if (t < T) *reinterpret_cast<gm_f32x4*>(y + (int64_t)t * D + r0 + 4 * o) = acc[0][j] * hsc[t];
  }
}

constexpr size_t kGemmSmem = 2 * (size_t)kTileG + 256 * 4 + 128 * 16 + 2 * kSegTok * 4;

template <int QTG, int QTD>
int prefill_t(const gm_moe_layer* L, const float* x, float* y, int T, int flags, uint8_t* ws, const GmMoeWs& lay,
              hipStream_t s) {
  const int D = L->D, FF = L->FF, E = L->E, k = L->k;
  float* logits = reinterpret_cast<float*>(ws + lay.logits);
  float* shg = reinterpret_cast<float*>(ws + lay.shg);
  int32_t* ids = reinterpret_cast<int32_t*>(ws + lay.ids);
  float* wts = reinterpret_cast<float*>(ws + lay.wts);
  PfWs w = pf_layout(L, T, ws + lay.pre, nullptr);
  const bool has_sh = L->gate_sh != nullptr;
  const bool sh_apart = pf_shared_apart(L);
  const bool sh_gemm = has_sh && !sh_apart;          // the shared expert as the GEMMs' ninth unit
  // a shared expert in I8 rows: its own f16 MFMA GEMMs; other formats (bf16): the fp32 pass
  const bool sh_i8 = sh_apart && L->q_gate_sh == GM_QTYPE_I8 && L->q_up_sh == GM_QTYPE_I8 &&
                     L->q_down_sh == GM_QTYPE_I8;
  const bool sh_f32 = sh_apart && !sh_i8;
  const size_t P = (size_t)T * k;
  const int nrows = E + (L->sh_gate_inp ? 1 : 0);
  const int ldp = router_ld(L);
  const int nsplit = router_split(D);
  {
    const int nrb = (nrows + 63) / 64, ntb = (T + 15) / 16, n_rt = nrb * ntb * nsplit;
    const dim3 g((unsigned)(n_rt + T));
    const bool f32 = L->q_router == GM_QTYPE_F32;
    float* xn32 = sh_f32 ? w.xn : nullptr;
#define GM_PR(NK, F32)                                                                                       \
  hipLaunchKernelGGL((k_pf_prep_router<NK, F32>), g, dim3(256), 0, s, L->router, L->sh_gate_inp, x, L->norm_w, \
                     L->norm_eps, T, D, E, ldp, w.part, nrb, ntb, n_rt, w.xh, w.xsc, xn32, w.rmsv)
    if (router_krange(D) == 512 && f32) GM_PR(4, true);
    else if (router_krange(D) == 512) GM_PR(4, false);
    else if (f32) GM_PR(2, true);
    else GM_PR(2, false);
#undef GM_PR
  }
  GM_TRY(hipGetLastError());
  {
    const int hg = L->sh_gate_inp ? 1 : 0;
    const dim3 g((T + 3) / 4);
    if (E <= 256 && nsplit <= 4)
      hipLaunchKernelGGL((k_pf_topk<4, 4>), g, dim3(256), 0, s, w.part, ldp, nsplit, T, E, k, hg, L->router_bias,
                         w.rmsv, logits, shg, ids, wts);
    else if (E <= 256 && nsplit <= 8)
      hipLaunchKernelGGL((k_pf_topk<4, 8>), g, dim3(256), 0, s, w.part, ldp, nsplit, T, E, k, hg, L->router_bias,
                         w.rmsv, logits, shg, ids, wts);
    else if (E <= 256)
      hipLaunchKernelGGL((k_pf_topk<4, 16>), g, dim3(256), 0, s, w.part, ldp, nsplit, T, E, k, hg, L->router_bias,
                         w.rmsv, logits, shg, ids, wts);
    else if (nsplit <= 8)
      hipLaunchKernelGGL((k_pf_topk<8, 8>), g, dim3(256), 0, s, w.part, ldp, nsplit, T, E, k, hg, L->router_bias,
                         w.rmsv, logits, shg, ids, wts);
    else
      hipLaunchKernelGGL((k_pf_topk<8, 16>), g, dim3(256), 0, s, w.part, ldp, nsplit, T, E, k, hg, L->router_bias,
                         w.rmsv, logits, shg, ids, wts);
  }
  GM_TRY(hipGetLastError());
  if (int rc = gm_launch_dispatch_seg(ids, T, k, E, w.counts, w.offsets, w.sorted, w.inv, w.segs, kSegTok,
                                     sh_gemm ? T : 0, s))
    return rc;
  if (sh_f32) {                                      // shared expert rows yp[P + t], fp32
    if (int rc = gm_launch_gateup(L->q_gate_sh, L->gate_sh, L->up_sh, FF, D, w.xn, T, w.hsh, s)) return rc;
    if (int rc = gm_launch_matvec(L->q_down_sh, L->down_sh, D, FF, w.hsh, T, w.yp + P * D, s)) return rc;
  }
  const int nseg = max_segments(T, k, E);
  {
    const int nrt = FF / 64;
    const int nb = (nseg + 7) / 8 * 8 * nrt;
    if (int rc = gm_set_smem(k_pf_gateup<QTG>, kGemmSmem)) return rc;
    hipLaunchKernelGGL(k_pf_gateup<QTG>, dim3(nb), dim3(256), kGemmSmem, s, *L, w.segs, w.offsets, w.sorted, w.xh,
                       w.xsc, w.hb, T, nrt);
    GM_TRY(hipGetLastError());
  }
  if (sh_i8) {                                       // shared SwiGLU rows hb[P + t] (D % 256 == 0)
    const int nkw = sh_kparts(D / 32), tok = 16 * kShTiles * (4 / nkw);    // tokens per block
    hipLaunchKernelGGL(k_pfs_gateup_i8, dim3(FF / 16, (T + tok - 1) / tok), dim3(256), 0, s,
                       static_cast<const uint8_t*>(L->gate_sh), static_cast<const uint8_t*>(L->up_sh), FF, D, w.xh,
                       w.xsc, T, nkw, w.hb + P * FF);
    GM_TRY(hipGetLastError());
  }
  {
    const int rows = T * k + (sh_gemm || sh_i8 ? T : 0);
    hipLaunchKernelGGL(k_pf_h16, dim3((rows + 3) / 4), dim3(256), 0, s, w.hb, rows, FF, w.hh, w.hsc);
    GM_TRY(hipGetLastError());
  }
  {
    constexpr int kGroupsPerBlock = 2;
    const int n_blk = ((D + 127) / 128 + kGroupsPerBlock - 1) / kGroupsPerBlock;
    const int nb = (nseg + 7) / 8 * 8 * n_blk;
    const size_t smem = kSegTok * (2 * (size_t)FF + 16) + 256 * 4 + 128 * 16 + kSegTok * 4;
    switch (FF / kChunk) {
      case 1:
        if (int rc = gm_set_smem(k_pf_down<QTD, 1>, smem)) return rc;
        hipLaunchKernelGGL((k_pf_down<QTD, 1>), dim3(nb), dim3(256), smem, s, *L, w.segs, w.offsets, w.hh, w.hsc, w.yp,
                           T, n_blk, kGroupsPerBlock);
        break;
      case 2:
        if (int rc = gm_set_smem(k_pf_down<QTD, 2>, smem)) return rc;
        hipLaunchKernelGGL((k_pf_down<QTD, 2>), dim3(nb), dim3(256), smem, s, *L, w.segs, w.offsets, w.hh, w.hsc, w.yp,
                           T, n_blk, kGroupsPerBlock);
        break;
      default:
        if (int rc = gm_set_smem(k_pf_down<QTD, 4>, smem)) return rc;
        hipLaunchKernelGGL((k_pf_down<QTD, 4>), dim3(nb), dim3(256), smem, s, *L, w.segs, w.offsets, w.hh, w.hsc, w.yp,
                           T, n_blk, kGroupsPerBlock);
        break;
    }
    GM_TRY(hipGetLastError());
  }
  if (sh_i8) {                                       // shared expert rows yp[P + t] (FF % 256 == 0)
    const int nkw = sh_kparts(FF / 32), tok = 16 * kShTiles * (4 / nkw);
    hipLaunchKernelGGL(k_pfs_down_i8, dim3(D / 16, (T + tok - 1) / tok), dim3(256), 0, s,
                       static_cast<const uint8_t*>(L->down_sh), D, FF, w.hh + P * FF, w.hsc + P, T, nkw,
                       w.yp + P * D);
    GM_TRY(hipGetLastError());
  }
  hipLaunchKernelGGL(k_pf_combine, dim3(T), dim3(256), 0, s, x, w.yp, w.inv, wts, shg, T, k, D, has_sh ? 1 : 0,
                     flags, y);
  GM_TRY(hipGetLastError());
  return GM_OK;
}

}  // namespace

size_t gm_prefill_scratch_bytes(const gm_moe_layer* L, int T) {
  size_t total = 0;
  pf_layout(L, T, nullptr, &total);
  return total;
}

int gm_pf_run(const gm_moe_layer* L, const float* x, float* y, int T, int flags, uint8_t* ws, const GmMoeWs& lay,
              hipStream_t s) {
  if (L->D % kChunk || L->FF % kChunk || L->FF > 4 * kChunk)
    return gm_fail_arg("gm_moe_forward: prefill needs D and FF multiples of %d and FF <= %d", kChunk, 4 * kChunk);
  if (router_split(L->D) > kRouterSplit)
    return gm_fail_arg("gm_moe_forward: prefill supports D <= 8192 (a multiple of 512 above 4096); D=%d", L->D);
  const int qg = L->q_gate, qd = L->q_down;
  if (qg == GM_QTYPE_IQ4_XS && qd == GM_QTYPE_IQ3_XXS) return prefill_t<GM_QTYPE_IQ4_XS, GM_QTYPE_IQ3_XXS>(L, x, y, T, flags, ws, lay, s);
  if (qg == GM_QTYPE_IQ3_XXS && qd == GM_QTYPE_IQ4_XS) return prefill_t<GM_QTYPE_IQ3_XXS, GM_QTYPE_IQ4_XS>(L, x, y, T, flags, ws, lay, s);
  if (qg == GM_QTYPE_IQ4_XS && qd == GM_QTYPE_IQ4_XS) return prefill_t<GM_QTYPE_IQ4_XS, GM_QTYPE_IQ4_XS>(L, x, y, T, flags, ws, lay, s);
  if (qg == GM_QTYPE_IQ3_XXS && qd == GM_QTYPE_IQ3_XXS) return prefill_t<GM_QTYPE_IQ3_XXS, GM_QTYPE_IQ3_XXS>(L, x, y, T, flags, ws, lay, s);
  return gm_fail_arg("gm_moe_forward: unsupported routed formats gate/up %d down %d", qg, qd);
}
