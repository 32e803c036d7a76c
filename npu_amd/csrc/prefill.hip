// MoE block, prefill path (T > 8 tokens): grouped dequant-to-bf16 MFMA GEMMs.
//
//   1. router logits + top-k (router.hip), dispatch: histogram -> exclusive scan
//      -> stable scatter of (token, slot) pairs by expert (dispatch.hip), plus the
//      inverse permutation
//   2. k_pf_segments: split every expert's token list (and the shared expert's,
//      which takes all T tokens) into segments of <= 64 tokens
//   3. k_pf_prep_x:   xn = rmsnorm(x) (or x), rounded to bf16
//   4. k_pf_gateup:   per (segment, 64-row tile): h = silu(G x) * (U x) with the
//                     weights dequantised to bf16 in registers straight into
//                     v_mfma_f32_16x16x32_bf16 operands, token tiles staged in LDS;
//                     h stored as bf16 in expert-sorted row order
//   5. k_pf_down:     per (segment, 64-row tile): y_pair = Down_e h, fp32
//   6. k_pf_combine:  y[t] = sum over t's experts in ascending id of w * y_pair
//                     + sigmoid gate * y_shared (+ x); fixed order, no atomics
//
// Reference semantics: the CPU loop of qwen/forward.py:622-663 (prefill takes
// that path in the reference; its NPU kernels are T = 1 only).
#include "moe_common.h"

using namespace gm_moe;

typedef __bf16 gm_bf16x8 __attribute__((ext_vector_type(8)));

namespace {

constexpr int kSegTok = 64;      // tokens per segment (4 MFMA column tiles)
constexpr int kRowTile = 64;     // weight rows per block (4 waves x 16)
constexpr int kChunk = 256;      // K elements staged per step (one superblock column)
constexpr int kPitch = kChunk + 8;  // bf16 row pitch in LDS (pad against bank conflicts)

struct PfWs {
  int32_t* counts;    // [E]
  int32_t* offsets;   // [E + 1]
  int32_t* sorted;    // [P]
  int32_t* inv;       // [P]   position of pair p in sorted order
  int32_t* segs;      // [1 + 4 * max_seg]  n_seg, then (expert, start, n, unused)
  uint16_t* xb;       // [T][D]   bf16 xn
  uint16_t* hb;       // [P + T][FF]  bf16 SwiGLU rows (sorted pairs, then shared per token)
  float* yp;          // [P + T][D]   fp32 per-pair / shared outputs
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

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
  w.xb = reinterpret_cast<uint16_t*>(take((size_t)T * L->D * 2));
  w.hb = reinterpret_cast<uint16_t*>(take((P + T) * (size_t)L->FF * 2));
  w.yp = reinterpret_cast<float*>(take((P + T) * (size_t)L->D * 4));
  if (total) *total = o;
  return w;
}

// ---------------------------------------------------------------- segments
__global__ void __launch_bounds__(1024) k_pf_segments(const int32_t* __restrict__ counts, int E, int T, int shared,
                                                      int32_t* __restrict__ segs) {
  __shared__ int32_t nseg[1024 + 1];
  __shared__ int32_t base[1024 + 1];
  const int n_units = E + (shared ? 1 : 0);
  for (int u = threadIdx.x; u < n_units; u += blockDim.x) {
    const int n = u < E ? counts[u] : T;
    nseg[u] = (n + kSegTok - 1) / kSegTok;
  }
  __syncthreads();
  if (threadIdx.x == 0) {            // n_units <= 513: a serial scan is cheap
    int run = 0;
    for (int u = 0; u < n_units; ++u) { base[u] = run; run += nseg[u]; }
    segs[0] = run;
  }
  __syncthreads();
  for (int u = threadIdx.x; u < n_units; u += blockDim.x) {
    const int n = u < E ? counts[u] : T;
    for (int j = 0; j < nseg[u]; ++j) {
      int32_t* s = segs + 1 + 4 * (base[u] + j);
      s[0] = u;
      s[1] = j * kSegTok;
      s[2] = min(kSegTok, n - j * kSegTok);
      s[3] = 0;
    }
  }
}

// ---------------------------------------------------------------- prep x
__global__ void __launch_bounds__(256) k_pf_prep_x(const float* __restrict__ x, int D, const float* __restrict__ norm_w,
                                                   float eps, uint16_t* __restrict__ xb) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const float* xr = x + (int64_t)t * D;
  float rms = 1.f;
  if (norm_w) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < D; i += 256) ss = fmaf(xr[i], xr[i], ss);
    ss = gm_wave_sum64(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    rms = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
  }
  for (int i = threadIdx.x; i < D; i += 256) {
    const float v = norm_w ? (xr[i] * rms) * norm_w[i] : xr[i];
    xb[(int64_t)t * D + i] = (uint16_t)gm_f2bf(v);
  }
}

// ------------------------------------------------------- A operand decode
// MFMA 16x16x32 operand layout: lane l holds 8 values of row (l % 16) at
// k-slots 8*(l/16) .. 8*(l/16)+7 of the 32-wide step.  Weights and
// activations must use the same slot -> k map within a sub-block:
//   IQ3_XXS: slot 8q+i -> k = 8q+i (sign group q, grid points qs[2q], qs[2q+1])
//   IQ4_XS:  slot 8q+i -> k = 4q+i (i < 4, low nibbles of qs bytes 4q..4q+3)
//                         k = 16+4q+(i-4) (i >= 4, high nibbles of the same bytes)
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) { return gm_f2bf(a) | (gm_f2bf(b) << 16); }

template <int QT>
__device__ __forceinline__ gm_bf16x8 decode_a(const uint8_t* __restrict__ sbp, int s, int q,
                                              const uint32_t* __restrict__ grid) {
  uint32_t w4[4];
  if constexpr (QT == GM_QTYPE_IQ4_XS) {
    const uint2 hdr = *reinterpret_cast<const uint2*>(sbp);
    const uint32_t qw = *reinterpret_cast<const uint32_t*>(sbp + 8 + 16 * s + 4 * q);
    const float d = gm_h2f(hdr.x & 0xffffu);
    const uint32_t sl = (hdr.y >> (8 * (s >> 1) + 4 * (s & 1))) & 15u;
    const int ls = (int)(sl | (((hdr.x >> 16 >> (2 * s)) & 3u) << 4));
    const float dl = d * (float)(ls - 32);
    const uint32_t lo = gm_iq4nl_lut4(qw & 0x0f0f0f0fu);
    const uint32_t hi = gm_iq4nl_lut4((qw >> 4) & 0x0f0f0f0fu);
    w4[0] = pk_bf16(dl * gm_sbyte(lo, 0), dl * gm_sbyte(lo, 1));
    w4[1] = pk_bf16(dl * gm_sbyte(lo, 2), dl * gm_sbyte(lo, 3));
    w4[2] = pk_bf16(dl * gm_sbyte(hi, 0), dl * gm_sbyte(hi, 1));
    w4[3] = pk_bf16(dl * gm_sbyte(hi, 2), dl * gm_sbyte(hi, 3));
  } else {
    const uint16_t* h16 = reinterpret_cast<const uint16_t*>(sbp);
    const float d = gm_h2f(h16[0]);
    const uint32_t qq = h16[1 + 4 * s + q];                       // qs[8s+2q], qs[8s+2q+1]
    const uint32_t w = (uint32_t)h16[33 + 2 * s] | ((uint32_t)h16[34 + 2 * s] << 16);
    const float db = d * (0.5f + (float)(w >> 28)) * 0.5f;
    const uint32_t ga = grid[qq & 0xffu], gb = grid[qq >> 8];
    const uint32_t sg = gm_ksigns((w >> (7 * q)) & 127u);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float m = gm_ubyte(i < 4 ? ga : gb, i & 3);
      v[i] = db * (((sg >> i) & 1u) ? -m : m);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) w4[j] = pk_bf16(v[2 * j], v[2 * j + 1]);
  }
  gm_bf16x8 r;
  __builtin_memcpy(&r, w4, 16);
  return r;
}

// B operand: 8 activations of LDS row `col` at the same slot -> k map.
template <int QT>
__device__ __forceinline__ gm_bf16x8 load_b(const uint16_t* __restrict__ xrow, int s, int q) {
  uint32_t w4[4];
  if constexpr (QT == GM_QTYPE_IQ4_XS) {
    const uint2 a = *reinterpret_cast<const uint2*>(xrow + 32 * s + 4 * q);
    const uint2 b = *reinterpret_cast<const uint2*>(xrow + 32 * s + 16 + 4 * q);
    w4[0] = a.x; w4[1] = a.y; w4[2] = b.x; w4[3] = b.y;
  } else {
    const uint4 a = *reinterpret_cast<const uint4*>(xrow + 32 * s + 8 * q);
    w4[0] = a.x; w4[1] = a.y; w4[2] = a.z; w4[3] = a.w;
  }
  gm_bf16x8 r;
  __builtin_memcpy(&r, w4, 16);
  return r;
}

// Stage the segment's activation rows [c0, c0+256) into LDS (zero past n).
__device__ __forceinline__ void stage_b(uint16_t* __restrict__ lds, const uint16_t* __restrict__ src, int K,
                                        const int32_t* __restrict__ rows, int n, int c0) {
  // 64 rows x 256 bf16 = 64 x 32 uint4
  for (int i = threadIdx.x; i < kSegTok * (kChunk / 8); i += blockDim.x) {
    const int r = i / (kChunk / 8), c = i % (kChunk / 8);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (r < n) v = *reinterpret_cast<const uint4*>(src + (int64_t)rows[r] * K + c0 + 8 * c);
    *reinterpret_cast<uint4*>(lds + r * kPitch + 8 * c) = v;
  }
}

// -------------------------------------------------------------- gate/up
template <int QT>
__global__ void __launch_bounds__(256) k_pf_gateup(gm_moe_layer P, const int32_t* __restrict__ segs,
                                                   const int32_t* __restrict__ offsets,
                                                   const int32_t* __restrict__ sorted, const uint16_t* __restrict__ xb,
                                                   uint16_t* __restrict__ hb, int T, int n_row_tiles) {
  __shared__ uint32_t grid[256];
  __shared__ int32_t tok_row[kSegTok];
  __shared__ int32_t out_row[kSegTok];
  __shared__ __attribute__((aligned(16))) uint16_t xl[kSegTok * kPitch];
  const int seg = blockIdx.x / n_row_tiles, rt = blockIdx.x - seg * n_row_tiles;
  if (seg >= segs[0]) return;
  const int e = segs[1 + 4 * seg], start = segs[2 + 4 * seg], n = segs[3 + 4 * seg];
  const int D = P.D, FF = P.FF, k = P.k, E = P.E;
  const int Ptot = T * k;
  const bool shared = e == E;
  if constexpr (QT == GM_QTYPE_IQ3_XXS) gm_stage_grid(grid);
  if (threadIdx.x < kSegTok) {
    const int c = threadIdx.x;
    int tr = 0, orow = 0;
    if (c < n) {
      if (shared) { tr = start + c; orow = Ptot + start + c; }
      else { const int pos = offsets[e] + start + c; tr = sorted[pos] / k; orow = pos; }
    }
    tok_row[c] = tr;
    out_row[c] = orow;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, l16 = lane & 15;
  const int row = rt * kRowTile + wave * 16 + l16;
  const bool live_row = row < FF;
  const int64_t rb = gm_row_bytes(QT, D);
  const uint8_t* gbase = shared ? static_cast<const uint8_t*>(P.gate_sh) : static_cast<const uint8_t*>(P.gate_exps) + (int64_t)e * FF * rb;
  const uint8_t* ubase = shared ? static_cast<const uint8_t*>(P.up_sh) : static_cast<const uint8_t*>(P.up_exps) + (int64_t)e * FF * rb;
  const uint8_t* grow = gbase + (int64_t)(live_row ? row : 0) * rb;
  const uint8_t* urow = ubase + (int64_t)(live_row ? row : 0) * rb;
  const int ntiles = (n + 15) / 16;
  gm_f32x4 ag[4], au[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) { ag[j] = gm_f32x4{0, 0, 0, 0}; au[j] = gm_f32x4{0, 0, 0, 0}; }
  for (int c0 = 0; c0 < D; c0 += kChunk) {
    __syncthreads();
    stage_b(xl, xb, D, tok_row, n, c0);
    __syncthreads();
    const int sb = c0 / GM_QK;
    const uint8_t* gsb = grow + sb * gm_block_bytes(QT);
    const uint8_t* usb = urow + sb * gm_block_bytes(QT);
#pragma unroll 2
    for (int s = 0; s < 8; ++s) {
      const gm_bf16x8 wg = decode_a<QT>(gsb, s, q, grid);
      const gm_bf16x8 wu = decode_a<QT>(usb, s, q, grid);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j < ntiles) {
          const gm_bf16x8 b = load_b<QT>(xl + (j * 16 + l16) * kPitch, s, q);
          ag[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wg, b, ag[j], 0, 0, 0);
          au[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wu, b, au[j], 0, 0, 0);
        }
      }
    }
  }
  // C layout: lane l holds rows 4*(l/16)+i (i = 0..3) of the 16-row tile, column l % 16
  const int r0 = rt * kRowTile + wave * 16 + 4 * q;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = j * 16 + l16;
    if (j < ntiles && col < n && r0 < FF) {
      uint32_t h01 = pk_bf16(gm_silu(ag[j][0]) * au[j][0], gm_silu(ag[j][1]) * au[j][1]);
      uint32_t h23 = pk_bf16(gm_silu(ag[j][2]) * au[j][2], gm_silu(ag[j][3]) * au[j][3]);
      *reinterpret_cast<uint2*>(hb + (int64_t)out_row[col] * FF + r0) = make_uint2(h01, h23);
    }
  }
}

// ------------------------------------------------------------------ down
template <int QT>
__global__ void __launch_bounds__(256) k_pf_down(gm_moe_layer P, const int32_t* __restrict__ segs,
                                                 const int32_t* __restrict__ offsets, const uint16_t* __restrict__ hb,
                                                 float* __restrict__ yp, int T, int n_row_tiles) {
  __shared__ uint32_t grid[256];
  __shared__ int32_t in_row[kSegTok];
  __shared__ __attribute__((aligned(16))) uint16_t hl[kSegTok * kPitch];
  const int seg = blockIdx.x / n_row_tiles, rt = blockIdx.x - seg * n_row_tiles;
  if (seg >= segs[0]) return;
  const int e = segs[1 + 4 * seg], start = segs[2 + 4 * seg], n = segs[3 + 4 * seg];
  const int D = P.D, FF = P.FF, k = P.k, E = P.E;
  const bool shared = e == E;
  const int row0 = shared ? T * k + start : offsets[e] + start;    // rows of hb / yp
  if constexpr (QT == GM_QTYPE_IQ3_XXS) gm_stage_grid(grid);
  if (threadIdx.x < kSegTok) in_row[threadIdx.x] = row0 + (threadIdx.x < n ? threadIdx.x : 0);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, l16 = lane & 15;
  const int row = rt * kRowTile + wave * 16 + l16;
  const bool live_row = row < D;
  const int64_t rb = gm_row_bytes(QT, FF);
  const uint8_t* base = shared ? static_cast<const uint8_t*>(P.down_sh) : static_cast<const uint8_t*>(P.down_exps) + (int64_t)e * D * rb;
  const uint8_t* wrow = base + (int64_t)(live_row ? row : 0) * rb;
  const int ntiles = (n + 15) / 16;
  gm_f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = gm_f32x4{0, 0, 0, 0};
  for (int c0 = 0; c0 < FF; c0 += kChunk) {
    __syncthreads();
    stage_b(hl, hb, FF, in_row, n, c0);
    __syncthreads();
    const uint8_t* sbp = wrow + (c0 / GM_QK) * gm_block_bytes(QT);
#pragma unroll 2
    for (int s = 0; s < 8; ++s) {
      const gm_bf16x8 w = decode_a<QT>(sbp, s, q, grid);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j < ntiles) {
          const gm_bf16x8 b = load_b<QT>(hl + (j * 16 + l16) * kPitch, s, q);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, b, acc[j], 0, 0, 0);
        }
      }
    }
  }
  const int r0 = rt * kRowTile + wave * 16 + 4 * q;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = j * 16 + l16;
    if (j < ntiles && col < n && r0 < D)
      *reinterpret_cast<float4*>(yp + (int64_t)(row0 + col) * D + r0) =
          make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
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
  const int Ptot = T * k;
  for (int d = threadIdx.x; d < D; d += 256) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < k) acc = fmaf(w[j], yp[(int64_t)pos[j] * D + d], acc);
    if (has_sh) acc += sg * yp[(int64_t)(Ptot + t) * D + d];
    if (flags & GM_MOE_RESIDUAL) acc = x[(int64_t)t * D + d] + acc;
    y[(int64_t)t * D + d] = acc;
  }
}

template <int QTG, int QTD, int QTSG, int QTSD>
int prefill_t(const gm_moe_layer* L, const float* x, float* y, int T, int flags, uint8_t* ws, const GmMoeWs& lay,
              hipStream_t s) {
  const int D = L->D, FF = L->FF, E = L->E, k = L->k;
  float* logits = reinterpret_cast<float*>(ws + lay.logits);
  float* shg = reinterpret_cast<float*>(ws + lay.shg);
  int32_t* ids = reinterpret_cast<int32_t*>(ws + lay.ids);
  float* wts = reinterpret_cast<float*>(ws + lay.wts);
  PfWs w = pf_layout(L, T, ws + lay.pre, nullptr);
  const bool has_sh = L->gate_sh != nullptr;
  if (int rc = gm_launch_router(L->router, L->router_bias, x, T, D, E, L->sh_gate_inp, L->norm_w, L->norm_eps,
                                logits, shg, s)) return rc;
  if (int rc = gm_launch_topk(logits, T, E, k, ids, wts, s)) return rc;
  if (int rc = gm_launch_dispatch_inv(ids, T, k, E, w.counts, w.offsets, w.sorted, w.inv, s)) return rc;
  hipLaunchKernelGGL(k_pf_segments, dim3(1), dim3(1024), 0, s, w.counts, E, T, has_sh ? 1 : 0, w.segs);
  GM_TRY(hipGetLastError());
  hipLaunchKernelGGL(k_pf_prep_x, dim3(T), dim3(256), 0, s, x, D, L->norm_w, L->norm_eps, w.xb);
  GM_TRY(hipGetLastError());
  const int nseg = max_segments(T, k, E);
  {
    const int nrt = (FF + kRowTile - 1) / kRowTile;
    hipLaunchKernelGGL(k_pf_gateup<QTG>, dim3(nseg * nrt), dim3(256), 0, s, *L, w.segs, w.offsets, w.sorted, w.xb,
                       w.hb, T, nrt);
    GM_TRY(hipGetLastError());
  }
  {
    const int nrt = (D + kRowTile - 1) / kRowTile;
    hipLaunchKernelGGL(k_pf_down<QTD>, dim3(nseg * nrt), dim3(256), 0, s, *L, w.segs, w.offsets, w.hb, w.yp, T, nrt);
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

int gm_pf_run(const gm_moe_layer* L, const float* x, float* y, int T, int flags, uint8_t* ws,
                   const GmMoeWs& lay, hipStream_t s) {
  if (L->gate_sh && (L->q_gate_sh != L->q_gate || L->q_down_sh != L->q_down))
    return gm_fail_arg("gm_moe_forward: the prefill path needs the shared expert in the routed formats"),
           GM_EUNSUPPORTED;
  if (L->D % kChunk || L->FF % kChunk)
    return gm_fail_arg("gm_moe_forward: prefill needs D and FF multiples of %d", kChunk);
  const int qg = L->q_gate, qd = L->q_down;
  if (qg == GM_QTYPE_IQ4_XS && qd == GM_QTYPE_IQ3_XXS)
    return prefill_t<GM_QTYPE_IQ4_XS, GM_QTYPE_IQ3_XXS, 0, 0>(L, x, y, T, flags, ws, lay, s);
  if (qg == GM_QTYPE_IQ3_XXS && qd == GM_QTYPE_IQ4_XS)
    return prefill_t<GM_QTYPE_IQ3_XXS, GM_QTYPE_IQ4_XS, 0, 0>(L, x, y, T, flags, ws, lay, s);
  if (qg == GM_QTYPE_IQ4_XS && qd == GM_QTYPE_IQ4_XS)
    return prefill_t<GM_QTYPE_IQ4_XS, GM_QTYPE_IQ4_XS, 0, 0>(L, x, y, T, flags, ws, lay, s);
  if (qg == GM_QTYPE_IQ3_XXS && qd == GM_QTYPE_IQ3_XXS)
    return prefill_t<GM_QTYPE_IQ3_XXS, GM_QTYPE_IQ3_XXS, 0, 0>(L, x, y, T, flags, ws, lay, s);
  return gm_fail_arg("gm_moe_forward: unsupported routed formats gate/up %d down %d", qg, qd);
}
