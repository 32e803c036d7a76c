// Device routines shared by the MoE kernels: activation staging in LDS (with
// the RMSNorm of qwen/forward.py:58-61), wave-level top-k with renormalised
// softmax weights, and the per-expert grouping table.
#pragma once
#include "iq_decode.h"
#include "kernels.h"

namespace gm_moe {

// ---------------------------------------------------------------- LDS layout
// Activation rows live in LDS "quad-interleaved by sub-block": element k of a
// row of K values (sub = k / 32, j = k % 32) sits at float index
//     ((j / 4) * (K / 32) + sub) * 4 + (j % 4).
// The 16 lanes of a weight row read sub-blocks lir, lir+16, ...; with this
// layout the float4 they read for the same j/4 are consecutive 16-byte chunks,
// so ds_read_b128 is bank-conflict free (a contiguous layout puts them 128 B
// apart: a 16-way conflict).
__device__ __forceinline__ int il_index4(int q, int sub, int nsub) { return q * nsub + sub; }

// 32-wide dot of decoded weights with sub-block `sub` of an interleaved row.
__device__ __forceinline__ float gm_dot32_il(const float (&wv)[32], const float* __restrict__ row, int sub, int nsub) {
  const float4* r4 = reinterpret_cast<const float4*>(row);
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int q = 0; q < 8; q += 2) {
    const float4 a = r4[il_index4(q, sub, nsub)];
    const float4 b = r4[il_index4(q + 1, sub, nsub)];
    s0 = fmaf(wv[4 * q + 0], a.x, s0); s1 = fmaf(wv[4 * q + 4], b.x, s1);
    s0 = fmaf(wv[4 * q + 1], a.y, s0); s1 = fmaf(wv[4 * q + 5], b.y, s1);
    s0 = fmaf(wv[4 * q + 2], a.z, s0); s1 = fmaf(wv[4 * q + 6], b.z, s1);
    s0 = fmaf(wv[4 * q + 3], a.w, s0); s1 = fmaf(wv[4 * q + 7], b.w, s1);
  }
  return s0 + s1;
}

// Block-wide sum (every thread gets the total); red needs blockDim/64 floats.
__device__ __forceinline__ float block_sum(float v, float* __restrict__ red) {
  v = gm_wave_sum64(v);
  const int nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
  for (int w = 0; w < nw; ++w) s += red[w];
  return s;
}

// Stage rows t0 .. t0+nt-1 of x [.][D] into xs (NT interleaved rows of D floats),
// zero rows past nt; when norm_w != NULL apply xn = (x * rms) * w with
// rms = 1/sqrt(mean(x^2) + eps).  red: >= 16 + NT floats of LDS.  All threads call.
template <int NT>
__device__ __forceinline__ void stage_xn(const float* __restrict__ x, int t0, int nt, int D,
                                         const float* __restrict__ norm_w, float eps, float* __restrict__ xs,
                                         float* __restrict__ red) {
  const int nq = D >> 2, nsub = D >> 5;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4* xs4 = reinterpret_cast<float4*>(xs);
  float ss[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    ss[t] = 0.f;
    for (int c = threadIdx.x; c < nq; c += blockDim.x) {
      const float4 v = t < nt ? x4[(int64_t)(t0 + t) * nq + c] : make_float4(0.f, 0.f, 0.f, 0.f);
      ss[t] = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss[t]))));
      xs4[t * nq + il_index4(c & 7, c >> 3, nsub)] = v;
    }
  }
  if (norm_w != nullptr) {
    const float4* w4 = reinterpret_cast<const float4*>(norm_w);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < nt) {
        const float rms = 1.0f / sqrtf(block_sum(ss[t], red) / (float)D + eps);
        for (int c = threadIdx.x; c < nq; c += blockDim.x) {
          float4* p = &xs4[t * nq + il_index4(c & 7, c >> 3, nsub)];
          float4 v = *p;
          const float4 w = w4[c];
          v.x = (v.x * rms) * w.x; v.y = (v.y * rms) * w.y; v.z = (v.z * rms) * w.z; v.w = (v.w * rms) * w.w;
          *p = v;
        }
      }
    }
  }
  __syncthreads();
}

// Stage n contiguous rows of K floats (global) into interleaved LDS rows.
__device__ __forceinline__ void stage_rows_il(const float* __restrict__ src, int n, int K, float* __restrict__ dst) {
  const int nq = K >> 2, nsub = K >> 5;
  const float4* s4 = reinterpret_cast<const float4*>(src);
  float4* d4 = reinterpret_cast<float4*>(dst);
  for (int r = 0; r < n; ++r)
    for (int c = threadIdx.x; c < nq; c += blockDim.x) d4[r * nq + il_index4(c & 7, c >> 3, nsub)] = s4[(int64_t)r * nq + c];
}

// ------------------------------------------------------------------ top-k
// One wave: top-k of E logits (descending, ties -> lower id), softmax over all
// E, renormalised top-k probabilities (qwen/forward.py:609-611).  Each lane
// sorts its MAXV values once; every round takes the wave-wide best lane head
// (DPP inside 16-lane rows, readlane across rows) and pops it.
template <int CTRL>
__device__ __forceinline__ void dpp_argmax_step(float& bv, int& bi) {
  const float ov = GM_DPP_F(bv, CTRL);
  const int oi = GM_DPP_I(bi, CTRL);
  if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) { return av > bv || (av == bv && ai < bi); }

template <int MAXV>
__device__ __forceinline__ void wave_topk(const float* __restrict__ lg, int E, int k, int32_t* __restrict__ ids,
                                          float* __restrict__ wts) {
  const int lane = threadIdx.x & 63;
  float v[MAXV];
  int ix[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    ix[i] = lane + 64 * i;
    v[i] = ix[i] < E ? lg[ix[i]] : -INFINITY;
  }
  // per-lane sort, descending (ties: lower index first)
#pragma unroll
  for (int a = 0; a < MAXV; ++a)
#pragma unroll
    for (int b = MAXV - 1; b > a; --b)
      if (better(v[b], ix[b], v[b - 1], ix[b - 1])) {
        const float tv = v[b]; v[b] = v[b - 1]; v[b - 1] = tv;
        const int ti = ix[b]; ix[b] = ix[b - 1]; ix[b - 1] = ti;
      }
  // softmax normaliser over all E (max = best head)
  float m = v[0];
  m = fmaxf(m, GM_DPP_F(m, GM_ROW_ROR8));
  m = fmaxf(m, GM_DPP_F(m, GM_ROW_ROR4));
  m = fmaxf(m, GM_DPP_F(m, GM_QPERM_2301));
  m = fmaxf(m, GM_DPP_F(m, GM_QPERM_1032));
  {
    const int b = __builtin_bit_cast(int, m);
    m = fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)),
                    __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))),
              fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)),
                    __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48))));
  }
  float z = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i)
    if (ix[i] < E) z += expf(v[i] - m);
  z = gm_wave_sum64(z);
  float psum = 0.f, myp = 0.f;
  int myid = 0;
  for (int r = 0; r < k; ++r) {
    float bv = v[0];
    int bi = ix[0];
    dpp_argmax_step<GM_ROW_ROR8>(bv, bi);
    dpp_argmax_step<GM_ROW_ROR4>(bv, bi);
    dpp_argmax_step<GM_QPERM_2301>(bv, bi);
    dpp_argmax_step<GM_QPERM_1032>(bv, bi);
    const int bb = __builtin_bit_cast(int, bv);
    float wv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bb, 0));
    int wi = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
    for (int row = 16; row < 64; row += 16) {
      const float rv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bb, row));
      const int ri = __builtin_amdgcn_readlane(bi, row);
      if (better(rv, ri, wv, wi)) { wv = rv; wi = ri; }
    }
    if ((wi & 63) == lane) {         // pop the winner's head
#pragma unroll
      for (int i = 0; i + 1 < MAXV; ++i) { v[i] = v[i + 1]; ix[i] = ix[i + 1]; }
      v[MAXV - 1] = -INFINITY;
      ix[MAXV - 1] = 0x7fffffff;
    }
    const float p = expf(wv - m) / z;
    psum += p;
    if (lane == r) { myp = p; myid = wi; }
  }
  const float den = fmaxf(psum, 1e-20f);
  if (lane < k) {
    ids[lane] = myid;
    wts[lane] = myp / den;
  }
}

// --------------------------------------------------------------- grouping
// Grouping of (token, slot) pairs by expert into LDS (all threads call; pairs
// are handled by wave 0): g[0] = n_unique, g[1+u] = expert of slot u
// (ascending), g[65+u] = member count, g[129 + 8u + m] = pair index t*k + j
// of member m (tokens ascending).
__device__ __forceinline__ void block_group(const int32_t* __restrict__ ids, int P, int E, int32_t* __restrict__ g,
                                            uint32_t* __restrict__ bits) {
  const int nwords = (E + 31) / 32;
  for (int i = threadIdx.x; i < nwords; i += blockDim.x) bits[i] = 0u;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const bool w0 = threadIdx.x < 64;
  const int e = (w0 && lane < P) ? ids[lane] : -1;
  if (e >= 0) atomicOr(&bits[e >> 5], 1u << (e & 31));
  __syncthreads();
  if (w0) {
    int nu = 0, rank = 0;
    for (int w = 0; w < nwords; ++w) {
      const uint32_t b = bits[w];
      nu += __builtin_popcount(b);
      if (e >= 0 && (w << 5) < e) {
        const int hi = e - (w << 5);
        rank += hi >= 32 ? __builtin_popcount(b) : __builtin_popcount(b & ((1u << hi) - 1u));
      }
    }
    int m = 0, cnt = 0;
    for (int q = 0; q < P; ++q) {
      const int eq = __builtin_amdgcn_readlane(e, q);
      if (eq == e) {
        cnt += 1;
        if (q < lane) m += 1;
      }
    }
    if (lane == 0) g[0] = nu;
    if (e >= 0) {
      g[1 + rank] = e;
      g[1 + GM_GRP_MAXU + rank] = cnt;
      g[1 + 2 * GM_GRP_MAXU + rank * GM_GRP_MAXM + m] = lane;
    }
  }
  __syncthreads();
}

}  // namespace gm_moe
