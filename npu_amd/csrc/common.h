// Shared definitions for the gfx950 MoE-block kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/npu_amd.h"

#define GM_QK 256            // weights per superblock (GGUF QK_K)
#define GM_SUB 32            // weights per sub-block (one scale)
#define GM_IQ4XS_BYTES 136   // GGUF block_iq4_xs
#define GM_IQ3XXS_BYTES 98   // GGUF block_iq3_xxs
#define GM_WAVE 64

// Host-side launch-check helper: every entry point returns an int status.
#define GM_TRY(expr)                                   \
  do {                                                 \
    hipError_t e_ = (expr);                            \
    if (e_ != hipSuccess) return gm_fail_hip(e_, #expr); \
  } while (0)

int gm_fail_hip(hipError_t e, const char* what);
int gm_fail_arg(const char* fmt, ...);

// Bytes per superblock (256 weights) for a weight format, 0 if unsupported.
__host__ __device__ inline int gm_block_bytes(int qtype) {
  return qtype == GM_QTYPE_IQ4_XS ? GM_IQ4XS_BYTES
       : qtype == GM_QTYPE_IQ3_XXS ? GM_IQ3XXS_BYTES
       : qtype == GM_QTYPE_BF16 ? 2 * GM_QK
       : qtype == GM_QTYPE_F32 ? 4 * GM_QK : 0;
}

__host__ __device__ inline int64_t gm_row_bytes(int qtype, int K) {
  return (int64_t)(K / GM_QK) * gm_block_bytes(qtype);
}

__device__ __forceinline__ float gm_h2f(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

__device__ __forceinline__ float gm_bf2f(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN-preserving).
__device__ __forceinline__ uint32_t gm_f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float gm_silu(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ float gm_sigmoid(float g) { return 1.0f / (1.0f + __expf(-g)); }

template <typename T>
__device__ __forceinline__ T gm_wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over aligned groups of L lanes (L a power of two <= 64).
template <int L>
__device__ __forceinline__ float gm_group_sum(float v) {
#pragma unroll
  for (int o = L / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Dynamic LDS above 64 KB needs an explicit opt-in per kernel (gfx950 has 160 KB).
template <typename K>
inline int gm_set_smem(K kern, size_t bytes) {
  if (bytes > 65536) GM_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
  return GM_OK;
}
