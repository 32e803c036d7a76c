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

// Native 4 x f32 vector.  Staging copies use it instead of HIP's float4
// struct: a struct load + store pair is turned into a memcpy by the optimiser,
// which then issues every load right before its store.
typedef float gm_f32x4 __attribute__((ext_vector_type(4)));
typedef double gm_f64x2 __attribute__((ext_vector_type(2)));
typedef uint32_t gm_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t gm_u32x2 __attribute__((ext_vector_type(2)));

// Weight loads.  ST = true: a nontemporal load, for weight bytes a decode
// launch streams once (routed and shared experts, the router, dense
// projection rows); activations and tables keep the default policy.  Measured
// on MI355X: 17.06 -> 15.85 us per T = 1 MoE block.  The prefill GEMMs, whose
// expert rows several token segments re-read, keep the default (nontemporal
// there took 226 -> 292 us per block).
template <bool ST, typename T>
__device__ __forceinline__ T gm_ld(const T* p) {
  if constexpr (ST) return __builtin_nontemporal_load(p);
  else return *p;
}

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
       : qtype == GM_QTYPE_I8 ? 384
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

// ---- DPP reductions (VALU-rate; no LDS round trips) ----------------------
#define GM_DPP_F(v, ctrl) __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, false))
#define GM_DPP_I(v, ctrl) __builtin_amdgcn_update_dpp(0, (v), (ctrl), 0xF, 0xF, false)
#define GM_ROW_ROR8 0x128
#define GM_ROW_ROR4 0x124
#define GM_QPERM_2301 0x4E
#define GM_QPERM_1032 0xB1

// Sum over each 16-lane row; every lane of the row receives the row total.
__device__ __forceinline__ float gm_row_sum16(float v) {
  v += GM_DPP_F(v, GM_ROW_ROR8);
  v += GM_DPP_F(v, GM_ROW_ROR4);
  v += GM_DPP_F(v, GM_QPERM_2301);
  v += GM_DPP_F(v, GM_QPERM_1032);
  return v;
}

// Sum over all 64 lanes (wave-uniform result).
__device__ __forceinline__ float gm_wave_sum64(float v) {
  v = gm_row_sum16(v);
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

// Sum over aligned groups of L lanes, L in {16, 64} via DPP, else shuffles.
template <int L>
__device__ __forceinline__ float gm_lane_group_sum(float v) {
  if constexpr (L == 16) return gm_row_sum16(v);
  else if constexpr (L == 64) return gm_wave_sum64(v);
  else return gm_group_sum<L>(v);
}

// Dynamic LDS above 64 KB needs an explicit opt-in per kernel (gfx950 has 160 KB).
template <typename K>
inline int gm_set_smem(K kern, size_t bytes) {
  if (bytes > 65536) GM_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
  return GM_OK;
}
