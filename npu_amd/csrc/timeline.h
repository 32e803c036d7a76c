// Per-block timestamps for the decode kernels (a profiling build only).
//
// Built with -DGM_TIMELINE=1 (python -m npu_amd.build --timeline ->
// libnpu_amd_tl.so), every instrumented kernel takes one extra argument, a
// pointer into the caller's workspace, and thread 0 of each block writes one
// 64-byte record there: the s_memrealtime counter (100 MHz, one clock for the
// whole chip) at block entry, at two kernel-specific marks, and at the end,
// plus the HW_ID and XCC_ID registers of the wave.  Record layout (u64):
//   [0] entry  [1] mark 1  [2] mark 2  [3] end  [4] HW_ID | XCC_ID << 32
//   [5] s_memtime (shader clock) at entry  [6] s_memtime at the end
//   [7] mark 3 (an optional earlier mark, 0 if unused)
// Each workspace holds GM_TL_KERNELS x GM_TL_MAXB records, so every layer of
// a chain keeps its own stamps.  Slots: T = 1 router 0, gate/up 1, down 2;
// T > 1 router partials 4, routing 5, gate/up 6, down 7, combine 3.  In the normal build the macros expand to
// nothing and the kernels are unchanged.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define GM_TL_KERNELS 8
#define GM_TL_MAXB 2560
#define GM_TL_REC 8   // u64 per record

#if defined(GM_TIMELINE) && GM_TIMELINE

__device__ __forceinline__ uint64_t gm_tl_now() {
  uint64_t t;
  asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t)::"memory");
  return t;
}

// The stamp is taken after `dep` has been computed.
template <typename T>
__device__ __forceinline__ uint64_t gm_tl_after(const T& dep) {
  const float d = (float)dep;
  asm volatile("" ::"v"(d));
  return gm_tl_now();
}

__device__ __forceinline__ uint64_t gm_tl_clock() {
  uint64_t t;
  asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t)::"memory");
  return t;
}

__device__ __forceinline__ void gm_tl_flush(uint64_t* __restrict__ buf, int slot, uint64_t t0, uint64_t t1,
                                            uint64_t t2, uint64_t c0, uint64_t t3m) {
  const uint64_t t3 = gm_tl_now();
  const uint64_t c1 = gm_tl_clock();
  const uint32_t blk = blockIdx.x + blockIdx.y * gridDim.x;           // linear block id (2-D grids)
  if (threadIdx.x == 0 && blk < GM_TL_MAXB) {
    const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);     // HW_ID
    const uint32_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);   // XCC_ID
    uint64_t* r = buf + ((int64_t)slot * GM_TL_MAXB + blk) * GM_TL_REC;
    r[0] = t0;
    r[1] = t1;
    r[2] = t2;
    r[3] = t3;
    r[4] = (uint64_t)hw | ((uint64_t)xcc << 32);
    r[5] = c0;
    r[6] = c1;
    r[7] = t3m;
  }
}

#define GM_TL_PARAM , uint64_t* __restrict__ gm_tl
#define GM_TL_ARG(p) , (p)
#define GM_TL_BEGIN() uint64_t gm_tl_t0 = gm_tl_now(), gm_tl_c0 = gm_tl_clock(), gm_tl_t1 = 0, gm_tl_t2 = 0, gm_tl_t3 = 0
#define GM_TL_MARK1(dep) (gm_tl_t1 = gm_tl_after(dep))
#define GM_TL_MARK2(dep) (gm_tl_t2 = gm_tl_after(dep))
#define GM_TL_MARK3(dep) (gm_tl_t3 = gm_tl_after(dep))
#define GM_TL_END(slot) gm_tl_flush(gm_tl, (slot), gm_tl_t0, gm_tl_t1, gm_tl_t2, gm_tl_c0, gm_tl_t3)
#define GM_TL_BYTES ((size_t)GM_TL_KERNELS * GM_TL_MAXB * GM_TL_REC * 8)

#else

#define GM_TL_PARAM
#define GM_TL_ARG(p)
#define GM_TL_BEGIN() ((void)0)
#define GM_TL_MARK1(dep) ((void)0)
#define GM_TL_MARK2(dep) ((void)0)
#define GM_TL_MARK3(dep) ((void)0)
#define GM_TL_END(slot) ((void)0)
#define GM_TL_BYTES ((size_t)0)

#endif
