// Per-sub-block (32 weights) load and decode of raw GGUF superblocks.
//
// A row of an [M x K] weight is K/256 consecutive superblocks.  Sub-block
// `sub` (0 .. K/32-1) of a row is sub-block (sub % 8) of superblock (sub / 8).
// load_sub<QT>() fetches the raw bytes one lane needs for one sub-block;
// decode_sub<QT>() turns them into 32 unscaled fp32 weights plus the
// sub-block scale, so that  weight[i] == scale * wv[i]  exactly (every
// product involved is exact in fp32; see the layout notes per format).
#pragma once
#include "common.h"
#include "iq_tables.h"

// kvalues_iq4nl as 16 int8 bytes, entry n in byte (n % 4) of word (n / 4).
constexpr uint32_t kGmKv[4] = {GM_IQ4NL_PACKED_INIT};
#define GM_KV0 kGmKv[0]
#define GM_KV1 kGmKv[1]
#define GM_KV2 kGmKv[2]
#define GM_KV3 kGmKv[3]

// Four IQ4 nibbles (one per byte, values 0..15) -> four int8 kvalues, in two
// v_perm_b32 lookups and an XOR.  v_perm_b32 picks bytes 0..7 of an 8-byte
// pool for selector bytes 0..7 and returns fixed bytes for the others: 8..11
// the sign of pool byte 1, 3, 5, 7 spread to 0x00 / 0xff, 12 zero, >= 13
// 0xff.  With selector n the pool P answers nibbles n < 8 and gives such a
// fixed byte f(n) for n >= 8; with selector n ^ 8 the pool Q answers n >= 8
// and gives a fixed byte g(n) for n < 8.  So P[n] = kv[n] ^ g(n) and
// Q[n - 8] = kv[n] ^ f(n) make perm(P, n) ^ perm(Q, n ^ 8) = kv[n] for every
// n.  f reads the signs of P[1, 3, 5, 7] and g those of Q[1, 3, 5, 7]; the
// entries are solved in dependency order below (those with a constant f or g
// first) and the result is checked for all 16 nibbles at compile time.
namespace gm_iq4_xor {
struct Tabs { uint32_t p0, p1, q0, q1; };

// Table entry n of a 16-byte table given as 4 words (entry n in byte n % 4 of word n / 4).
constexpr uint32_t entry(const uint32_t (&t)[4], int n) { return (t[n >> 2] >> (8 * (n & 3))) & 0xffu; }
constexpr uint32_t sgn(uint32_t b) { return (b & 0x80u) ? 0xffu : 0u; }

constexpr Tabs solve(const uint32_t (&t)[4]) {
  // fixed bytes with constant selectors: g(4) = 0, g(5..7) = ff; f(12) = 0, f(13..15) = ff
  const uint32_t P4 = entry(t, 4), P5 = entry(t, 5) ^ 0xffu, P6 = entry(t, 6) ^ 0xffu, P7 = entry(t, 7) ^ 0xffu;
  const uint32_t Q4 = entry(t, 12), Q5 = entry(t, 13) ^ 0xffu, Q6 = entry(t, 14) ^ 0xffu, Q7 = entry(t, 15) ^ 0xffu;
  // g(n) = sign of Q[2n + 1] for n < 4, f(n) = sign of P[2(n - 8) + 1] for 8 <= n < 12
  const uint32_t P3 = entry(t, 3) ^ sgn(Q7), P2 = entry(t, 2) ^ sgn(Q5);
  const uint32_t Q3 = entry(t, 11) ^ sgn(P7), Q2 = entry(t, 10) ^ sgn(P5);
  const uint32_t P1 = entry(t, 1) ^ sgn(Q3), Q1 = entry(t, 9) ^ sgn(P3);
  const uint32_t P0 = entry(t, 0) ^ sgn(Q1), Q0 = entry(t, 8) ^ sgn(P1);
  return Tabs{P0 | P1 << 8 | P2 << 16 | P3 << 24, P4 | P5 << 8 | P6 << 16 | P7 << 24,
              Q0 | Q1 << 8 | Q2 << 16 | Q3 << 24, Q4 | Q5 << 8 | Q6 << 16 | Q7 << 24};
}

// v_perm_b32 on one selector byte, as the ISA defines it (pool bytes 0-3 = lo, 4-7 = hi).
constexpr uint32_t perm_byte(uint32_t hi, uint32_t lo, uint32_t sel) {
  const uint64_t pool = (uint64_t)hi << 32 | lo;
  return sel >= 13 ? 0xffu : sel == 12 ? 0u
       : sel >= 8 ? (((pool >> (8 * (2 * (sel - 8) + 1) + 7)) & 1u) ? 0xffu : 0u)
                  : (uint32_t)((pool >> (8 * sel)) & 0xffu);
}
constexpr bool check(const uint32_t (&t)[4], Tabs x) {
  for (uint32_t n = 0; n < 16; ++n)
    if ((perm_byte(x.p1, x.p0, n) ^ perm_byte(x.q1, x.q0, n ^ 8u)) != entry(t, (int)n)) return false;
  return true;
}
constexpr Tabs kKv = solve(kGmKv);
static_assert(check(kGmKv, kKv), "IQ4 XOR lookup tables do not reproduce kvalues_iq4nl");
}  // namespace gm_iq4_xor

// Lookup of four nibbles in a 16-entry byte table through its solved pools.
__device__ __forceinline__ uint32_t gm_lut16_xor(gm_iq4_xor::Tabs t, uint32_t nib) {
  return __builtin_amdgcn_perm(t.p1, t.p0, nib) ^ __builtin_amdgcn_perm(t.q1, t.q0, nib ^ 0x08080808u);
}

__device__ __forceinline__ uint32_t gm_iq4nl_lut4(uint32_t nib) { return gm_lut16_xor(gm_iq4_xor::kKv, nib); }

__device__ __forceinline__ float gm_sbyte(uint32_t v, int i) {
  return (float)(int)(int8_t)(uint8_t)(v >> (8 * i));
}

__device__ __forceinline__ float gm_ubyte(uint32_t v, int i) {
  return (float)(uint32_t)((v >> (8 * i)) & 0xffu);
}

// ---------------------------------------------------------------- IQ4_XS
// block_iq4_xs (136 B): fp16 d | u16 scales_h | u8 scales_l[4] | u8 qs[128].
// ls_s = ((scales_l[s/2] >> 4*(s%2)) & 15) | (((scales_h >> 2s) & 3) << 4),
// dl_s = d * (ls_s - 32); qs[16s + j]: low nibble -> weight 32s+j,
// high nibble -> weight 32s+16+j.  (Reference: npu/quant_mv_iq4.py:180-202.)
struct RawIq4 {
  uint32_t h0, h1;      // d | scales_h, scales_l[0..3]
  uint32_t q[4];        // 16 qs bytes of the sub-block
};

template <bool ST = false>
__device__ __forceinline__ RawIq4 gm_load_iq4(const uint8_t* __restrict__ row, int sub) {
  const uint8_t* blk = row + (sub >> 3) * GM_IQ4XS_BYTES;     // 8-byte aligned
  const gm_u32x2 h = gm_ld<ST>(reinterpret_cast<const gm_u32x2*>(blk));
  const gm_u32x2* qp = reinterpret_cast<const gm_u32x2*>(blk + 8 + 16 * (sub & 7));
  const gm_u32x2 a = gm_ld<ST>(qp), b = gm_ld<ST>(qp + 1);
  RawIq4 r;
  r.h0 = h.x; r.h1 = h.y;
  r.q[0] = a.x; r.q[1] = a.y; r.q[2] = b.x; r.q[3] = b.y;
  return r;
}

__device__ __forceinline__ float gm_decode_iq4(const RawIq4& r, int sub, float (&wv)[32]) {
  const int s = sub & 7;
  const float d = gm_h2f(r.h0 & 0xffffu);
  const uint32_t sh = r.h0 >> 16;
  const uint32_t sl = (r.h1 >> (8 * (s >> 1) + 4 * (s & 1))) & 15u;
  const int ls = (int)(sl | (((sh >> (2 * s)) & 3u) << 4));
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t lo = gm_iq4nl_lut4(r.q[w] & 0x0f0f0f0fu);
    const uint32_t hi = gm_iq4nl_lut4((r.q[w] >> 4) & 0x0f0f0f0fu);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wv[4 * w + i] = gm_sbyte(lo, i);
      wv[16 + 4 * w + i] = gm_sbyte(hi, i);
    }
  }
  return d * (float)(ls - 32);
}

// --------------------------------------------------------------- IQ3_XXS
// block_iq3_xxs (98 B): fp16 d | u8 qs[64] | u32 scale/sign words[8].
// Fields are only 2-byte aligned (98 is not a multiple of 4), so they are
// fetched as 16-bit words.  Sub-block s: qs[8s .. 8s+7], word w_s;
// db = d * (0.5 + (w_s >> 28)) * 0.5; group g uses sign byte
// ksigns[(w_s >> 7g) & 127] and grid points qs[8s+2g], qs[8s+2g+1].
// (Reference: npu/iq3_xxs.py:4-15, 97-119.)
struct RawIq3 {
  uint32_t d;      // fp16 bits
  uint32_t q0, q1; // 8 grid indices
  uint32_t w;      // scale/sign word
};

// Superblocks are 2-byte aligned (98 B each), so every field offset is 0 or
// 2 mod 4.  Fields are fetched with aligned dword loads (global memory or
// LDS) and re-aligned with v_alignbyte_b32; every dword read contains at
// least one byte of this superblock, so no load crosses into an unmapped page.
// gm_load_iq3_words issues the loads only; gm_iq3_align re-aligns them.  A
// kernel that issues many rows' loads before an issue fence keeps the words
// raw until it decodes them, so no ALU work on loaded values (which would
// wait for the loads) sits in front of the fence.
struct RawIq3Words {
  uint32_t d0, q0, q1, q2, w0, w1;
  uint32_t rq;     // 2 when the superblock starts at 0 mod 4 (d in the low half), else 0
};

template <bool ST = false>
__device__ __forceinline__ RawIq3Words gm_load_iq3_words(const uint8_t* __restrict__ row, int sub) {
  const int sb = sub >> 3, s = sub & 7;
  const uint8_t* base = row + sb * GM_IQ3XXS_BYTES;
  const int odd = (int)((reinterpret_cast<uintptr_t>(base) >> 1) & 1);   // base % 4 == 2 * odd
  const uint32_t* dp = reinterpret_cast<const uint32_t*>(base - 2 * odd);
  RawIq3Words t;
  t.d0 = gm_ld<ST>(dp);
  // qs at base + 2 + 8s: offset % 4 == 2 when sb is even, 0 when odd
  const int rq = odd ? 0 : 2;
  t.rq = (uint32_t)rq;
  const uint32_t* qp = reinterpret_cast<const uint32_t*>(base + 2 + 8 * s - rq);
  t.q0 = gm_ld<ST>(qp);
  t.q1 = gm_ld<ST>(qp + 1);
  t.q2 = gm_ld<ST>(qp + (rq ? 2 : 1));
  // word at base + 66 + 4s: same parity rule
  const uint32_t* wp = reinterpret_cast<const uint32_t*>(base + 66 + 4 * s - rq);
  t.w0 = gm_ld<ST>(wp);
  t.w1 = gm_ld<ST>(wp + (rq ? 1 : 0));
  return t;
}

__device__ __forceinline__ RawIq3 gm_iq3_align(const RawIq3Words& t) {
  RawIq3 r;
  r.d = t.rq ? (t.d0 & 0xffffu) : (t.d0 >> 16);
  r.q0 = __builtin_amdgcn_alignbyte(t.q1, t.q0, t.rq);
  r.q1 = __builtin_amdgcn_alignbyte(t.q2, t.q1, t.rq);
  r.w = __builtin_amdgcn_alignbyte(t.w1, t.w0, t.rq);
  return r;
}

template <bool ST = false>
__device__ __forceinline__ RawIq3 gm_load_iq3(const uint8_t* __restrict__ row, int sub) {
  return gm_iq3_align(gm_load_iq3_words<ST>(row, sub));
}

// ksigns byte for a 7-bit index: the 7 explicit sign bits plus a parity bit
// that makes the byte's popcount even.
__device__ __forceinline__ uint32_t gm_ksigns(uint32_t s7) {
  return s7 | ((__builtin_popcount(s7) & 1u) << 7);
}

__device__ __forceinline__ float gm_decode_iq3(const RawIq3& r, const uint32_t* __restrict__ grid,
                                               float (&wv)[32]) {
  const float d = gm_h2f(r.d);
  const float db = d * (0.5f + (float)(r.w >> 28)) * 0.5f;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t qw = g < 2 ? r.q0 : r.q1;
    const uint32_t ga = grid[(qw >> (16 * (g & 1))) & 0xffu];
    const uint32_t gb = grid[(qw >> (16 * (g & 1) + 8)) & 0xffu];
    const uint32_t sg = gm_ksigns((r.w >> (7 * g)) & 127u);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float m = gm_ubyte(i < 4 ? ga : gb, i & 3);
      wv[8 * g + i] = ((sg >> i) & 1u) ? -m : m;
    }
  }
  return db;
}

// ------------------------------------------------------------------ BF16
struct RawBf16 {
  uint4 v[4];   // 32 bf16 values
};

template <bool ST = false>
__device__ __forceinline__ RawBf16 gm_load_bf16(const uint8_t* __restrict__ row, int sub) {
  const gm_u32x4* p = reinterpret_cast<const gm_u32x4*>(row + sub * 64);
  RawBf16 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const gm_u32x4 v = gm_ld<ST>(p + i);
    r.v[i] = uint4{v.x, v.y, v.z, v.w};
  }
  return r;
}

__device__ __forceinline__ float gm_decode_bf16(const RawBf16& r, float (&wv)[32]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t u[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wv[8 * i + 2 * j] = __uint_as_float(u[j] << 16);
      wv[8 * i + 2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
    }
  }
  return 1.0f;
}

// -------------------------------------------------------------------- I8
// Transcoded K-quant / Q8_0 rows (GM_QTYPE_I8, written by k_transcode_i8): a
// 32-weight sub-block is 48 bytes, int8 q[32] (weight k = byte k), fp32 s0
// (scale of weights 0-15), fp32 s1 (16-31), fp32 off, 4 zero bytes;
// weight k = s_{k / 16} q[k] + off.
struct RawI8 {
  gm_u32x4 q0, q1, s;   // q[0..15], q[16..31], {s0, s1, off, 0}
};

template <bool ST = false>
__device__ __forceinline__ RawI8 gm_load_i8(const uint8_t* __restrict__ row, int sub) {
  const gm_u32x4* p = reinterpret_cast<const gm_u32x4*>(row + sub * 48);
  return RawI8{gm_ld<ST>(p), gm_ld<ST>(p + 1), gm_ld<ST>(p + 2)};
}

__device__ __forceinline__ float gm_decode_i8row(const RawI8& r, float (&wv)[32]) {
  const float s0 = __uint_as_float(r.s.x), s1 = __uint_as_float(r.s.y), off = __uint_as_float(r.s.z);
  const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[4 * c + i] = fmaf(c < 4 ? s0 : s1, gm_sbyte(q[c], i), off);
  return 1.0f;
}

// ---------------------------------------------------------- generic front
template <int QT> struct RawSub;
template <> struct RawSub<GM_QTYPE_IQ4_XS> { using T = RawIq4; };
template <> struct RawSub<GM_QTYPE_IQ3_XXS> { using T = RawIq3; };
template <> struct RawSub<GM_QTYPE_BF16> { using T = RawBf16; };
template <> struct RawSub<GM_QTYPE_I8> { using T = RawI8; };

template <int QT, bool ST = false>
__device__ __forceinline__ typename RawSub<QT>::T gm_load_sub(const uint8_t* __restrict__ row, int sub) {
  if constexpr (QT == GM_QTYPE_IQ4_XS) return gm_load_iq4<ST>(row, sub);
  else if constexpr (QT == GM_QTYPE_IQ3_XXS) return gm_load_iq3<ST>(row, sub);
  else if constexpr (QT == GM_QTYPE_I8) return gm_load_i8<ST>(row, sub);
  else return gm_load_bf16<ST>(row, sub);
}

template <int QT>
__device__ __forceinline__ float gm_decode_sub(const typename RawSub<QT>::T& r, int sub,
                                               const uint32_t* __restrict__ grid, float (&wv)[32]) {
  if constexpr (QT == GM_QTYPE_IQ4_XS) return gm_decode_iq4(r, sub, wv);
  else if constexpr (QT == GM_QTYPE_IQ3_XXS) return gm_decode_iq3(r, grid, wv);
  else if constexpr (QT == GM_QTYPE_I8) return gm_decode_i8row(r, wv);
  else return gm_decode_bf16(r, wv);
}

// The IQ3_XXS grid (256 x 4 magnitudes) in global constant memory.
static __device__ const uint32_t gm_iq3xxs_grid[256] = {GM_IQ3XXS_GRID_INIT};

// Stage the IQ3_XXS grid in LDS (1 KB); every thread of the block must call.
__device__ __forceinline__ void gm_stage_grid(uint32_t* grid_lds) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) grid_lds[i] = gm_iq3xxs_grid[i];
}

// IQ3_XXS decode tables in LDS (3 KB): the grid as packed byte magnitudes,
// and per 7-bit ksigns index the byte masks of its 8 signs (0x00 / 0xff) with
// the same masks & 0x01 per byte: {signs 0-3, signs 4-7, low 0-3, low 4-7}.
struct Iq3Tab {
  uint32_t grid[256];
  gm_u32x4 sgn[128];
};

// Threads 0..255 each load one grid word (step 1) and store it with the sign
// masks (step 2); the block size must be >= 256.
__device__ __forceinline__ uint32_t gm_iq3_tab_load() {
  return threadIdx.x < 256 ? gm_iq3xxs_grid[threadIdx.x] : 0u;
}

__device__ __forceinline__ void gm_iq3_tab_store(uint32_t g, Iq3Tab* __restrict__ tab) {
  if (threadIdx.x < 256) tab->grid[threadIdx.x] = g;
  if (threadIdx.x < 128) {
    const uint32_t s = gm_ksigns(threadIdx.x);
    uint32_t m0 = 0, m1 = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      m0 |= ((s >> b) & 1u) ? 0xffu << (8 * b) : 0u;
      m1 |= ((s >> (b + 4)) & 1u) ? 0xffu << (8 * b) : 0u;
    }
    tab->sgn[threadIdx.x] = gm_u32x4{m0, m1, m0 & 0x01010101u, m1 & 0x01010101u};
  }
}

// Sign byte masks of a 7-bit ksigns index computed in registers: the byte
// with the parity bit (bit 7) is s = idx | (popcount(idx) & 1) << 7; byte i
// of o0 / o1 is bit i / i + 4 of s (the multiply spreads 4 bits to the low
// bit of 4 bytes without carries), and m0 / m1 are those bytes times 0xff.
// The same values as Iq3Tab::sgn[idx], for kernels where LDS traffic, not
// VALU issue, is the limit.
__device__ __forceinline__ gm_u32x4 gm_iq3_sign_masks(uint32_t idx7) {
  const uint32_t s = idx7 | ((__builtin_popcount(idx7) & 1u) << 7);
  const uint32_t o0 = ((s & 15u) * 0x00204081u) & 0x01010101u;
  const uint32_t o1 = ((s >> 4) * 0x00204081u) & 0x01010101u;
  return gm_u32x4{o0 * 0xffu, o1 * 0xffu, o0, o1};
}

// Signed int8 weights of one sub-block in k order (byte i of w[c] is weight
// 4c + i) and the sub-block scale: weight[k] == scale * int8 exactly.
//   IQ4_XS: kvalues (npu/quant_mv_iq4.py:194-197), scale d (ls - 32);
//   IQ3_XXS: +-grid magnitude (<= 62, never 0, so the byte negation
//            (g ^ 0xff) + 1 cannot carry), scale d (0.5 + s4) / 2; the sign
//            masks from the LDS table, or computed (ARITH).
template <int QT, bool ARITH = false>
__device__ __forceinline__ float gm_decode_i8(const typename RawSub<QT>::T& r, int sub, const Iq3Tab* __restrict__ tab,
                                              uint32_t (&w)[8]) {
  if constexpr (QT == GM_QTYPE_IQ4_XS) {
    const int s = sub & 7;
    const float d = gm_h2f(r.h0 & 0xffffu);
    const uint32_t sh = r.h0 >> 16;
    const uint32_t sl = (r.h1 >> (8 * (s >> 1) + 4 * (s & 1))) & 15u;
    const int ls = (int)(sl | (((sh >> (2 * s)) & 3u) << 4));
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      w[c] = gm_iq4nl_lut4(r.q[c] & 0x0f0f0f0fu);
      w[4 + c] = gm_iq4nl_lut4((r.q[c] >> 4) & 0x0f0f0f0fu);
    }
    return d * (float)(ls - 32);
  } else {
    const float d = gm_h2f(r.d);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t qw = (g < 2 ? r.q0 : r.q1) >> (16 * (g & 1));
      const uint32_t ga = tab->grid[qw & 0xffu], gb = tab->grid[(qw >> 8) & 0xffu];
      const gm_u32x4 m = ARITH ? gm_iq3_sign_masks((r.w >> (7 * g)) & 127u) : tab->sgn[(r.w >> (7 * g)) & 127u];
      w[2 * g] = (ga ^ m.x) + m.z;
      w[2 * g + 1] = (gb ^ m.y) + m.w;
    }
    return d * (0.5f + (float)(r.w >> 28)) * 0.5f;
  }
}

// Float weights (scale excluded) with the LDS tables where a format needs them.
template <int QT>
__device__ __forceinline__ float gm_decode_sub_t(const typename RawSub<QT>::T& r, int sub,
                                                 const Iq3Tab* __restrict__ tab, float (&wv)[32]) {
  if constexpr (QT == GM_QTYPE_IQ3_XXS || QT == GM_QTYPE_IQ4_XS) {
    uint32_t w[8];
    const float sc = gm_decode_i8<QT>(r, sub, tab, w);
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) wv[4 * c + i] = gm_sbyte(w[c], i);
    return sc;
  } else {
    return gm_decode_sub<QT>(r, sub, nullptr, wv);
  }
}

// 32-wide dot of decoded weights with x (LDS or registers).
__device__ __forceinline__ float gm_dot32(const float (&wv)[32], const float* __restrict__ x) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = 0; i < 32; i += 8) {
    const float4 a = *reinterpret_cast<const float4*>(x + i);
    const float4 b = *reinterpret_cast<const float4*>(x + i + 4);
    s0 = fmaf(wv[i + 0], a.x, s0); s1 = fmaf(wv[i + 4], b.x, s1);
    s0 = fmaf(wv[i + 1], a.y, s0); s1 = fmaf(wv[i + 5], b.y, s1);
    s0 = fmaf(wv[i + 2], a.z, s0); s1 = fmaf(wv[i + 6], b.z, s1);
    s0 = fmaf(wv[i + 3], a.w, s0); s1 = fmaf(wv[i + 7], b.w, s1);
  }
  return s0 + s1;
}
