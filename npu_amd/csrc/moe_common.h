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

// Max over lanes 8j .. 8j+7: the two quad swaps, then the half-row mirror.
__device__ __forceinline__ float gm_max8(float m) {
  m = fmaxf(m, GM_DPP_F(m, GM_QPERM_1032));
  m = fmaxf(m, GM_DPP_F(m, GM_QPERM_2301));
  return fmaxf(m, GM_DPP_F(m, 0x141));                       // row_half_mirror
}

// Sum over lanes 8j .. 8j+7 (the same value in all of them: each step adds a
// lane's partner, so all 8 lanes add the same terms, in the same order per pair).
__device__ __forceinline__ float gm_sum8(float v) {
  v += GM_DPP_F(v, GM_QPERM_1032);
  v += GM_DPP_F(v, GM_QPERM_2301);
  return v + GM_DPP_F(v, 0x141);                             // row_half_mirror
}

// ------------------------------------------------------------------ top-k
// One wave: top-k of E logits (descending, ties -> lower id), softmax over all
// E, renormalised top-k probabilities (qwen/forward.py:609-611).
// Lane values of one wave's top-k input: logits lane + 64 i (clamped loads,
// so every lane issues the same MAXV loads; out-of-range entries are masked
// by topk_keys).
template <int MAXV>
__device__ __forceinline__ void topk_load(const float* __restrict__ lg, int E, float (&v)[MAXV], int (&ix)[MAXV]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    ix[i] = lane + 64 * i;
    v[i] = lg[ix[i] < E ? ix[i] : E - 1];
  }
}

// Unsigned key with the order of the float values: NaN of either sign is the
// largest (torch.topk ranks NaN above every number), -0 and +0 are equal, and
// every value has a key >= 0x007fffff (-inf), so 0 marks an absent entry.
// Branch-free (selects only), so a wave's keys cost a few VALU per value.
__device__ __forceinline__ uint32_t ukey(float f) {
  const uint32_t b = __float_as_uint(f);
  const uint32_t flip = (uint32_t)((int32_t)b >> 31) | 0x80000000u;   // negative: all bits, else the sign bit
  uint32_t k = b ^ flip;
  k = b == 0x80000000u ? 0x80000000u : k;                             // -0: the key of +0
  return (b & 0x7fffffffu) > 0x7f800000u ? 0xffffffffu : k;          // NaN of either sign: the largest
}

// Value back from a key (NaN keys give a NaN, -0 comes back as +0).
__device__ __forceinline__ float ukey_inv(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

template <int MAXV>
__device__ __forceinline__ void topk_keys(const float (&v)[MAXV], const int (&ix)[MAXV], int E, uint32_t (&u)[MAXV]) {
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const uint32_t kv = ukey(v[i]);                      // computed for every lane, then masked
    u[i] = ix[i] < E ? kv : 0u;
  }
}

// Wave-uniform selection: on return bit l of sel[i] is set iff entry
// lane l + 64 i is one of the k largest keys, exact ties at the k-th value
// going to the lowest ids.  Bisection over the key bits, most significant
// first, for a threshold with exactly k keys at or above it: each step is one
// compare and ballot per value and scalar popcounts, and it stops as soon as
// such a threshold is found (after about 14 of the 32 steps for random
// logits).  If the k-th and (k+1)-th keys are equal it ends with the k-th key
// itself, and the keys equal to it are taken in ascending id order.
template <int MAXV>
__device__ __forceinline__ void topk_masks_bisect(const uint32_t (&u)[MAXV], int k, uint64_t (&sel)[MAXV]) {
  uint32_t ans = 0;
  int cnt = 0x7fffffff;                                  // keys >= ans (once ans > 0)
  for (uint32_t bit = 0x80000000u; bit != 0u; bit >>= 1) {
    // the threshold is wave-uniform: readfirstlane keeps it (and the loop) scalar
    const uint32_t cand = (uint32_t)__builtin_amdgcn_readfirstlane((int)(ans | bit));
    int c = 0;
#pragma unroll
    for (int i = 0; i < MAXV; ++i) c += __popcll(__ballot(u[i] >= cand));
    if (c >= k) {
      ans = cand;
      cnt = c;
      if (c == k) break;
    }
  }
  if (cnt == k) {
#pragma unroll
    for (int i = 0; i < MAXV; ++i) sel[i] = __ballot(u[i] >= ans);
    return;
  }
  int need = k;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    sel[i] = __ballot(u[i] > ans);
    need -= __popcll(sel[i]);
  }
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    uint64_t eq = __ballot(u[i] == ans);
    while (need > 0 && eq != 0) {
      const uint64_t low = eq & (~eq + 1ull);
      sel[i] |= low;
      eq ^= low;
      --need;
    }
  }
}

// Candidate network (the fast path of topk_masks).  An entry is a pair (key,
// id) held as two words, hi = key and lo = ~id: the order of the 64-bit value
// hi:lo is the selection order (larger key first, then lower id).
__device__ __forceinline__ uint64_t tk_pair(uint32_t hi, uint32_t lo) { return ((uint64_t)hi << 32) | lo; }

// Compare-exchange with the partner's pair (phi, plo): a lane with `up` set
// keeps the smaller pair, any other lane the larger.
__device__ __forceinline__ void tk_ce(uint32_t& hi, uint32_t& lo, uint32_t phi, uint32_t plo, bool up) {
  const bool take = (tk_pair(phi, plo) > tk_pair(hi, lo)) != up;
  hi = take ? phi : hi;
  lo = take ? plo : lo;
}

// DPP move; a lane whose source lies outside its row reads 0 (bound_ctrl), so
// no old value has to be set up.
template <int CTRL>
__device__ __forceinline__ uint32_t tk_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}

// Partner through one DPP pattern.
template <int CTRL>
__device__ __forceinline__ void tk_stage(uint32_t& hi, uint32_t& lo, bool up) {
  tk_ce(hi, lo, tk_dpp<CTRL>(hi), tk_dpp<CTRL>(lo), up);
}

// Partner lane ^ 4 within 8 lanes: row_shl:4 brings lane + 4 to the lower
// four, row_shr:4 lane - 4 to the upper four (the upper four keep the smaller).
__device__ __forceinline__ void tk_stage_x4(uint32_t& hi, uint32_t& lo) {
  const bool up = (threadIdx.x & 4) != 0;
  const uint32_t ah = tk_dpp<0x104>(hi), al = tk_dpp<0x104>(lo);
  const uint32_t bh = tk_dpp<0x114>(hi), bl = tk_dpp<0x114>(lo);
  tk_ce(hi, lo, up ? bh : ah, up ? bl : al, up);
}

// Fast path of topk_masks.  t0 = the smallest of the eight 8-lane group
// maxima: the eight maxima are distinct entries >= t0, so the k <= 8 largest
// entries are all >= t0.  When at most 32 entries are >= t0 they are compacted
// into lanes 0 .. 31 (ds_permute, other lanes hold 0:0) and a bitonic network
// on DPP leaves the 8 largest pairs, sorted, in lanes 0 .. 7: each 8-lane
// group is sorted, then groups are merged two at a time (a mirrored compare
// keeps the larger half in the lower group, then half-cleaners at distances
// 4, 2, 1).  Merges that only meet empty groups are skipped.  The k-th pair
// then selects, exactly as the bisection does.  Returns false (sel untouched)
// when a group holds no entry or more than 32 entries are >= t0.
template <int MAXV>
__device__ __forceinline__ bool topk_masks_net(const uint32_t (&u)[MAXV], int k, uint64_t (&sel)[MAXV]) {
  const int lane = threadIdx.x & 63;
  uint32_t m = u[0];
#pragma unroll
  for (int i = 1; i < MAXV; ++i) m = max(m, u[i]);
  m = max(m, (uint32_t)GM_DPP_I((int)m, GM_QPERM_1032));
  m = max(m, (uint32_t)GM_DPP_I((int)m, GM_QPERM_2301));
  m = max(m, (uint32_t)GM_DPP_I((int)m, 0x141));             // row_half_mirror: the 8-lane group maximum
  m = min(m, (uint32_t)GM_DPP_I((int)m, 0x140));             // row_mirror: the smaller of the row's two groups
  const uint32_t t0 = min(min((uint32_t)__builtin_amdgcn_readlane((int)m, 0), (uint32_t)__builtin_amdgcn_readlane((int)m, 16)),
                          min((uint32_t)__builtin_amdgcn_readlane((int)m, 32), (uint32_t)__builtin_amdgcn_readlane((int)m, 48)));
  if (t0 == 0u) return false;                                // a group without entries
  uint64_t cm[MAXV];
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    cm[i] = __ballot(u[i] >= t0);
    cnt += __popcll(cm[i]);
  }
  if (cnt > 32) return false;
  uint32_t hi = 0u, lo = 0u;
  int base = 0;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const uint64_t c = cm[i];
    const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(c >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)c, 0u));
    const int dst = ((c >> lane) & 1ull) ? base + below : 63;   // lane 63 receives no candidate
    const uint32_t kv = (uint32_t)__builtin_amdgcn_ds_permute(dst << 2, (int)u[i]);
    const uint32_t iv = (uint32_t)__builtin_amdgcn_ds_permute(dst << 2, ~(lane + 64 * i));
    const int n = __popcll(c);
    const bool here = lane >= base && lane < base + n;
    hi = here ? kv : hi;
    lo = here ? iv : lo;
    base += n;
  }
  const int l = lane & 7;
  tk_stage<GM_QPERM_1032>(hi, lo, (l & 1) != 0);             // sort 8: pairs
  tk_stage<0x1B>(hi, lo, (l & 3) >= 2);                      // quads: quad_perm [3,2,1,0]
  tk_stage<GM_QPERM_1032>(hi, lo, (l & 1) != 0);
  tk_stage<0x141>(hi, lo, l >= 4);                           // eights: row_half_mirror
  tk_stage<GM_QPERM_2301>(hi, lo, (l & 2) != 0);
  tk_stage<GM_QPERM_1032>(hi, lo, (l & 1) != 0);
  if (cnt > 8) {                                             // lanes 8j .. 8j+7 with 8j+8 < 16: merge 16
    tk_stage<0x140>(hi, lo, (lane & 8) != 0);                // row_mirror
    tk_stage_x4(hi, lo);
    tk_stage<GM_QPERM_2301>(hi, lo, (l & 2) != 0);
    tk_stage<GM_QPERM_1032>(hi, lo, (l & 1) != 0);
  }
  if (cnt > 16) {                                            // lanes 0 .. 7 with lanes 23 .. 16 (lane ^ 0x17)
    const uint32_t phi = (uint32_t)__builtin_amdgcn_ds_swizzle((int)hi, 0x5C1F);
    const uint32_t plo = (uint32_t)__builtin_amdgcn_ds_swizzle((int)lo, 0x5C1F);
    tk_ce(hi, lo, phi, plo, (lane & 16) != 0);
    tk_stage_x4(hi, lo);
    tk_stage<GM_QPERM_2301>(hi, lo, (l & 2) != 0);
    tk_stage<GM_QPERM_1032>(hi, lo, (l & 1) != 0);
  }
  const uint64_t kth = tk_pair((uint32_t)__builtin_amdgcn_readlane((int)hi, k - 1),
                               (uint32_t)__builtin_amdgcn_readlane((int)lo, k - 1));
#pragma unroll
  for (int i = 0; i < MAXV; ++i) sel[i] = __ballot(tk_pair(u[i], ~(uint32_t)(lane + 64 * i)) >= kth);
  return true;
}

template <int MAXV>
__device__ __forceinline__ void topk_masks(const uint32_t (&u)[MAXV], int k, uint64_t (&sel)[MAXV]) {
  if (!topk_masks_net<MAXV>(u, k, sel)) topk_masks_bisect<MAXV>(u, k, sel);
}

// Expert id of rank r (0-based, ascending id) among the selected entries
// (wave-uniform r).
template <int MAXV>
__device__ __forceinline__ int topk_rank_id(const uint64_t (&sel)[MAXV], int r) {
  int id = 0;
  bool done = false;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = __popcll(sel[i]);
    if (!done && r < c) {
      uint64_t m = sel[i];
      for (int j = 0; j < r; ++j) m &= m - 1ull;
      id = 64 * i + __builtin_ctzll(m);
      done = true;
    }
    if (!done) r -= c;
  }
  return id;
}

// Lane r < k ends with the selected entry of rank r in ascending id order: its
// key and id (other lanes: key 0, id 0x7fffffff).  Per key word, each lane
// pushes its selected entry to lane (selected entries before it) with
// ds_permute; unselected lanes push to lane 63, which holds no rank (k <= 8).
template <int MAXV>
__device__ __forceinline__ void topk_compact(const uint64_t (&sel)[MAXV], const uint32_t (&u)[MAXV], int k,
                                             uint32_t& rkey, int& rid) {
  const int lane = threadIdx.x & 63;
  uint32_t key = 0u;
  int id = 0x7fffffff;
  int base = 0;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const uint64_t m = sel[i];
    const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    const int dst = ((m >> lane) & 1ull) ? base + below : 63;
    const uint32_t kv = (uint32_t)__builtin_amdgcn_ds_permute(dst << 2, (int)u[i]);
    const int iv = __builtin_amdgcn_ds_permute(dst << 2, lane + 64 * i);
    const int cnt = __popcll(m);
    const bool here = lane >= base && lane < base + cnt;
    key = here ? kv : key;
    id = here ? iv : id;
    base += cnt;
  }
  rkey = lane < k ? key : 0u;
  rid = lane < k ? id : 0x7fffffff;
}

// Renormalised softmax weight of the pick in lane r < k (key rkey, lanes >= k
// hold key 0): softmax over all valid entries with the largest key as the
// maximum, then p / max(sum of the k picks, 1e-20) (qwen/forward.py:609-611).
// Other lanes return 0.
template <int MAXV>
__device__ __forceinline__ float topk_weight(const uint32_t (&u)[MAXV], uint32_t rkey, int k) {
  const int lane = threadIdx.x & 63;
  uint32_t mk = rkey;                                     // max over lanes 0 .. 7 (the picks)
  mk = max(mk, (uint32_t)GM_DPP_I((int)mk, GM_QPERM_1032));
  mk = max(mk, (uint32_t)GM_DPP_I((int)mk, GM_QPERM_2301));
  mk = max(mk, (uint32_t)GM_DPP_I((int)mk, 0x141));       // row_half_mirror
  const float m = ukey_inv((uint32_t)__builtin_amdgcn_readlane((int)mk, 0));
  float z = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const float e = expf(ukey_inv(u[i]) - m);
    z += u[i] != 0u ? e : 0.f;
  }
  z = gm_wave_sum64(z);
  const float p = lane < k ? expf(ukey_inv(rkey) - m) / z : 0.f;
  const float den = fmaxf(gm_sum8(p), 1e-20f);           // lanes 0 .. 7: the sum of the k picks
  return p / den;
}

// One compare-exchange stage of an 8-lane bitonic sort: the partner's pick via
// DPP (CTRL), the lower lane of the pair keeps the better one (larger key,
// then lower id).
template <int CTRL>
__device__ __forceinline__ void sort8_stage(uint32_t& key, int& id, float& w, bool lower) {
  const uint32_t pk = (uint32_t)GM_DPP_I((int)key, CTRL);
  const int pi = GM_DPP_I(id, CTRL);
  const float pw = GM_DPP_F(w, CTRL);
  const bool pbetter = pk > key || (pk == key && pi < id);
  const bool take = lower ? pbetter : !pbetter;
  key = take ? pk : key;
  id = take ? pi : id;
  w = take ? pw : w;
}

// Sorts each group of 8 lanes by (key descending, id ascending), carrying w:
// bitonic merges of 2, 4 and 8 lanes, each opened by a mirrored compare
// (partner 2^s - 1 - i) so that every stage sorts in the same direction.
__device__ __forceinline__ void topk_sort8(uint32_t& key, int& id, float& w) {
  const int l = threadIdx.x & 7;
  sort8_stage<GM_QPERM_1032>(key, id, w, (l & 1) == 0);   // pairs (mirror of 2 = xor 1)
  sort8_stage<0x1B>(key, id, w, (l & 3) < 2);              // quads: quad_perm [3,2,1,0]
  sort8_stage<GM_QPERM_1032>(key, id, w, (l & 1) == 0);
  sort8_stage<0x141>(key, id, w, l < 4);                   // eights: row_half_mirror
  sort8_stage<GM_QPERM_2301>(key, id, w, (l & 2) == 0);
  sort8_stage<GM_QPERM_1032>(key, id, w, (l & 1) == 0);
}

// Lane s < k ends with pick s in descending order (larger keys first, equal
// keys in ascending id order): its expert id and renormalised weight (other
// lanes: id 0x7fffffff, weight 0).
template <int MAXV>
__device__ __forceinline__ void topk_finish(const float (&v)[MAXV], const int (&ix)[MAXV], int E, int k,
                                            int& out_id, float& out_w) {
  const int lane = threadIdx.x & 63;
  uint32_t u[MAXV];
  uint64_t sel[MAXV];
  topk_keys<MAXV>(v, ix, E, u);
  topk_masks<MAXV>(u, k, sel);
  uint32_t key;
  int id;
  topk_compact<MAXV>(sel, u, k, key, id);
  float w = topk_weight<MAXV>(u, key, k);
  topk_sort8(key, id, w);
  out_id = lane < k ? id : 0x7fffffff;
  out_w = lane < k ? w : 0.f;
}

template <int MAXV>
__device__ __forceinline__ void wave_topk(const float* __restrict__ lg, int E, int k, int32_t* __restrict__ ids,
                                          float* __restrict__ wts) {
  float v[MAXV];
  int ix[MAXV];
  topk_load<MAXV>(lg, E, v, ix);
  int id;
  float w;
  topk_finish<MAXV>(v, ix, E, k, id, w);
  const int lane = threadIdx.x & 63;
  if (lane < k) {
    ids[lane] = id;
    wts[lane] = w;
  }
}

// --------------------------------------------------------------- grouping
// Grouping of (token, slot) pairs by expert into LDS: g[0] = n_unique,
// g[1+u] = expert of unique slot u (ascending), g[65+u] = member count,
// g[129 + 8u + m] = pair index t*k + j of member m (pairs ascending).  Wave 0
// does the work (P <= 64 pairs, one per lane): the lanes sharing a lane's
// expert are found with one ballot per bit of the id, the rank of the expert
// among the unique ones from an LDS bitmap (bits[0..15]) and its prefix counts
// (bits[16..31]; E <= 512).  All threads call; ends with a barrier.
__device__ __forceinline__ void block_group(const int32_t* __restrict__ ids, int P, int E, int32_t* __restrict__ g,
                                            uint32_t* __restrict__ bits) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int nwords = (E + 31) / 32;
    if (lane < nwords) bits[lane] = 0u;
    const int e = lane < P ? ids[lane] : -1;
    const uint64_t valid = __ballot(e >= 0);
    uint64_t same = valid;
    for (int b = 0; (1 << b) < E; ++b) {
      const uint64_t bm = __ballot((e >> b) & 1);
      same &= ((e >> b) & 1) ? bm : ~bm;
    }
    const int m = __popcll(same & ((1ull << lane) - 1ull));   // members of my expert before me
    const int cnt = __popcll(same);
    if (e >= 0 && m == 0) atomicOr(&bits[e >> 5], 1u << (e & 31));   // same wave: LDS ops stay in order
    // prefix popcounts of the bitmap words (lane w < 16 holds the count of
    // unique experts below word w), then one read of each per lane
    const uint32_t bw = lane < 16 ? bits[lane] : 0u;
    const int pc = lane < nwords ? __builtin_popcount(bw) : 0;
    int incl = pc;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int up = __shfl_up(incl, o, 64);
      incl += (lane & 15) >= o ? up : 0;
    }
    if (lane < 16) bits[16 + lane] = (uint32_t)(incl - pc);
    int rank = 0;
    if (e >= 0) rank = (int)bits[16 + (e >> 5)] + __builtin_popcount(bits[e >> 5] & ((1u << (e & 31)) - 1u));
    const int nu = __popcll(__ballot(e >= 0 && m == 0));       // ballot with every lane active
    if (lane == 0) g[0] = nu;
    if (e >= 0) {
      g[1 + rank] = e;
      g[1 + GM_GRP_MAXU + rank] = cnt;
      g[1 + 2 * GM_GRP_MAXU + rank * GM_GRP_MAXM + m] = lane;
    }
  }
  __syncthreads();
}

// Keeps the compiler's scheduler from moving instructions across this point:
// placed after a kernel has issued all of its loads, so that none is sunk
// next to its first use (where, behind the weight loads in the in-order
// vmcnt queue, each would wait for everything issued before it), and between
// independent passes to bound register pressure.
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

// ------------------------------------------------------------ router rows
// The router and the shared scalar gate come as bf16 bits or as fp32
// (gm_moe_layer.q_router; the reference reads both in fp32,
// qwen/forward.py:41-47, 599, 608).  A lane takes 8 consecutive values of a
// row: one 16-byte load of bf16, two of fp32.
template <bool F32>
using RouterChunk = gm_u32x4[F32 ? 2 : 1];

template <bool F32>
__device__ __forceinline__ const void* router_row(const void* base, int64_t row, int D) {
  return static_cast<const char*>(base) + row * D * (F32 ? 4 : 2);
}

template <bool F32, bool ST>
__device__ __forceinline__ void router_load8(const void* row, int kk, RouterChunk<F32>& r) {
  if constexpr (F32) {
    const gm_u32x4* p = reinterpret_cast<const gm_u32x4*>(static_cast<const float*>(row) + kk);
    r[0] = gm_ld<ST>(p);
    r[1] = gm_ld<ST>(p + 1);
  } else {
    r[0] = gm_ld<ST>(reinterpret_cast<const gm_u32x4*>(static_cast<const uint16_t*>(row) + kk));
  }
}

template <bool F32>
__device__ __forceinline__ void router_unpack8(const RouterChunk<F32>& r, float (&w)[8]) {
  if constexpr (F32) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      w[4 * h + 0] = __uint_as_float(r[h].x);
      w[4 * h + 1] = __uint_as_float(r[h].y);
      w[4 * h + 2] = __uint_as_float(r[h].z);
      w[4 * h + 3] = __uint_as_float(r[h].w);
    }
  } else {
    const uint32_t v[4] = {r[0].x, r[0].y, r[0].z, r[0].w};
#pragma unroll
    for (int j = 0; j < 8; ++j)
      w[j] = (j & 1) ? __uint_as_float(v[j >> 1] & 0xffff0000u) : __uint_as_float(v[j >> 1] << 16);
  }
}

// --------------------------------------------------------- I8 x limbs
// One I8 sub-block (int8 q, scales s0 / s1 of its halves, offset off) against
// the limbs of one activation sub-block: s0 sum_{k<16} q_k a_k + s1 sum_{k>=16}
// q_k a_k + off sum_k a_k, the products on v_dot4_i32_i8 (exact int32 sums per
// half and limb), the activation sum stored with the limbs.
__device__ __forceinline__ float gm_i8_limb_dot(const RawI8& r, const uint32_t (&l0)[8], const uint32_t (&l1)[8],
                                               const uint32_t (&l2)[8], float hscale, float asum) {
  const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
  int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    a0 = __builtin_amdgcn_sdot4((int)q[c], (int)l0[c], a0, false);
    a1 = __builtin_amdgcn_sdot4((int)q[c], (int)l1[c], a1, false);
    a2 = __builtin_amdgcn_sdot4((int)q[c], (int)l2[c], a2, false);
    b0 = __builtin_amdgcn_sdot4((int)q[4 + c], (int)l0[4 + c], b0, false);
    b1 = __builtin_amdgcn_sdot4((int)q[4 + c], (int)l1[4 + c], b1, false);
    b2 = __builtin_amdgcn_sdot4((int)q[4 + c], (int)l2[4 + c], b2, false);
  }
  const float va = fmaf((float)a2, 65536.f, fmaf((float)a1, 256.f, (float)a0));
  const float vb = fmaf((float)b2, 65536.f, fmaf((float)b1, 256.f, (float)b0));
  const float s0 = __uint_as_float(r.s.x), s1 = __uint_as_float(r.s.y), off = __uint_as_float(r.s.z);
  return fmaf(hscale, fmaf(s0, va, s1 * vb), off * asum);
}

// The same with the activation sub-block read from its limb row (LDS).
__device__ __forceinline__ float gm_i8_dot_limbs(const RawI8& r, const uint8_t* __restrict__ s) {
  const gm_u32x4* p = reinterpret_cast<const gm_u32x4*>(s);
  const gm_u32x4 l0a = p[0], l0b = p[1], l1a = p[2], l1b = p[3], l2a = p[4], l2b = p[5];
  const uint32_t l0[8] = {l0a.x, l0a.y, l0a.z, l0a.w, l0b.x, l0b.y, l0b.z, l0b.w};
  const uint32_t l1[8] = {l1a.x, l1a.y, l1a.z, l1a.w, l1b.x, l1b.y, l1b.z, l1b.w};
  const uint32_t l2[8] = {l2a.x, l2a.y, l2a.z, l2a.w, l2b.x, l2b.y, l2b.z, l2b.w};
  const float2 hs = *reinterpret_cast<const float2*>(s + 96);
  return gm_i8_limb_dot(r, l0, l1, l2, hs.x, hs.y);
}

// --------------------------------------------------------- row streaming
// The decode kernels issue every weight load a lane needs before they wait on
// anything: SPL sub-blocks per lane and row, at sub = lir + LR * i.  Indices
// past the row are clamped to its last sub-block (a harmless duplicate load
// whose result is skipped), so the loads are unconditional and straight-line
// and the compiler can count them instead of draining the queue before each.
// What a fetch keeps until the decode: the raw sub-block, or for IQ3_XXS its
// unaligned words (gm_iq3_align at decode time), so that no ALU work on
// loaded values, which would wait for the loads, is issued with the loads.
template <int QT> struct FetchRaw { using T = typename RawSub<QT>::T; };
template <> struct FetchRaw<GM_QTYPE_IQ3_XXS> { using T = RawIq3Words; };

template <int QT, bool ST = false>
__device__ __forceinline__ typename FetchRaw<QT>::T gm_fetch_sub(const uint8_t* __restrict__ row, int sub) {
  if constexpr (QT == GM_QTYPE_IQ3_XXS) return gm_load_iq3_words<ST>(row, sub);
  else return gm_load_sub<QT, ST>(row, sub);
}

template <int QT>
__device__ __forceinline__ typename RawSub<QT>::T gm_fetched(const typename FetchRaw<QT>::T& t) {
  if constexpr (QT == GM_QTYPE_IQ3_XXS) return gm_iq3_align(t);
  else return t;
}

template <int QT, int SPL>
struct RowFetch {
  typename FetchRaw<QT>::T r[SPL];
};

template <int QT, int LR, int SPL, bool ST = false>
__device__ __forceinline__ void fetch_subs(RowFetch<QT, SPL>& f, const uint8_t* __restrict__ row, int lir, int nsub) {
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    const int sub = lir + LR * i;
    f.r[i] = gm_fetch_sub<QT, ST>(row, sub < nsub ? sub : nsub - 1);
  }
}

// Makes fetched raw weights opaque to the optimiser at this point, so that
// their decode stays inside a loop instead of being hoisted out of it with
// every decoded value kept live across iterations.
template <int QT, int SPL>
__device__ __forceinline__ void opaque(RowFetch<QT, SPL>& f) {
  static_assert(sizeof(typename RawSub<QT>::T) % 4 == 0, "raw sub-block is whole dwords");
  uint32_t* w = reinterpret_cast<uint32_t*>(&f.r[0]);
#pragma unroll
  for (int i = 0; i < SPL * (int)sizeof(typename RawSub<QT>::T) / 4; ++i) asm volatile("" : "+v"(w[i]));
}

// acc[m] += W_row . act[idx[m]] over the fetched sub-blocks, m < nt; act rows
// are interleaved LDS rows of K floats.
template <int QT, int LR, int SPL, int NT>
__device__ __forceinline__ void dot_subs(const RowFetch<QT, SPL>& f, int lir, int nsub, const float* __restrict__ act,
                                         int K, const int (&idx)[NT], int nt, const Iq3Tab* __restrict__ tab,
                                         float (&acc)[NT]) {
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    const int sub = lir + LR * i;
    if (sub < nsub) {
      float wv[32];
      const float sc = gm_decode_sub_t<QT>(gm_fetched<QT>(f.r[i]), sub, tab, wv);
#pragma unroll
      for (int m = 0; m < NT; ++m)
        if (m < nt) acc[m] = fmaf(sc, gm_dot32_il(wv, act + idx[m] * K, sub, nsub), acc[m]);
    }
  }
}

// ------------------------------------------------- int8-limb activations
// The decode kernels multiply the int8 weights of gm_decode_i8 with
// activations split into three int8 limbs on v_dot4_i32_i8.  A sub-block of
// 32 activations a_k with |a_k| < 2^E is held as q_k = rne(a_k 2^(22-E)),
// q_k = L2 2^16 + L1 2^8 + L0 (L0, L1 in [-128, 127], |L2| <= 65), so that
// a_k = 2^(E-22) q_k to within 2^(E-23) and every partial dot product
// sum_k w_k L_k (|w| <= 127, 32 terms) is an exact int32 below 2^24.
// LDS layout per sub-block, GM_LSUB = 112 bytes (a 28-dword stride spreads 16
// consecutive sub-blocks over all 64 banks): plane L0 (32 bytes, byte i of
// dword c = k 4c + i), plane L1, plane L2, float 2^(E-22), float sum of the
// 32 activations (the offset term of I8 weights), 8 spare bytes.
constexpr int GM_LSUB = 112;

__host__ __device__ inline int gm_limb_row_bytes(int K) { return (K / GM_SUB) * GM_LSUB; }

// Low bytes of four int32 -> one dword.
__device__ __forceinline__ uint32_t gm_pack_lo4(int a, int b, int c, int d) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000c0cu);
  return lo | hi;
}

// rne(v * up) and its three limb bytes, packed per plane for 4 values.
__device__ __forceinline__ void gm_limb_planes(gm_f32x4 v, float up, uint32_t& p0, uint32_t& p1, uint32_t& p2) {
  int q[4];
  const float f[4] = {v.x * up, v.y * up, v.z * up, v.w * up};
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = __float_as_int(f[i] + 12582912.0f) - 0x4B400000;   // rne, |f| < 2^22
  int t1[4], t2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) { t1[i] = (q[i] + 128) >> 8; t2[i] = (t1[i] + 128) >> 8; }
  p0 = gm_pack_lo4(q[0], q[1], q[2], q[3]);
  p1 = gm_pack_lo4(t1[0], t1[1], t1[2], t1[3]);
  p2 = gm_pack_lo4(t2[0], t2[1], t2[2], t2[3]);
}

// Exponent E (|a| < 2^E for the block max m, clamped below at -100) and the
// quantisation factor 2^(22 - E) / sub-block scale 2^(E - 22); NaN scale for
// a non-finite m.
__device__ __forceinline__ void gm_limb_scale(float m, float& up, float& scale) {
  const int E = m > 0.f && m <= 3.4e38f ? max(__builtin_amdgcn_frexp_expf(m), -100) : 0;
  up = __builtin_ldexpf(1.0f, 22 - E);
  scale = m <= 3.4e38f ? __builtin_ldexpf(1.0f, E - 22) : __builtin_nanf("");
}

__device__ __forceinline__ float gm_absmax4(gm_f32x4 v) {
  const float ax = fabsf(v.x), ay = fabsf(v.y), az = fabsf(v.z), aw = fabsf(v.w);
  const bool fin = ax <= 3.4e38f && ay <= 3.4e38f && az <= 3.4e38f && aw <= 3.4e38f;
  return fin ? fmaxf(fmaxf(ax, ay), fmaxf(az, aw)) : __builtin_inff();
}

// Limbs of activations 4c .. 4c+7 (c even) of a row into `row`: as
// gm_put_limbs4 with 4 lanes per sub-block (lanes 4j .. 4j+3, c / 2 % 4 ==
// lane % 4).
// The limbs, scale and activation sum of 8 values (a, b), computed by 4 lanes
// per sub-block as gm_put_limbs8 describes; stored with gm_store_limbs8.
struct GmLimbs8 {
  uint32_t a0, a1, a2, b0, b1, b2;
  float scale, sum;
};

__device__ __forceinline__ GmLimbs8 gm_limbs8(gm_f32x4 a, gm_f32x4 b) {
  float m = fmaxf(gm_absmax4(a), gm_absmax4(b));
  m = fmaxf(m, GM_DPP_F(m, GM_QPERM_1032));
  m = fmaxf(m, GM_DPP_F(m, GM_QPERM_2301));
  float up;
  GmLimbs8 l;
  gm_limb_scale(m, up, l.scale);
  gm_limb_planes(a, up, l.a0, l.a1, l.a2);
  gm_limb_planes(b, up, l.b0, l.b1, l.b2);
  float sum = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
  sum += GM_DPP_F(sum, GM_QPERM_1032);
  sum += GM_DPP_F(sum, GM_QPERM_2301);
  l.sum = sum;
  return l;
}

__device__ __forceinline__ void gm_store_limbs8(const GmLimbs8& l, int c, uint8_t* __restrict__ row) {
  uint8_t* sb = row + (c >> 3) * GM_LSUB + 4 * (c & 7);
  *reinterpret_cast<uint2*>(sb) = make_uint2(l.a0, l.b0);
  *reinterpret_cast<uint2*>(sb + 32) = make_uint2(l.a1, l.b1);
  *reinterpret_cast<uint2*>(sb + 64) = make_uint2(l.a2, l.b2);
  *reinterpret_cast<float2*>(row + (c >> 3) * GM_LSUB + 96) = make_float2(l.scale, l.sum);   // same from all 4 lanes
}

__device__ __forceinline__ void gm_put_limbs8(gm_f32x4 a, gm_f32x4 b, int c, uint8_t* __restrict__ row) {
  gm_store_limbs8(gm_limbs8(a, b), c, row);
}

// Limbs of activations 4c .. 4c+3 of a row into `row` (limb layout).  The 8
// lanes holding the float4s of one sub-block must be lanes 8j .. 8j+7 of one
// wave (c % 8 == lane % 8), all executing this call (store to a spare
// sub-block when c is past the row).  A non-finite activation makes the
// sub-block's scale NaN.
__device__ __forceinline__ void gm_put_limbs4(gm_f32x4 v, int c, uint8_t* __restrict__ row) {
  const float ax = fabsf(v.x), ay = fabsf(v.y), az = fabsf(v.z), aw = fabsf(v.w);
  const bool fin = ax <= 3.4e38f && ay <= 3.4e38f && az <= 3.4e38f && aw <= 3.4e38f;
  const float m = gm_max8(fin ? fmaxf(fmaxf(ax, ay), fmaxf(az, aw)) : __builtin_inff());
  // m in [2^(E-1), 2^E); below 2^-100 the sub-block is quantised against 2^-100
  const int E = m > 0.f && m <= 3.4e38f ? max(__builtin_amdgcn_frexp_expf(m), -100) : 0;
  const float up = __builtin_ldexpf(1.0f, 22 - E);
  const float scale = m <= 3.4e38f ? __builtin_ldexpf(1.0f, E - 22) : __builtin_nanf("");
  int q[4];
  const float f[4] = {v.x * up, v.y * up, v.z * up, v.w * up};
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = __float_as_int(f[i] + 12582912.0f) - 0x4B400000;   // rne, |f| < 2^22
  int t1[4], t2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) { t1[i] = (q[i] + 128) >> 8; t2[i] = (t1[i] + 128) >> 8; }
  const float sum = gm_sum8((v.x + v.y) + (v.z + v.w));
  uint8_t* sb = row + (c >> 3) * GM_LSUB + 4 * (c & 7);
  *reinterpret_cast<uint32_t*>(sb) = gm_pack_lo4(q[0], q[1], q[2], q[3]);
  *reinterpret_cast<uint32_t*>(sb + 32) = gm_pack_lo4(t1[0], t1[1], t1[2], t1[3]);
  *reinterpret_cast<uint32_t*>(sb + 64) = gm_pack_lo4(t2[0], t2[1], t2[2], t2[3]);
  *reinterpret_cast<float2*>(row + (c >> 3) * GM_LSUB + 96) = make_float2(scale, sum);   // same from all 8 lanes
}

// One wave stages x [D] (XW float4 per lane, RMSNorm'd when norm_w != NULL)
// as a limb row `row` (gm_limb_row_bytes(D) + GM_LSUB bytes); no block barrier.
template <int XW>
__device__ __forceinline__ void stage_limbs_wave(const float* __restrict__ x, int D, const float* __restrict__ norm_w,
                                                 float eps, uint8_t* __restrict__ row) {
  const int lane = threadIdx.x & 63, nq = D >> 2;
  const gm_f32x4* x4 = reinterpret_cast<const gm_f32x4*>(x);
  const gm_f32x4* w4 = reinterpret_cast<const gm_f32x4*>(norm_w);
  gm_f32x4 v[XW], w[XW];
#pragma unroll
  for (int i = 0; i < XW; ++i) {
    const int c = lane + 64 * i;
    v[i] = x4[c < nq ? c : nq - 1];
  }
  if (norm_w != nullptr) {
#pragma unroll
    for (int i = 0; i < XW; ++i) {
      const int c = lane + 64 * i;
      w[i] = w4[c < nq ? c : nq - 1];
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < XW; ++i)
      if (lane + 64 * i < nq) ss = fmaf(v[i].x, v[i].x, fmaf(v[i].y, v[i].y, fmaf(v[i].z, v[i].z, fmaf(v[i].w, v[i].w, ss))));
    const float rms = 1.0f / sqrtf(gm_wave_sum64(ss) / (float)D + eps);
#pragma unroll
    for (int i = 0; i < XW; ++i) {
      v[i].x = (v[i].x * rms) * w[i].x; v[i].y = (v[i].y * rms) * w[i].y;
      v[i].z = (v[i].z * rms) * w[i].z; v[i].w = (v[i].w * rms) * w[i].w;
    }
  }
#pragma unroll
  for (int i = 0; i < XW; ++i) {
    const int c = lane + 64 * i;
    gm_put_limbs4(v[i], c < nq ? c : nq + (c & 7), row);
  }
}

// One wave copies a limb row of D <= 1024 DC activations (rbytes bytes) from
// global memory into the LDS row `row` (+ its spare sub-block): every lane
// issues all of its 16-byte loads before its first store.
template <int DC>
__device__ __forceinline__ void copy_limbs_wave(const uint8_t* __restrict__ src, int rbytes,
                                                uint8_t* __restrict__ row) {
  constexpr int CPL = (32 * DC * GM_LSUB / 16 + 63) / 64;
  const int lane = threadIdx.x & 63, n16 = rbytes >> 4;
  const gm_u32x4* s4 = reinterpret_cast<const gm_u32x4*>(src);
  gm_u32x4* d4 = reinterpret_cast<gm_u32x4*>(row);
  gm_u32x4 r[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    r[i] = s4[c < n16 ? c : n16 - 1];
  }
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    d4[c < n16 ? c : n16 + (c & 3)] = r[i];
  }
}

// acc[m] += W_row . act[idx[m]] over the fetched sub-blocks, m < nt; act rows
// are limb rows of row_bytes bytes.  BF16 weights (a shared expert kept in
// bf16) take the activations back to fp32 from their limbs.
template <int QT, int LR, int SPL, int NT, bool ARITH = false>
__device__ __forceinline__ void dot_subs_i8(const RowFetch<QT, SPL>& f, int lir, int nsub,
                                            const uint8_t* __restrict__ act, int row_bytes, const int (&idx)[NT],
                                            int nt, const Iq3Tab* __restrict__ tab, float (&acc)[NT]) {
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    const int sub = lir + LR * i;
    if (sub < nsub) {
      if constexpr (QT == GM_QTYPE_I8) {
#pragma unroll
        for (int m = 0; m < NT; ++m)
          if (m < nt) acc[m] += gm_i8_dot_limbs(f.r[i], act + idx[m] * row_bytes + sub * GM_LSUB);
      } else if constexpr (QT == GM_QTYPE_BF16) {
        float wv[32];
        gm_decode_bf16(f.r[i], wv);
#pragma unroll
        for (int m = 0; m < NT; ++m) {
          if (m < nt) {
            const uint8_t* s = act + idx[m] * row_bytes + sub * GM_LSUB;
            const gm_u32x4* p = reinterpret_cast<const gm_u32x4*>(s);
            const gm_u32x4 l0a = p[0], l0b = p[1], l1a = p[2], l1b = p[3], l2a = p[4], l2b = p[5];
            const uint32_t l0[8] = {l0a.x, l0a.y, l0a.z, l0a.w, l0b.x, l0b.y, l0b.z, l0b.w};
            const uint32_t l1[8] = {l1a.x, l1a.y, l1a.z, l1a.w, l1b.x, l1b.y, l1b.z, l1b.w};
            const uint32_t l2[8] = {l2a.x, l2a.y, l2a.z, l2a.w, l2b.x, l2b.y, l2b.z, l2b.w};
            float sacc = 0.f;
#pragma unroll
            for (int c = 0; c < 8; ++c)
#pragma unroll
              for (int b = 0; b < 4; ++b) {
                const float a = fmaf(gm_sbyte(l2[c], b), 65536.f, fmaf(gm_sbyte(l1[c], b), 256.f, gm_sbyte(l0[c], b)));
                sacc = fmaf(wv[4 * c + b], a, sacc);
              }
            acc[m] = fmaf(*reinterpret_cast<const float*>(s + 96), sacc, acc[m]);
          }
        }
      } else {
        uint32_t w[8];
        const float ws = gm_decode_i8<QT, ARITH>(gm_fetched<QT>(f.r[i]), sub, tab, w);
#pragma unroll
        for (int m = 0; m < NT; ++m) {
          if (m < nt) {
            const uint8_t* s = act + idx[m] * row_bytes + sub * GM_LSUB;
            const gm_u32x4* p = reinterpret_cast<const gm_u32x4*>(s);
            const gm_u32x4 l0a = p[0], l0b = p[1], l1a = p[2], l1b = p[3], l2a = p[4], l2b = p[5];
            const uint32_t l0[8] = {l0a.x, l0a.y, l0a.z, l0a.w, l0b.x, l0b.y, l0b.z, l0b.w};
            const uint32_t l1[8] = {l1a.x, l1a.y, l1a.z, l1a.w, l1b.x, l1b.y, l1b.z, l1b.w};
            const uint32_t l2[8] = {l2a.x, l2a.y, l2a.z, l2a.w, l2b.x, l2b.y, l2b.z, l2b.w};
            int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              s0 = __builtin_amdgcn_sdot4((int)w[c], (int)l0[c], s0, false);
              s1 = __builtin_amdgcn_sdot4((int)w[c], (int)l1[c], s1, false);
              s2 = __builtin_amdgcn_sdot4((int)w[c], (int)l2[c], s2, false);
            }
            const float r = fmaf((float)s2, 65536.f, fmaf((float)s1, 256.f, (float)s0));
            acc[m] = fmaf(ws * *reinterpret_cast<const float*>(s + 96), r, acc[m]);
          }
        }
      }
    }
  }
}

// Sum over the LR lanes of a row (LR = 16, 32 or 64), result in every lane.
template <int LR>
__device__ __forceinline__ float row_sum(float v) {
  if constexpr (LR == 64) return gm_wave_sum64(v);
  v = gm_row_sum16(v);
  if constexpr (LR == 32) v += __shfl_xor(v, 16, 64);
  return v;
}

// ------------------------------------------------------ activation rows
// Up to NT activation rows of D floats (plus the RMSNorm weight) held in
// registers: XPT float4 per thread per row, thread-strided (blockDim 256).
template <int NT, int XPT>
struct XRegs {
  gm_f32x4 v[NT][XPT];
  gm_f32x4 w[XPT];
};

// Rows tok[m], m < nt, of x [.][D]; rows past nt re-load row tok[0] (the
// loads stay unconditional and straight-line: a load under a branch would
// end in a full wait at the join).
template <int NT, int XPT>
__device__ __forceinline__ void load_x(XRegs<NT, XPT>& r, const float* __restrict__ x, const int (&tok)[NT], int nt,
                                       int D, const float* __restrict__ norm_w) {
  const int nq = D >> 2;
  const gm_f32x4* x4 = reinterpret_cast<const gm_f32x4*>(x);
#pragma unroll
  for (int m = 0; m < NT; ++m) {
    const int t = m < nt ? tok[m] : tok[0];
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int c = threadIdx.x + 256 * i;
      r.v[m][i] = x4[(int64_t)t * nq + (c < nq ? c : nq - 1)];
    }
  }
  if (norm_w != nullptr) {
    const gm_f32x4* w4 = reinterpret_cast<const gm_f32x4*>(norm_w);
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int c = threadIdx.x + 256 * i;
      r.w[i] = w4[c < nq ? c : nq - 1];
    }
  }
}

// Write the rows to interleaved LDS rows xs[m][D], applying
// xn = (x * rms) * w with rms = 1/sqrt(mean(x^2) + eps) when norm_w != NULL
// (qwen/forward.py:58-61).  One barrier for all rows.  red: 4 * NT floats.
// xs holds NT * D + 4 floats: lanes past the row store into the last float4,
// so the stores are unconditional and the loads feeding them are not sunk
// into branches (where each would end in a full wait).  All 256 threads
// call; ends with a barrier.
template <int NT, int XPT>
__device__ __forceinline__ void stage_x_regs(XRegs<NT, XPT>& r, int nt, int D, const float* __restrict__ norm_w,
                                             float eps, float* __restrict__ xs, float* __restrict__ red) {
  const int nq = D >> 2, nsub = D >> 5;
  gm_f32x4* xs4 = reinterpret_cast<gm_f32x4*>(xs);
  if (norm_w != nullptr) {
    float ss[NT];
#pragma unroll
    for (int m = 0; m < NT; ++m) {
      ss[m] = 0.f;
      if (m < nt) {
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
          const int c = threadIdx.x + 256 * i;
          const gm_f32x4 v = r.v[m][i];
          if (c < nq) ss[m] = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss[m]))));
        }
      }
      ss[m] = gm_wave_sum64(ss[m]);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
      for (int m = 0; m < NT; ++m) red[wave * NT + m] = ss[m];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < NT; ++m) {
      if (m < nt) {
        const float tot = (red[m] + red[NT + m]) + (red[2 * NT + m] + red[3 * NT + m]);
        const float rms = 1.0f / sqrtf(tot / (float)D + eps);
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
          const int c = threadIdx.x + 256 * i;
          gm_f32x4 v = r.v[m][i];
          const gm_f32x4 w = r.w[i];
          v.x = (v.x * rms) * w.x; v.y = (v.y * rms) * w.y; v.z = (v.z * rms) * w.z; v.w = (v.w * rms) * w.w;
          xs4[c < nq ? m * nq + il_index4(c & 7, c >> 3, nsub) : NT * nq] = v;
        }
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < NT; ++m) {
      if (m < nt) {
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
          const int c = threadIdx.x + 256 * i;
          xs4[c < nq ? m * nq + il_index4(c & 7, c >> 3, nsub) : NT * nq] = r.v[m][i];
        }
      }
    }
  }
  __syncthreads();
}

// As stage_x_regs, into limb rows: row m of xs at m * gm_limb_row_bytes(D);
// lanes past the row store into the spare sub-block after row NT - 1.
template <int NT, int XPT>
__device__ __forceinline__ void stage_limbs_regs(XRegs<NT, XPT>& r, int nt, int D, const float* __restrict__ norm_w,
                                                 float eps, uint8_t* __restrict__ xs, float* __restrict__ red) {
  const int nq = D >> 2, rbytes = gm_limb_row_bytes(D);
  float rms[NT];
#pragma unroll
  for (int m = 0; m < NT; ++m) rms[m] = 1.f;
  if (norm_w != nullptr) {
    float ss[NT];
#pragma unroll
    for (int m = 0; m < NT; ++m) {
      ss[m] = 0.f;
      if (m < nt) {
#pragma unroll
        for (int i = 0; i < XPT; ++i) {
          const int c = threadIdx.x + 256 * i;
          const gm_f32x4 v = r.v[m][i];
          if (c < nq) ss[m] = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss[m]))));
        }
      }
      ss[m] = gm_wave_sum64(ss[m]);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
      for (int m = 0; m < NT; ++m) red[wave * NT + m] = ss[m];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < NT; ++m) {
      const float tot = (red[m] + red[NT + m]) + (red[2 * NT + m] + red[3 * NT + m]);
      rms[m] = 1.0f / sqrtf(tot / (float)D + eps);
    }
  }
#pragma unroll
  for (int m = 0; m < NT; ++m) {
    if (m < nt) {
#pragma unroll
      for (int i = 0; i < XPT; ++i) {
        const int c = threadIdx.x + 256 * i;
        gm_f32x4 v = r.v[m][i];
        if (norm_w != nullptr) {
          const gm_f32x4 w = r.w[i];
          v.x = (v.x * rms[m]) * w.x; v.y = (v.y * rms[m]) * w.y; v.z = (v.z * rms[m]) * w.z; v.w = (v.w * rms[m]) * w.w;
        }
        gm_put_limbs4(v, c < nq ? c : (c & 7), xs + (c < nq ? m : NT) * rbytes);   // unconditional (DPP inside)
      }
    }
  }
  __syncthreads();
}

// One wave stages x [D] (XW float4 per lane, RMSNorm'd when norm_w != NULL)
// into the interleaved LDS row xs [D + 4]; no block barrier involved.
template <int XW>
__device__ __forceinline__ void stage_x_wave(const float* __restrict__ x, int D, const float* __restrict__ norm_w,
                                             float eps, float* __restrict__ xs) {
  const int lane = threadIdx.x & 63, nq = D >> 2, nsub = D >> 5;
  const gm_f32x4* x4 = reinterpret_cast<const gm_f32x4*>(x);
  const gm_f32x4* w4 = reinterpret_cast<const gm_f32x4*>(norm_w);
  gm_f32x4 v[XW], w[XW];
#pragma unroll
  for (int i = 0; i < XW; ++i) {
    const int c = lane + 64 * i;
    v[i] = x4[c < nq ? c : nq - 1];
  }
  if (norm_w != nullptr) {
#pragma unroll
    for (int i = 0; i < XW; ++i) {
      const int c = lane + 64 * i;
      w[i] = w4[c < nq ? c : nq - 1];
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < XW; ++i)
      if (lane + 64 * i < nq) ss = fmaf(v[i].x, v[i].x, fmaf(v[i].y, v[i].y, fmaf(v[i].z, v[i].z, fmaf(v[i].w, v[i].w, ss))));
    const float rms = 1.0f / sqrtf(gm_wave_sum64(ss) / (float)D + eps);
#pragma unroll
    for (int i = 0; i < XW; ++i) {
      v[i].x = (v[i].x * rms) * w[i].x; v[i].y = (v[i].y * rms) * w[i].y;
      v[i].z = (v[i].z * rms) * w[i].z; v[i].w = (v[i].w * rms) * w[i].w;
    }
  }
  gm_f32x4* xs4 = reinterpret_cast<gm_f32x4*>(xs);
#pragma unroll
  for (int i = 0; i < XW; ++i) {
    const int c = lane + 64 * i;
    xs4[c < nq ? il_index4(c & 7, c >> 3, nsub) : nq] = v[i];
  }
}

}  // namespace gm_moe
