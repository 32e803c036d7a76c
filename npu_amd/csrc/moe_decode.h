// Decode-path (T <= 8) launchers shared by moe_decode*.hip.
#pragma once
#include "kernels.h"

// Device pointers into the MoE workspace for one call.
struct GmDecArgs {
  float* logits;    // [T][E]
  float* shg;       // [T]
  int32_t* ids;     // [T][k]
  float* wts;       // [T][k]
  int32_t* grp;     // grouping table, see kernels.h; words GM_GRP_WORDS.. hold the T = 1
                    // routing weights in ascending-expert order
  float* h;         // [T * k][FF], directly followed by hsh
  float* hsh;       // [T][FF]
  float* yp;        // [T * k + T][D] per-pair / shared partial outputs (general path)
  float* part;      // [nz][T][gm_dec_part_ld] router partials (general path, inside yp)
  float* ssq;       // [nz][T] partial sums of x^2 (general path, inside yp)
  int nz;           // router partial ranges: gm_dec_nz(D), or gm_dec_link_nz(D) when the previous
                    // layer's combine kernel wrote them
  float* rms;       // [T] RMSNorm factors (general path, inside yp)
  uint8_t* xl;      // [T + 1] limb rows of x w_norm (general path, inside yp)
  uint64_t* tl;     // per-block timestamps (profiling build)
  double* acc;      // T = 1 router accumulators of this layer (see gm_acc_ld), read by the gate/up kernel
  double* acc_zero; // accumulators the gate/up kernel clears for the next layer's down kernel (or NULL)
};

// T = 1 router accumulators: GM_ACC_COPIES copies of gm_acc_ld(E) doubles.
// Word e < E: the raw router dot product sum_d W[e][d] (x[d] w_norm[d]) of
// expert e (no RMSNorm factor, no bias); word E: the same for the shared gate
// vector; word E + 1: sum_d x[d]^2.  The value of a word is the fp64 sum of
// its copies, added in copy order.  Either the router kernel writes copy 0 and
// zeros the others, or the previous layer's down kernel (block b) adds its
// rows' fp32 partials into copy b % 8 with fp64 atomics, which spreads the
// 256-way contention on one address over 8 addresses.  Each copy receives 32
// fp32 terms; their fp64 sum is exact, hence independent of the order the
// atomics land in, when the terms' exponents lie within 24 binades of each
// other (24 significant bits + 24 binades + log2(32) = 5 bits of growth fit
// fp64's 53).  Partials that cancel to tiny values can exceed that span; then
// one fp64 rounding can differ with the atomics' order, a 2^-53-relative
// difference.  So replays are bit-identical in practice, not by construction.
// (GM_ACC_COPIES, gm_acc_ld and gm_acc_bytes are in kernels.h.)

// The next layer's router, for the T = 1 down kernel of a chain: block b adds
// its 8 output rows' share of the next layer's accumulators (router rows and
// the shared gate vector at columns r0 .. r0 + 7, times the next layer's
// RMSNorm weight, and the sum of squares of the rows).
struct GmNextRouter {
  const void* w;     // gm_moe_layer.router_t: [D/8][E+1][8], bf16 bits or fp32 (f32 != 0)
  const float* nw;   // [D] RMSNorm weight, or NULL
  double* acc;       // GM_ACC_COPIES x ld accumulators, zeroed by this layer's gate/up kernel
  int E, ld, f32;
};

// The next layer's router inputs, for the T > 1 combine kernel of a chain
// (k_dec_combine_nx): the router partials of 256-column slices, the slices'
// sums of x^2 and the limb rows, written into the next layer's workspace where
// its routing and gate/up kernels read them (gm_dec_part_ptrs).
struct GmNextB8 {
  const void* w;     // gm_moe_layer.router_t of the next layer: [D/8][E+1][8], bf16 bits or fp32 (f32 != 0)
  const float* nw;   // [D] RMSNorm weight, or NULL
  float* part;       // [D / 256][T][ldp]
  float* ssq;        // [D / 256][T]
  uint8_t* xl;       // [T + 1] limb rows (row T: spare)
  int E, ldp, f32;
};

// gm_dec_chain_ok (kernels.h): the T = 1 layers that run on the accumulator
// kernels (router, k_dec_gateup1w, k_dec_down1), which a chain links by the
// down kernel feeding the next layer's accumulators.

// Row stride of the router partials: E rows + the shared gate row, padded to 4.
inline int gm_dec_part_ld(const gm_moe_layer* P) { return (P->E + 1 + 3) & ~3; }

// K range of the T > 1 router partials: 512 values when 512 divides D, else 256
// (D % 256 == 0), so a D <= 4096 splits into at most 16 ranges.
inline int gm_dec_kr(int D) { return D % 512 == 0 ? 512 : 256; }
inline int gm_dec_nz(int D) { return D / gm_dec_kr(D); }
constexpr int GM_DEC_MAX_NZ = 16;

// Partials of a T > 1 chain's combine kernel: 256-column slices.
constexpr int GM_DEC_LINK_KR = 256;
inline int gm_dec_link_nz(int D) { return D / GM_DEC_LINK_KR; }

// Where the T > 1 router inputs sit in a layer's workspace (inside yp, which
// the down stage overwrites only after the gate/up stage has read them): nz
// partial ranges of [T][ldp], then GM_DEC_MAX_NZ x T sums of x^2, T RMSNorm
// factors (16 words), T + 1 limb rows.  Returns false when they do not fit.
bool gm_dec_part_ptrs(const gm_moe_layer* P, int T, int nz, uint8_t* ws, const GmMoeWs& lay, float** part,
                      float** ssq, float** rms, uint8_t** xl);
// Whether those inputs fit a T-token workspace of P with nz ranges.
bool gm_dec_part_fits(const gm_moe_layer* P, int T, int nz);

// Weight-row chunk sizes: D and FF in units of 1024 and 512 elements.
inline int gm_dec_dc(int D) { return D <= 1024 ? 1 : D <= 2048 ? 2 : 4; }
inline int gm_dec_fc(int FF) { return FF <= 512 ? 1 : FF <= 1024 ? 2 : 4; }

// Stage 2: top-k + grouping + routed gate/up.  fast1: the T = 1 kernel that
// recomputes the top-k in every block; otherwise one routing block, then the
// grouped gate/up kernel.
int gm_dec_gateup(const gm_moe_layer* P, const float* x, int T, bool fast1, const GmDecArgs& a, hipStream_t s);
// Stage 3: down projections and the weighted combine (+ shared expert, + x).
// With next8 (T > 1 chains) the combine also writes the next layer's router inputs.
int gm_dec_down(const gm_moe_layer* P, const float* x, float* y, int T, int flags, bool fast1, const GmDecArgs& a,
                hipStream_t s, const GmNextRouter* next = nullptr, const GmNextB8* next8 = nullptr);
