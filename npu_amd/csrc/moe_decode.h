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
  float* part;      // [gm_dec_nz(D)][T][gm_dec_part_ld] router partials (general path, inside yp)
  float* ssq;       // [gm_dec_nz(D)][T] partial sums of x^2 (general path, inside yp)
  float* rms;       // [T] RMSNorm factors (general path, inside yp)
  uint8_t* xl;      // [T + 1] limb rows of x w_norm (general path, inside yp)
  uint64_t* tl;     // per-block timestamps (profiling build)
};

// Row stride of the router partials: E rows + the shared gate row, padded to 4.
inline int gm_dec_part_ld(const gm_moe_layer* P) { return (P->E + 1 + 3) & ~3; }

// K range of the T > 1 router partials: 512 values when 512 divides D, else 256
// (D % 256 == 0), so a D <= 4096 splits into at most 16 ranges.
inline int gm_dec_kr(int D) { return D % 512 == 0 ? 512 : 256; }
inline int gm_dec_nz(int D) { return D / gm_dec_kr(D); }
constexpr int GM_DEC_MAX_NZ = 16;

// Weight-row chunk sizes: D and FF in units of 1024 and 512 elements.
inline int gm_dec_dc(int D) { return D <= 1024 ? 1 : D <= 2048 ? 2 : 4; }
inline int gm_dec_fc(int FF) { return FF <= 512 ? 1 : FF <= 1024 ? 2 : 4; }

// Stage 2: top-k + grouping + routed gate/up.  fast1: the T = 1 kernel that
// recomputes the top-k in every block; otherwise one routing block, then the
// grouped gate/up kernel.
int gm_dec_gateup(const gm_moe_layer* P, const float* x, int T, bool fast1, const GmDecArgs& a, hipStream_t s);
// Stage 3: down projections and the weighted combine (+ shared expert, + x).
int gm_dec_down(const gm_moe_layer* P, const float* x, float* y, int T, int flags, bool fast1, const GmDecArgs& a,
                hipStream_t s);
