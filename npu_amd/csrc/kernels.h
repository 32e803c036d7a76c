// Internal launchers (host side).  All return GM_OK or an error status.
#pragma once
#include "common.h"
#include "timeline.h"

int gm_launch_dequant(int qtype, const void* raw, int64_t n_sb, float* out, hipStream_t s);

// Q8_0 / Q4_K / Q5_K / Q6_K: weights and bytes per block (0 for other types).
struct GmKBlock { int weights, bytes; };
inline GmKBlock gm_kquant_block(int qtype) {
  switch (qtype) {
    case GM_QTYPE_Q8_0: return {32, 34};
    case GM_QTYPE_Q4_K: return {256, 144};
    case GM_QTYPE_Q5_K: return {256, 176};
    case GM_QTYPE_Q6_K: return {256, 210};
    default: return {0, 0};
  }
}
int gm_launch_dequant_k(int qtype, const void* raw, int64_t n_blocks, float* out, hipStream_t s);
int gm_launch_transcode_i8(int qtype, const void* raw, int64_t n_blocks, void* out, hipStream_t s);
int gm_launch_matvec(int qtype, const void* w, int M, int K, const float* x, int n_tok, float* y,
                     hipStream_t s);
// Dense bf16 matvec (K % 256 == 0, K <= 16384, 16-byte aligned w and x).
int gm_launch_mv_bf16(const uint16_t* w, int M, int K, const float* x, int n_tok, float* y, hipStream_t s);
int gm_launch_gateup(int qtype, const void* wg, const void* wu, int FF, int D, const float* x, int n_tok,
                     float* h, hipStream_t s);
// One token, y = add + W x (add may be NULL); with nx (a MoE block's router,
// moe_decode.h) y also feeds that block's T = 1 router accumulators.
struct GmNextRouter;
int gm_launch_mv_bf16_add(const uint16_t* w, int M, int K, const float* x, float* y, const float* add,
                          hipStream_t s, const GmNextRouter* nx = nullptr);
// One token: h = RMSNorm(x) (norm_w, eps; none when norm_w is null), y = W h and,
// when w2 is given, y2 = W2 h with W2's M2 rows in the same launch; zacc: zn
// doubles the launch clears (NULL: none).
int gm_launch_mv_bf16_norm2(const uint16_t* w, int M, const uint16_t* w2, int M2, int K, const float* x,
                            const float* norm_w, float eps, float* y, float* y2, hipStream_t s,
                            double* zacc = nullptr, int zn = 0);
int gm_launch_rms_row(const float* x, const float* w, int D, int n_rows, float eps, float* y, hipStream_t s);

// Core-layer decode workspaces (core_decode.hip), byte offsets, 256-byte aligned.
struct GmAttnWs {
  size_t h, qkv, qr, part, out, total;
  int nch;         // attention partial slots per head (max_pos / chunk, rounded up)
};
GmAttnWs gm_attn_ws_layout(const gm_attn_layer* L, int max_pos);
// With moe (the following MoE block's router, its T = 1 accumulators): the
// layer's first launch clears the accumulators and its output projection adds
// the router inputs of its output into them.
int gm_attn_run(const gm_attn_layer* L, const float* x, float* y, float* kc, float* vc, int pos, int max_pos,
                const float* cosr, const float* sinr, int flags, uint8_t* ws, hipStream_t s,
                const GmNextRouter* moe = nullptr);
struct GmSsmWs {
  size_t h, mixed, z, gb, conv, o, o2, total;
};
GmSsmWs gm_ssm_ws_layout(const gm_ssm_layer* L);
int gm_ssm_run(const gm_ssm_layer* L, const float* x, float* y, float* conv_state, float* rec_state, int flags,
               uint8_t* ws, hipStream_t s, const GmNextRouter* moe = nullptr);

// MoE workspace layout for T tokens (offsets in bytes, 256-byte aligned).
struct GmMoeWs {
  size_t logits;   // f32 [T][E]
  size_t shg;      // f32 [T]       sigmoid(shared scalar gate)
  size_t ids;      // i32 [T][k]
  size_t wts;      // f32 [T][k]
  size_t grp;      // i32 grouping table (decode) / dispatch tables (prefill)
  size_t h;        // f32 [T][k][FF]  routed SwiGLU activations (decode)
  size_t hsh;      // f32 [T][FF_sh]  shared SwiGLU activations (directly after h)
  size_t yp;       // f32 [T * k + T][D]  per-pair / shared partial outputs (decode, T > 1)
  size_t pre;      // prefill scratch (see prefill.hip)
  size_t acc;      // T = 1 router accumulators, two buffers of gm_acc_bytes(E) (moe_decode.h)
  size_t tl;       // per-block timestamps (profiling build only, else empty); last region
  size_t total;
};

// T = 1 router accumulators (layout in moe_decode.h): GM_ACC_COPIES copies of
// gm_acc_ld(E) doubles, each copy a whole number of 128-byte lines.  Word e < E
// (expert e) sits at position MV (e % 64) + e / 64 (MV = 4 for E <= 256, else
// 8), so that lane l of the selecting wave reads its words l, l + 64, ... as
// MV consecutive doubles; words E (shared gate) and E + 1 (sum of squares)
// follow at 64 MV and 64 MV + 1.
constexpr int GM_ACC_COPIES = 8;
__host__ __device__ inline int gm_acc_mv(int E) { return E <= 256 ? 4 : 8; }
__host__ __device__ inline int gm_acc_ld(int E) { return 64 * gm_acc_mv(E) + 16; }
__host__ __device__ inline int gm_acc_pos(int e, int E) {
  const int mv = gm_acc_mv(E);
  return e < E ? mv * (e & 63) + (e >> 6) : 64 * mv + (e - E);
}
inline size_t gm_acc_bytes(int E) { return (size_t)GM_ACC_COPIES * gm_acc_ld(E) * sizeof(double); }

// One layer of a linked gm_moe_chain.  T = 1 (accumulator path): the router
// accumulators the gate/up kernel reads (acc), those it clears for the next
// layer (acc_zero, or NULL) and the next layer for the down kernel (next, or
// NULL).  T > 1: the next layer's router inputs for the combine kernel (next8,
// or NULL).  Either way, whether the router kernel runs first (the chain's
// first layer; the others find their router inputs in their workspace).
struct GmNextRouter;
struct GmNextB8;
struct GmChainStep {
  double* acc;
  double* acc_zero;
  const GmNextRouter* next;
  bool router;
  const GmNextB8* next8;
};
bool gm_dec_chain_ok(const gm_moe_layer* P);

GmMoeWs gm_moe_ws_layout(const gm_moe_layer* L, int T);
size_t gm_prefill_scratch_bytes(const gm_moe_layer* L, int T);

// Decode grouping table (int32 words) written to ws.grp by the gate/up kernel:
//   [0]            n_unique
//   [1 .. 64]      expert id of unique slot u (ascending)
//   [65 .. 128]    member count of slot u
//   [129 .. 640]   members: slot u, member m -> (token * k + topk_slot), tokens ascending
//   [641 .. 648]   T = 1 only: routing weight of slot u (float bits)
#define GM_GRP_MAXU 64
#define GM_GRP_MAXM 8
#define GM_GRP_WORDS (1 + 2 * GM_GRP_MAXU + GM_GRP_MAXU * GM_GRP_MAXM)
#define GM_DECODE_MAX_T 8

int gm_launch_router(const uint16_t* w_router, const float* bias, const float* x, int T, int D, int E,
                     const uint16_t* w_sh_gate, const float* norm_w, float eps, float* logits,
                     float* sh_gate, hipStream_t s);
int gm_launch_topk(const float* logits, int T, int E, int k, int32_t* ids, float* wts, hipStream_t s);
int gm_dec_run(const gm_moe_layer* L, const float* x, float* y, int T, int flags, uint8_t* ws,
                  const GmMoeWs& lay, hipStream_t s, int stage = 0, const GmChainStep* cs = nullptr);
int gm_pf_run(const gm_moe_layer* L, const float* x, float* y, int T, int flags, uint8_t* ws,
                   const GmMoeWs& lay, hipStream_t s);
int gm_launch_dispatch(const int32_t* ids, int T, int k, int E, int32_t* counts, int32_t* offsets,
                       int32_t* sorted_pairs, hipStream_t s);
// Dispatch plus (inv != NULL) the inverse permutation and (segs != NULL) the
// segment list: segs[0] = count, then (unit, start, n, 0) per segment of at
// most seg_tok pairs; unit E is a shared unit of shared_T tokens (0: none).
int gm_launch_dispatch_seg(const int32_t* ids, int T, int k, int E, int32_t* counts, int32_t* offsets,
                           int32_t* sorted_pairs, int32_t* inv, int32_t* segs, int seg_tok, int shared_T,
                           hipStream_t s);
