/*
 * npu_amd.h -- C ABI of the gfx950 (MI355X) Qwen MoE-block hot path.
 *
 * Drop-in boundary for the path BojanFaletic/NPU runs through
 * qwen/forward.py:moe_forward (563-665) and the npu.* operator wrappers it
 * calls.  Every entry point:
 *   - takes DEVICE pointers (owned by the caller, e.g. torch tensors) and plain
 *     sizes; weights stay in raw GGUF layout (IQ4_XS 136-byte / IQ3_XXS 98-byte
 *     superblocks, row-major [out][in/256 superblocks], experts outermost);
 *   - enqueues on the caller's hipStream_t passed as `void* stream` and never
 *     synchronises;
 *   - allocates no device memory (scratch comes from the caller's workspace);
 *   - returns 0 on success, a negative GM_E* code for a rejected argument, or
 *     a positive hipError_t; gm_last_error() returns a thread-local message.
 * No exceptions cross the ABI; the only global state is constant codebooks.
 */
#ifndef NPU_AMD_H
#define NPU_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight formats: ggml type ids (gguf GGMLQuantizationType). */
#define GM_QTYPE_F32 0
#define GM_QTYPE_F16 1
#define GM_QTYPE_Q8_0 8
#define GM_QTYPE_Q4_K 12
#define GM_QTYPE_Q5_K 13
#define GM_QTYPE_Q6_K 14
#define GM_QTYPE_IQ3_XXS 18
#define GM_QTYPE_IQ4_XS 23
#define GM_QTYPE_BF16 30
/* Not a GGML type: K-quant / Q8_0 rows transcoded by gm_transcode_i8.  Per 32
 * weights 48 bytes: int8 q[32], fp32 s0 (scale of q[0..15]), fp32 s1 (scale of
 * q[16..31]), fp32 off, 4 zero bytes; weight k = s_{k/16} * q[k] + off. */
#define GM_QTYPE_I8 100

/* Status codes (negative = argument errors). */
#define GM_OK 0
#define GM_EINVAL (-1)
#define GM_EUNSUPPORTED (-2)
#define GM_EWORKSPACE (-3)

/* Flags for gm_moe_forward. */
#define GM_MOE_RESIDUAL 1   /* y = x + moe(rmsnorm(x)) instead of y = moe(rmsnorm(x)) */

/* Message for the last failing call on this thread ("" if none). */
const char* gm_last_error(void);

/* ABI version (bumped on any signature or struct change). */
int gm_abi_version(void);

/*
 * Dequantise n_superblocks raw blocks of `qtype` to fp32: IQ4_XS, IQ3_XXS,
 * Q4_K, Q5_K, Q6_K (256 values per block) or Q8_0 (32 values per block).
 * Every product is exact in fp32; Q4_K / Q5_K round once when subtracting the
 * min term.  Replaces gguf.quants.dequantize as called by TensorStore.get /
 * get_expert (qwen/model.py:212, 266) and npu/iq3_xxs.py:dequant_rows (97-119).
 * IQ4_XS / IQ3_XXS need raw 8-byte and out 16-byte aligned; the other types
 * only 4-byte aligned out.
 */
int gm_dequant_f32(int qtype, const void* raw, int64_t n_superblocks, float* out, void* stream);

/*
 * Transcode n_blocks raw Q8_0 / Q4_K / Q5_K / Q6_K blocks into GM_QTYPE_I8
 * sub-blocks (48 bytes per 32 weights, in weight order, so a row of K weights
 * becomes a row of K / 32 * 48 bytes).  s * q + off reproduces gm_dequant_f32
 * bit for bit.  The MoE kernels multiply I8 rows on v_dot4_i32_i8 with the
 * int8 activation limbs.  Replaces the per-call dequant of K-quant expert and
 * shared-expert tensors (qwen/forward.py:480-491 dequant_one, :495-498 for the
 * Q5_K / Q6_K outlier layers, :465-468 for the shared expert).  out must be
 * 16-byte aligned.
 */
int gm_transcode_i8(int qtype, const void* raw, int64_t n_blocks, void* out, void* stream);

/*
 * y[t][m] = sum_k W[m][k] * x[t][k] for t < n_tok, W given as M rows of raw
 * `qtype` superblocks (IQ4_XS, IQ3_XXS) or bf16 (BF16), fp32 x/y, fp32
 * accumulate.  K must be a multiple of 256.
 * Replaces NpuQuantMatVec.__call__ (npu/quant_mv.py:419-463),
 * NpuIQ4MatVec.__call__ (npu/quant_mv_iq4.py:317-361),
 * NpuIQ4PackedMatVec.__call__ (npu/quant_mv_iq4_packed.py:320-364) and,
 * with qtype BF16, NpuMatVec / NpuConcatMatVec.__call__ (npu/mv.py:222-347).
 * The reference takes one vector (n_tok == 1); n_tok >= 1 is accepted.
 */
int gm_matvec(int qtype, const void* w, int M, int K, const float* x, int n_tok, float* y,
              void* stream);

/*
 * SwiGLU MLP: y[t] = W_down (silu(W_gate x[t]) * (W_up x[t])), gate/up
 * [FF][D] of qtype q_gu, down [D][FF] of qtype q_down; h is an fp32
 * [n_tok][FF] scratch buffer.  Weights aligned to 16 (bf16), 8 (IQ4_XS) or
 * 2 (IQ3_XXS) bytes; h 16-byte aligned when the down matrix is bf16.
 * Replaces NpuFusedMLP.__call__
 * (npu/mlp.py:413-466) and the shared-expert F.linear chain
 * (qwen/forward.py:592-598).
 */
int gm_swiglu_mlp(int q_gu, const void* w_gate, const void* w_up, int q_down, const void* w_down,
                  int D, int FF, const float* x, int n_tok, float* h, float* y, void* stream);

/*
 * Router: logits[t][e] = W_router[e] . xn[t] (+ bias[e]), then softmax over E,
 * top-k (ties -> lower expert id) and renormalisation of the k probabilities;
 * also sh_gate[t] = sigmoid(w_sh_gate . xn[t]) when w_sh_gate != NULL.
 * xn = rmsnorm(x, norm_w, eps) when norm_w != NULL, else x.
 * W_router and w_sh_gate are bf16 bits.  `logits` may be NULL.
 * Replaces qwen/forward.py:599-611 (router F.linear / NpuMatVec, softmax,
 * topk, renormalise) and the shared scalar gate.
 */
int gm_router_topk(const uint16_t* w_router, const float* bias, const float* x, int T, int D, int E,
                   int k, const uint16_t* w_sh_gate, const float* norm_w, float eps, int32_t* ids,
                   float* weights, float* logits, float* sh_gate, void* stream);

/*
 * Token -> expert dispatch: counts[E] = pairs per expert, offsets[E+1] =
 * exclusive prefix sum, sorted_pairs[T*k] = (token*k + slot) grouped by
 * ascending expert, tokens ascending within an expert (stable).
 * Replaces qwen/forward.py:612, 623-629 (torch.unique + nonzero per expert).
 */
int gm_moe_dispatch(const int32_t* ids, int T, int k, int E, int32_t* counts, int32_t* offsets,
                    int32_t* sorted_pairs, void* stream);

/*
 * One MoE block's resident weights (device pointers) and shape.  Routed and
 * shared formats: IQ4_XS or IQ3_XXS superblocks, or BF16 rows (how experts
 * stored in Q8_0 / Q4_K / Q5_K / Q6_K are held: dequantised once at load, as
 * the reference keeps its Q5_K / Q6_K outlier layers on a dequant + F.linear
 * path, qwen/forward.py:495-498).  gate and up share one format.
 */
typedef struct gm_moe_layer {
  const void* gate_exps;        /* [E][FF][row_bytes(q_gate, D)]  raw GGUF bytes */
  const void* up_exps;          /* [E][FF][row_bytes(q_up, D)] */
  const void* down_exps;        /* [E][D][row_bytes(q_down, FF)] */
  const void* gate_sh;          /* [FF_sh][row_bytes(q_gate_sh, D)] */
  const void* up_sh;            /* [FF_sh][row_bytes(q_up_sh, D)] */
  const void* down_sh;          /* [D][row_bytes(q_down_sh, FF_sh)] */
  const void* router;           /* [E][D] in q_router: bf16 bits, or fp32 as the GGUF holds it */
  const void* sh_gate_inp;      /* [D] in q_router (shared-expert scalar gate), or NULL */
  const float* router_bias;     /* [E] added to logits, or NULL (not in the reference model) */
  const float* norm_w;          /* [D] RMSNorm weight applied to x, or NULL */
  float norm_eps;
  int32_t q_gate, q_up, q_down;
  int32_t q_gate_sh, q_up_sh, q_down_sh;
  int32_t D, FF, FF_sh, E, k;
  int32_t q_router;             /* GM_QTYPE_BF16 or GM_QTYPE_F32 (= 0): format of router and sh_gate_inp */
  /* Optional (NULL allowed): router and shared gate vector transposed in groups
   * of 8 columns, [D/8][E+1][8] in q_router: group j holds columns 8j .. 8j+7 of
   * router rows 0 .. E-1, then of sh_gate_inp (zeros without one).  Only
   * gm_moe_chain reads it (layers 1 .. n-1 at T = 1); without it the chain runs
   * its layers one gm_moe_forward at a time. */
  const void* router_t;
} gm_moe_layer;

/* Workspace bytes gm_moe_forward needs for T tokens (0 on bad arguments). */
size_t gm_moe_workspace_bytes(const gm_moe_layer* L, int T);

/*
 * Byte offsets inside the workspace of the per-call intermediates, for
 * stage-wise checks: router logits fp32 [T][E], top-k ids int32 [T][k],
 * renormalised weights fp32 [T][k], shared gate fp32 [T].
 */
int gm_moe_workspace_offsets(const gm_moe_layer* L, int T, size_t* off_logits, size_t* off_ids,
                             size_t* off_weights, size_t* off_sh_gate);

/*
 * The whole MoE block for T tokens: y = moe(xn) (+ x with GM_MOE_RESIDUAL),
 * xn = rmsnorm(x) when L->norm_w != NULL.  Routing, dispatch, expert
 * products, shared expert and the combine all run on the device from
 * device-resident ids (no host synchronisation).  T <= 8 uses the decode
 * kernels (fp32 accumulate); larger T uses the grouped MFMA prefill.
 * x and y must not alias.  x, y, the weight pointers, L->norm_w and
 * L->sh_gate_inp must be 16-byte aligned (torch allocations are).
 * Replaces qwen/forward.py:moe_forward (563-665).
 */
int gm_moe_forward(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws,
                   size_t ws_bytes, void* stream);

/*
 * gm_moe_forward forced onto one path.  gm_moe_decode: the fp32-accumulate
 * decode kernels, 1 <= T <= 8 (the reference's NPU expert path is T = 1:
 * qwen/forward.py:494-560 via _npu_routed_expert).  gm_moe_prefill: the
 * grouped f16/bf16-MFMA GEMMs for any T >= 1 (the reference runs prefill through
 * the CPU loop of qwen/forward.py:622-663); a layer with BF16 or I8 routed
 * experts runs its tokens as decode chunks of at most 8 instead.  A shared
 * expert in other formats than the (IQ) routed ones, such as the real
 * model's K-quant shared experts held as I8 rows, runs as an fp32 pass of
 * its own beside the routed GEMMs.  Same workspace as gm_moe_forward.
 */
int gm_moe_decode(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws,
                  size_t ws_bytes, void* stream);
int gm_moe_prefill(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws,
                   size_t ws_bytes, void* stream);

/*
 * One stage of gm_moe_forward, for stage-wise checks and per-kernel timing:
 * stage 1 = router logits and shared scalar gate (+ shared expert gate/up),
 * 2 = top-k, grouping and routed gate/up + SwiGLU, 3 = down + combine
 * (+ residual); stage 0 runs all three.
 * Stages must run in order on the same workspace.  Decode path (T <= 8) only.
 * Mirrors the stage boundaries of qwen/compare.py:compare_moe (191-297).
 */
int gm_moe_forward_stage(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws,
                         size_t ws_bytes, int stage, void* stream);

/*
 * n_layers MoE blocks in sequence (the decoder loop's MoE
 * step x = x + moe_forward(rms_norm(x)) of qwen/forward.py:880-884 repeated
 * over consecutive layers): x_{l+1} = moe_l(x_l) (+ x_l with
 * GM_MOE_RESIDUAL), x_0 = x, x_n written to y.  Layer l writes y when
 * n_layers - 1 - l is even and buf otherwise (buf: [T][D], may be NULL for one
 * layer); x is not written.  ws[l] is layer l's workspace of ws_bytes[l] >=
 * gm_moe_workspace_bytes(&layers[l], T) bytes (the same workspace may serve
 * every layer).  Every layer must have the same D.  At T = 1, when all layers
 * share E, fit the one-block-per-CU gate/up kernel (e.g. FF = 512, k = 8) and
 * layers 1 .. n-1 carry router_t,
 * each layer's down kernel also computes the next layer's router dot products
 * (fp64 accumulators in the next layer's workspace), so the chain runs one
 * router launch and then two launches per layer; results equal gm_moe_forward
 * layer by layer to fp32 rounding (the logits are the same dot products added
 * in another order).  At 2 <= T <= 8 (decode path), when D is a multiple of
 * 256 up to 4096, layers 1 .. n-1 carry router_t and consecutive layers'
 * workspaces do not overlap, each layer's combine kernel also forms the next
 * layer's router partials over 256-column slices, sums of x^2 and activation
 * limb rows in the next layer's workspace, so the chain runs one router
 * launch and then four launches per layer (routing, gate/up, down, combine),
 * again equal to gm_moe_forward layer by layer to fp32 rounding.  Otherwise
 * each layer runs as gm_moe_forward.  After the
 * call each workspace holds its layer's intermediates
 * (gm_moe_workspace_offsets) when the layers' workspaces are distinct.
 */
int gm_moe_chain(const gm_moe_layer* layers, int n_layers, const float* x, float* y, float* buf, int T,
                 int flags, void* const* ws, const size_t* ws_bytes, void* stream);

/*
 * Which path gm_moe_chain takes for these layers and T, without running it:
 * 1 = the accumulator-linked T = 1 kernels (one router launch, then two
 * launches per layer), 2 = the combine-linked 2 <= T <= 8 kernels (one router
 * launch, then four launches per layer, when the layers' workspaces are
 * distinct), 0 = one gm_moe_forward per layer, negative = a rejected layer
 * (GM_E*).  No counterpart in the reference (its decoder loop
 * runs one block at a time); for callers and tests that must know the fast
 * path is the one that runs.
 */
int gm_moe_chain_fused(const gm_moe_layer* layers, int n_layers, int T);

/*
 * The core layers beside the MoE block in every decoder layer, one decode
 * token (qwen/forward.py:834-893 runs x = x + core(x) and then the MoE step).
 * fp32 activations and state; the large projections are bf16 weights, as the
 * reference's NPU operators stage them for these sites (qwen/forward.py:813-831).
 */

/* Gated attention layer (the reference's AttnLayer, qwen/forward.py:100-130). */
typedef struct gm_attn_layer {
  const void* wqkv;         /* bf16 [(2 n_head + 2 n_head_kv) head_dim][D]: attn_q (q and gate
                               interleaved per head, [q_h | gate_h]), then attn_k, then attn_v */
  const void* wo;           /* bf16 [D][n_head head_dim] (attn_output) */
  const float* attn_norm;   /* [D], 16-byte aligned */
  const float* q_norm;      /* [head_dim] */
  const float* k_norm;      /* [head_dim] */
  float eps;
  int32_t D, n_head, n_head_kv, head_dim, rope_dim;
} gm_attn_layer;

/* Workspace bytes of gm_attn_decode for caches of max_pos positions (0 on bad arguments). */
size_t gm_attn_workspace_bytes(const gm_attn_layer* L, int max_pos);

/*
 * y = attn(x) (+ x with GM_MOE_RESIDUAL) for one token at position pos:
 * RMSNorm, the q / gate / k / v projection, per-head RMSNorm of q and k,
 * partial RoPE with rows pos of rope_cos / rope_sin ([max_pos][rope_dim], the
 * reference's build_partial_rope_cache tables), k and v written to row pos of
 * k_cache / v_cache ([max_pos][n_head_kv][head_dim] fp32: one row per kv head,
 * the reference repeats each kv head over its n_head / n_head_kv q heads), the
 * softmax over positions 0 .. pos, the output times sigmoid(gate), and wo.
 * head_dim in {64, 128, 256, 512}, rope_dim even and <= head_dim, D and
 * n_head head_dim multiples of 32.  x and y must not alias.
 * Replaces qwen/forward.py:attn_forward (133-239) at T = 1.
 */
int gm_attn_decode(const gm_attn_layer* L, const float* x, float* y, float* k_cache, float* v_cache, int pos,
                   int max_pos, const float* rope_cos, const float* rope_sin, int flags, void* ws, size_t ws_bytes,
                   void* stream);

/* Gated DeltaNet layer (the reference's SSMLayer, qwen/forward.py:242-284). */
typedef struct gm_ssm_layer {
  const void* w_in;         /* bf16 [2 n_k_heads d_state + n_v_heads d_state][D] (attn_qkv) */
  const void* w_gate;       /* bf16 [n_v_heads d_state][D] (attn_gate) */
  const void* w_out;        /* bf16 [D][n_v_heads d_state] (ssm_out) */
  const float* alpha;       /* [n_v_heads][D] (ssm_alpha), 16-byte aligned */
  const float* beta;        /* [n_v_heads][D] (ssm_beta), 16-byte aligned */
  const float* conv1d;      /* [conv channels][conv_k] (ssm_conv1d) */
  const float* a;           /* [n_v_heads] (ssm_a) */
  const float* dt_bias;     /* [n_v_heads] (ssm_dt.bias) */
  const float* ssm_norm;    /* [d_state] */
  const float* attn_norm;   /* [D], 16-byte aligned */
  float eps;
  int32_t D, n_k_heads, n_v_heads, d_state, conv_k;
} gm_ssm_layer;

/* Workspace bytes of gm_ssm_decode (0 on bad arguments). */
size_t gm_ssm_workspace_bytes(const gm_ssm_layer* L);

/*
 * y = ssm(x) (+ x with GM_MOE_RESIDUAL) for one token, updating in place
 * conv_state ([conv channels][conv_k - 1] fp32) and rec_state ([n_v_heads]
 * [d_state][d_state] fp32, the reference's [H][K][V] layout).  d_state in {64,
 * 128, 256}, n_v_heads a multiple of n_k_heads, conv_k in 1 .. 8.  x and y must
 * not alias.  Replaces qwen/forward.py:ssm_forward (292-431) at T = 1.
 */
int gm_ssm_decode(const gm_ssm_layer* L, const float* x, float* y, float* conv_state, float* rec_state, int flags,
                  void* ws, size_t ws_bytes, void* stream);

/*
 * A core layer linked to the MoE block that follows it in the decoder layer
 * (qwen/forward.py:880-884 runs x = x + moe_forward(rms_norm(x, post_norm)) on
 * the core layer's output): as gm_attn_decode / gm_ssm_decode, and the layer's
 * output projection also forms that block's router inputs from its output y
 * (the raw router dot products of y * moe->norm_w and the sum of y^2, added into
 * the block's T = 1 router accumulators in moe_ws), so gm_moe_forward_acc then
 * runs the block on y without a router launch.  moe must fit the T = 1
 * accumulator kernels (gm_moe_chain_fused(moe, 1, 1) == 1), have the core
 * layer's D and carry a 16-byte aligned router_t; moe_ws is the block's
 * workspace (>= gm_moe_workspace_bytes(moe, 1) bytes, 256-byte aligned).  The
 * call clears the accumulators itself (its first launch), so the pair is
 * self-contained; the logits equal gm_moe_forward's to fp32 rounding (the same
 * dot products added in another order).  No counterpart in the reference (its
 * decoder loop calls the router per MoE block); for decoder loops that run a
 * core layer and its MoE block back to back.
 */
int gm_attn_decode_moe(const gm_attn_layer* L, const float* x, float* y, float* k_cache, float* v_cache, int pos,
                       int max_pos, const float* rope_cos, const float* rope_sin, int flags, void* ws,
                       size_t ws_bytes, const gm_moe_layer* moe, void* moe_ws, size_t moe_ws_bytes, void* stream);
int gm_ssm_decode_moe(const gm_ssm_layer* L, const float* x, float* y, float* conv_state, float* rec_state, int flags,
                      void* ws, size_t ws_bytes, const gm_moe_layer* moe, void* moe_ws, size_t moe_ws_bytes,
                      void* stream);

/*
 * One token through a MoE block whose router inputs the preceding
 * gm_attn_decode_moe / gm_ssm_decode_moe call formed in ws (same block, same
 * workspace, x = that call's y): gm_moe_forward at T = 1 without the router
 * launch (gate/up and down).  flags as gm_moe_forward.  No counterpart in the
 * reference; see gm_attn_decode_moe.
 */
int gm_moe_forward_acc(const gm_moe_layer* L, const float* x, float* y, int flags, void* ws, size_t ws_bytes,
                       void* stream);

/* y[r] = rmsnorm(x[r], w, eps) for n_rows rows of D (qwen/forward.py:58-61; the
 * decoder's output norm, :887-888). */
int gm_rms_norm(const float* x, const float* w, int D, int n_rows, float eps, float* y, void* stream);

/* Size of the static scratch gm_moe_forward_noalloc works in: 16 MiB per GPU. */
#define GM_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/*
 * gm_moe_forward without a workspace argument and without any allocation
 * (no hipMalloc / hipFree, no allocating library call): the workspace is a
 * static device array of GM_NOALLOC_SCRATCH_BYTES that every GPU running the
 * library holds until the process ends.  No counterpart in the reference; it
 * is for callers that cannot allocate (code under stream / graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same kernels and
 * results as gm_moe_forward.  Returns GM_EWORKSPACE when
 * gm_moe_workspace_bytes(L, T) > GM_NOALLOC_SCRATCH_BYTES (config 5: T <= 8
 * needs 1.7 MiB, prefill fits up to T = 111).  stream must belong to the
 * current device.  The first call on each device resolves the array's address
 * (hipGetSymbolAddress, which may load the code object) and so must happen
 * outside stream capture; later calls may be captured.  All calls on one GPU share that GPU's array, which keeps
 * the last call's contents: calls that overlap on one GPU (other streams,
 * other threads) race and must be serialised by the caller.
 */
int gm_moe_forward_noalloc(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NPU_AMD_H */
