// extern "C" entry points: argument validation, error reporting, workspace
// layout.  Kernels live in matvec.hip, moe_decode.hip, dispatch.hip and
// prefill.hip.
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "kernels.h"
#include "moe_decode.h"

static thread_local char g_err[512] = "";

int gm_fail_hip(hipError_t e, const char* what) {
  snprintf(g_err, sizeof g_err, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
  return (int)e;
}

int gm_fail_arg(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return GM_EINVAL;
}

static inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static bool is_quant(int q) { return q == GM_QTYPE_IQ4_XS || q == GM_QTYPE_IQ3_XXS; }
static bool is_weight_fmt(int q) { return is_quant(q) || q == GM_QTYPE_BF16 || q == GM_QTYPE_I8; }

// K must be a multiple of 256 for superblock formats and of 32 for bf16.
static int check_k(const char* fn, int qtype, int K) {
  if (K <= 0) return gm_fail_arg("%s: K=%d must be positive", fn, K);
  if (is_quant(qtype) && K % GM_QK) return gm_fail_arg("%s: K=%d must be a multiple of %d", fn, K, GM_QK);
  if (qtype == GM_QTYPE_BF16 && K % GM_SUB) return gm_fail_arg("%s: K=%d must be a multiple of %d", fn, K, GM_SUB);
  return GM_OK;
}

GmMoeWs gm_moe_ws_layout(const gm_moe_layer* L, int T) {
  GmMoeWs w{};
  size_t o = 0;
  const size_t Tz = (size_t)T, E = (size_t)L->E, k = (size_t)L->k;
  w.logits = o; o = align256(o + Tz * E * 4);
  w.shg = o; o = align256(o + Tz * 4);
  w.ids = o; o = align256(o + Tz * k * 4);
  w.wts = o; o = align256(o + Tz * k * 4);
  w.grp = o; o = align256(o + ((size_t)GM_GRP_WORDS + 8 + 2 * E + 1 + Tz * k) * 4);
  w.h = o; o = o + Tz * k * (size_t)L->FF * 4;     // FF % 256 == 0: h_sh starts 256-byte aligned
  w.hsh = o; o = align256(o + Tz * (size_t)(L->FF_sh > 0 ? L->FF_sh : 0) * 4);
  const size_t Td = T < GM_DECODE_MAX_T ? Tz : (size_t)GM_DECODE_MAX_T;   // decode chunk (bf16 routed experts)
  w.yp = o; o = align256(o + (Td * k + Td) * (size_t)L->D * 4);
  w.pre = o; o = align256(o + gm_prefill_scratch_bytes(L, T));     // every T: gm_moe_prefill takes any T
  w.acc = o; o = align256(o + 2 * gm_acc_bytes(L->E));
  w.tl = o; o = align256(o + GM_TL_BYTES);                   // last: the timeline tool reads the end
  w.total = o;
  return w;
}

static int check_layer(const gm_moe_layer* L) {
  if (!L) return gm_fail_arg("gm_moe_forward: layer is NULL");
  if (L->D <= 0 || L->FF <= 0 || L->E <= 0 || L->k <= 0)
    return gm_fail_arg("gm_moe_forward: bad shape D=%d FF=%d E=%d k=%d", L->D, L->FF, L->E, L->k);
  if (L->k > 8 || L->k > L->E) return gm_fail_arg("gm_moe_forward: k=%d must be <= min(8, E=%d)", L->k, L->E);
  if (L->E > 512) return gm_fail_arg("gm_moe_forward: E=%d > 512 is not supported", L->E);
  if (!L->gate_exps || !L->up_exps || !L->down_exps || !L->router)
    return gm_fail_arg("gm_moe_forward: routed expert / router weights must be non-NULL");
  if (!is_weight_fmt(L->q_gate) || L->q_up != L->q_gate || !is_weight_fmt(L->q_down))
    return gm_fail_arg("gm_moe_forward: routed formats gate %d up %d down %d unsupported (gate == up, "
                       "IQ4_XS, IQ3_XXS, BF16 or I8)", L->q_gate, L->q_up, L->q_down);
  if (L->D % GM_QK || L->FF % GM_QK)
    return gm_fail_arg("gm_moe_forward: D=%d and FF=%d must be multiples of %d", L->D, L->FF, GM_QK);
  if (L->q_router != GM_QTYPE_BF16 && L->q_router != GM_QTYPE_F32)
    return gm_fail_arg("gm_moe_forward: q_router=%d must be GM_QTYPE_BF16 or GM_QTYPE_F32", L->q_router);
  const bool has_sh = L->gate_sh || L->up_sh || L->down_sh;
  if (has_sh) {
    if (!L->gate_sh || !L->up_sh || !L->down_sh)
      return gm_fail_arg("gm_moe_forward: shared expert needs gate, up and down");
    if (L->FF_sh != L->FF) return gm_fail_arg("gm_moe_forward: FF_sh=%d must equal FF=%d", L->FF_sh, L->FF);
    if (!is_weight_fmt(L->q_gate_sh) || L->q_up_sh != L->q_gate_sh || !is_weight_fmt(L->q_down_sh))
      return gm_fail_arg("gm_moe_forward: shared formats gate %d up %d down %d unsupported", L->q_gate_sh,
                         L->q_up_sh, L->q_down_sh);
  }
  if (L->norm_w && !(L->norm_eps >= 0.f)) return gm_fail_arg("gm_moe_forward: norm_eps must be >= 0");
  const void* wptrs[] = {L->gate_exps, L->up_exps, L->down_exps, L->gate_sh,     L->up_sh,
                         L->down_sh,    L->router, L->norm_w,    L->sh_gate_inp};
  for (const void* p : wptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16)
      return gm_fail_arg("gm_moe_forward: weight, norm_w and sh_gate_inp pointers must be 16-byte aligned");
  return GM_OK;
}

extern "C" {

const char* gm_last_error(void) { return g_err; }

int gm_abi_version(void) { return 6; }

int gm_dequant_f32(int qtype, const void* raw, int64_t n_superblocks, float* out, void* stream) {
  if (gm_kquant_block(qtype).bytes)
    return n_superblocks < 0 || !raw || !out ? gm_fail_arg("gm_dequant_f32: bad arguments")
                                            : gm_launch_dequant_k(qtype, raw, n_superblocks, out, as_stream(stream));
  if (!is_quant(qtype))
    return gm_fail_arg("gm_dequant_f32: qtype %d is not IQ4_XS(23)/IQ3_XXS(18)/Q8_0(8)/Q4_K(12)/Q5_K(13)/Q6_K(14)",
                       qtype);
  if (n_superblocks < 0) return gm_fail_arg("gm_dequant_f32: negative n_superblocks");
  if (n_superblocks == 0) return GM_OK;
  if (!raw || !out) return gm_fail_arg("gm_dequant_f32: NULL pointer");
  if (reinterpret_cast<uintptr_t>(raw) % 8 || reinterpret_cast<uintptr_t>(out) % 16)
    return gm_fail_arg("gm_dequant_f32: raw must be 8-byte and out 16-byte aligned");
  return gm_launch_dequant(qtype, raw, n_superblocks, out, as_stream(stream));
}

int gm_transcode_i8(int qtype, const void* raw, int64_t n_blocks, void* out, void* stream) {
  if (!gm_kquant_block(qtype).bytes)
    return gm_fail_arg("gm_transcode_i8: qtype %d is not Q8_0(8)/Q4_K(12)/Q5_K(13)/Q6_K(14)", qtype);
  if (n_blocks < 0) return gm_fail_arg("gm_transcode_i8: negative n_blocks");
  if (n_blocks == 0) return GM_OK;
  if (!raw || !out) return gm_fail_arg("gm_transcode_i8: NULL pointer");
  if (reinterpret_cast<uintptr_t>(out) % 16) return gm_fail_arg("gm_transcode_i8: out must be 16-byte aligned");
  return gm_launch_transcode_i8(qtype, raw, n_blocks, out, as_stream(stream));
}

int gm_matvec(int qtype, const void* w, int M, int K, const float* x, int n_tok, float* y, void* stream) {
  if (!is_quant(qtype) && qtype != GM_QTYPE_BF16) return gm_fail_arg("gm_matvec: unsupported qtype %d", qtype);
  if (int rc = check_k("gm_matvec", qtype, K)) return rc;
  if (M < 0 || n_tok < 0) return gm_fail_arg("gm_matvec: negative size");
  if (M == 0 || n_tok == 0) return GM_OK;
  if (!w || !x || !y) return gm_fail_arg("gm_matvec: NULL pointer");
  if (K > 16384) return gm_fail_arg("gm_matvec: K=%d > 16384 not supported", K);
  if (reinterpret_cast<uintptr_t>(w) % 16 || reinterpret_cast<uintptr_t>(x) % 16)
    return gm_fail_arg("gm_matvec: w and x must be 16-byte aligned");
  return gm_launch_matvec(qtype, w, M, K, x, n_tok, y, as_stream(stream));
}

int gm_swiglu_mlp(int q_gu, const void* w_gate, const void* w_up, int q_down, const void* w_down, int D, int FF,
                  const float* x, int n_tok, float* h, float* y, void* stream) {
  if (!is_weight_fmt(q_gu) || !is_weight_fmt(q_down))
    return gm_fail_arg("gm_swiglu_mlp: unsupported qtypes %d / %d", q_gu, q_down);
  if (int rc = check_k("gm_swiglu_mlp", q_gu, D)) return rc;
  if (int rc = check_k("gm_swiglu_mlp", q_down, FF)) return rc;
  if (D > 16384 || FF > 16384) return gm_fail_arg("gm_swiglu_mlp: D/FF > 16384 not supported");
  if (n_tok < 0) return gm_fail_arg("gm_swiglu_mlp: negative n_tok");
  if (n_tok == 0) return GM_OK;
  if (!w_gate || !w_up || !w_down || !x || !h || !y) return gm_fail_arg("gm_swiglu_mlp: NULL pointer");
  // each weight aligned to its format's load width; h is read with 16-byte loads by the bf16 down kernel
  auto width = [](int q) -> uintptr_t { return q == GM_QTYPE_BF16 ? 16 : q == GM_QTYPE_IQ4_XS ? 8 : 2; };
  if (reinterpret_cast<uintptr_t>(w_gate) % width(q_gu) || reinterpret_cast<uintptr_t>(w_up) % width(q_gu) ||
      reinterpret_cast<uintptr_t>(w_down) % width(q_down) ||
      (q_down == GM_QTYPE_BF16 && reinterpret_cast<uintptr_t>(h) % 16))
    return gm_fail_arg("gm_swiglu_mlp: weights must be aligned to 16 (bf16), 8 (IQ4_XS) or 2 (IQ3_XXS) bytes, "
                       "and h to 16 bytes when the down matrix is bf16");
  hipStream_t s = as_stream(stream);
  if (int rc = gm_launch_gateup(q_gu, w_gate, w_up, FF, D, x, n_tok, h, s)) return rc;
  return gm_launch_matvec(q_down, w_down, D, FF, h, n_tok, y, s);
}

int gm_router_topk(const uint16_t* w_router, const float* bias, const float* x, int T, int D, int E, int k,
                   const uint16_t* w_sh_gate, const float* norm_w, float eps, int32_t* ids, float* weights,
                   float* logits, float* sh_gate, void* stream) {
  if (T < 0 || D <= 0 || E <= 0 || k <= 0) return gm_fail_arg("gm_router_topk: bad sizes");
  if (E > 512 || k > 8 || k > E) return gm_fail_arg("gm_router_topk: need E <= 512 and k <= min(8, E)");
  if (D % GM_SUB) return gm_fail_arg("gm_router_topk: D=%d must be a multiple of 32", D);
  if (D > 16384) return gm_fail_arg("gm_router_topk: D > 16384 not supported");
  if (T == 0) return GM_OK;
  if (!w_router || !x || !ids || !weights || !logits) return gm_fail_arg("gm_router_topk: NULL pointer");
  if (w_sh_gate && !sh_gate) return gm_fail_arg("gm_router_topk: sh_gate output missing");
  hipStream_t s = as_stream(stream);
  if (int rc = gm_launch_router(w_router, bias, x, T, D, E, w_sh_gate, norm_w, eps, logits, sh_gate, s)) return rc;
  return gm_launch_topk(logits, T, E, k, ids, weights, s);
}

int gm_moe_dispatch(const int32_t* ids, int T, int k, int E, int32_t* counts, int32_t* offsets,
                    int32_t* sorted_pairs, void* stream) {
  if (T < 0 || k <= 0 || E <= 0) return gm_fail_arg("gm_moe_dispatch: bad sizes");
  if (!ids || !counts || !offsets || !sorted_pairs) return gm_fail_arg("gm_moe_dispatch: NULL pointer");
  return gm_launch_dispatch(ids, T, k, E, counts, offsets, sorted_pairs, as_stream(stream));
}

size_t gm_moe_workspace_bytes(const gm_moe_layer* L, int T) {
  if (T < 0 || check_layer(L) != GM_OK) return 0;
  return gm_moe_ws_layout(L, T).total;
}

int gm_moe_workspace_offsets(const gm_moe_layer* L, int T, size_t* off_logits, size_t* off_ids,
                             size_t* off_weights, size_t* off_sh_gate) {
  if (int rc = check_layer(L)) return rc;
  const GmMoeWs w = gm_moe_ws_layout(L, T);
  if (off_logits) *off_logits = w.logits;
  if (off_ids) *off_ids = w.ids;
  if (off_weights) *off_weights = w.wts;
  if (off_sh_gate) *off_sh_gate = w.shg;
  return GM_OK;
}

enum { kPathAuto = 0, kPathDecode = 1, kPathPrefill = 2 };

static int moe_forward_impl(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws,
                            size_t ws_bytes, int stage, int path, void* stream);

int gm_moe_forward(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws, size_t ws_bytes,
                   void* stream) {
  return moe_forward_impl(L, x, y, T, flags, ws, ws_bytes, 0, kPathAuto, stream);
}

int gm_moe_decode(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws, size_t ws_bytes,
                  void* stream) {
  if (T > GM_DECODE_MAX_T) return gm_fail_arg("gm_moe_decode: T=%d > %d (use gm_moe_prefill)", T, GM_DECODE_MAX_T);
  return moe_forward_impl(L, x, y, T, flags, ws, ws_bytes, 0, kPathDecode, stream);
}

int gm_moe_prefill(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws, size_t ws_bytes,
                   void* stream) {
  return moe_forward_impl(L, x, y, T, flags, ws, ws_bytes, 0, kPathPrefill, stream);
}

int gm_moe_forward_stage(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws,
                         size_t ws_bytes, int stage, void* stream) {
  if (stage < 0 || stage > 3) return gm_fail_arg("gm_moe_forward_stage: stage %d not in 0..3", stage);
  return moe_forward_impl(L, x, y, T, flags, ws, ws_bytes, stage, kPathAuto, stream);
}

// Layers l = 0 .. n-1 in sequence: x_{l+1} = moe_l(x_l) (+ x_l with
// GM_MOE_RESIDUAL), x_0 = x; layer l writes y when n - 1 - l is even, else
// buf, so that the last layer writes y.  At T = 1, when every layer fits the
// accumulator kernels and the layers agree on D and E, the router runs once
// (layer 0) and each layer's down kernel adds the next layer's router dot
// products into accumulators in that layer's workspace (buffer l % 2, cleared
// by layer l - 1's gate/up kernel): two launches per layer instead of three.
// Otherwise every layer runs as gm_moe_forward.
// Whether layer l of a T-token chain can run on the accumulator-linked kernels.
static bool chain_layer_fused(const gm_moe_layer* layers, int l, int T) {
  const gm_moe_layer* L = layers + l;
  return T == 1 && L->E == layers[0].E && L->D <= 4096 && L->FF <= 2048 && L->k <= 8 && gm_dec_chain_ok(L) &&
         (l == 0 || L->router_t != nullptr);
}

// Whether layers l and l + 1 of a T-token chain (2 <= T <= 8, decode path)
// can be linked through layer l's combine kernel, which then writes layer
// l + 1's router inputs (partials over 256-column slices, sums of x^2, limb
// rows) into layer l + 1's workspace: both take the decode path, D splits
// into at most 16 slices, layer l + 1 has router_t and its workspace holds the
// inputs.  gm_moe_chain also needs the two workspaces not to overlap (the
// combine reads layer l's partial rows while it writes layer l + 1's inputs).
static bool chain_pair_linkable(const gm_moe_layer* layers, int l, int T) {
  const gm_moe_layer* A = layers + l;
  const gm_moe_layer* B = layers + l + 1;
  auto decode = [&](const gm_moe_layer* L) {
    return T >= 2 && T <= GM_DECODE_MAX_T && T * L->k <= GM_GRP_MAXU && L->D % 256 == 0 && L->FF % 256 == 0 &&
           L->D <= 4096 && L->FF <= 2048 && L->k <= 8;
  };
  if (!decode(A) || !decode(B) || A->D % GM_DEC_LINK_KR || gm_dec_link_nz(A->D) > GM_DEC_MAX_NZ) return false;
  return B->router_t != nullptr && B->D == A->D && gm_dec_part_fits(B, T, gm_dec_link_nz(B->D));
}

static bool ws_disjoint(const void* a, size_t na, const void* b, size_t nb) {
  const uint8_t* pa = static_cast<const uint8_t*>(a);
  const uint8_t* pb = static_cast<const uint8_t*>(b);
  return pa + na <= pb || pb + nb <= pa;
}

int gm_moe_chain_fused(const gm_moe_layer* layers, int n_layers, int T) {
  if (!layers || n_layers < 1 || T < 0) return gm_fail_arg("gm_moe_chain_fused: bad arguments");
  bool fused = true, linked = n_layers > 1;
  for (int l = 0; l < n_layers; ++l) {
    if (int rc = check_layer(layers + l)) return rc;
    fused = fused && chain_layer_fused(layers, l, T);
    if (l + 1 < n_layers) linked = linked && chain_pair_linkable(layers, l, T);
  }
  return fused ? 1 : linked ? 2 : 0;
}

int gm_moe_chain(const gm_moe_layer* layers, int n_layers, const float* x, float* y, float* buf, int T, int flags,
                 void* const* ws, const size_t* ws_bytes, void* stream) {
  if (!layers || !ws || !ws_bytes) return gm_fail_arg("gm_moe_chain: NULL layers or workspace array");
  if (n_layers < 1) return gm_fail_arg("gm_moe_chain: n_layers=%d < 1", n_layers);
  if (T < 0) return gm_fail_arg("gm_moe_chain: negative T");
  if (!x || !y || (n_layers > 1 && !buf)) return gm_fail_arg("gm_moe_chain: NULL x, y or buf");
  if (x == y || x == buf || y == buf) return gm_fail_arg("gm_moe_chain: x, y and buf must not alias");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 16 ||
      reinterpret_cast<uintptr_t>(buf) % 16)
    return gm_fail_arg("gm_moe_chain: x, y and buf must be 16-byte aligned");
  bool fused = T == 1;
  for (int l = 0; l < n_layers; ++l) {
    const gm_moe_layer* L = layers + l;
    if (int rc = check_layer(L)) return rc;
    if (L->D != layers[0].D) return gm_fail_arg("gm_moe_chain: layer %d has D=%d, layer 0 D=%d", l, L->D, layers[0].D);
    if (!ws[l]) return gm_fail_arg("gm_moe_chain: workspace %d is NULL", l);
    if (reinterpret_cast<uintptr_t>(ws[l]) % 256) return gm_fail_arg("gm_moe_chain: workspace %d not 256-byte aligned", l);
    const size_t need = gm_moe_ws_layout(L, T).total;
    if (ws_bytes[l] < need)
      return gm_fail_arg("gm_moe_chain: workspace %d has %zu bytes < %zu needed", l, ws_bytes[l], need), GM_EWORKSPACE;
    fused = fused && chain_layer_fused(layers, l, T);
    if (L->router_t && reinterpret_cast<uintptr_t>(L->router_t) % 16)
      return gm_fail_arg("gm_moe_chain: layer %d router_t must be 16-byte aligned", l);
  }
  if (T == 0) return GM_OK;
  hipStream_t s = as_stream(stream);
  const float* in = x;
  bool linked_in = false;                                   // layer l's router inputs come from layer l - 1
  for (int l = 0; l < n_layers; ++l) {
    const gm_moe_layer* L = layers + l;
    float* out = (n_layers - 1 - l) % 2 == 0 ? y : buf;
    uint8_t* w = static_cast<uint8_t*>(ws[l]);
    const GmMoeWs lay = gm_moe_ws_layout(L, T);
    const bool linked_out = !fused && l + 1 < n_layers && chain_pair_linkable(layers, l, T) &&
                            ws_disjoint(ws[l], ws_bytes[l], ws[l + 1], ws_bytes[l + 1]);
    if (!fused && (linked_in || linked_out)) {
      GmNextB8 nx8{};
      GmChainStep cs{nullptr, nullptr, nullptr, !linked_in, nullptr};
      if (linked_out) {
        const gm_moe_layer* N = layers + l + 1;
        float* rms;
        if (!gm_dec_part_ptrs(N, T, gm_dec_link_nz(N->D), static_cast<uint8_t*>(ws[l + 1]), gm_moe_ws_layout(N, T),
                              &nx8.part, &nx8.ssq, &rms, &nx8.xl))
          return gm_fail_arg("gm_moe_chain: internal workspace layout error (linked)");
        nx8.w = N->router_t;
        nx8.nw = N->norm_w;
        nx8.E = N->E;
        nx8.ldp = gm_dec_part_ld(N);
        nx8.f32 = N->q_router == GM_QTYPE_F32 ? 1 : 0;
        cs.next8 = &nx8;
      }
      if (int rc = gm_dec_run(L, in, out, T, flags, w, lay, s, 0, &cs)) return rc;
      linked_in = linked_out;
    } else if (!fused) {
      if (int rc = moe_forward_impl(L, in, out, T, flags, w, ws_bytes[l], 0, kPathAuto, stream)) return rc;
      linked_in = false;
    } else {
      auto acc_of = [&](int j) {
        const GmMoeWs lj = gm_moe_ws_layout(layers + j, T);
        return reinterpret_cast<double*>(static_cast<uint8_t*>(ws[j]) + lj.acc) +
               (size_t)(j % 2) * gm_acc_bytes(layers[j].E) / sizeof(double);
      };
      GmNextRouter nx{};
      GmChainStep cs{acc_of(l), nullptr, nullptr, l == 0, nullptr};
      if (l + 1 < n_layers) {
        const gm_moe_layer* N = layers + l + 1;
        nx.w = N->router_t;
        nx.nw = N->norm_w;
        nx.acc = acc_of(l + 1);
        nx.E = N->E;
        nx.ld = gm_acc_ld(N->E);
        nx.f32 = N->q_router == GM_QTYPE_F32 ? 1 : 0;
        cs.acc_zero = nx.acc;
        cs.next = &nx;
      }
      if (int rc = gm_dec_run(L, in, out, T, flags, w, lay, s, 0, &cs)) return rc;
    }
    in = out;
  }
  return GM_OK;
}

// ------------------------------------------------------------ core layers
static int check_attn(const gm_attn_layer* L) {
  if (!L) return gm_fail_arg("gm_attn_decode: layer is NULL");
  if (!L->wqkv || !L->wo || !L->attn_norm || !L->q_norm || !L->k_norm)
    return gm_fail_arg("gm_attn_decode: weights and norms must be non-NULL");
  const int Dh = L->head_dim;
  if (Dh != 64 && Dh != 128 && Dh != 256 && Dh != 512)
    return gm_fail_arg("gm_attn_decode: head_dim=%d must be 64, 128, 256 or 512", Dh);
  if (L->n_head <= 0 || L->n_head_kv <= 0 || L->n_head % L->n_head_kv)
    return gm_fail_arg("gm_attn_decode: n_head=%d must be a positive multiple of n_head_kv=%d", L->n_head,
                       L->n_head_kv);
  if (L->rope_dim < 0 || L->rope_dim % 2 || L->rope_dim > Dh)
    return gm_fail_arg("gm_attn_decode: rope_dim=%d must be even and <= head_dim", L->rope_dim);
  if (L->D <= 0 || L->D % GM_SUB || L->D > 16384 || (L->n_head * Dh) > 16384)
    return gm_fail_arg("gm_attn_decode: D=%d must be a multiple of 32 up to 16384", L->D);
  if (!(L->eps >= 0.f)) return gm_fail_arg("gm_attn_decode: eps must be >= 0");
  if (reinterpret_cast<uintptr_t>(L->wqkv) % 16 || reinterpret_cast<uintptr_t>(L->wo) % 16 ||
      reinterpret_cast<uintptr_t>(L->attn_norm) % 16)
    return gm_fail_arg("gm_attn_decode: wqkv, wo and attn_norm must be 16-byte aligned");
  return GM_OK;
}

static int check_ssm(const gm_ssm_layer* L) {
  if (!L) return gm_fail_arg("gm_ssm_decode: layer is NULL");
  if (!L->w_in || !L->w_gate || !L->w_out || !L->alpha || !L->beta || !L->conv1d || !L->a || !L->dt_bias ||
      !L->ssm_norm || !L->attn_norm)
    return gm_fail_arg("gm_ssm_decode: weights must be non-NULL");
  const int S = L->d_state;
  if (S != 64 && S != 128 && S != 256) return gm_fail_arg("gm_ssm_decode: d_state=%d must be 64, 128 or 256", S);
  if (L->n_k_heads <= 0 || L->n_v_heads <= 0 || L->n_v_heads % L->n_k_heads)
    return gm_fail_arg("gm_ssm_decode: n_v_heads=%d must be a positive multiple of n_k_heads=%d", L->n_v_heads,
                       L->n_k_heads);
  if (L->conv_k < 1 || L->conv_k > 8) return gm_fail_arg("gm_ssm_decode: conv_k=%d must be in 1..8", L->conv_k);
  if (L->D <= 0 || L->D % GM_SUB || L->D > 16384 || L->n_v_heads * S > 16384)
    return gm_fail_arg("gm_ssm_decode: D=%d must be a multiple of 32 up to 16384", L->D);
  if (!(L->eps >= 0.f)) return gm_fail_arg("gm_ssm_decode: eps must be >= 0");
  const void* w[] = {L->w_in, L->w_gate, L->w_out, L->attn_norm, L->alpha, L->beta};
  for (const void* p : w)
    if (reinterpret_cast<uintptr_t>(p) % 16)
      return gm_fail_arg("gm_ssm_decode: bf16 weights, alpha, beta and attn_norm must be 16-byte aligned");
  return GM_OK;
}

static int check_io(const char* fn, const float* x, const float* y) {
  if (!x || !y) return gm_fail_arg("%s: NULL x or y", fn);
  if (x == y) return gm_fail_arg("%s: x and y must not alias", fn);
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 16)
    return gm_fail_arg("%s: x and y must be 16-byte aligned", fn);
  return GM_OK;
}

size_t gm_attn_workspace_bytes(const gm_attn_layer* L, int max_pos) {
  if (max_pos < 1 || check_attn(L) != GM_OK) return 0;
  return gm_attn_ws_layout(L, max_pos).total;
}

int gm_attn_decode(const gm_attn_layer* L, const float* x, float* y, float* k_cache, float* v_cache, int pos,
                   int max_pos, const float* rope_cos, const float* rope_sin, int flags, void* ws, size_t ws_bytes,
                   void* stream) {
  if (int rc = check_attn(L)) return rc;
  if (int rc = check_io("gm_attn_decode", x, y)) return rc;
  if (max_pos < 1 || pos < 0 || pos >= max_pos)
    return gm_fail_arg("gm_attn_decode: pos=%d must be in [0, max_pos=%d)", pos, max_pos);
  if (!k_cache || !v_cache || !ws || (L->rope_dim > 0 && (!rope_cos || !rope_sin)))
    return gm_fail_arg("gm_attn_decode: NULL cache, rope table or workspace");
  const size_t need = gm_attn_ws_layout(L, max_pos).total;
  if (ws_bytes < need)
    return gm_fail_arg("gm_attn_decode: workspace %zu bytes < %zu needed", ws_bytes, need), GM_EWORKSPACE;
  if (reinterpret_cast<uintptr_t>(ws) % 256) return gm_fail_arg("gm_attn_decode: workspace must be 256-byte aligned");
  return gm_attn_run(L, x, y, k_cache, v_cache, pos, max_pos, rope_cos, rope_sin, flags, static_cast<uint8_t*>(ws),
                     as_stream(stream));
}

size_t gm_ssm_workspace_bytes(const gm_ssm_layer* L) {
  if (check_ssm(L) != GM_OK) return 0;
  return gm_ssm_ws_layout(L).total;
}

int gm_ssm_decode(const gm_ssm_layer* L, const float* x, float* y, float* conv_state, float* rec_state, int flags,
                  void* ws, size_t ws_bytes, void* stream) {
  if (int rc = check_ssm(L)) return rc;
  if (int rc = check_io("gm_ssm_decode", x, y)) return rc;
  if (!rec_state || !ws || (L->conv_k > 1 && !conv_state))
    return gm_fail_arg("gm_ssm_decode: NULL state or workspace");
  const size_t need = gm_ssm_ws_layout(L).total;
  if (ws_bytes < need)
    return gm_fail_arg("gm_ssm_decode: workspace %zu bytes < %zu needed", ws_bytes, need), GM_EWORKSPACE;
  if (reinterpret_cast<uintptr_t>(ws) % 256) return gm_fail_arg("gm_ssm_decode: workspace must be 256-byte aligned");
  return gm_ssm_run(L, x, y, conv_state, rec_state, flags, static_cast<uint8_t*>(ws), as_stream(stream));
}

// The MoE block that follows a core layer, for the linked entry points: it must
// run on the T = 1 accumulator kernels (gm_moe_chain_fused(&moe, 1, 1) == 1),
// share the core layer's D and carry router_t; its workspace holds the
// accumulators the core layer's launches clear and fill.
static int moe_link(const char* fn, const gm_moe_layer* M, int D, void* ws, size_t ws_bytes, GmNextRouter* nx) {
  if (int rc = check_layer(M)) return rc;
  if (!chain_layer_fused(M, 0, 1) || M->D != D || !M->router_t)
    return gm_fail_arg("%s: the MoE block must fit the T = 1 accumulator kernels, have D=%d and carry router_t", fn,
                       D);
  if (reinterpret_cast<uintptr_t>(M->router_t) % 16) return gm_fail_arg("%s: router_t must be 16-byte aligned", fn);
  if (!ws || reinterpret_cast<uintptr_t>(ws) % 256) return gm_fail_arg("%s: MoE workspace NULL or not 256-byte aligned", fn);
  const GmMoeWs lay = gm_moe_ws_layout(M, 1);
  if (ws_bytes < lay.total)
    return gm_fail_arg("%s: MoE workspace %zu bytes < %zu needed", fn, ws_bytes, lay.total), GM_EWORKSPACE;
  nx->w = M->router_t;
  nx->nw = M->norm_w;
  nx->acc = reinterpret_cast<double*>(static_cast<uint8_t*>(ws) + lay.acc);
  nx->E = M->E;
  nx->ld = gm_acc_ld(M->E);
  nx->f32 = M->q_router == GM_QTYPE_F32 ? 1 : 0;
  return GM_OK;
}

int gm_attn_decode_moe(const gm_attn_layer* L, const float* x, float* y, float* k_cache, float* v_cache, int pos,
                       int max_pos, const float* rope_cos, const float* rope_sin, int flags, void* ws,
                       size_t ws_bytes, const gm_moe_layer* moe, void* moe_ws, size_t moe_ws_bytes, void* stream) {
  if (int rc = check_attn(L)) return rc;
  if (int rc = check_io("gm_attn_decode_moe", x, y)) return rc;
  if (max_pos < 1 || pos < 0 || pos >= max_pos)
    return gm_fail_arg("gm_attn_decode_moe: pos=%d must be in [0, max_pos=%d)", pos, max_pos);
  if (!k_cache || !v_cache || !ws || (L->rope_dim > 0 && (!rope_cos || !rope_sin)))
    return gm_fail_arg("gm_attn_decode_moe: NULL cache, rope table or workspace");
  const size_t need = gm_attn_ws_layout(L, max_pos).total;
  if (ws_bytes < need)
    return gm_fail_arg("gm_attn_decode_moe: workspace %zu bytes < %zu needed", ws_bytes, need), GM_EWORKSPACE;
  if (reinterpret_cast<uintptr_t>(ws) % 256) return gm_fail_arg("gm_attn_decode_moe: workspace must be 256-byte aligned");
  GmNextRouter nx{};
  if (int rc = moe_link("gm_attn_decode_moe", moe, L->D, moe_ws, moe_ws_bytes, &nx)) return rc;
  return gm_attn_run(L, x, y, k_cache, v_cache, pos, max_pos, rope_cos, rope_sin, flags, static_cast<uint8_t*>(ws),
                     as_stream(stream), &nx);
}

int gm_ssm_decode_moe(const gm_ssm_layer* L, const float* x, float* y, float* conv_state, float* rec_state, int flags,
                      void* ws, size_t ws_bytes, const gm_moe_layer* moe, void* moe_ws, size_t moe_ws_bytes,
                      void* stream) {
  if (int rc = check_ssm(L)) return rc;
  if (int rc = check_io("gm_ssm_decode_moe", x, y)) return rc;
  if (!rec_state || !ws || (L->conv_k > 1 && !conv_state))
    return gm_fail_arg("gm_ssm_decode_moe: NULL state or workspace");
  const size_t need = gm_ssm_ws_layout(L).total;
  if (ws_bytes < need)
    return gm_fail_arg("gm_ssm_decode_moe: workspace %zu bytes < %zu needed", ws_bytes, need), GM_EWORKSPACE;
  if (reinterpret_cast<uintptr_t>(ws) % 256) return gm_fail_arg("gm_ssm_decode_moe: workspace must be 256-byte aligned");
  GmNextRouter nx{};
  if (int rc = moe_link("gm_ssm_decode_moe", moe, L->D, moe_ws, moe_ws_bytes, &nx)) return rc;
  return gm_ssm_run(L, x, y, conv_state, rec_state, flags, static_cast<uint8_t*>(ws), as_stream(stream), &nx);
}

int gm_moe_forward_acc(const gm_moe_layer* L, const float* x, float* y, int flags, void* ws, size_t ws_bytes,
                       void* stream) {
  if (int rc = check_layer(L)) return rc;
  if (!chain_layer_fused(L, 0, 1) || !L->router_t)
    return gm_fail_arg("gm_moe_forward_acc: the block must fit the T = 1 accumulator kernels and carry router_t");
  if (!x || !y || !ws) return gm_fail_arg("gm_moe_forward_acc: NULL pointer");
  if (x == y) return gm_fail_arg("gm_moe_forward_acc: x and y must not alias");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 16)
    return gm_fail_arg("gm_moe_forward_acc: x and y must be 16-byte aligned");
  const GmMoeWs lay = gm_moe_ws_layout(L, 1);
  if (ws_bytes < lay.total)
    return gm_fail_arg("gm_moe_forward_acc: workspace %zu bytes < %zu needed", ws_bytes, lay.total), GM_EWORKSPACE;
  if (reinterpret_cast<uintptr_t>(ws) % 256) return gm_fail_arg("gm_moe_forward_acc: workspace must be 256-byte aligned");
  uint8_t* w = static_cast<uint8_t*>(ws);
  GmChainStep cs{reinterpret_cast<double*>(w + lay.acc), nullptr, nullptr, false, nullptr};
  return gm_dec_run(L, x, y, 1, flags, w, lay, as_stream(stream), 0, &cs);
}

int gm_rms_norm(const float* x, const float* w, int D, int n_rows, float eps, float* y, void* stream) {
  if (D <= 0 || n_rows < 0 || !(eps >= 0.f)) return gm_fail_arg("gm_rms_norm: bad sizes or eps");
  if (n_rows == 0) return GM_OK;
  if (!x || !w || !y) return gm_fail_arg("gm_rms_norm: NULL pointer");
  return gm_launch_rms_row(x, w, D, n_rows, eps, y, as_stream(stream));
}

}  // extern "C"

// gm_moe_forward_noalloc's workspace: a file-scope device array.  Every GPU that
// loads this code object holds its own copy, at its own address, until the
// process ends.  In host code `scratch` names a host-side stand-in, never the
// device memory: the per-device address comes from hipGetSymbolAddress once, on
// the first call on each device, and only that address is passed on.
static __device__ __align__(256) uint8_t scratch[GM_NOALLOC_SCRATCH_BYTES];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_address(int dev, void** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return gm_fail_hip(e, "gm_moe_forward_noalloc: hipGetSymbolAddress(scratch)");
    if (!ptr || reinterpret_cast<uintptr_t>(ptr) % 256)
      return gm_fail_arg("gm_moe_forward_noalloc: scratch address %p is not 256-byte aligned", ptr);
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GM_OK;
}

extern "C" int gm_moe_forward_noalloc(const gm_moe_layer* L, const float* x, float* y, int T, int flags,
                                      void* stream) {
  if (int rc = check_layer(L)) return rc;
  if (T < 0) return gm_fail_arg("gm_moe_forward_noalloc: negative T");
  const size_t need = gm_moe_ws_layout(L, T).total;
  if (need > GM_NOALLOC_SCRATCH_BYTES)
    return gm_fail_arg("gm_moe_forward_noalloc: T=%d needs %zu workspace bytes, more than the %zu of the static "
                       "scratch (use gm_moe_forward with a workspace)", T, need, (size_t)GM_NOALLOC_SCRATCH_BYTES),
           GM_EWORKSPACE;
  if (T == 0) return GM_OK;
  int dev = -1;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return gm_fail_hip(e, "gm_moe_forward_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return gm_fail_arg("gm_moe_forward_noalloc: device %d >= %d", dev, kMaxDevices);
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipError_t e = hipStreamGetDevice(as_stream(stream), &sdev); e != hipSuccess)
      return gm_fail_hip(e, "gm_moe_forward_noalloc: hipStreamGetDevice");
    if (sdev != dev)
      return gm_fail_arg("gm_moe_forward_noalloc: stream is on device %d but device %d is current", (int)sdev, dev);
  }
  void* ptr = nullptr;
  if (int rc = scratch_address(dev, &ptr)) return rc;
  // No region of the workspace has to start at zero: every kernel writes what it
  // later reads within the same call.
  return moe_forward_impl(L, x, y, T, flags, ptr, GM_NOALLOC_SCRATCH_BYTES, 0, kPathAuto, stream);
}

static int moe_forward_impl(const gm_moe_layer* L, const float* x, float* y, int T, int flags, void* ws,
                            size_t ws_bytes, int stage, int path, void* stream) {
  if (int rc = check_layer(L)) return rc;
  if (T < 0) return gm_fail_arg("gm_moe_forward: negative T");
  if (T == 0) return GM_OK;
  if (!x || !y || !ws) return gm_fail_arg("gm_moe_forward: NULL pointer");
  if (x == y) return gm_fail_arg("gm_moe_forward: x and y must not alias");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 16)
    return gm_fail_arg("gm_moe_forward: x and y must be 16-byte aligned");
  const GmMoeWs lay = gm_moe_ws_layout(L, T);
  if (ws_bytes < lay.total)
    return gm_fail_arg("gm_moe_forward: workspace %zu bytes < %zu needed", ws_bytes, lay.total), GM_EWORKSPACE;
  if (reinterpret_cast<uintptr_t>(ws) % 256) return gm_fail_arg("gm_moe_forward: workspace must be 256-byte aligned");
  uint8_t* w = static_cast<uint8_t*>(ws);
  hipStream_t s = as_stream(stream);
  const bool decode = path == kPathDecode || (path == kPathAuto && T <= GM_DECODE_MAX_T && T * L->k <= GM_GRP_MAXU);
  if (decode) return gm_dec_run(L, x, y, T, flags, w, lay, s, stage);
  if (stage != 0) return gm_fail_arg("gm_moe_forward_stage: stages are only defined for the decode path (T <= 8)");
  if (!is_quant(L->q_gate) || !is_quant(L->q_down)) {
    // Routed experts held as bf16 or I8 rows (K-quant expert tensors): the
    // prefill GEMMs decode IQ4_XS / IQ3_XXS only, so the tokens run as decode
    // chunks of at most 8 (every token's MoE output is independent of the
    // others).  Each chunk writes its logits / ids / weights / shared gate into
    // its rows of the full-T arrays.  (A shared expert in other formats than IQ
    // routed experts stays on the prefill path: gm_pf_run runs it as a pass of
    // its own.)
    const int D = L->D, E = L->E, k = L->k;
    for (int t0 = 0; t0 < T; t0 += GM_DECODE_MAX_T) {
      const int tc = T - t0 < GM_DECODE_MAX_T ? T - t0 : GM_DECODE_MAX_T;
      GmMoeWs lc = lay;
      lc.logits += (size_t)t0 * E * 4;
      lc.shg += (size_t)t0 * 4;
      lc.ids += (size_t)t0 * k * 4;
      lc.wts += (size_t)t0 * k * 4;
      lc.hsh = lc.h + (size_t)tc * k * L->FF * 4;                      // h_sh directly after the chunk's h
      if (int rc = gm_dec_run(L, x + (size_t)t0 * D, y + (size_t)t0 * D, tc, flags, w, lc, s, 0)) return rc;
    }
    return GM_OK;
  }
  return gm_pf_run(L, x, y, T, flags, w, lay, s);
}
