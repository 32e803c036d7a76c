// MoE block, prefill path (T > 8): grouped dequant-to-bf16 MFMA GEMMs.
#include "kernels.h"

size_t gm_prefill_scratch_bytes(const gm_moe_layer* L, int T) {
  (void)L;
  (void)T;
  return 0;
}

int gm_moe_prefill(const gm_moe_layer* L, const float* x, float* y, int T, int flags, uint8_t* ws,
                   const GmMoeWs& lay, hipStream_t s) {
  (void)L; (void)x; (void)y; (void)flags; (void)ws; (void)lay; (void)s;
  return gm_fail_arg("gm_moe_forward: prefill (T=%d > 8) not built yet", T), GM_EUNSUPPORTED;
}
