"""CPU oracle for the Qwen MoE-block hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's arithmetic for the path
(BojanFaletic/NPU ``qwen/forward.py:563-665`` and the gguf-py 0.18.0 dequant
routines it calls through ``qwen/model.py:230-277``).  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker / CPU baseline.  The product package
(``npu_amd``) never imports it and has no CPU fallback.

Modules
-------
tables   IQ3_XXS grid, ksigns and kvalues_iq4nl codebooks.
quants   IQ4_XS / IQ3_XXS superblock dequantisation (numpy, fp32 exact).
moe      ``moe_forward`` restated in torch fp32 (per-call dequant, as the
         reference CPU path does), RMSNorm, router top-k, bf16 helpers.

Pinning status (what each function is checked against) is listed in the
header of each module.
"""
