"""npu_amd -- MI355X (gfx950) implementation of BojanFaletic/NPU's Qwen MoE-block hot path.

Hand-written HIP kernels (``csrc/``) behind a C ABI (``include/npu_amd.h``),
loaded with ctypes (``_lib``).  Python mirrors of the reference's operator
surface live in the modules named after the reference's ``npu/*.py`` files
(``quant_mv``, ``quant_mv_iq4``, ``quant_mv_iq4_packed``, ``mv``, ``mlp``,
``iq3_xxs``, ``profiler``) and in ``qwen_moe`` (``MoELayer``, ``moe_forward``,
``enable_npu`` of ``qwen/forward.py``).
"""
__all__ = ["ops", "moe", "synth", "gguf_types"]
