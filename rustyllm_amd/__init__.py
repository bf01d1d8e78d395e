"""rustyllm_amd — MI355X-native decode-step backend for RustyLLM.

The product is librusty_hip.so (include/rusty_hip.h): hand-written gfx950
kernels for the quantized GEMVs (Q8_0, Q4_K, Q6_K, MXFP4), split-K GQA decode
attention and the fused small ops, behind a C ABI that mirrors the reference's
Metal seam (src/metal.rs).  `rustyllm_amd.hip` binds it with ctypes;
`rustyllm_amd.synth` writes seeded synthetic models; `rustyllm_amd.gguf`
reads and writes GGUF files.
"""
__all__ = ["hip", "synth", "gguf", "build"]
