"""rustyllm_amd — MI355X-native decode-step backend for RustyLLM.

The product is librusty_hip.so (include/rusty_hip.h): hand-written gfx950
kernels for the quantized GEMVs (Q8_0, Q4_K, Q6_K, MXFP4), GQA decode
attention (the reference's serial order, or split-K) and the fused small ops,
the resident per-token decoder and the batched prefill, behind a C ABI that
mirrors the reference's Metal seam (src/metal.rs), plus a native GGUF loader
into the resident decoder.  `rustyllm_amd.hip` binds it with ctypes;
`rustyllm_amd.synth` makes seeded synthetic models; `rustyllm_amd.gguf`
reads and writes GGUF v3 files.
"""
__all__ = ["hip", "synth", "gguf", "build"]
