"""MI355X (gfx950) backend for llm-runner's DiT hot path: GGUF Q8_0/Q4_K
dequant-GEMM and non-causal flash attention behind a C-ABI (include/llmr_hip.h).

`capi` binds the C-ABI, `ops` mirrors the reference's op interface on torch
device tensors, `gguf` holds the block formats and quantizers, `synth` the
deterministic input generator.
"""
from . import gguf, synth  # noqa: F401

__all__ = ["gguf", "synth", "capi", "ops"]
