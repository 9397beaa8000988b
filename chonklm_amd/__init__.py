"""chonklm_amd — MI355X-native decode path of the llama-webgpu runtime.

The compute lives in libchonk.so (HIP kernels for gfx950 + C++ engine behind
the C ABI in include/chonk.h); this package is the host-side mirror of the
reference runtime module API (see runtime.py).
"""
from .registry import ModelDef, Workload, WORKLOADS
from .runtime import (
    ChonkError,
    LlamaWgslEngine,
    LoadedLlamaWgslModel,
    dispose_llama_wgsl,
    generate_llama_wgsl,
    load_llama_wgsl_model,
    reset_llama_wgsl_conversation,
    shard_gguf,
    write_synthetic_gguf,
)

__all__ = [
    "ModelDef", "Workload", "WORKLOADS", "ChonkError", "LlamaWgslEngine", "LoadedLlamaWgslModel",
    "dispose_llama_wgsl", "generate_llama_wgsl", "load_llama_wgsl_model", "reset_llama_wgsl_conversation",
    "shard_gguf", "write_synthetic_gguf",
]
