"""chonklm_amd — MI355X-native decode path of the llama-webgpu runtime (and the gpt-webgpu,
lfm2-webgpu and granite-webgpu runtimes on the same kernels).

The compute lives in libchonk.so (HIP kernels for gfx950 + C++ engine behind
the C ABI in include/chonk.h); this package is the host-side mirror of the
reference runtime module API (see runtime.py).
"""
from .registry import ModelDef, Workload, WORKLOADS
from .runtime import (
    ChonkError,
    LlamaWgslEngine,
    LoadedGptWgslModel,
    LoadedGraniteWgslModel,
    LoadedLfmWgslModel,
    LoadedLlamaWgslModel,
    dispose_gpt_wgsl,
    dispose_granite_wgsl,
    dispose_lfm_wgsl,
    dispose_llama_wgsl,
    generate_gpt_wgsl,
    generate_granite_wgsl,
    generate_lfm_wgsl,
    load_gpt_wgsl_model,
    load_granite_wgsl_model,
    load_lfm_wgsl_model,
    reset_granite_wgsl_conversation,
    reset_lfm_wgsl_conversation,
    reset_gpt_wgsl_conversation,
    generate_llama_wgsl,
    load_llama_wgsl_model,
    reset_llama_wgsl_conversation,
    shard_gguf,
    write_synthetic_gguf,
)

__all__ = [
    "ModelDef", "Workload", "WORKLOADS", "ChonkError", "LlamaWgslEngine", "LoadedLlamaWgslModel",
    "dispose_llama_wgsl", "generate_llama_wgsl", "load_llama_wgsl_model", "reset_llama_wgsl_conversation",
    "shard_gguf", "write_synthetic_gguf", "LoadedGptWgslModel", "load_gpt_wgsl_model", "generate_gpt_wgsl",
    "reset_gpt_wgsl_conversation", "dispose_gpt_wgsl", "LoadedLfmWgslModel", "load_lfm_wgsl_model",
    "generate_lfm_wgsl", "reset_lfm_wgsl_conversation", "dispose_lfm_wgsl", "LoadedGraniteWgslModel",
    "load_granite_wgsl_model", "generate_granite_wgsl", "reset_granite_wgsl_conversation", "dispose_granite_wgsl",
]
