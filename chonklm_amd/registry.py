"""Model definitions of the decode workloads.

``ModelDef`` carries the fields of the reference's registry entry that the
llama-webgpu runtime reads (src/lib/registry.ts:14-46): id, vocab, layers,
maxContext, eosIds, defaultRepetitionPenalty, and the artefact location (a
GGUF file or a shard directory instead of base + gguf URL).

``WORKLOADS`` are the synthetic decoders the benchmark and tests use: random
weights (N(0, 0.02) linear weights, 1 + N(0, 0.02) norm weights) quantized
with the Q4_K_M or Q8_0 recipe. Their maxContext covers prompt + decode
(the reference's registry caps Qwen3 at 2048 and Gemma-3 at 512 positions,
registry.ts:191 and :129, which the long-prompt workloads exceed).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional


@dataclass
class ModelDef:
    id: str
    vocab: int
    layers: int
    max_context: int
    eos_ids: list[int] = field(default_factory=list)
    path: str = ""  # GGUF file or shard directory (manifest.json + NNNN.bin)
    default_repetition_penalty: Optional[float] = None
    runtime: str = "llama-webgpu"
    kv_dtype: str = "f16"  # "f16" or "f32" (the reference's fp32 cache)
    device: int = 0


@dataclass
class SynthSpec:
    arch: str
    recipe: str
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    ffn: int
    vocab: int
    head_dim: int = 0  # 0: hidden // heads, no key_length metadata
    context_length: int = 32768
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5
    sliding_window: int = 0
    seed: int = 1234
    # openelm: per-layer head / kv-head / feed-forward counts (heads, kv_heads
    # and ffn above are then their maxima)
    layer_heads: Optional[list[int]] = None
    layer_kv_heads: Optional[list[int]] = None
    layer_ffn: Optional[list[int]] = None


@dataclass
class Workload:
    name: str
    spec: SynthSpec
    max_context: int
    eos_ids: list[int]
    prompt_tokens: int
    decode_tokens: int
    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0
    description: str = ""

    def prompt(self, seed: int = 1234, n: Optional[int] = None) -> list[int]:
        """Seeded uniform token ids: the workload's prompt (n defaults to prompt_tokens)."""
        import numpy as np

        return np.random.default_rng(seed).integers(0, self.spec.vocab, self.prompt_tokens if n is None else n).tolist()

    def model_def(self, path: str, kv_dtype: str = "f16", device: int = 0) -> ModelDef:
        runtime = {"gpt2": "gpt-webgpu", "lfm2": "lfm2-webgpu", "granitehybrid": "granite-webgpu"}.get(
            self.spec.arch, "llama-webgpu")
        return ModelDef(id=self.name, vocab=self.spec.vocab, layers=self.spec.layers, max_context=self.max_context,
                        eos_ids=list(self.eos_ids), path=path, kv_dtype=kv_dtype, device=device, runtime=runtime)


SMOLLM2 = dict(arch="llama", hidden=576, layers=30, heads=9, kv_heads=3, ffn=1536, vocab=49152,
               context_length=8192, rope_theta=100000.0, norm_eps=1e-5)
QWEN3 = dict(arch="qwen3", hidden=1024, layers=28, heads=16, kv_heads=8, head_dim=128, ffn=3072, vocab=151936,
             context_length=40960, rope_theta=1000000.0, norm_eps=1e-6)
GEMMA3 = dict(arch="gemma3", hidden=640, layers=18, heads=4, kv_heads=1, head_dim=256, ffn=2048, vocab=262144,
              context_length=32768, rope_theta=1000000.0, norm_eps=1e-6, sliding_window=512)

# OpenELM-270M-shaped: per-layer query / kv heads as the reference registry
# lists them (registry.ts:55-58, 589-630; groups of 4), feed-forward widths
# from multipliers 0.5..4.0 of the hidden size rounded to multiples of 256
OPENELM_270M = dict(arch="openelm", hidden=1280, layers=16, heads=20, kv_heads=5, head_dim=64, ffn=5120, vocab=32000,
                    context_length=2048, rope_theta=10000.0, norm_eps=1e-6,
                    layer_heads=[12] * 5 + [16] * 7 + [20] * 4, layer_kv_heads=[3] * 5 + [4] * 7 + [5] * 4,
                    layer_ffn=[768, 1024, 1280, 1536, 1792, 2048, 2560, 2816, 3072, 3328, 3584, 3840, 4352, 4608,
                               4864, 5120])

# LFM2.5-350M-shaped (registry.ts:61-112; the runtime's fixed shape,
# lfm-wgsl-runtime.ts:457-462): convolution and attention layers in the
# registry's order, 8 kv heads on the attention layers (0 marks a convolution
# layer, as lfm2.attention.head_count_kv does)
LFM2_TYPES = ["conv", "conv", "attention", "conv", "conv", "attention", "conv", "conv", "attention", "conv",
              "attention", "conv", "attention", "conv", "attention", "conv"]
LFM2_350M = dict(arch="lfm2", hidden=1024, layers=16, heads=16, kv_heads=8, head_dim=64, ffn=4608, vocab=65536,
                 context_length=128000, rope_theta=1000000.0, norm_eps=1e-5,
                 layer_kv_heads=[8 if t == "attention" else 0 for t in LFM2_TYPES])

# Granite-4.0-H-350M-shaped (registry.ts:48-53, :271-319; the runtime's fixed
# shape, granite-wgsl-runtime.ts:335-345, :526-533): Mamba2 and NoPE attention
# layers in the registry's order (0 kv heads marks a Mamba2 layer, as
# granitehybrid.attention.head_count_kv does), 12 q / 4 kv heads of 64, SSM
# inner size 1536 (48 heads of 32, 128 states)
GRANITE_TYPES = (["mamba"] * 10 + ["attention"] + ["mamba"] * 2 + ["attention"] + ["mamba"] * 3 + ["attention"] +
                 ["mamba"] * 9 + ["attention"] + ["mamba"] * 4)
GRANITE_350M = dict(arch="granitehybrid", hidden=768, layers=32, heads=12, kv_heads=4, head_dim=64, ffn=2048,
                    vocab=100352, context_length=32768, norm_eps=1e-5,
                    layer_kv_heads=[4 if t == "attention" else 0 for t in GRANITE_TYPES])

WORKLOADS: dict[str, Workload] = {
    w.name: w
    for w in [
        Workload("smollm2-135m-q4_k_m", SynthSpec(recipe="q4_k_m", **SMOLLM2), max_context=512, eos_ids=[2],
                 prompt_tokens=32, decode_tokens=128,
                 description="SmolLM2-135M-shaped llama decoder, Q4_K_M, 32-token prompt, greedy 128"),
        Workload("smollm2-135m-q8_0", SynthSpec(recipe="q8_0", **SMOLLM2), max_context=512, eos_ids=[2],
                 prompt_tokens=32, decode_tokens=128,
                 description="SmolLM2-135M-shaped llama decoder, Q8_0, 32-token prompt, greedy 128"),
        Workload("qwen3-0.6b-q4_k_m", SynthSpec(recipe="q4_k_m", **QWEN3), max_context=2048 + 256,
                 eos_ids=[151645, 151643], prompt_tokens=2048, decode_tokens=256,
                 description="Qwen3-0.6B-shaped decoder, Q4_K_M, 2048-token prompt, greedy 256, fp16 KV"),
        Workload("gemma3-270m-q4_k_m", SynthSpec(recipe="q4_k_m", **GEMMA3), max_context=1024 + 128,
                 eos_ids=[1, 106], prompt_tokens=1024, decode_tokens=128, temperature=0.8, top_k=40,
                 description="Gemma-3-270M-shaped decoder, Q4_K_M (Q8_0 lm_head), 1024-token prompt, "
                             "top-k 40 / T 0.8 sampling, 128 tokens"),
        Workload("gpt2-124m-q4_k_m", SynthSpec(arch="gpt2", recipe="q4_k_m", hidden=768, layers=12, heads=12,
                                               kv_heads=12, ffn=3072, vocab=50257, context_length=1024, seed=29),
                 max_context=1024, eos_ids=[50256], prompt_tokens=512, decode_tokens=128,
                 description="GPT-2-124M-shaped decoder (gpt2 runtime), Q4_K_M, 512-token prompt, greedy 128"),
        Workload("openelm-270m-q4_k_m", SynthSpec(recipe="q4_k_m", seed=37, **OPENELM_270M), max_context=512,
                 eos_ids=[2], prompt_tokens=32, decode_tokens=128,
                 description="OpenELM-270M-shaped decoder (fused q|k|v, per-layer heads 12-20 / kv heads 3-5 / "
                             "feed-forward 768-5120), Q4_K_M, 32-token prompt, greedy 128"),
        Workload("lfm2.5-350m-q4_k_m", SynthSpec(recipe="q4_k_m", seed=41, **LFM2_350M), max_context=4096,
                 eos_ids=[7, 2], prompt_tokens=32, decode_tokens=128,
                 description="LFM2.5-350M-shaped hybrid decoder (10 short-convolution and 6 attention layers, "
                             "lfm2 runtime), Q4_K_M, 32-token prompt, greedy 128"),
        Workload("lfm2.5-350m-q8_0", SynthSpec(recipe="q8_0", seed=41, **LFM2_350M), max_context=4096,
                 eos_ids=[7, 2], prompt_tokens=32, decode_tokens=128,
                 description="LFM2.5-350M-shaped hybrid decoder (lfm2 runtime), Q8_0, 32-token prompt, greedy 128"),
        Workload("granite-4.0-h-350m-q4_k_m", SynthSpec(recipe="q4_k_m", seed=53, **GRANITE_350M), max_context=4096,
                 eos_ids=[100257, 100265], prompt_tokens=32, decode_tokens=128,
                 description="Granite-4.0-H-350M-shaped hybrid decoder (28 Mamba2 and 4 attention layers, "
                             "granite runtime), Q4_K_M, 32-token prompt, greedy 128"),
        Workload("granite-4.0-h-350m-q8_0", SynthSpec(recipe="q8_0", seed=53, **GRANITE_350M), max_context=4096,
                 eos_ids=[100257, 100265], prompt_tokens=32, decode_tokens=128,
                 description="Granite-4.0-H-350M-shaped hybrid decoder (granite runtime), Q8_0, 32-token prompt, "
                             "greedy 128"),
        # small decoders for oracle parity (each exercises a different type mix)
        Workload("tiny-qwen3", SynthSpec(arch="qwen3", recipe="q4_k_m", hidden=256, layers=3, heads=4, kv_heads=2,
                                         head_dim=64, ffn=512, vocab=1200, context_length=4096,
                                         rope_theta=1000000.0, norm_eps=1e-6, seed=7),
                 max_context=160, eos_ids=[1199], prompt_tokens=24, decode_tokens=32),
        Workload("tiny-qwen3-hd128", SynthSpec(arch="qwen3", recipe="q4_k_m", hidden=256, layers=2, heads=4,
                                               kv_heads=2, head_dim=128, ffn=512, vocab=900, context_length=4096,
                                               rope_theta=1000000.0, norm_eps=1e-6, seed=19),
                 max_context=400, eos_ids=[899], prompt_tokens=150, decode_tokens=40),
        Workload("tiny-gpt2", SynthSpec(arch="gpt2", recipe="q4_k_m", hidden=256, layers=3, heads=4, kv_heads=4,
                                        ffn=1024, vocab=800, context_length=256, norm_eps=1e-5, seed=23),
                 max_context=160, eos_ids=[799], prompt_tokens=24, decode_tokens=24),
        Workload("tiny-llama", SynthSpec(arch="llama", recipe="q4_k_m", hidden=192, layers=3, heads=6, kv_heads=2,
                                         ffn=512, vocab=1000, context_length=4096, rope_theta=100000.0,
                                         norm_eps=1e-5, seed=11),
                 max_context=160, eos_ids=[2], prompt_tokens=24, decode_tokens=32),
        Workload("tiny-llama-q8", SynthSpec(arch="llama", recipe="q8_0", hidden=192, layers=2, heads=6, kv_heads=2,
                                            ffn=384, vocab=700, context_length=4096, rope_theta=100000.0,
                                            norm_eps=1e-5, seed=13),
                 max_context=160, eos_ids=[2], prompt_tokens=16, decode_tokens=24),
        Workload("tiny-openelm", SynthSpec(arch="openelm", recipe="q4_k_m", hidden=256, layers=4, heads=4,
                                           kv_heads=2, head_dim=64, ffn=768, vocab=1000, context_length=2048,
                                           rope_theta=10000.0, norm_eps=1e-6, seed=31,
                                           layer_heads=[2, 3, 4, 4], layer_kv_heads=[1, 1, 1, 2],
                                           layer_ffn=[256, 384, 512, 768]),
                 max_context=160, eos_ids=[2], prompt_tokens=24, decode_tokens=32),
        Workload("tiny-lfm2", SynthSpec(arch="lfm2", recipe="q4_k_m", hidden=256, layers=4, heads=4, kv_heads=2,
                                        head_dim=64, ffn=512, vocab=1024, context_length=4096,
                                        rope_theta=1000000.0, norm_eps=1e-5, seed=43, layer_kv_heads=[0, 2, 0, 2]),
                 max_context=160, eos_ids=[7, 2], prompt_tokens=24, decode_tokens=32),
        Workload("tiny-lfm2-q8", SynthSpec(arch="lfm2", recipe="q8_0", hidden=192, layers=3, heads=6, kv_heads=2,
                                           head_dim=32, ffn=384, vocab=700, context_length=4096,
                                           rope_theta=1000000.0, norm_eps=1e-5, seed=47, layer_kv_heads=[0, 0, 2]),
                 max_context=160, eos_ids=[7, 2], prompt_tokens=16, decode_tokens=24),
        Workload("tiny-granite", SynthSpec(arch="granitehybrid", recipe="q4_k_m", hidden=256, layers=4, heads=4,
                                           kv_heads=2, head_dim=64, ffn=512, vocab=1024, context_length=4096,
                                           norm_eps=1e-5, seed=59, layer_kv_heads=[0, 2, 0, 0]),
                 max_context=160, eos_ids=[7, 2], prompt_tokens=24, decode_tokens=32),
        Workload("tiny-granite-q8", SynthSpec(arch="granitehybrid", recipe="q8_0", hidden=192, layers=3, heads=3,
                                              kv_heads=1, head_dim=64, ffn=384, vocab=700, context_length=4096,
                                              norm_eps=1e-5, seed=61, layer_kv_heads=[0, 1, 0]),
                 max_context=160, eos_ids=[7, 2], prompt_tokens=16, decode_tokens=24),
        Workload("tiny-gemma3", SynthSpec(arch="gemma3", recipe="q4_k_m", hidden=320, layers=7, heads=4,
                                          kv_heads=1, head_dim=128, ffn=512, vocab=1500, context_length=4096,
                                          rope_theta=1000000.0, norm_eps=1e-6, sliding_window=16, seed=17),
                 max_context=96, eos_ids=[1, 106], prompt_tokens=40, decode_tokens=24, temperature=0.8, top_k=40),
        # long-context decode attention with 512-position windows (5 of 6 layers) past 8192
        # positions, where each attention workgroup walks several 64-position sub-chunks:
        # head_dim 256 with a 4-head group (Gemma-3's geometry) and head_dim 64
        Workload("tiny-gemma3-hd256", SynthSpec(arch="gemma3", recipe="q4_k_m", hidden=512, layers=6, heads=4,
                                                kv_heads=1, head_dim=256, ffn=512, vocab=1000, context_length=16384,
                                                rope_theta=1000000.0, norm_eps=1e-6, sliding_window=512, seed=71),
                 max_context=9000, eos_ids=[1, 106], prompt_tokens=16, decode_tokens=16),
        Workload("tiny-gemma3-hd64", SynthSpec(arch="gemma3", recipe="q4_k_m", hidden=256, layers=6, heads=8,
                                               kv_heads=2, head_dim=64, ffn=512, vocab=1000, context_length=16384,
                                               rope_theta=1000000.0, norm_eps=1e-6, sliding_window=512, seed=73),
                 max_context=9000, eos_ids=[1, 106], prompt_tokens=16, decode_tokens=16),
    ]
}
