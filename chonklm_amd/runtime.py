"""Host-side mirror of the reference's llama-webgpu runtime module API.

Reference: src/lib/llama-wgsl-runtime.ts
  loadLlamaWgslModel(model, onProgress?, onStep?)        :184-240  -> load_llama_wgsl_model
  generateLlamaWgsl(loaded, promptIds, opts)             :242-314  -> generate_llama_wgsl
  disposeLlamaWgsl(loaded)                               :316-318  -> dispose_llama_wgsl
  resetLlamaWgslConversation(loaded)                     :320-324  -> reset_llama_wgsl_conversation
  LlamaWgslEngine.runToken / reset / position / dispose  :1011-1215 -> LlamaWgslEngine
PleIAs aliases (src/lib/pleias-wgsl-runtime.ts:1-6) are exported under the
same names with the pleias prefix.

Everything below calls libchonk.so through its C ABI (include/chonk.h); there
is no other execution path. Token ids in, token ids out: text decoding is the
caller's tokenizer's job (the reference's tokenizer is not on this path), so
``text`` is produced only when a ``decode`` callable is supplied.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Callable, Optional, Sequence

import numpy as np

from . import _lib
from ._lib import ChonkError, check, lib
from .registry import ModelDef, Workload, WORKLOADS


def _i32_array(values: Sequence[int]):
    arr = (C.c_int32 * max(1, len(values)))(*values)
    return arr, len(values)


def _sampling(temperature=None, top_p=None, top_k=None, repetition_penalty=None, seed: int = 0) -> _lib.SamplingC:
    s = _lib.SamplingC()
    s.temperature = 0.0 if temperature is None else float(temperature)
    s.top_p = 1.0 if top_p is None else float(top_p)
    s.top_k = 0 if top_k is None or not np.isfinite(top_k) else int(max(0, int(top_k)))
    s.repetition_penalty = -1.0 if repetition_penalty is None else float(repetition_penalty)
    s.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    return s


class LlamaWgslEngine:
    """One decode engine on one GPU (LlamaWgslEngine, :619-1693)."""

    def __init__(self, model: ModelDef):
        L = lib()
        eos, n_eos = _i32_array(model.eos_ids)
        d = _lib.ModelDefC()
        d.id = model.id.encode()
        d.vocab = model.vocab
        d.layers = model.layers
        d.max_context = model.max_context
        d.eos_ids = C.cast(eos, C.POINTER(C.c_int32))
        d.n_eos = n_eos
        d.default_repetition_penalty = float(model.default_repetition_penalty or 0.0)
        d.kv_dtype = _lib.KV_F32 if model.kv_dtype == "f32" else _lib.KV_F16
        d.device = model.device
        handle = C.c_void_p()
        check(L.chonk_engine_create(C.byref(d), model.path.encode(), C.byref(handle)))
        self._h = handle
        self.model = model
        info = _lib.EngineInfoC()
        check(L.chonk_engine_info_get(self._h, C.byref(info)), self._h)
        self.info = {name: getattr(info, name) for name, _ in info._fields_}

    # -- reference API --------------------------------------------------------------
    def run_token(self, token_id: int, need_logits: bool, temperature=None, top_p=None, top_k=None,
                  repetition_penalty=None, penalized_token_ids: Optional[Sequence[int]] = None,
                  seen_ids: Optional[Sequence[int]] = None, seed: int = 0) -> int:
        s = _sampling(temperature, top_p, top_k, 1.0 if repetition_penalty is None else repetition_penalty, seed)
        pen, n_pen = _i32_array(penalized_token_ids or [])
        seen, n_seen = _i32_array(seen_ids or [])
        out = C.c_int32()
        check(lib().chonk_engine_run_token(self._h, int(token_id), 1 if need_logits else 0, C.byref(s),
                                           C.cast(pen, C.POINTER(C.c_int32)), n_pen,
                                           C.cast(seen, C.POINTER(C.c_int32)), n_seen, C.byref(out)), self._h)
        return int(out.value)

    def prefill(self, token_ids: Sequence[int]) -> None:
        """runToken(id, false) for every id, computed as row batches (no logits)."""
        arr, n = _i32_array(list(token_ids))
        check(lib().chonk_engine_prefill(self._h, C.cast(arr, C.POINTER(C.c_int32)), n), self._h)

    def prefill_noalloc(self, token_ids: Sequence[int]) -> None:
        """prefill() with the row buffers in the library's per-GPU scratch (no device
        allocation); at most info['noalloc_prefill_rows'] tokens per call."""
        arr, n = _i32_array(list(token_ids))
        check(lib().chonk_engine_prefill_noalloc(self._h, C.cast(arr, C.POINTER(C.c_int32)), n), self._h)

    def reset(self) -> None:
        check(lib().chonk_engine_reset(self._h), self._h)

    @property
    def position(self) -> int:
        v = C.c_int32()
        check(lib().chonk_engine_position(self._h, C.byref(v)), self._h)
        return int(v.value)

    def dispose(self) -> None:
        if self._h:
            check(lib().chonk_engine_destroy(self._h))
            self._h = None

    # -- additions for parity tests and measurement ---------------------------------
    def read_logits(self) -> np.ndarray:
        out = np.empty(self.info["vocab"], dtype=np.float32)
        check(lib().chonk_engine_read_logits(self._h, out.ctypes.data_as(C.POINTER(C.c_float)), out.size), self._h)
        return out

    def read_buffer(self, which: int) -> np.ndarray:
        i = self.info
        # lfm2 / granitehybrid: one slot per residue class
        slots = 256 if i["architecture"] in (5, 6) else (i["vocab"] + 255) // 256
        sizes = {0: i["hidden"] * 4, 1: i["heads"] * i["head_dim"] * 4, 2: slots * 8,
                 3: (i["heads"] + 2 * i["kv_heads"]) * i["head_dim"] * 4}
        buf = np.empty(sizes[which], dtype=np.uint8)
        check(lib().chonk_engine_read_buffer(self._h, which, buf.ctypes.data, buf.size), self._h)
        return buf.view(np.float32) if which != 2 else buf

    def read_kv(self, layer: int, is_value: bool, pos: int) -> np.ndarray:
        out = np.empty(self.info["kv_heads"] * self.info["head_dim"], dtype=np.float32)
        check(lib().chonk_engine_read_kv(self._h, layer, 1 if is_value else 0, pos,
                                         out.ctypes.data_as(C.POINTER(C.c_float))), self._h)
        return out

    def bench_kernel_cold(self, kernel_id: int, reps: int, flush_bytes: int = 768 << 20) -> tuple[float, float]:
        """(cold, warm) mean microseconds of one launch of a step kernel, caches flushed or not."""
        cold, warm = C.c_double(), C.c_double()
        check(lib().chonk_engine_bench_kernel_cold(self._h, kernel_id, reps, flush_bytes, C.byref(cold),
                                                   C.byref(warm)), self._h)
        return float(cold.value), float(warm.value)

    def fake_context(self, pos: int, seed: int = 1) -> None:
        check(lib().chonk_engine_fake_context(self._h, pos, seed), self._h)

    def bench_decode(self, warmup: int, steps: int) -> float:
        ms = C.c_double()
        check(lib().chonk_engine_bench_decode(self._h, warmup, steps, C.byref(ms)), self._h)
        return float(ms.value)

    def time_kernels(self, ids: list[int], rounds: int = 1) -> float:
        """Mean microseconds per launch of the step kernels `ids` launched back to back."""
        arr = (C.c_int32 * len(ids))(*ids)
        us = C.c_double()
        check(lib().chonk_engine_time_kernels(self._h, arr, len(ids), rounds, C.byref(us)), self._h)
        return float(us.value)

    def bench_kernel(self, kernel_id: int, reps: int) -> tuple[str, float, int]:
        us = C.c_double()
        name = C.create_string_buffer(64)
        nbytes = C.c_uint64()
        check(lib().chonk_engine_bench_kernel(self._h, kernel_id, reps, C.byref(us), name, 64, C.byref(nbytes)),
              self._h)
        return name.value.decode(), float(us.value), int(nbytes.value)

    def conversation(self) -> tuple[list[int], Optional[int]]:
        n = C.c_size_t()
        nxt = C.c_int32()
        check(lib().chonk_engine_conversation(self._h, None, 0, C.byref(n), C.byref(nxt)), self._h)
        buf = (C.c_int32 * max(1, n.value))()
        check(lib().chonk_engine_conversation(self._h, buf, n.value, C.byref(n), C.byref(nxt)), self._h)
        return list(buf[: n.value]), (None if nxt.value < 0 else int(nxt.value))

    def __del__(self):
        try:
            self.dispose()
        except Exception:
            pass


@dataclass
class LoadedLlamaWgslModel:
    """LoadedLlamaWgslModel (:174-182); ``ep`` names the execution provider."""

    def_: ModelDef
    engine: LlamaWgslEngine
    tokenizer: object = None
    runtime: str = "llama-webgpu"
    ep: str = "hip"
    cached_token_ids: list[int] = field(default_factory=list)
    cached_next_id: Optional[int] = None


def load_llama_wgsl_model(model: ModelDef, on_progress: Optional[Callable] = None,
                          on_step: Optional[Callable] = None, tokenizer: object = None) -> LoadedLlamaWgslModel:
    if model.runtime != "llama-webgpu":
        raise ValueError(f"loadLlamaWgslModel: {model.id} is not configured for the Llama WGSL runtime")
    if on_step:
        on_step({"step": "weights", "detail": "uploading GGUF tensors to the GPU"})
    engine = LlamaWgslEngine(model)
    arch = {3: "gpt2", 5: "lfm2", 6: "granitehybrid"}.get(engine.info["architecture"])
    if arch:
        engine.dispose()
        raise ValueError(f"Llama GGUF WGSL does not support architecture {arch}")
    if on_step:
        on_step({"step": "ready", "detail": "Llama HIP runtime ready"})
    return LoadedLlamaWgslModel(def_=model, engine=engine, tokenizer=tokenizer)


class LlamaWgslBatch:
    """Independent sequences decoded together over one engine's weights (no
    counterpart in the reference, which runs one sequence per engine): each
    sequence has its own paged fp16 K/V cache; a step appends one token to any
    subset of them and returns their greedy next ids (chonk_batch_*)."""

    def __init__(self, engine: LlamaWgslEngine, max_seqs: int, max_tokens: int):
        self.engine = engine
        self.vocab = engine.info["vocab"]
        h = C.c_void_p()
        check(lib().chonk_batch_create(engine._h, int(max_seqs), int(max_tokens), C.byref(h)), engine._h)
        self._h = h

    def prefill(self, seq: int, token_ids: Sequence[int]) -> int:
        arr, n = _i32_array(list(token_ids))
        out = C.c_int32()
        check(lib().chonk_batch_prefill(self._h, int(seq), C.cast(arr, C.POINTER(C.c_int32)), n, C.byref(out)),
              self.engine._h)
        return int(out.value)

    def step(self, seqs: Sequence[int], token_ids: Sequence[int]) -> list[int]:
        s_arr, n = _i32_array(list(seqs))
        t_arr, m = _i32_array(list(token_ids))
        if n != m:
            raise ValueError("seqs and token_ids differ in length")
        out = (C.c_int32 * max(1, n))()
        check(lib().chonk_batch_step(self._h, C.cast(s_arr, C.POINTER(C.c_int32)), C.cast(t_arr, C.POINTER(C.c_int32)),
                                     n, C.cast(out, C.POINTER(C.c_int32))), self.engine._h)
        return [int(out[i]) for i in range(n)]

    def position(self, seq: int) -> int:
        v = C.c_int32()
        check(lib().chonk_batch_position(self._h, int(seq), C.byref(v)))
        return int(v.value)

    def read_logits(self, row: int) -> np.ndarray:
        out = np.empty(self.vocab, dtype=np.float32)
        check(lib().chonk_batch_read_logits(self._h, int(row), out.ctypes.data_as(C.POINTER(C.c_float)), out.size),
              self.engine._h)
        return out

    def close(self) -> None:
        if self._h:
            check(lib().chonk_batch_destroy(self._h), self.engine._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def generate_llama_wgsl(loaded: LoadedLlamaWgslModel, prompt_ids: Sequence[int], max_new_tokens: Optional[int] = None,
                        temperature=None, top_p=None, top_k=None, repetition_penalty=None,
                        on_token: Optional[Callable[[dict], None]] = None,
                        should_stop: Optional[Callable[[], bool]] = None, seed: int = 0,
                        decode: Optional[Callable[[list[int]], str]] = None) -> dict:
    """generateLlamaWgsl (:242-314).

    Without callbacks the whole call runs on the device (no per-token host
    round trip). With ``on_token`` / ``should_stop`` the loop is stepped
    from the host as in the reference, one readback per token.
    """
    L = lib()
    eng = loaded.engine
    s = _sampling(temperature, top_p, top_k, repetition_penalty, seed)
    prompt, n_prompt = _i32_array(list(prompt_ids))
    # maxNewTokens ?? 128 (:255); the ABI takes a negative value for "not given"
    max_arg = -1 if max_new_tokens is None else max(0, int(max_new_tokens))
    cap = 128 if max_arg < 0 else max(1, max_arg)
    out = (C.c_int32 * cap)()
    n_out = C.c_size_t()
    stats = _lib.GenStatsC()
    generated: list[int] = []
    cumulative = [""]

    if on_token is None and should_stop is None:
        check(L.chonk_engine_generate(eng._h, C.cast(prompt, C.POINTER(C.c_int32)), n_prompt,
                                      max_arg, C.byref(s), out, cap, C.byref(n_out),
                                      C.byref(stats)), eng._h)
        generated = list(out[: n_out.value])
    else:
        def _cb(_user, event, token):
            if event == 0:
                return 1 if (should_stop and should_stop()) else 0
            generated.append(int(token))
            if on_token:
                text = decode(generated) if decode else ""
                piece = text[len(cumulative[0]):]
                cumulative[0] = text
                on_token({"id": int(token), "text": piece, "cumulative": text})
            return 0

        cb = _lib.TOKEN_CALLBACK(_cb)
        check(L.chonk_engine_generate_stepped(eng._h, C.cast(prompt, C.POINTER(C.c_int32)), n_prompt,
                                              max_arg, C.byref(s), C.cast(cb, C.c_void_p), None,
                                              out, cap, C.byref(n_out), C.byref(stats)), eng._h)
        generated = list(out[: n_out.value])
    loaded.cached_token_ids, loaded.cached_next_id = eng.conversation()
    text = decode(generated) if decode else ""
    return {"text": text, "ids": generated, "tokensPerSec": stats.tokens_per_sec,
            "prefillMs": stats.prefill_ms, "decodeMs": stats.decode_ms}


def dispose_llama_wgsl(loaded: LoadedLlamaWgslModel) -> None:
    loaded.engine.dispose()


def reset_llama_wgsl_conversation(loaded: LoadedLlamaWgslModel) -> None:
    check(lib().chonk_engine_reset_conversation(loaded.engine._h), loaded.engine._h)
    loaded.cached_token_ids = []
    loaded.cached_next_id = None


# ---- GPT-2 runtime (src/lib/gpt-wgsl-runtime.ts) ------------------------------------
# The same engine runs the gpt2 architecture (LayerNorm with bias, learned positions,
# biased linears, GELU-tanh MLP, clamped residual, its argmax rule and generate loop); the
# architecture comes from the GGUF file, the runtime tag from the model definition.

@dataclass
class LoadedGptWgslModel(LoadedLlamaWgslModel):
    """LoadedGptWgslModel (gpt-wgsl-runtime.ts:120-128)."""

    runtime: str = "gpt-webgpu"


def load_gpt_wgsl_model(model: ModelDef, on_progress: Optional[Callable] = None,
                        on_step: Optional[Callable] = None, tokenizer: object = None) -> LoadedGptWgslModel:
    """loadGptWgslModel (:130-180): rejects a definition not tagged for the GPT runtime and a
    GGUF file whose architecture is not gpt2."""
    if model.runtime != "gpt-webgpu":
        raise ValueError(f"loadGptWgslModel: unsupported model {model.id}")
    if on_step:
        on_step({"step": "weights", "detail": "uploading GGUF tensors to the GPU"})
    engine = LlamaWgslEngine(model)
    if engine.info["architecture"] != 3:
        engine.dispose()
        raise ValueError(f"loadGptWgslModel: {model.id} is not a gpt2 GGUF file")
    if on_step:
        on_step({"step": "ready", "detail": "GPT HIP runtime ready"})
    return LoadedGptWgslModel(def_=model, engine=engine, tokenizer=tokenizer)


def generate_gpt_wgsl(loaded: LoadedGptWgslModel, prompt_ids: Sequence[int], max_new_tokens: Optional[int] = None,
                      **kw) -> dict:
    """generateGptWgsl (:182-249): the engine follows the GPT loop (an empty suffix needs a
    cached next id; one more step runs after the last generated token)."""
    return generate_llama_wgsl(loaded, prompt_ids, max_new_tokens, **kw)


def reset_gpt_wgsl_conversation(loaded: LoadedGptWgslModel) -> None:
    """resetGptWgslConversation (:251-255)."""
    reset_llama_wgsl_conversation(loaded)


def dispose_gpt_wgsl(loaded: LoadedGptWgslModel) -> None:
    """disposeGptWgsl (:257-260)."""
    dispose_llama_wgsl(loaded)


# ---- LFM2 runtime (src/lib/lfm-wgsl-runtime.ts) -----------------------------------
# The same engine runs the lfm2 architecture (gated short-convolution layers beside
# GQA attention layers, the embedding as lm_head, TOPK256 candidates, its generate
# loop); the architecture comes from the GGUF file, the runtime tag from the model
# definition.

@dataclass
class LoadedLfmWgslModel(LoadedLlamaWgslModel):
    """LoadedLfmWgslModel (lfm-wgsl-runtime.ts:159-167)."""

    runtime: str = "lfm2-webgpu"


def load_lfm_wgsl_model(model: ModelDef, on_progress: Optional[Callable] = None,
                        on_step: Optional[Callable] = None, tokenizer: object = None) -> LoadedLfmWgslModel:
    """loadLfmWgslModel (:169-217): rejects a definition not tagged for the LFM runtime and
    a GGUF file whose architecture is not lfm2 (openGgufLfmSource, :318-322)."""
    if model.runtime != "lfm2-webgpu":
        raise ValueError(f"loadLfmWgslModel: unsupported model {model.id}")
    if on_step:
        on_step({"step": "weights", "detail": "uploading GGUF tensors to the GPU"})
    engine = LlamaWgslEngine(model)
    if engine.info["architecture"] != 5:
        arch = {0: "llama", 1: "qwen3", 2: "gemma3", 3: "gpt2", 4: "openelm"}.get(engine.info["architecture"])
        engine.dispose()
        raise ValueError(f"unsupported LFM GGUF architecture: {arch}")
    if on_step:
        on_step({"step": "ready", "detail": "LFM HIP runtime ready"})
    return LoadedLfmWgslModel(def_=model, engine=engine, tokenizer=tokenizer)


def generate_lfm_wgsl(loaded: LoadedLfmWgslModel, prompt_ids: Sequence[int], max_new_tokens: Optional[int] = None,
                      **kw) -> dict:
    """generateLfmWgsl (:219-306): the engine follows the LFM loop (one more step runs after
    the last generated token; repetitionPenalty defaults to 1, not to the definition's)."""
    return generate_llama_wgsl(loaded, prompt_ids, max_new_tokens, **kw)


def reset_lfm_wgsl_conversation(loaded: LoadedLfmWgslModel) -> None:
    """resetLfmWgslConversation (:312-316)."""
    reset_llama_wgsl_conversation(loaded)


def dispose_lfm_wgsl(loaded: LoadedLfmWgslModel) -> None:
    """disposeLfmWgsl (:308-310)."""
    dispose_llama_wgsl(loaded)


@dataclass
class LoadedGraniteWgslModel(LoadedLlamaWgslModel):
    """LoadedGraniteWgslModel (granite-wgsl-runtime.ts:158-166)."""

    runtime: str = "granite-webgpu"


def load_granite_wgsl_model(model: ModelDef, on_progress: Optional[Callable] = None,
                            on_step: Optional[Callable] = None, tokenizer: object = None) -> LoadedGraniteWgslModel:
    """loadGraniteWgslModel (:168-221): rejects a definition not tagged for the Granite runtime
    and a GGUF file whose architecture is not granitehybrid (validateGraniteGguf, :359-371)."""
    if model.runtime != "granite-webgpu":
        raise ValueError(f"loadGraniteWgslModel: unsupported model {model.id}")
    if on_step:
        on_step({"step": "weights", "detail": "uploading GGUF tensors to the GPU"})
    engine = LlamaWgslEngine(model)
    if engine.info["architecture"] != 6:
        arch = {0: "llama", 1: "qwen3", 2: "gemma3", 3: "gpt2", 4: "openelm", 5: "lfm2"}.get(engine.info["architecture"])
        engine.dispose()
        raise ValueError(f"Granite WGSL {model.id}: expected GGUF architecture granitehybrid, got {arch}")
    if on_step:
        on_step({"step": "ready", "detail": "Granite HIP runtime ready"})
    return LoadedGraniteWgslModel(def_=model, engine=engine, tokenizer=tokenizer)


def generate_granite_wgsl(loaded: LoadedGraniteWgslModel, prompt_ids: Sequence[int],
                          max_new_tokens: Optional[int] = None, **kw) -> dict:
    """generateGraniteWgsl (:223-292): the engine follows the Granite loop (one more step runs
    after the last generated token; repetitionPenalty defaults to 1, not to the definition's)."""
    return generate_llama_wgsl(loaded, prompt_ids, max_new_tokens, **kw)


def reset_granite_wgsl_conversation(loaded: LoadedGraniteWgslModel) -> None:
    """resetGraniteWgslConversation (:298-302)."""
    reset_llama_wgsl_conversation(loaded)


def dispose_granite_wgsl(loaded: LoadedGraniteWgslModel) -> None:
    """disposeGraniteWgsl (:294-296)."""
    dispose_llama_wgsl(loaded)


# PleIAs aliases (src/lib/pleias-wgsl-runtime.ts:1-6)
load_pleias_wgsl_model = load_llama_wgsl_model
generate_pleias_wgsl = generate_llama_wgsl
dispose_pleias_wgsl = dispose_llama_wgsl


# ---- model files ------------------------------------------------------------------

def write_synthetic_gguf(workload: Workload | str, path: str, threads: int = 8) -> str:
    w = WORKLOADS[workload] if isinstance(workload, str) else workload
    sp = w.spec
    c = _lib.SynthConfigC()
    c.arch = sp.arch.encode()
    c.recipe = sp.recipe.encode()
    c.hidden, c.layers, c.heads, c.kv_heads = sp.hidden, sp.layers, sp.heads, sp.kv_heads
    c.head_dim, c.ffn, c.vocab, c.context_length = sp.head_dim, sp.ffn, sp.vocab, sp.context_length
    c.rope_theta, c.norm_eps, c.sliding_window, c.seed = sp.rope_theta, sp.norm_eps, sp.sliding_window, sp.seed
    keep = []
    for fld in ("layer_heads", "layer_kv_heads", "layer_ffn"):
        vals = getattr(sp, fld)
        if vals is not None:
            arr = (C.c_int32 * len(vals))(*vals)
            keep.append(arr)
            setattr(c, fld, C.cast(arr, C.POINTER(C.c_int32)))
    check(lib().chonk_write_synthetic_gguf(C.byref(c), str(path).encode(), int(threads)))
    return str(path)


def shard_gguf(gguf_path: str, out_dir: str, shard_size: int = 24 * 1024 * 1024, quant: str = "") -> str:
    """scripts/shard-gguf.mjs: <out_dir>/NNNN.bin + manifest.json (24 MiB default shards)."""
    check(lib().chonk_write_shards(str(gguf_path).encode(), str(out_dir).encode(), int(shard_size), quant.encode()))
    return str(out_dir)


__all__ = [
    "ChonkError", "LlamaWgslEngine", "LoadedLlamaWgslModel", "ModelDef", "load_llama_wgsl_model",
    "generate_llama_wgsl", "dispose_llama_wgsl", "LlamaWgslBatch", "reset_llama_wgsl_conversation", "write_synthetic_gguf",
    "shard_gguf", "LoadedLfmWgslModel", "load_lfm_wgsl_model", "generate_lfm_wgsl", "reset_lfm_wgsl_conversation",
    "dispose_lfm_wgsl", "LoadedGraniteWgslModel", "load_granite_wgsl_model", "generate_granite_wgsl",
    "reset_granite_wgsl_conversation", "dispose_granite_wgsl",
]
