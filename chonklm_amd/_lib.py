"""ctypes binding of libchonk.so (include/chonk.h).

The library is the product: there is no fallback. Loading fails loudly when
``chonklm_amd/_lib/libchonk.so`` has not been built.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libchonk.so"

CHONK_OK = 0
CHONK_EINVAL = -1
CHONK_EIO = -2
CHONK_EHIP = -3
CHONK_ECONTEXT = -4
CHONK_EBUSY = -5
CHONK_ELOST = -6
CHONK_ENOMEM = -7
KV_F16 = 0
KV_F32 = 1

STATUS_NAMES = {
    CHONK_EINVAL: "EINVAL",
    CHONK_EIO: "EIO",
    CHONK_EHIP: "EHIP",
    CHONK_ECONTEXT: "ECONTEXT",
    CHONK_EBUSY: "EBUSY",
    CHONK_ELOST: "ELOST",
    CHONK_ENOMEM: "ENOMEM",
}


class ModelDefC(C.Structure):
    _fields_ = [
        ("id", C.c_char_p),
        ("vocab", C.c_int32),
        ("layers", C.c_int32),
        ("max_context", C.c_int32),
        ("eos_ids", C.POINTER(C.c_int32)),
        ("n_eos", C.c_int32),
        ("default_repetition_penalty", C.c_float),
        ("kv_dtype", C.c_int32),
        ("device", C.c_int32),
    ]


class SamplingC(C.Structure):
    _fields_ = [
        ("temperature", C.c_double),
        ("top_p", C.c_double),
        ("top_k", C.c_int32),
        ("repetition_penalty", C.c_double),
        ("seed", C.c_uint64),
    ]


class EngineInfoC(C.Structure):
    _fields_ = [
        ("hidden", C.c_int32),
        ("ffn", C.c_int32),
        ("vocab", C.c_int32),
        ("layers", C.c_int32),
        ("heads", C.c_int32),
        ("kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("context", C.c_int32),
        ("architecture", C.c_int32),
        ("qk_norm", C.c_int32),
        ("interleaved_rope", C.c_int32),
        ("kv_dtype", C.c_int32),
        ("weight_bytes_per_token", C.c_uint64),
        ("device_bytes", C.c_uint64),
        ("kernels_per_step", C.c_int32),
        ("persistent_step", C.c_int32),
        ("noalloc_prefill_rows", C.c_int32),
        ("spin_attention", C.c_int32),
        ("fused_attention", C.c_int32),
    ]


class GenStatsC(C.Structure):
    _fields_ = [
        ("prefill_ms", C.c_double),
        ("decode_ms", C.c_double),
        ("prompt_tokens", C.c_int32),
        ("generated_tokens", C.c_int32),
        ("tokens_per_sec", C.c_double),
    ]


class SynthConfigC(C.Structure):
    _fields_ = [
        ("arch", C.c_char_p),
        ("recipe", C.c_char_p),
        ("hidden", C.c_int32),
        ("layers", C.c_int32),
        ("heads", C.c_int32),
        ("kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("ffn", C.c_int32),
        ("vocab", C.c_int32),
        ("context_length", C.c_int32),
        ("rope_theta", C.c_float),
        ("norm_eps", C.c_float),
        ("sliding_window", C.c_int32),
        ("seed", C.c_uint64),
        ("weight_std", C.c_float),
        ("norm_std", C.c_float),
        ("layer_heads", C.POINTER(C.c_int32)),
        ("layer_kv_heads", C.POINTER(C.c_int32)),
        ("layer_ffn", C.POINTER(C.c_int32)),
    ]


P = C.c_void_p
I32P = C.POINTER(C.c_int32)
TOKEN_CALLBACK = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_int32, C.c_int32)
F32P = C.POINTER(C.c_float)

# (name, restype, argtypes) for every symbol declared in include/chonk.h
SIGNATURES = [
    ("chonk_last_error", C.c_char_p, []),
    ("chonk_engine_last_error", C.c_char_p, [P]),
    ("chonk_engine_create", C.c_int, [C.POINTER(ModelDefC), C.c_char_p, C.POINTER(P)]),
    ("chonk_engine_create_from_memory", C.c_int, [C.POINTER(ModelDefC), P, C.c_size_t, C.POINTER(P)]),
    ("chonk_engine_destroy", C.c_int, [P]),
    ("chonk_engine_info_get", C.c_int, [P, C.POINTER(EngineInfoC)]),
    ("chonk_engine_run_token", C.c_int,
     [P, C.c_int32, C.c_int32, C.POINTER(SamplingC), I32P, C.c_size_t, I32P, C.c_size_t, I32P]),
    ("chonk_engine_generate", C.c_int,
     [P, I32P, C.c_size_t, C.c_int32, C.POINTER(SamplingC), I32P, C.c_size_t, C.POINTER(C.c_size_t),
      C.POINTER(GenStatsC)]),
    ("chonk_engine_generate_stepped", C.c_int,
     [P, I32P, C.c_size_t, C.c_int32, C.POINTER(SamplingC), P, P, I32P, C.c_size_t, C.POINTER(C.c_size_t),
      C.POINTER(GenStatsC)]),
    ("chonk_engine_prefill", C.c_int, [P, I32P, C.c_size_t]),
    ("chonk_engine_prefill_noalloc", C.c_int, [P, I32P, C.c_size_t]),
    ("chonk_engine_conversation", C.c_int, [P, I32P, C.c_size_t, C.POINTER(C.c_size_t), I32P]),
    ("chonk_engine_reset", C.c_int, [P]),
    ("chonk_engine_debug_fail_next_launch", C.c_int, [P]),
    ("chonk_engine_reset_conversation", C.c_int, [P]),
    ("chonk_engine_position", C.c_int, [P, I32P]),
    ("chonk_engine_read_logits", C.c_int, [P, F32P, C.c_size_t]),
    ("chonk_engine_read_buffer", C.c_int, [P, C.c_int32, P, C.c_size_t]),
    ("chonk_engine_read_kv", C.c_int, [P, C.c_int32, C.c_int32, C.c_int32, F32P]),
    ("chonk_engine_bench_decode", C.c_int, [P, C.c_int32, C.c_int32, C.POINTER(C.c_double)]),
    ("chonk_batch_create", C.c_int, [P, C.c_int32, C.c_int32, C.POINTER(P)]),
    ("chonk_batch_destroy", C.c_int, [P]),
    ("chonk_batch_prefill", C.c_int, [P, C.c_int32, I32P, C.c_size_t, I32P]),
    ("chonk_batch_step", C.c_int, [P, I32P, I32P, C.c_size_t, I32P]),
    ("chonk_batch_position", C.c_int, [P, C.c_int32, I32P]),
    ("chonk_batch_read_logits", C.c_int, [P, C.c_int32, F32P, C.c_size_t]),
    ("chonk_engine_time_kernels", C.c_int, [P, I32P, C.c_int32, C.c_int32, C.POINTER(C.c_double)]),
    ("chonk_engine_bench_kernel", C.c_int,
     [P, C.c_int32, C.c_int32, C.POINTER(C.c_double), C.c_char_p, C.c_size_t, C.POINTER(C.c_uint64)]),
    ("chonk_engine_fake_context", C.c_int, [P, C.c_int32, C.c_uint64]),
    ("chonk_engine_bench_kernel_cold", C.c_int,
     [P, C.c_int32, C.c_int32, C.c_uint64, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    ("chonk_dequant", C.c_int, [C.c_int32, C.c_uint32, P, C.c_int64, C.c_int64, F32P]),
    ("chonk_matvec", C.c_int,
     [C.c_int32, C.c_uint32, P, C.c_int64, C.c_int64, F32P, F32P, C.c_int32, C.POINTER(C.c_double)]),
    ("chonk_gemm", C.c_int,
     [C.c_int32, C.c_uint32, P, C.c_int64, C.c_int64, F32P, C.c_int64, F32P, C.c_int32, C.POINTER(C.c_double)]),
    ("chonk_write_synthetic_gguf", C.c_int, [C.POINTER(SynthConfigC), C.c_char_p, C.c_int32]),
    ("chonk_write_shards", C.c_int, [C.c_char_p, C.c_char_p, C.c_uint64, C.c_char_p]),
]


class ChonkError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status
        self.status_name = STATUS_NAMES.get(status, str(status))


_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    """Loads libchonk.so once; raises if it is missing."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m chonklm_amd.build` (hipcc, gfx950)")
        handle = C.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(status: int, engine: C.c_void_p | None = None) -> None:
    if status == CHONK_OK:
        return
    L = lib()
    msg = L.chonk_engine_last_error(engine) if engine else L.chonk_last_error()
    raise ChonkError(status, (msg or b"").decode("utf-8", "replace"))
