"""ORACLE — TEST INFRASTRUCTURE ONLY.

ctypes wrapper of oracle/_build/liborc.so, the CPU restatement of the
reference's llama-webgpu decode path (see oracle.h). Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use it; it is the
checker, never the thing measured or shipped.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path
from typing import Callable, Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liborc.so"

GGML = {"F32": 0, "F16": 1, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}
BLOCK = {0: (1, 4), 1: (1, 2), 6: (32, 22), 7: (32, 24), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


class _Def(C.Structure):
    _fields_ = [("vocab", C.c_int32), ("layers", C.c_int32), ("max_context", C.c_int32), ("kv_f16", C.c_int32),
                ("n_threads", C.c_int32)]


class _Samp(C.Structure):
    _fields_ = [("temperature", C.c_double), ("top_p", C.c_double), ("top_k", C.c_int32),
                ("repetition_penalty", C.c_double)]


_L = None


def lib():
    global _L
    if _L is None:
        if not LIB_PATH.exists():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        L = C.CDLL(str(LIB_PATH))
        P = C.c_void_p
        I32P = C.POINTER(C.c_int32)
        L.orc_dequant.argtypes = [C.c_uint32, P, C.c_int64, P]
        L.orc_matvec.argtypes = [C.c_uint32, P, C.c_int64, C.c_int64, P, P, C.c_int]
        L.orc_decode_rows.argtypes = [C.c_uint32, P, C.c_int64, C.c_int64, P]
        L.orc_model_load.restype = P
        L.orc_model_load.argtypes = [C.c_char_p, C.POINTER(_Def), C.c_char_p, C.c_size_t]
        L.orc_model_free.argtypes = [P]
        L.orc_model_context.argtypes = [P]
        L.orc_model_is_gpt.argtypes = [P]
        L.orc_model_is_lfm.argtypes = [P]
        L.orc_model_is_granite.argtypes = [P]
        L.orc_lfm_select.argtypes = [P, C.c_int64, P, I32P]
        L.orc_model_vocab.argtypes = [P]
        L.orc_model_position.argtypes = [P]
        L.orc_model_reset.argtypes = [P]
        L.orc_model_run_token.argtypes = [P, C.c_int32, C.c_int32, C.POINTER(_Samp), I32P, C.c_int64, I32P,
                                          C.c_int64, C.c_double, I32P, C.c_char_p, C.c_size_t]
        L.orc_model_read.argtypes = [P, C.c_int, P, C.c_int64]
        L.orc_model_read_kv.argtypes = [P, C.c_int, C.c_int, C.c_int, P]
        L.orc_model_fake_context.argtypes = [P, C.c_int, C.c_uint64]
        L.orc_sample_candidates.restype = C.c_int32
        L.orc_sample_candidates.argtypes = [P, C.c_int64, C.POINTER(_Samp), I32P, C.c_int64, C.c_double]
        L.orc_argmax.argtypes = [P, C.c_int64, I32P, C.c_int64, C.c_double, P, I32P]
        L.orc_argmax_gpt.argtypes = [P, C.c_int64, I32P, C.c_int64, C.c_double, P, I32P]
        L.orc_uniform.restype = C.c_double
        L.orc_uniform.argtypes = [C.c_uint64, C.c_uint64]
        _L = L
    return _L


def dequant(type_id: int, blocks: bytes | np.ndarray, n: int) -> np.ndarray:
    raw = np.frombuffer(bytes(blocks), dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if lib().orc_dequant(type_id, raw.ctypes.data, n, out.ctypes.data) != 0:
        raise ValueError("bad dequant arguments")
    return out


def decode_rows(type_id: int, blocks: bytes | np.ndarray, n_rows: int, row_len: int) -> np.ndarray:
    """Row-wise block decode used inside the oracle's matvec (must equal dequant)."""
    raw = np.frombuffer(bytes(blocks), dtype=np.uint8)
    out = np.empty(n_rows * row_len, dtype=np.float32)
    if lib().orc_decode_rows(type_id, raw.ctypes.data, n_rows, row_len, out.ctypes.data) != 0:
        raise ValueError("bad decode arguments")
    return out


def matvec(type_id: int, blocks: bytes | np.ndarray, n_rows: int, row_len: int, x: np.ndarray,
           threads: int = 8) -> np.ndarray:
    raw = np.frombuffer(bytes(blocks), dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n_rows, dtype=np.float32)
    if lib().orc_matvec(type_id, raw.ctypes.data, n_rows, row_len, x.ctypes.data, y.ctypes.data, threads) != 0:
        raise ValueError("bad matvec arguments")
    return y


def argmax(logits: np.ndarray, penalized: Sequence[int] = (), repetition_penalty: float = 1.0):
    """(token, candidate pairs as uint8[groups*8])."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    groups = (lg.size + 255) // 256
    pairs = np.zeros(groups * 8, dtype=np.uint8)
    arr = (C.c_int32 * max(1, len(penalized)))(*penalized)
    tok = C.c_int32()
    lib().orc_argmax(lg.ctypes.data, lg.size, arr, len(penalized), repetition_penalty, pairs.ctypes.data,
                     C.byref(tok))
    return int(tok.value), pairs


def argmax_gpt(logits: np.ndarray, penalized: Sequence[int] = (), repetition_penalty: float = 1.0):
    """The GPT-2 runtime's argmax: (token, candidate pairs as uint8[groups*8])."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    groups = (lg.size + 255) // 256
    pairs = np.zeros(groups * 8, dtype=np.uint8)
    arr = (C.c_int32 * max(1, len(penalized)))(*penalized)
    tok = C.c_int32()
    if lib().orc_argmax_gpt(lg.ctypes.data, lg.size, arr, len(penalized), repetition_penalty, pairs.ctypes.data,
                            C.byref(tok)) != 0:
        raise ValueError("vocab outside 1..65536")
    return int(tok.value), pairs


def lfm_select(logits: np.ndarray):
    """The LFM runtime's TOPK256 / ARGMAX: (greedy token, 256 candidate pairs as uint8[2048])."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    pairs = np.zeros(256 * 8, dtype=np.uint8)
    tok = C.c_int32()
    lib().orc_lfm_select(lg.ctypes.data, lg.size, pairs.ctypes.data, C.byref(tok))
    return int(tok.value), pairs


def uniform(seed: int, step: int) -> float:
    return float(lib().orc_uniform(seed & 0xFFFFFFFFFFFFFFFF, step))


def sample_candidates(pairs: np.ndarray, temperature: float, top_p: float, top_k: int, repetition_penalty: float,
                      seen: Sequence[int], u: float) -> int:
    raw = np.ascontiguousarray(pairs).view(np.uint8)
    s = _Samp(temperature, top_p, top_k, repetition_penalty)
    arr = (C.c_int32 * max(1, len(seen)))(*seen)
    return int(lib().orc_sample_candidates(raw.ctypes.data, raw.size // 8, C.byref(s), arr, len(seen), u))


class OracleModel:
    """CPU restatement of LlamaWgslEngine + generateLlamaWgsl, for a gpt2 GGUF
    of GptWgslEngine + generateGptWgsl (gpt-wgsl-runtime.ts), for an lfm2 GGUF
    of LfmWgslEngine + generateLfmWgsl (lfm-wgsl-runtime.ts), for a
    granitehybrid GGUF of GraniteWgslEngine + generateGraniteWgsl
    (granite-wgsl-runtime.ts)."""

    def __init__(self, path: str, vocab: int, layers: int, max_context: int, kv_f16: bool = True,
                 threads: int = 8, eos_ids: Sequence[int] = (), default_repetition_penalty: Optional[float] = None):
        err = C.create_string_buffer(512)
        d = _Def(vocab, layers, max_context, 1 if kv_f16 else 0, threads)
        self._h = lib().orc_model_load(str(path).encode(), C.byref(d), err, 512)
        if not self._h:
            raise RuntimeError(err.value.decode())
        self.gpt = bool(lib().orc_model_is_gpt(self._h))
        self.lfm = bool(lib().orc_model_is_lfm(self._h))
        self.granite = bool(lib().orc_model_is_granite(self._h))
        self.vocab = int(lib().orc_model_vocab(self._h))
        self.max_context = max_context
        self.eos_ids = set(eos_ids)
        self.default_repetition_penalty = default_repetition_penalty
        self.cached_token_ids: list[int] = []
        self.cached_next_id: Optional[int] = None

    def close(self):
        if self._h:
            lib().orc_model_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def position(self) -> int:
        return int(lib().orc_model_position(self._h))

    @property
    def context(self) -> int:
        return int(lib().orc_model_context(self._h))

    def reset(self) -> None:
        lib().orc_model_reset(self._h)

    def fake_context(self, pos: int, seed: int = 1) -> None:
        lib().orc_model_fake_context(self._h, pos, seed)

    def run_token(self, token: int, need_logits: bool, temperature: float = 0.0, top_p: float = 1.0,
                  top_k: int = 0, repetition_penalty: float = 1.0, penalized: Sequence[int] = (),
                  seen: Sequence[int] = (), seed: int = 0) -> int:
        s = _Samp(temperature, top_p, top_k, repetition_penalty)
        pen = (C.c_int32 * max(1, len(penalized)))(*penalized)
        sn = (C.c_int32 * max(1, len(seen)))(*seen)
        u = uniform(seed, self.position)
        out = C.c_int32()
        err = C.create_string_buffer(512)
        rc = lib().orc_model_run_token(self._h, int(token), 1 if need_logits else 0, C.byref(s), pen, len(penalized),
                                       sn, len(seen), u, C.byref(out), err, 512)
        if rc != 0:
            raise RuntimeError(err.value.decode())
        return int(out.value)

    def read(self, which: int, n: int, dtype=np.float32) -> np.ndarray:
        buf = np.empty(n, dtype=dtype)
        got = lib().orc_model_read(self._h, which, buf.ctypes.data, buf.nbytes)
        if got < 0:
            raise ValueError("bad buffer id or size")
        return buf

    def logits(self) -> np.ndarray:
        return self.read(0, self.vocab)

    def read_kv(self, layer: int, is_value: bool, pos: int, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        if lib().orc_model_read_kv(self._h, layer, 1 if is_value else 0, pos, out.ctypes.data) != 0:
            raise ValueError("bad layer/position")
        return out

    def generate(self, prompt_ids: Sequence[int], max_new_tokens: Optional[int] = None, temperature=None,
                 top_p=None, top_k=None, repetition_penalty=None, seed: int = 0,
                 margins: Optional[list] = None,
                 on_logits: Optional[Callable[[int, np.ndarray], None]] = None) -> list[int]:
        """generateLlamaWgsl (llama-wgsl-runtime.ts:242-314); generateGptWgsl
        (gpt-wgsl-runtime.ts:182-249) for gpt2, which also runs the token after
        the last generated one and refuses an empty prompt with no cached token;
        generateLfmWgsl (lfm-wgsl-runtime.ts:219-306) for lfm2 and
        generateGraniteWgsl (granite-wgsl-runtime.ts:223-292) for granitehybrid,
        which run the token after the last generated one, start an empty prompt
        with no cached token from id 0 and ignore the definition's default
        penalty. ``on_logits(i, logits)`` sees the logits that pick generated
        id i (i = 0: those of the last prompt token)."""
        prompt = list(prompt_ids)
        mx = min(128 if max_new_tokens is None else max_new_tokens, self.max_context - len(prompt))
        t = 0.0 if temperature is None else temperature
        tp = 1.0 if top_p is None else top_p
        tk = 0 if top_k is None else top_k
        rp = repetition_penalty if repetition_penalty is not None else (
            1.0 if self.lfm or self.granite else (self.default_repetition_penalty or 1.0))
        n = 0
        while n < min(len(self.cached_token_ids), len(prompt)) and self.cached_token_ids[n] == prompt[n]:
            n += 1
        prefix = n
        if prefix != len(self.cached_token_ids):
            self.reset()
            self.cached_token_ids = []
            self.cached_next_id = None
            prefix = 0
        suffix = prompt[prefix:]
        next_id = 0
        if not suffix and self.gpt and self.cached_next_id is None:
            raise RuntimeError("GPT WGSL has no cached next token for an empty prompt")
        if not suffix and self.cached_next_id is not None:
            next_id = self.cached_next_id
        else:
            for i, tok in enumerate(suffix):
                need = i == len(suffix) - 1
                ids = prompt[: prefix + i + 1] if need else []
                next_id = self.run_token(tok, need, t, tp, tk, rp, ids, ids, seed)
                if need and margins is not None:
                    margins.append(self._margin())
                if need and on_logits is not None:
                    on_logits(0, self.logits())
        generated: list[int] = []
        for step in range(mx):
            generated.append(next_id)
            if next_id in self.eos_ids:
                break
            if step + 1 >= mx and not self.gpt and not self.lfm and not self.granite:
                break
            ids = prompt + generated
            next_id = self.run_token(next_id, True, t, tp, tk, rp, ids, ids, seed)
            if margins is not None:
                margins.append(self._margin())
            if on_logits is not None:
                on_logits(step + 1, self.logits())
        self.cached_token_ids = prompt + generated
        self.cached_next_id = None if (generated and generated[-1] in self.eos_ids) else next_id
        return generated

    def _margin(self) -> float:
        lg = self.logits()
        top2 = np.partition(lg, -2)[-2:]
        return float(abs(top2[1] - top2[0]))
