"""The C ABI without a GPU: exports, host mirror completeness, error paths.

Every function declared in include/chonk.h must be exported by
chonklm_amd/_lib/libchonk.so and described in the ctypes table of
chonklm_amd/_lib.py. Engine creation fails with the reference's error text
before any device call when the file is missing, is not GGUF, or declares an
architecture the llama runtime rejects (llama-wgsl-runtime.ts:331-332).
"""
from __future__ import annotations

import ctypes as C
import re
import struct
from pathlib import Path

import pytest

from chonklm_amd import _lib
from chonklm_amd._lib import lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "chonk.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(chonk_\w+)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if not n.endswith("_t")))


def test_header_declares_the_engine_api():
    names = declared_functions()
    for must in ("chonk_engine_create", "chonk_engine_run_token", "chonk_engine_generate", "chonk_engine_reset",
                 "chonk_engine_position", "chonk_engine_read_logits", "chonk_engine_destroy", "chonk_last_error"):
        assert must in names


@pytest.mark.parametrize("name", declared_functions())
def test_library_exports(name):
    assert hasattr(lib(), name), f"{name} declared in chonk.h but not exported"


def test_ctypes_table_covers_header():
    table = {s[0] for s in _lib.SIGNATURES}
    assert set(declared_functions()) <= table


def _def(vocab=1000, ctx=64):
    d = _lib.ModelDefC()
    d.id = b"t"
    d.vocab = vocab
    d.layers = 2
    d.max_context = ctx
    d.n_eos = 0
    d.default_repetition_penalty = 1.0
    d.kv_dtype = _lib.KV_F16
    d.device = 0
    return d


def _create(path: str):
    h = C.c_void_p()
    rc = lib().chonk_engine_create(C.byref(_def()), str(path).encode(), C.byref(h))
    return rc, lib().chonk_last_error().decode()


def test_missing_file_is_eio(tmp_path):
    rc, msg = _create(tmp_path / "nope.gguf")
    assert rc == _lib.CHONK_EIO and "nope.gguf" in msg


def test_not_gguf_is_rejected(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"NOTGGUF" + bytes(100))
    rc, msg = _create(p)
    assert rc == _lib.CHONK_EINVAL and "could not parse GGUF header" in msg


def _gguf_with_arch(arch: str) -> bytes:
    def s(x: str) -> bytes:
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    kv = s("general.architecture") + struct.pack("<I", 8) + s(arch)
    head = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + kv
    return head + bytes(4096 - len(head))


def test_unsupported_architecture(tmp_path):
    p = tmp_path / "arch.gguf"
    p.write_bytes(_gguf_with_arch("mamba"))
    rc, msg = _create(p)
    assert rc == _lib.CHONK_EINVAL and "does not support architecture mamba" in msg


def test_null_arguments():
    assert lib().chonk_engine_destroy(None) == 0
    h = C.c_void_p()
    assert lib().chonk_engine_create(C.byref(_def()), None, C.byref(h)) == _lib.CHONK_EINVAL


def test_shard_size_mismatch_uses_the_reference_wording(synth, tmp_path):
    """A shard whose byte size differs from its manifest entry is refused before any device
    work, with fetchShardCached's message (cache.ts:568-573)."""
    from chonklm_amd import shard_gguf

    out = tmp_path / "shards"
    shard_gguf(synth("tiny-qwen3"), str(out), shard_size=65536)
    victim = sorted(out.glob("*.bin"))[1]
    size = victim.stat().st_size
    victim.write_bytes(victim.read_bytes()[: size - 10])
    rc, msg = _create(out)
    assert rc == _lib.CHONK_EIO
    assert f"shard {victim}: expected {size} bytes, got {size - 10}" in msg

