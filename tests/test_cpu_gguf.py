"""GGUF writing/reading, the Q4_K_M type recipe and shard manifests (host code only).

The synthetic writer (chonklm_amd/csrc/host/synth.cpp) and the sharder
(chonklm_amd/csrc/host/gguf.cpp, the scripts/shard-gguf.mjs:102-167 format)
are checked through an independent Python GGUF reader (tests/ggufpy.py): the
header fields the reference reads (src/lib/gguf.ts:42-130, data offset
aligned to 32), tensor byte lengths per block type, the llama.cpp Q4_K_M
type choices, the weight statistics of the seeded init, and the byte-exact
reassembly of shards.
"""
from __future__ import annotations

import json
import os
from pathlib import Path

import numpy as np
import pytest

from chonklm_amd import WORKLOADS, shard_gguf
from tests import ggufpy

BLOCK = {0: (1, 4), 1: (1, 2), 6: (32, 22), 7: (32, 24), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def use_more_bits(i: int, n: int) -> bool:
    # llama.cpp llama_tensor_get_type, Q4_K_M: attn_v / ffn_down layers that keep Q6_K
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


def q4_k_m_type(role: str, layer: int, n_layers: int, row_len: int) -> int:
    t = 12
    if role == "output":
        return 8 if row_len % 256 else 14
    if role in ("attn_v", "ffn_down") and use_more_bits(layer, n_layers):
        t = 14
    if row_len % 256:
        t = {12: 6, 14: 8}[t]
    return t


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama", "tiny-gemma3", "tiny-llama-q8"])
def test_header_and_tensor_table(name, synth):
    w = WORKLOADS[name]
    sp = w.spec
    path = synth(name)
    g = ggufpy.read_gguf(path)
    a = g.kv["general.architecture"]
    assert a == sp.arch
    assert g.kv[a + ".block_count"] == sp.layers and g.kv[a + ".embedding_length"] == sp.hidden
    assert g.kv[a + ".attention.head_count"] == sp.heads and g.kv[a + ".attention.head_count_kv"] == sp.kv_heads
    assert g.kv[a + ".feed_forward_length"] == sp.ffn
    assert g.data_offset % 32 == 0
    size = os.path.getsize(path)
    for t in g.tensors.values():
        be, bb = BLOCK[t.type]
        n = int(np.prod(t.shape))
        assert n % be == 0
        assert t.offset % 32 == 0
        assert g.data_offset + t.offset + n // be * bb <= size


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama", "tiny-gemma3"])
def test_q4_k_m_recipe(name, synth):
    sp = WORKLOADS[name].spec
    g = ggufpy.read_gguf(synth(name))
    H = sp.hidden
    assert g.tensors["token_embd.weight"].type == q4_k_m_type("output", -1, sp.layers, H)
    for i in range(sp.layers):
        for role in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
            t = g.tensors[f"blk.{i}.{role}.weight"]
            assert t.type == q4_k_m_type(role, i, sp.layers, t.shape[0]), (role, i)
        assert g.tensors[f"blk.{i}.attn_norm.weight"].type == 0


def test_seeded_weights_have_the_stated_distribution(synth):
    g = ggufpy.read_gguf(synth("tiny-qwen3"))
    w = ggufpy.matrix(g, "blk.1.ffn_up.weight").astype(np.float64)
    assert abs(w.mean()) < 1e-3 and abs(w.std() - 0.02) < 1.5e-3
    n = ggufpy.matrix(g, "blk.1.attn_norm.weight").astype(np.float64)
    assert abs(n.mean() - 1.0) < 5e-3


def test_writer_is_deterministic(synth, tmp_path):
    from chonklm_amd import write_synthetic_gguf

    a = Path(synth("tiny-llama-q8")).read_bytes()
    p = tmp_path / "again.gguf"
    write_synthetic_gguf("tiny-llama-q8", str(p), threads=3)
    assert p.read_bytes() == a


@pytest.mark.parametrize("shard_size", [4096, 65536, 1 << 30])
def test_shards_reassemble_byte_exact(synth, tmp_path, shard_size):
    path = synth("tiny-qwen3")
    out = tmp_path / f"s{shard_size}"
    shard_gguf(path, str(out), shard_size=shard_size, quant="Q4_K_M")
    m = json.loads((out / "manifest.json").read_text())
    data = Path(path).read_bytes()
    assert m["totalSize"] == len(data) and m["shardSize"] == shard_size and m["quant"] == "Q4_K_M"
    assert m["shardCount"] == len(m["shards"]) == -(-len(data) // shard_size)
    joined = b""
    for i, s in enumerate(m["shards"]):
        assert s["index"] == i and s["offset"] == len(joined)
        blob = (out / s["name"]).read_bytes()
        assert len(blob) == s["size"] <= shard_size
        joined += blob
    assert joined == data
