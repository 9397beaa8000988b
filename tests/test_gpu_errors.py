"""Failure handling of the C ABI on the GPU, forced from the host.

A HIP error marks the engine lost and every later call that uses the device
fails fast with CHONK_ELOST (the deviceLost rule of the reference's LFM
runtime, lfm-wgsl-runtime.ts:704-707, :729-731). The error is forced through
the chonk_engine_debug_fail_next_launch hook, which makes the engine's next
launch report a HIP error without running anything on the device.
"""
from __future__ import annotations

import pytest

from chonklm_amd import WORKLOADS, ChonkError, generate_llama_wgsl, load_llama_wgsl_model
from chonklm_amd import _lib
from chonklm_amd._lib import check, lib

pytestmark = pytest.mark.gpu


def _loaded(synth):
    w = WORKLOADS["tiny-qwen3"]
    return w, load_llama_wgsl_model(w.model_def(synth("tiny-qwen3")))


def _status(fn):
    with pytest.raises(ChonkError) as ei:
        fn()
    return ei.value.status, str(ei.value)


@pytest.mark.parametrize("where", ["step", "generate", "prefill"])
def test_injected_hip_error_then_lost(synth, where):
    w, loaded = _loaded(synth)
    eng = loaded.engine
    assert eng.run_token(5, True) >= 0  # healthy before
    check(lib().chonk_engine_debug_fail_next_launch(eng._h), eng._h)
    first = {"step": lambda: eng.run_token(6, True),
             "generate": lambda: generate_llama_wgsl(loaded, [1, 2, 3], 4),
             "prefill": lambda: eng.prefill([7, 8, 9])}[where]
    status, msg = _status(first)
    assert status == _lib.CHONK_EHIP and "injected" in msg
    for later in (lambda: eng.run_token(6, True), lambda: generate_llama_wgsl(loaded, [1, 2], 2), eng.reset,
                  eng.read_logits, lambda: eng.prefill([1, 2])):
        status, msg = _status(later)
        assert status == _lib.CHONK_ELOST and "lost" in msg
    eng.dispose()  # a lost engine is still freed


def test_lost_engine_does_not_affect_another(synth):
    w, a = _loaded(synth)
    _, b = _loaded(synth)
    check(lib().chonk_engine_debug_fail_next_launch(a.engine._h), a.engine._h)
    assert _status(lambda: a.engine.run_token(1, True))[0] == _lib.CHONK_EHIP
    prompt = w.prompt(3, 10)
    assert len(generate_llama_wgsl(b, prompt, 5)["ids"]) == 5
    a.engine.dispose()
    b.engine.dispose()


def test_shard_range_out_of_bounds(synth, tmp_path):
    """A shard manifest whose totalSize stops before the tensor data: the tensor read is
    refused by the range check of fetchShardedRange, with its wording (cache.ts:429-433)."""
    import json

    from chonklm_amd import shard_gguf

    w = WORKLOADS["tiny-qwen3"]
    out = tmp_path / "shards"
    shard_gguf(synth("tiny-qwen3"), str(out), shard_size=65536)
    m = json.loads((out / "manifest.json").read_text())
    m["shards"] = m["shards"][:1]
    m["shardCount"] = 1
    m["totalSize"] = m["shards"][0]["size"]
    (out / "manifest.json").write_text(json.dumps(m))
    md = w.model_def(str(out))
    status, msg = _status(lambda: load_llama_wgsl_model(md))
    assert status == _lib.CHONK_EIO
    assert f"range out of bounds for {out}: offset=" in msg and f"totalSize={m['totalSize']}" in msg
