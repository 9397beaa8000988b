"""The Node host (chonklm_amd/node/llama-hip-runtime.js over the N-API addon) without a GPU.

Checks the module's exports against the reference module
(src/lib/llama-wgsl-runtime.ts and the PleIAs aliases) and the load-time
errors that happen before any device call: wrong runtime, missing file,
non-GGUF file, unsupported architecture.
"""
from __future__ import annotations

import json
import shutil
import subprocess
from pathlib import Path

import pytest

from tests.test_cpu_abi import _gguf_with_arch

ROOT = Path(__file__).resolve().parents[1]
ADDON = ROOT / "chonklm_amd" / "_lib" / "chonk_napi.node"

pytestmark = pytest.mark.skipif(shutil.which("node") is None or not ADDON.exists(),
                                reason="node or the N-API addon is not available")


def run_driver(job: dict, timeout: int = 120) -> dict:
    p = subprocess.run(["node", str(ROOT / "tests" / "node_driver.js"), json.dumps(job)], capture_output=True,
                       text=True, timeout=timeout)
    lines = [ln for ln in p.stdout.splitlines() if ln.startswith("{")]
    assert lines, f"no output: rc={p.returncode} stderr={p.stderr[-2000:]}"
    out = json.loads(lines[-1])
    assert "fatal" not in out, out["fatal"]
    return out


def model(gguf: str, **kw) -> dict:
    d = {"id": "t", "runtime": "llama-webgpu", "eosIds": [2], "vocab": 1000, "layers": 2, "maxContext": 64,
         "base": "", "gguf": gguf}
    d.update(kw)
    return d


def test_exports_and_load_errors(tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"NOTGGUF" + bytes(100))
    arch = tmp_path / "arch.gguf"
    arch.write_bytes(_gguf_with_arch("rwkv"))
    out = run_driver({"kind": "errors", "models": [
        model("x.gguf", runtime="gemma-webgpu"),
        model(str(tmp_path / "missing.gguf")),
        model(str(bad)),
        model("arch.gguf", base=str(tmp_path)),
    ]})
    assert out["exports"] == sorted(["LlamaWgslEngine", "loadLlamaWgslModel", "generateLlamaWgsl",
                                     "disposeLlamaWgsl", "resetLlamaWgslConversation", "loadPleiasWgslModel",
                                     "generatePleiasWgsl", "disposePleiasWgsl", "loadGptWgslModel",
                                     "generateGptWgsl", "disposeGptWgsl", "resetGptWgslConversation",
                                     "loadLfmWgslModel", "generateLfmWgsl", "disposeLfmWgsl",
                                     "resetLfmWgslConversation", "loadGraniteWgslModel", "generateGraniteWgsl",
                                     "disposeGraniteWgsl", "resetGraniteWgslConversation"])
    e = out["errors"]
    assert not e[0]["ok"] and "is not configured for the Llama WGSL runtime" in e[0]["message"]
    assert e[1]["code"] == "EIO" and "missing.gguf" in e[1]["message"]
    assert e[2]["code"] == "EINVAL" and "could not parse GGUF header" in e[2]["message"]
    assert e[3]["code"] == "EINVAL" and "does not support architecture rwkv" in e[3]["message"]
