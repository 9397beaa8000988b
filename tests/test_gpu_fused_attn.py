"""The q|k|v matvec inside the decode attention launch (k_qkv_attn).

On every attention layer after the first whose q|k|v matvec is the
three-matrix row kernel with the RMSNorm prologue, the engine runs that matvec
in the attention's launch: the matvec workgroups come first in the grid and
store each row as a word tagged with its kv head's epoch, and each attention
workgroup polls its group's q, k and v words while its K/V rows are in flight.
The rows are computed by the same row-kernel code as the separate launch, so
the fused engine's logits equal those of the engine with separate launches
(CHONK_FUSE=0) bit for bit. Checked at the Qwen3-0.6B shape (group 2,
head_dim 128, q/k RMSNorm) over 1-36 chunks per kv head and at the SmolLM2
shape (group 3, head_dim 64, interleaved rotary, Q6_K v rows); both engines
also follow the oracle (the oracle comparison at every chunk count is
test_decode_attention_across_chunk_counts, which decodes through the fused
launch).
"""
from __future__ import annotations

import numpy as np
import pytest

from chonklm_amd import WORKLOADS, load_llama_wgsl_model
from oracle.oracle import OracleModel
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

CASES = {
    "qwen3-0.6b-q4_k_m": (2304, (1, 63, 64, 700, 2047, 2048, 2112, 2302)),
    "smollm2-135m-q4_k_m": (640, (1, 31, 64, 300, 637)),
}


def _decode(path, w, ctx, positions, steps=2):
    md = w.model_def(path)
    md.max_context = ctx
    eng = load_llama_wgsl_model(md).engine
    info = eng.info
    out = []
    tok = 17
    for pos in positions:
        eng.fake_context(pos, seed=pos)
        for _ in range(steps):
            tok = eng.run_token(tok, True)
            out.append((pos, tok, eng.read_logits().copy()))
    eng.dispose()
    return info, out


@pytest.mark.parametrize("name", sorted(CASES))
def test_fused_launch_equals_separate_launches(synth, monkeypatch, name):
    w = WORKLOADS[name]
    path = synth(name)
    ctx, positions = CASES[name]
    monkeypatch.delenv("CHONK_FUSE", raising=False)
    info_f, fused = _decode(path, w, ctx, positions)
    monkeypatch.setenv("CHONK_FUSE", "0")
    info_s, sep = _decode(path, w, ctx, positions)
    monkeypatch.delenv("CHONK_FUSE")
    if info_f["spin_attention"] != 1:
        pytest.skip("another engine on this GPU holds the spin-merging attention")
    assert info_f["fused_attention"] == w.spec.layers - 1
    assert info_s["fused_attention"] == 0
    assert info_f["kernels_per_step"] == info_s["kernels_per_step"] - (w.spec.layers - 1)
    for (pa, ta, la), (pb, tb, lb) in zip(fused, sep):
        assert ta == tb, f"position {pa}: token {ta} != {tb}"
        assert np.array_equal(la, lb), f"position {pa}: logits differ (max |d| {np.max(np.abs(la - lb)):.3e})"


def test_fused_launch_follows_oracle_at_smollm2_shape(synth):
    name = "smollm2-135m-q4_k_m"
    w = WORKLOADS[name]
    path = synth(name)
    ctx, positions = CASES[name]
    md = w.model_def(path)
    md.max_context = ctx
    eng = load_llama_wgsl_model(md).engine
    if eng.info["fused_attention"] == 0:
        eng.dispose()
        pytest.skip("another engine on this GPU holds the spin-merging attention")
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, ctx, kv_f16=True, threads=16)
    tok = 5
    for pos in positions:
        eng.fake_context(pos, seed=pos)
        ref.fake_context(pos, seed=pos)
        for i in range(2):
            a = eng.run_token(tok, True)
            b = ref.run_token(tok, True)
            e = rel_err(eng.read_logits(), ref.logits())
            assert e <= 1e-3, f"position {pos + i}: logits rel err {e:.3e}"
            assert a == b, f"position {pos + i}: token {a} != {b}"
            tok = a
    eng.dispose()
    ref.close()
