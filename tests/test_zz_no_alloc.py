"""chonk_engine_prefill_noalloc: the prompt pass with its row buffers in the
library's per-GPU scratch array (no device allocation) gives what
chonk_engine_prefill gives: the same next token and logits within 1e-3 after
the pass, and the same K/V rows (to fp16 rounding of fp32-rounding-level
differences), on two calls in a row where the second takes fewer tokens (so
the scratch still holds the first call's larger contents), on two model
shapes; more tokens than one pass holds are refused with a clear error.
"""
from __future__ import annotations

import numpy as np
import pytest

from chonklm_amd import WORKLOADS, ChonkError
from chonklm_amd.runtime import LlamaWgslEngine
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,lengths", [("tiny-qwen3", (140, 37)), ("qwen3-0.6b-q4_k_m", (0, 200))])
def test_prefill_noalloc_matches_prefill(synth, name, lengths):
    w = WORKLOADS[name]
    md = w.model_def(synth(name))
    md.max_context = min(md.max_context, 1024)
    a = LlamaWgslEngine(md)
    b = LlamaWgslEngine(md)
    rows = b.info["noalloc_prefill_rows"]
    assert 16 <= rows <= 2048 and rows % 16 == 0  # (at most one full pass of 2048 rows)
    first, second = lengths
    first = first or min(rows, md.max_context - 8)
    assert second < first <= rows
    for call, n in enumerate((first, second)):
        a.reset()
        b.reset()
        p = w.prompt(100 + call, n + 1)
        a.prefill(p[:-1])
        b.prefill_noalloc(p[:-1])
        assert a.position == b.position == n
        for layer in (0, w.spec.layers - 1):
            for pos in (0, n // 2, n - 1):
                for is_v in (False, True):
                    ka = a_kv = a.read_kv(layer, is_v, pos)
                    kb = b.read_kv(layer, is_v, pos)
                    assert np.max(np.abs(ka - kb)) <= 2e-3 * max(1.0, float(np.max(np.abs(a_kv)))), (call, layer, pos)
        ta = a.run_token(p[-1], True)
        tb = b.run_token(p[-1], True)
        e = rel_err(b.read_logits(), a.read_logits())
        assert e <= 1e-3, f"call {call}: logits rel err {e:.3e}"
        assert ta == tb, f"call {call}: token {tb} != {ta}"
    with pytest.raises(ChonkError, match=f"at most {rows} tokens per call"):
        b.prefill_noalloc([1] * (rows + 1))
    a.dispose()
    b.dispose()
