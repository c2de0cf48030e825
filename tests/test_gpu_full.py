"""BASELINE config 4 at full size on the GPU: the 0.8B-shaped synthetic model,
greedy decode of 128 steps from token 9419.  The trace must equal the
compiled reference CPU path's (tests/golden/qwen35_0.8b_trace.*, written by
tests/golden/make_golden.py --full) and the first step's top-8 logits must
agree within 1e-3 of the top logit."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


@pytest.fixture(scope="module")
def full_model_path():
    # the same file bench.py uses, so one GPU session writes it once
    from fortai_amd import synth
    path = os.path.join(os.environ.get("TMPDIR", "/tmp"), "fortai_bench", "qwen35-0.8b.gguf")
    if not os.path.exists(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        synth.write_model(path + ".part", synth.CONFIGS["qwen35-0.8b"])
        os.replace(path + ".part", path)
    return path


def test_full_model_128_step_trace(full_model_path):
    from test_gpu_model import open_decoder
    with np.load(os.path.join(GOLDEN, "qwen35_0.8b_trace.npz")) as z:
        tokens, top_i, top_v = z["tokens"], z["top_index"], z["top_value"]
    with open(os.path.join(GOLDEN, "qwen35_0.8b_trace.json")) as f:
        meta = json.load(f)
    m = open_decoder(full_model_path, meta["context"])
    try:
        logits = m.forward(meta["token"], 0).copy()
        scale = float(abs(top_v[0, 0]))
        assert np.max(np.abs(logits[top_i[0]] - top_v[0])) <= 1e-3 * scale
        assert int(np.argmax(logits)) == int(tokens[0])
        m.reset()
        trace = m.generate(meta["token"], meta["steps"])
        first_diff = next((i for i in range(len(tokens)) if trace[i] != tokens[i]), None)
        assert first_diff is None, f"trace differs from step {first_diff}: {trace[first_diff]} vs {tokens[first_diff]}"
    finally:
        m.close()
