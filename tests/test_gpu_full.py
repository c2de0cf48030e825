"""BASELINE config 4 at full size on the GPU: the 0.8B-shaped synthetic model,
greedy decode from token 9419.  The traces must equal the compiled reference
CPU path's: 128 steps (tests/golden/qwen35_0.8b_trace.*, written by
tests/golden/make_golden.py --full; the first step's top-8 logits bit for
bit) and the whole 4096-position context of the headline config
(tests/golden/qwen35_0.8b_trace_4096.*, make_golden.py --trace4096; the last
64 steps' top-8 logits bit for bit)."""
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
        assert np.array_equal(logits[top_i[0]].view(np.uint32), top_v[0].view(np.uint32))
        assert int(np.argmax(logits)) == int(tokens[0])
        m.reset()
        trace = m.generate(meta["token"], meta["steps"])
        first_diff = next((i for i in range(len(tokens)) if trace[i] != tokens[i]), None)
        assert first_diff is None, f"trace differs from step {first_diff}: {trace[first_diff]} vs {tokens[first_diff]}"
    finally:
        m.close()


GOLDEN_4096 = os.path.join(GOLDEN, "qwen35_0.8b_trace_4096.npz")


@pytest.mark.skipif(not os.path.exists(GOLDEN_4096), reason="the 4096-step golden is not generated")
def test_full_model_4096_step_trace(full_model_path):
    """The headline config: the decoder's greedy trace over every position of
    the 4096-token context equals the compiled reference's, and the logits of
    the last 64 steps agree at their top 8 entries bit for bit."""
    from test_gpu_model import open_decoder
    with np.load(GOLDEN_4096) as z:
        tokens, top_i, top_v = z["tokens"], z["last_top_index"], z["last_top_value"]
    with open(GOLDEN_4096.replace(".npz", ".json")) as f:
        meta = json.load(f)
    n, last = meta["steps"], len(top_i)
    m = open_decoder(full_model_path, meta["context"])
    try:
        trace = m.generate(meta["token"], n - last)
        for k in range(last):
            pos = n - last + k
            nxt = m.decoder.forward(int(trace[-1]), pos)
            lg = m.decoder.logits
            assert np.array_equal(lg[top_i[k]].view(np.uint32), top_v[k].view(np.uint32)), f"logits at step {pos}"
            trace = np.append(trace, nxt)
        first_diff = next((i for i in range(n) if trace[i] != tokens[i]), None)
        assert first_diff is None, f"trace differs from step {first_diff}: {trace[first_diff]} vs {tokens[first_diff]}"
    finally:
        m.close()


def _golden_4096():
    with np.load(GOLDEN_4096) as z:
        tokens = z["tokens"].astype(np.int64)
    with open(GOLDEN_4096.replace(".npz", ".json")) as f:
        meta = json.load(f)
    return tokens, meta


@pytest.mark.skipif(not os.path.exists(GOLDEN_4096), reason="the 4096-step golden is not generated")
def test_batch_decoder_4096_step_trace(full_model_path):
    """The batched decoder (batch matvecs, the wide attention kernel) over the
    whole 4096-token context: two sequences from the reference's start token
    each reproduce the compiled reference's trace."""
    from fortai_amd.qwen35 import Qwen35Hip
    tokens, meta = _golden_4096()
    m = Qwen35Hip(full_model_path, max_context=meta["context"], batch=2)
    try:
        m.batch.reset()
        trace = m.batch.generate([meta["token"]] * 2, [0, 0], meta["steps"])
        for s in range(2):
            first_diff = next((i for i in range(len(tokens)) if trace[s][i] != tokens[i]), None)
            assert first_diff is None, f"sequence {s} differs from step {first_diff}"
    finally:
        m.close()


@pytest.mark.skipif(not os.path.exists(GOLDEN_4096), reason="the 4096-step golden is not generated")
def test_prefill_then_batch_decode_4096_step_trace(full_model_path):
    """The exact prompt prefill at the 0.8B shape: the first 512 tokens of the
    reference's trace as the prompt (the start token, then its greedy
    choices), whose next token must be the reference's 512th choice, then
    batched decoding to the end of the 4096-token context, token for token."""
    from fortai_amd.qwen35 import Qwen35Hip
    tokens, meta = _golden_4096()
    T = 512
    prompt = np.concatenate([[meta["token"]], tokens[:T - 1]]).astype(np.int64)
    m = Qwen35Hip(full_model_path, max_context=meta["context"], batch=2)
    try:
        m.batch.reset()
        nxt, _ = m.batch.prefill(np.stack([prompt, prompt]))
        assert nxt.tolist() == [int(tokens[T - 1])] * 2, "the prefill's next token"
        trace = m.batch.generate(nxt, [T, T], meta["steps"] - T)
        for s in range(2):
            want = tokens[T:]
            first_diff = next((i for i in range(len(want)) if trace[s][i] != want[i]), None)
            assert first_diff is None, f"sequence {s} differs from step {T + first_diff}"
    finally:
        m.close()
