"""BASELINE config 5 at full size: the Qwen3.5-4B shape (hidden 2560, 32
layers, FFN 9216, 16 q / 4 kv heads of 256, vocabulary 248320), 8
independent sequences, context 8192, a 512-token prompt per sequence.

The prefill (every projection on the matrix cores in the reference's lane
order, the exact causal attention) must leave each sequence exactly where
token-by-token decoding of its prompt leaves the single-sequence decoder:
the last prompt token's logits bit for bit and the greedy next token; the
batched decode steps that follow must then equal the single-sequence
decoder's steps.  The single-sequence decoder is itself bit-identical to the
reference CPU path (tests/test_gpu_model.py, tests/test_gpu_full.py)."""
from __future__ import annotations

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BATCH, PROMPT, CONTEXT, STEPS = 8, 512, 8192, 4


@pytest.fixture(scope="module")
def model_4b():
    from fortai_amd import synth
    from fortai_amd.qwen35 import Qwen35Hip
    # the file bench.py writes, so one GPU session writes it once
    path = os.path.join(os.environ.get("TMPDIR", "/tmp"), "fortai_bench", "qwen35-4b.gguf")
    if not os.path.exists(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        synth.write_model(path + ".part", synth.CONFIGS["qwen35-4b"])
        os.replace(path + ".part", path)
    m = Qwen35Hip(path, max_context=CONTEXT, batch=BATCH)
    yield m
    m.close()


def test_config5_prefill_and_decode_match_single_sequence(model_4b):
    m = model_4b
    d = m.d
    assert (d.hidden, d.layers, d.ffn, d.heads, d.kv_heads, d.head_size, d.vocab) == (2560, 32, 9216, 16, 4, 256, 248320)
    rng = np.random.default_rng(0x51E5)  # the prompts bench.py times
    prompts = rng.integers(0, d.vocab, size=(BATCH, PROMPT))
    m.batch.reset()
    nxt, ms = m.batch.prefill(prompts)
    logits = m.batch.logits.copy()
    trace = m.batch.generate(nxt, np.full(BATCH, PROMPT, dtype=np.int32), STEPS)
    print(f"config 5 prefill {BATCH} x {PROMPT} tokens in {ms:.1f} ms", flush=True)
    for s in range(BATCH):
        dec = m.decoder
        dec.reset()
        for pos in range(PROMPT - 1):
            dec.forward(int(prompts[s, pos]), pos, want_logits=False)
        want_next = dec.forward(int(prompts[s, -1]), PROMPT - 1)
        same = np.array_equal(logits[s].view(np.uint32), dec.logits.view(np.uint32))
        print(f"sequence {s}: logits identical {same}, next {int(nxt[s])} / {want_next}", flush=True)
        assert same, f"sequence {s}: prefill logits differ from token-by-token decoding"
        assert int(nxt[s]) == want_next
        assert dec.generate(want_next, PROMPT, STEPS).tolist() == trace[s].tolist(), f"sequence {s} decode steps"
