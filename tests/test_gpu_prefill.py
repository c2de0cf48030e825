"""Prompt prefill of a batch (512-token prefill per
sequence on the Q8_0 x Q8_0 token-block path) through the C ABI.

The reference has no prefill: it decodes the prompt one token at a time
(fortai_qwen35_cpu.f90:591-711), with the AVX2 eight-lane accumulation of
every Q8_0 dot.  The prefill computes each block dot exactly (int32, on the
matrix cores) but accumulates the scaled block dots in a different fp32 order,
so each projection agrees with the reference to ~1e-6 relative
(tests/test_gpu_mmq.py).  End to end, every layer re-quantizes its
activations to int8: a ~1e-7 difference now and then moves a value across an
int8 rounding boundary, and that one-step change propagates through the
recurrent state, the caches and the later layers (the 4B widths re-quantize
~18K values per token and layer, so at that shape most sequences see one).
Two bars follow:
- with FORTAI_HIP_PREFILL_EXACT=1 the projections run in the reference's
  lane order and everything else is the prefill's own code: the logits are
  then bit-identical to token-by-token decoding (one-token prompts by
  construction; longer prompts as measured) -- this validates the conv1d, the
  delta rule, RoPE and the KV append, the causal attention, the gating and
  the quantizers of the prefill;
- in the default (matrix-core) mode the logits stay within 1e-1 relative of
  token-by-token decoding and the greedy next token agrees for nearly every
  sequence.
The prefilled state continues decoding deterministically.
"""

import numpy as np
import pytest

from fortai_amd import synth
from fortai_amd.qwen35 import Qwen35Hip

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    want = np.asarray(want, dtype=np.float64)
    scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)) + 1e-30)
    return float(np.max(np.abs(np.asarray(got, np.float64) - want) / scale))


@pytest.fixture(scope="module")
def paths(tmp_path_factory):
    d = tmp_path_factory.mktemp("prefill_models")
    out = {}
    for name in ("qwen35-tiny", "qwen35-tiny-q8emb", "qwen35-4b-short"):
        out[name] = str(d / f"{name}.gguf")
        synth.write_model(out[name], synth.CONFIGS[name])
    return out


def decode_prompt(m, prompt):
    """The single-sequence decoder fed the prompt token by token."""
    m.decoder.reset()
    for pos, tok in enumerate(prompt):
        nxt = m.decoder.forward(int(tok), pos)
    return m.decoder.logits.copy(), nxt


@pytest.mark.parametrize("name,batch,lengths", [("qwen35-tiny", 4, (17, 24, 33, 48, 64, 70)),
                                                ("qwen35-tiny-q8emb", 4, (33, 65)),
                                                ("qwen35-4b-short", 8, (64,)),
                                                # many 32-key tiles of the matrix-core attention
                                                ("qwen35-tiny", 2, (511,)),
                                                ("qwen35-4b-short", 2, (300,))])
def test_prefill_close_to_token_by_token_decode(paths, name, batch, lengths):
    m = Qwen35Hip(paths[name], max_context=max(128, max(lengths) + 8), batch=batch)
    errs, agree, total = [], 0, 0
    try:
        for T in lengths:
            rng = np.random.default_rng(T * 13 + batch)
            prompts = rng.integers(0, m.d.vocab, size=(batch, T))
            m.batch.reset()
            nxt, _ = m.batch.prefill(prompts)
            logits = m.batch.logits.copy()
            for s in range(batch):
                want_logits, want_next = decode_prompt(m, prompts[s])
                errs.append(rel_err(logits[s], want_logits))
                agree += int(nxt[s]) == want_next
                total += 1
                print(f"{name} T {T} sequence {s}: rel {errs[-1]:.2e} next {int(nxt[s])} / {want_next}", flush=True)
    finally:
        m.close()
    assert max(errs) <= 1e-1
    assert agree >= total - max(1, total // 10)


@pytest.mark.parametrize("name,batch,T", [("qwen35-tiny", 3, 40), ("qwen35-4b-short", 8, 32)])
def test_prefilled_state_continues_exactly(paths, name, batch, T):
    """Prefill T-1 tokens then decode the last prompt token and 6 more: the
    same steps replayed after a second identical prefill give the same
    tokens (the prefill leaves a complete, deterministic decode state), and
    the decode steps after a prefill are the batch decoder's own."""
    m = Qwen35Hip(paths[name], max_context=128, batch=batch)
    try:
        rng = np.random.default_rng(T + batch)
        prompts = rng.integers(0, m.d.vocab, size=(batch, T))
        runs = []
        for _ in range(2):
            m.batch.reset()
            m.batch.prefill(prompts[:, :-1])
            runs.append(m.batch.generate(prompts[:, -1], np.full(batch, T - 1, dtype=np.int32), 7))
        assert np.array_equal(runs[0], runs[1])
        # prefill of all T tokens vs prefill of T-1 + one decode step: same next token
        m.batch.reset()
        nxt, _ = m.batch.prefill(prompts)
        agree = int(np.sum(nxt == runs[0][:, 0]))
        assert agree >= batch - 1
    finally:
        m.close()


def test_prefill_matches_oracle(paths, oracle):
    from oracle.oracle import OracleModel
    path = paths["qwen35-tiny"]
    m = Qwen35Hip(path, max_context=64, batch=2)
    try:
        prompts = np.array([[9, 8, 7, 100, 2000, 5, 4095, 17, 300, 9] * 3, [1] * 30], dtype=np.int64)
        m.batch.reset()
        nxt, _ = m.batch.prefill(prompts)
        ref = OracleModel(oracle, path, 64)
        for s in range(2):
            ref.reset()
            for pos, tok in enumerate(prompts[s]):
                want = ref.forward(int(tok), pos)
            err = rel_err(m.batch.logits[s], want)
            print(f"oracle sequence {s}: rel {err:.2e}", flush=True)
            assert err <= 1e-1
            assert int(nxt[s]) == int(np.argmax(want))
    finally:
        m.close()


@pytest.mark.parametrize("name,batch", [("qwen35-tiny", 8), ("qwen35-4b-short", 8)])
def test_exact_mode_prefill_matches_decode(paths, name, batch, monkeypatch):
    """FORTAI_HIP_PREFILL_EXACT=1 runs the projections in the reference's
    lane order; everything else is the prefill's own code.  A one-token prompt
    then has no order difference left anywhere (the single-key softmax is
    exact), so its logits must equal the decoder's bit for bit; with longer
    prompts only the attention's online softmax differs from the decoder's
    two-pass sums."""
    monkeypatch.setenv("FORTAI_HIP_PREFILL_EXACT", "1")
    m = Qwen35Hip(paths[name], max_context=64, batch=batch)
    try:
        rng = np.random.default_rng(7)
        prompts = rng.integers(0, m.d.vocab, size=(batch, 1))
        m.batch.reset()
        nxt, _ = m.batch.prefill(prompts)
        for s in range(batch):
            want_logits, want_next = decode_prompt(m, prompts[s])
            assert np.array_equal(m.batch.logits[s].view(np.uint32), want_logits.view(np.uint32)), f"sequence {s}"
            assert int(nxt[s]) == want_next
        errs = []
        for T in (2, 5, 24):
            prompts = rng.integers(0, m.d.vocab, size=(batch, T))
            m.batch.reset()
            nxt, _ = m.batch.prefill(prompts)
            for s in range(batch):
                want_logits, want_next = decode_prompt(m, prompts[s])
                errs.append(rel_err(m.batch.logits[s], want_logits))
                print(f"exact {name} T {T} sequence {s}: rel {errs[-1]:.2e}", flush=True)
        assert np.median(errs) <= 1e-5
    finally:
        m.close()
