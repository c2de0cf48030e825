"""End-to-end parity of the Qwen3.5 decode step on the GPU against the oracle
(the C restatement, itself bit-exact with the compiled reference on these
models -- tests/test_oracle.py).  The decode path keeps every rounding of
the reference, so logits, KV caches, GDN and conv states are compared bit
for bit."""

import os

import numpy as np
import pytest

from fortai_amd.qwen35 import Qwen35Hip

pytestmark = pytest.mark.gpu

REL = 1e-3


def rel_err(got, want):
    want = np.asarray(want, dtype=np.float64)
    scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)) + 1e-30)
    return float(np.max(np.abs(np.asarray(got, np.float64) - want) / scale))


def open_decoder(path, max_context):
    return Qwen35Hip(path, max_context=max_context)


def same_bits(got, want):
    return np.array_equal(np.asarray(got, np.float32).view(np.uint32), np.asarray(want, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def tiny(tiny_model_path):
    m = open_decoder(tiny_model_path, 64)
    yield m
    m.close()


def test_tiny_decoder_matches_oracle(tiny, oracle, tiny_model_path):
    from oracle.oracle import OracleModel
    ref = OracleModel(oracle, tiny_model_path, 64)
    tiny.reset()
    token = 9
    for pos in range(24):
        got = tiny.forward(token, pos).copy()
        want = ref.forward(token, pos)
        assert same_bits(got, want), f"step {pos}: logits differ (max rel {rel_err(got, want):.3e})"
        nxt = int(np.argmax(want))
        assert int(np.argmax(got)) == nxt, f"greedy token differs at step {pos}"
        token = nxt
    d = tiny.d
    for i, layer in enumerate(tiny.attention):
        if layer is None:
            continue
        k, v = layer.cache(24)
        assert np.array_equal(k, ref.kcache(i)[:k.size]), f"K cache of layer {i}"
        assert np.array_equal(v, ref.vcache(i)[:v.size]), f"V cache of layer {i}"
    for i, layer in enumerate(tiny.recurrent):
        if layer is None:
            continue
        gdn, conv = layer.state()
        assert same_bits(gdn, ref.gdn_state(i)), f"GDN state of layer {i}"
        assert same_bits(conv, ref.conv_state(i)), f"conv state of layer {i}"


def test_tiny_generate_trace_and_ops_path(tiny, oracle, tiny_model_path):
    from oracle.oracle import OracleModel
    ref = OracleModel(oracle, tiny_model_path, 64)
    want = ref.greedy(9, 48)
    tiny.reset()
    got = tiny.generate(9, 48)
    assert got.tolist() == want
    # the per-op reference ABI sequence gives the same logits
    tiny.reset()
    ref.reset()
    token = 9
    for pos in range(6):
        ops = tiny.forward_ops(token, pos)
        cpu = ref.forward(token, pos)
        assert rel_err(ops, cpu) <= REL, f"ops path step {pos}"
        token = int(np.argmax(cpu))


@pytest.fixture(scope="module")
def tiny_q8emb_path(tmp_path_factory):
    from fortai_amd import synth
    path = str(tmp_path_factory.mktemp("models") / "tiny_q8emb.gguf")
    synth.write_model(path, synth.CONFIGS["qwen35-tiny-q8emb"])
    return path


def test_q8_embedding_model_trace(oracle, tiny_q8emb_path):
    """Q8_0 tied embedding / LM head (the tensor types of llama.cpp Q8_0 exports)."""
    from oracle.oracle import OracleModel
    ref = OracleModel(oracle, tiny_q8emb_path, 64)
    m = open_decoder(tiny_q8emb_path, 64)
    try:
        token = 17
        for pos in range(12):
            got = m.forward(token, pos).copy()
            want = ref.forward(token, pos)
            assert same_bits(got, want), f"step {pos}: logits differ (max rel {rel_err(got, want):.3e})"
            token = int(np.argmax(want))
            assert int(np.argmax(got)) == token
        m.reset()
        ref.reset()
        assert m.generate(17, 40).tolist() == ref.greedy(17, 40)
    finally:
        m.close()


def same_values(got, want):
    """Bit-identical, NaNs only at the same places (their payloads are not
    part of the reference's arithmetic)."""
    a, b = np.asarray(got, np.float32), np.asarray(want, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def test_exponent31_value_cache_matches_oracle(oracle, tmp_path):
    """attn_v scaled so that about one value in ten leaves the fp16 range: the
    KV append (ties-away fp16 with overflow) must store the reference's
    exponent-31 halves bit for bit.  The reference reads them back as +-huge()
    (gguf_fp16_to_real, fortai_gguf_runtime.f90:770-788), which the o
    projection turns into inf and NaN, so from the first attention layer on
    every logit is NaN in both: this checks the caches, that the NaNs are the
    reference's (no finite value where it has NaN) and the greedy trace of
    first indices.  The flagged attention arithmetic itself is compared
    bit for bit in test_gpu_kernels.py::test_attention_output_kernels."""
    from fortai_amd import synth
    from oracle.oracle import OracleModel
    path = str(tmp_path / "hugev.gguf")
    synth.write_model(path, synth.CONFIGS["qwen35-tiny-hugev"])
    ref = OracleModel(oracle, path, 64)
    m = open_decoder(path, 64)
    try:
        token = 5
        for pos in range(20):
            got = m.forward(token, pos).copy()
            want = ref.forward(token, pos)
            assert same_values(got, want), f"step {pos}: logits differ"
            token = int(np.argmax(want))
            assert int(np.argmax(got)) == token, f"greedy token differs at step {pos}"
        flagged = 0
        for i, layer in enumerate(m.attention):
            if layer is None:
                continue
            k, v = layer.cache(20)
            assert np.array_equal(v, ref.vcache(i)[:v.size]), f"V cache of layer {i}"
            flagged += int(np.count_nonzero((v & 0x7c00) == 0x7c00))
        assert flagged > 0, "the V caches hold exponent-31 halves"
        print(f"exponent-31 halves in the V caches: {flagged}", flush=True)
        m.reset()
        ref.reset()
        assert m.generate(5, 48).tolist() == ref.greedy(5, 48)
    finally:
        m.close()


@pytest.fixture(scope="module")
def short_path(tmp_path_factory):
    """Every 0.8B layer shape (hidden 1024, FFN 3584, GDN 16x128, attention
    8/2 heads x 256) with 4 layers and a 16384-token vocabulary."""
    from fortai_amd import synth
    path = str(tmp_path_factory.mktemp("models") / "short.gguf")
    synth.write_model(path, synth.CONFIGS["qwen35-0.8b-short"])
    return path


def test_full_layer_shapes_long_context(oracle, short_path):
    """The decode step at the 0.8B layer shapes over 300 positions (several
    256-position segments of the attention chains): logits, caches, states
    and the trace follow the oracle bit for bit."""
    from oracle.oracle import OracleModel
    ctx = 320
    ref = OracleModel(oracle, short_path, ctx)
    m = open_decoder(short_path, ctx)
    try:
        token = 9419 % 16384
        for pos in range(8):
            got = m.forward(token, pos).copy()
            want = ref.forward(token, pos)
            assert same_bits(got, want), f"step {pos}: logits differ (max rel {rel_err(got, want):.3e})"
            token = int(np.argmax(want))
            assert int(np.argmax(got)) == token, f"step {pos}"
        trace = m.generate(token, 292, start=8)
        want = ref.greedy(token, 292, start=8)
        assert trace.tolist() == want
        for i, layer in enumerate(m.attention):
            if layer is None:
                continue
            k, v = layer.cache(300)
            assert np.array_equal(k, ref.kcache(i)[:k.size]), f"K cache of layer {i}"
            assert np.array_equal(v, ref.vcache(i)[:v.size]), f"V cache of layer {i}"
        for i, layer in enumerate(m.recurrent):
            if layer is None:
                continue
            gdn, conv = layer.state()
            assert same_bits(gdn, ref.gdn_state(i)), f"GDN state of layer {i}"
            assert same_bits(conv, ref.conv_state(i)), f"conv state of layer {i}"
    finally:
        m.close()


@pytest.fixture(scope="module")
def short4b_path(tmp_path_factory):
    """Every 4B layer shape (hidden 2560, FFN 9216, GDN 16 key / 32 value
    heads of 128, attention 16/4 heads x 256) with 4 layers and a
    16384-token vocabulary -- BASELINE config 5's layers."""
    from fortai_amd import synth
    path = str(tmp_path_factory.mktemp("models") / "short4b.gguf")
    synth.write_model(path, synth.CONFIGS["qwen35-4b-short"])
    return path


def test_4b_layer_shapes_match_oracle(oracle, short4b_path):
    """The single-sequence decoder at the 4B layer shapes against the oracle
    (fortai_qwen35_cpu.f90:231-235 grouped GDN heads, :801-918, :978-1035):
    logits of every step, then the K/V caches, GDN and conv states, bit for
    bit.  The batched decoder and the prefill are pinned to this decoder
    (test_gpu_batch.py, test_gpu_config5.py), so this closes their chain to
    the reference at config 5's own shapes."""
    from oracle.oracle import OracleModel
    ctx = 64
    steps = 16
    ref = OracleModel(oracle, short4b_path, ctx)
    m = open_decoder(short4b_path, ctx)
    try:
        token = 9419 % 16384
        for pos in range(steps):
            got = m.forward(token, pos).copy()
            want = ref.forward(token, pos)
            assert same_bits(got, want), f"step {pos}: logits differ (max rel {rel_err(got, want):.3e})"
            token = int(np.argmax(want))
            assert int(np.argmax(got)) == token, f"step {pos}"
        for i, layer in enumerate(m.attention):
            if layer is None:
                continue
            k, v = layer.cache(steps)
            assert np.array_equal(k, ref.kcache(i)[:k.size]), f"K cache of layer {i}"
            assert np.array_equal(v, ref.vcache(i)[:v.size]), f"V cache of layer {i}"
        for i, layer in enumerate(m.recurrent):
            if layer is None:
                continue
            gdn, conv = layer.state()
            assert same_bits(gdn, ref.gdn_state(i)), f"GDN state of layer {i}"
            assert same_bits(conv, ref.conv_state(i)), f"conv state of layer {i}"
    finally:
        m.close()
