"""The prompt prefill's causal attention by itself,
through fortai_hip_qwen35_attention_prefill_core_device.

The reference has no prefill: it runs fortai_qwen35_cpu.f90:990-1031 (q/k
RMSNorm, RoPE, fp16 KV append, two-pass softmax, P.V, sigmoid gate) once per
token.  The oracle's attention_core_step restates that step; run for
t = 0..T-1 it gives every prefill row.
- the exact kernel (the default prefill) must equal it bit for bit, outputs
  and the appended K/V cache;
- the fp16 matrix-core kernel (the 'fast' prefill mode) rounds q, k, v and
  the probabilities to fp16 (11-bit significands, relative 2^-11 = 4.9e-4
  each) and uses the hardware exp and reciprocal; its outputs are held to
  FAST_ATT_REL, relative to the output scale (rel_err below), and its K/V
  append must be bit-exact too.
"""

import numpy as np
import pytest

from fortai_amd import backend as B
from fortai_amd import synth

pytestmark = pytest.mark.gpu

# The fast prefill mode's attention against the reference's step.  fp16 q
# and k move a score by up to ~2^-11 x sum|q_i k_i| / sqrt(head), about 1e-3
# for these normalised heads, and a probability by as much relative to
# itself; P's own fp16 rounding adds 2^-11.  Measured here: 1.8e-3 (head
# 256, T 32), 3.0e-3 (256, 300), 3.6e-3 (256, 511), 3.2e-3 (64, 300),
# 2.0e-3 (128, 97).
FAST_ATT_REL = 6e-3


def rel_err(got, want):
    """max |got - want| / max(|want|, rms(want)) elementwise."""
    want = np.asarray(want, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)) + 1e-30)
    return float(np.max(np.abs(got - want) / scale))


def same_values(a, b):
    """Bit-identical, except that NaNs only have to sit at the same places
    (their payloads are not part of the reference's arithmetic)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


@pytest.mark.parametrize("head,T,big", [(256, 32, False), (256, 300, False), (256, 511, False), (64, 300, False),
                                        (128, 97, False), (256, 97, True), (64, 70, True)])
def test_prefill_attention_kernels(ctx, oracle, head, T, big):
    """big: some value entries beyond the fp16 range, so the cache holds
    exponent-31 halves (gguf_fp16_to_real reads them as +-huge,
    fortai_gguf_runtime.f90:770-788), the kv head is flagged and the exact
    kernel's flagged instance serves it."""
    rng = np.random.default_rng(head * 1000 + T)
    heads, kvh, H = 8, 2, 1024
    rope = 64 if head >= 128 else 16
    mk = lambda rows, width: B.Q8Weights(ctx, synth.q8_blocks(rng, rows, width), rows, width)
    ws = [mk(heads * 2 * head, H), mk(kvh * head, H), mk(kvh * head, H), mk(H, heads * head)]
    qn = (1 + 0.05 * rng.standard_normal(head)).astype(np.float32)
    kn = (1 + 0.05 * rng.standard_normal(head)).astype(np.float32)
    maxc = max(T, 64)
    A = B.Attention(ctx, *ws, qn, kn, heads, kvh, head, head, maxc, rope, 1.0e7, 1e-6)
    q = rng.standard_normal((T, heads * 2 * head)).astype(np.float32)
    k = rng.standard_normal((T, kvh * head)).astype(np.float32)
    v = rng.standard_normal((T, kvh * head)).astype(np.float32)
    if big:
        v[::7, : head // 3] *= np.float32(3e5)  # |v| > 65504 in places: exponent-31 halves in kv head 0

    # the reference, token by token
    kc = np.zeros(maxc * kvh * head, np.uint16)
    vc = np.zeros(maxc * kvh * head, np.uint16)
    scores = np.zeros(maxc, np.float32)
    want = np.zeros((T, heads * head), np.float32)
    for t in range(T):
        qw, kw = q[t].copy(), k[t].copy()
        oracle.attention_core_step(qw, kw, v[t].copy(), qn, kn, kc, vc, heads, kvh, head, head, t, rope,
                                   np.float32(1e7), np.float32(1e-6), scores, want[t])

    def run(matrix_cores):
        A.reset()
        dq, dk, dv = ctx.upload_array(q), ctx.upload_array(k), ctx.upload_array(v)
        do = ctx.alloc(T * heads * head * 4)
        ctx.call("fortai_hip_qwen35_attention_prefill_core_device", A.h, dq.ptr, dk.ptr, dv.ptr, T, matrix_cores,
                 do.ptr)
        got = do.download(np.float32).reshape(T, heads * head)
        cache = A.cache(T)
        for b in (dq, dk, dv, do):
            b.free()
        return got, cache

    try:
        exact, (gk, gv) = run(0)
        n = T * kvh * head
        assert np.array_equal(gk, kc[:n]) and np.array_equal(gv, vc[:n]), "appended K/V must be bit-exact"
        if big:
            assert np.any((vc[:n] & 0x7c00) == 0x7c00), "the cache holds exponent-31 halves"
        diff = [t for t in range(T) if not same_values(exact[t], want[t])]
        assert not diff, f"exact prefill attention differs from the reference step at rows {diff[:8]}"
        if big:
            return  # the matrix-core kernel hands flagged caches to its fp32 companion (no tolerance case)
        fast, (fk, fv) = run(1)
        assert np.array_equal(fk, kc[:n]) and np.array_equal(fv, vc[:n])
        err = rel_err(fast, want)
        print(f"head {head} T {T}: matrix-core attention rel err {err:.3e}", flush=True)
        assert err <= FAST_ATT_REL
        assert np.all(np.isfinite(fast))
    finally:
        A.free()
        for w in ws:
            w.free()
