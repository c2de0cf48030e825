"""Token-block Q8_0 x Q8_0 products on the matrix cores, through the C ABI.

The reference runs every token through the Q8 matvec
(fortai_gguf_runtime.f90:424-465).  Bars: the per-token quantization and
the int32 block dots bit-exact against the oracle; the lane-order product
(mmq_exact, the prefill's default) bit-identical to the oracle's AVX2 matvec
of every token; the whole-block product (mmq, the fast variant) within 1e-5
relative of it (the north star allows 1e-3).
"""

import ctypes

import numpy as np
import pytest

from fortai_amd import backend as B
from fortai_amd import synth

pytestmark = pytest.mark.gpu

REL = 1e-3


def rel_err(got, want):
    want = np.asarray(want, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)) + 1e-30)
    return float(np.max(np.abs(got - want) / scale))


def tokens_layout(ctx, buf, tokens, width):
    """Split an X8 buffer into q [blocks][tokens][32] and s [blocks][tokens]."""
    ld = (tokens + 127) // 128 * 128
    bp = (width // 32 + 3) // 4 * 4
    raw = buf.download(np.uint8, ld * bp * 36)
    q = raw[: ld * bp * 32].view(np.int8).reshape(bp, ld, 32)
    s = raw[ld * bp * 32:].view(np.float32).reshape(bp, ld)
    return q, s, ld, bp


@pytest.mark.parametrize("rows,width,tokens", [(13, 96, 5), (200, 1024, 37), (3584, 1024, 64), (1024, 3584, 70)])
def test_mmq_block_dots_and_outputs(ctx, oracle, rows, width, tokens):
    rng = np.random.default_rng(rows * 31 + width + tokens)
    w = synth.q8_blocks(rng, rows, width)
    x = rng.standard_normal((tokens, width)).astype(np.float32)
    x[0, :32] = 0.0  # an all-zero block
    nb = width // 32
    W = B.Q8Weights(ctx, w, rows, width)
    dx = ctx.upload_array(x)
    nbytes = B.load().fortai_hip_q8_tokens_bytes(tokens, width)
    dq = ctx.alloc(nbytes)
    ctx.call("fortai_hip_q8_quantize_tokens_device", ctx.h, dx.ptr, tokens, width, dq.ptr)
    q, s, ld, bp = tokens_layout(ctx, dq, tokens, width)
    # quantization: each token as the reference quantizer, zero padding
    for t in range(tokens):
        qr, sr = oracle.quantize(x[t])
        qr = qr.reshape(nb, 34)[:, 2:]
        assert np.array_equal(q[:nb, t], qr)
        assert np.array_equal(s[:nb, t].view(np.uint32), sr.view(np.uint32))
    assert not q[:, tokens:].any() and not s[:, tokens:].any()
    assert not q[nb:].any() and not s[nb:].any()
    # exact int32 block dots
    dd = ctx.alloc(tokens * rows * nb * 4)
    ctx.call("fortai_hip_q8_mmq_block_dots", ctx.h, W.h, dq.ptr, tokens, dd.ptr)
    dots = dd.download(np.int32).reshape(tokens, rows, nb)
    for t in range(tokens):
        qr, _ = oracle.quantize(x[t])
        assert np.array_equal(dots[t], oracle.block_dots(w, qr, rows, nb)), f"token {t}"
    # fp32 outputs against the reference matvec of every token; then the
    # residual epilogue in place
    out = ctx.alloc(tokens * rows * 4)
    ms = ctypes.c_float()
    ctx.call("fortai_hip_q8_mmq_device", ctx.h, W.h, dq.ptr, tokens, out.ptr, None, ctypes.byref(ms))
    got = out.download(np.float32).reshape(tokens, rows)
    want = np.stack([oracle.matvec(w, rows, width, x[t]) for t in range(tokens)])
    assert rel_err(got, want) <= REL
    assert rel_err(got, want) <= 1e-5  # the block dots are exact: only fp32 rounding differs
    resid = rng.standard_normal((tokens, rows)).astype(np.float32)
    dr = ctx.upload_array(resid)
    ctx.call("fortai_hip_q8_mmq_device", ctx.h, W.h, dq.ptr, tokens, dr.ptr, dr.ptr, None)
    got2 = dr.download(np.float32).reshape(tokens, rows)
    assert np.array_equal(got2, (got + resid).astype(np.float32))
    W.free()


def test_mmq_prefill_shape(ctx, oracle):
    """A 4B FFN gate shape (9216 x 2560) over 512 tokens; the oracle checks a
    sample of tokens (size-independent: every token's row vector is its own
    matvec)."""
    rows, width, tokens = 9216, 2560, 512
    rng = np.random.default_rng(5)
    w = synth.q8_blocks(rng, rows, width)
    x = rng.standard_normal((tokens, width)).astype(np.float32)
    W = B.Q8Weights(ctx, w, rows, width)
    dx = ctx.upload_array(x)
    dq = ctx.alloc(B.load().fortai_hip_q8_tokens_bytes(tokens, width))
    ctx.call("fortai_hip_q8_quantize_tokens_device", ctx.h, dx.ptr, tokens, width, dq.ptr)
    out = ctx.alloc(tokens * rows * 4)
    ctx.call("fortai_hip_q8_mmq_device", ctx.h, W.h, dq.ptr, tokens, out.ptr, None, None)
    got = out.download(np.float32).reshape(tokens, rows)
    for t in (0, 1, 63, 64, 255, 511):
        assert rel_err(got[t], oracle.matvec(w, rows, width, x[t])) <= 1e-5, f"token {t}"
    W.free()


@pytest.mark.parametrize("rows,width,tokens", [(13, 96, 5), (200, 1024, 37), (88, 256, 21), (3584, 1024, 64),
                                               (1024, 3584, 70), (9216, 2560, 130)])
def test_mmq_lane_order_bit_identical(ctx, oracle, rows, width, tokens):
    """q8_mmq_exact_kernel: every output equals the reference matvec of its
    token bit for bit (ragged rows, in the first or the second 16-row half of
    a wave's rows, partial token tiles, a 4B FFN shape); the
    residual epilogue adds in place."""
    rng = np.random.default_rng(rows + 7 * width + tokens)
    w = synth.q8_blocks(rng, rows, width)
    x = rng.standard_normal((tokens, width)).astype(np.float32)
    x[0, :32] = 0.0
    x[1 % tokens, 32:64] = 1e4
    W = B.Q8Weights(ctx, w, rows, width)
    dx = ctx.upload_array(x)
    dq = ctx.alloc(B.load().fortai_hip_q8_tokens_bytes(tokens, width))
    ctx.call("fortai_hip_q8_quantize_tokens_device", ctx.h, dx.ptr, tokens, width, dq.ptr)
    out = ctx.alloc(tokens * rows * 4)
    ctx.call("fortai_hip_q8_mmq_exact_device", ctx.h, W.h, dq.ptr, tokens, out.ptr, None, None)
    got = out.download(np.float32).reshape(tokens, rows)
    sample = range(tokens) if tokens <= 70 else (0, 1, 63, 64, 65, 127, 128, 129)
    for t in sample:
        want = oracle.matvec(w, rows, width, x[t])
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), \
            f"token {t}: max rel {rel_err(got[t], want):.2e}"
    resid = rng.standard_normal((tokens, rows)).astype(np.float32)
    dr = ctx.upload_array(resid)
    ctx.call("fortai_hip_q8_mmq_exact_device", ctx.h, W.h, dq.ptr, tokens, dr.ptr, dr.ptr, None)
    assert np.array_equal(dr.download(np.float32).reshape(tokens, rows), (got + resid).astype(np.float32))
    W.free()
