"""GPU parity of each hot-path kernel against the oracle, through the C ABI.

Bars: per-block int32 Q8_0 dots and KV-cache
contents bit-exact; fp32 outputs within 1e-3 relative.  Where this backend
reproduces the reference's lane order exactly (Q8 matvec, GDN step, F16 LM
head) the tests demand bit-identical floats, which is stricter.
"""

import os

import numpy as np
import pytest

from fortai_amd import backend as B
from fortai_amd import synth

pytestmark = pytest.mark.gpu

REL = 1e-3  # north_star fp32 tolerance


def rel_err(got, want):
    """max |got - want| / max(|want|, rms(want)) elementwise (1e-3 gate)."""
    want = np.asarray(want, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    scale = np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)) + 1e-30)
    return float(np.max(np.abs(got - want) / scale))


def quantize_case(n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32)
    x[:32] = 0.0                           # all-zero block -> scale 0, inverse 0
    x[32:64] = np.linspace(-3.5, 3.5, 32)  # values that land on .5 after scaling
    x[64:96] *= 1e-6                       # subnormal-range fp16 scales
    x[96:128] *= 1e4
    return x


@pytest.mark.parametrize("n", [128, 1024, 3584])
def test_quantize_bit_exact(ctx, oracle, n):
    x = quantize_case(n, 11 + n)
    q_ref, s_ref = oracle.quantize(x)
    dx = ctx.upload_array(x)
    dq = ctx.alloc(q_ref.nbytes)
    ds = ctx.alloc(s_ref.nbytes)
    ctx.call("fortai_hip_q8_quantize_device", ctx.h, dx.ptr, n, dq.ptr, ds.ptr)
    q = dq.download(np.int8)
    s = ds.download(np.float32)
    assert np.array_equal(q, q_ref)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("rows,width", [(3584, 1024), (13, 96), (1024, 3584), (16, 1024), (9216, 2560),
                                        (2560, 9216), (8192, 2560), (2560, 4096)])
def test_block_dots_and_matvec_bit_exact(ctx, oracle, rows, width):
    rng = np.random.default_rng(rows * 7 + width)
    w = synth.q8_blocks(rng, rows, width)
    x = rng.standard_normal(width).astype(np.float32)
    q, s = oracle.quantize(x)
    nb = width // 32
    W = B.Q8Weights(ctx, w, rows, width)
    dq = ctx.upload_array(q)
    dd = ctx.alloc(rows * nb * 4)
    ctx.call("fortai_hip_q8_block_dots_device", ctx.h, W.h, dq.ptr, dd.ptr)
    dots = dd.download(np.int32).reshape(rows, nb)
    assert np.array_equal(dots, oracle.block_dots(w, q, rows, nb))
    # resident matvec on the pre-quantized activation
    out = ctx.alloc(rows * 4)
    import ctypes
    ms = ctypes.c_float()
    ctx.call("fortai_hip_q8_matvec_resident", ctx.h, W.h, dq.ptr, out.ptr, ctypes.byref(ms))
    want = oracle.matvec(w, rows, width, x)
    got = out.download(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # f32 activation, quantized inside the kernel
    dx = ctx.upload_array(x)
    out2 = ctx.alloc(rows * 4)
    ctx.call("fortai_hip_q8_matvec_device_f32", ctx.h, W.h, dx.ptr, width, out2.ptr, rows)
    assert np.array_equal(out2.download(np.float32).view(np.uint32), want.view(np.uint32))
    W.free()


def test_matvec_denormal_and_zero_scales(ctx, oracle):
    """Weight scales that are fp16 subnormals (both signs) or zeros, and
    activation blocks so small that their Q8_0 scales are fp16 subnormals or
    zero: the scale products fl(f32(w_scale) * a_scale) widen the halves
    exactly whatever their class (F16C, fortai_q8_dot.c:305-318), so every
    matvec output is still bit-identical to the reference."""
    rng = np.random.default_rng(0xDE40)
    rows, width = 512, 2048
    w = synth.q8_blocks(rng, rows, width)
    nb = width // 32
    pick = rng.random((rows, nb))
    sub = (rng.integers(1, 0x400, size=(rows, nb)) | (rng.integers(0, 2, size=(rows, nb)) << 15)).astype(np.uint16)
    zero = np.where(rng.integers(0, 2, size=(rows, nb)) == 0, 0x0000, 0x8000).astype(np.uint16)
    bits = w[:, :, 0:2].copy().view(np.uint16)[..., 0]
    bits = np.where(pick < 0.3, sub, np.where(pick < 0.35, zero, bits)).astype(np.uint16)
    w[:, :, 0:2] = bits[..., None].view(np.uint8).reshape(rows, nb, 2)
    x = rng.standard_normal(width).astype(np.float32)
    tiny = rng.choice(nb, size=nb // 3, replace=False)
    for b in tiny:  # amax / 127 below the smallest normal half (6.1e-5), some below half the smallest subnormal
        x[32 * b:32 * b + 32] *= np.float32(rng.choice([1e-3, 1e-4, 1e-5, 1e-7]))
    q, s_ = oracle.quantize(x)
    assert np.any((s_ != 0) & (np.abs(s_) < 6.1e-5)) and np.any(s_ == 0), "the activation has subnormal and zero scales"
    want = oracle.matvec(w, rows, width, x)
    W = B.Q8Weights(ctx, w, rows, width)
    dx = ctx.upload_array(x)
    out = ctx.alloc(rows * 4)
    ctx.call("fortai_hip_q8_matvec_device_f32", ctx.h, W.h, dx.ptr, width, out.ptr, rows)
    got = out.download(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"max diff {np.max(np.abs(got - want))}"
    W.free()


def smoke_tensor(rows_scale):
    """The reference smoke test's Q8 tensors (test_fortai_smoke.f90:221-265)."""
    b = np.zeros((len(rows_scale), 34), dtype=np.uint8)
    for r, mult in enumerate(rows_scale):
        b[r, 1] = 0x3C                       # fp16 1.0
        b[r, 2:] = (np.arange(1, 33) * mult).astype(np.int8).view(np.uint8)
    return b


def test_reference_smoke_goldens_host_paths(ctx):
    """527.9677734375 / 1055.935546875 / 1583.9033203125 (test_fortai_smoke.f90:229-265)."""
    import ctypes
    from oracle.oracle import Oracle
    o = Oracle()
    t1 = B.Q8Weights(ctx, smoke_tensor([1]), 1, 32)
    t2 = B.Q8Weights(ctx, smoke_tensor([1, 2]), 2, 32)
    t3 = B.Q8Weights(ctx, smoke_tensor([3]), 1, 32)
    q, _ = o.quantize(np.ones(32, dtype=np.float32))
    ms = ctypes.c_float()
    out1 = np.zeros(1, np.float32)
    ctx.call("fortai_hip_q8_matvec_host", ctx.h, t1.h, q.ctypes.data, q.nbytes, out1.ctypes.data, 4, ctypes.byref(ms))
    assert abs(float(out1[0]) - 527.9677734375) < 1e-4
    o1, o2, o3 = np.zeros(1, np.float32), np.zeros(2, np.float32), np.zeros(1, np.float32)
    ctx.call("fortai_hip_q8_matvec_host_triplet", ctx.h, t1.h, t2.h, t3.h, q.ctypes.data, q.nbytes,
             o1.ctypes.data, 4, o2.ctypes.data, 8, o3.ctypes.data, 4, ctypes.byref(ms))
    got = np.concatenate([o1, o2, o3]).astype(np.float64)
    assert np.max(np.abs(got - [527.9677734375, 527.9677734375, 1055.935546875, 1583.9033203125])) < 1e-4
    flat = np.zeros(4, np.float32)
    ctx.call("fortai_hip_q8_matvec_host_triplet_contiguous", ctx.h, t1.h, t2.h, t3.h, q.ctypes.data, q.nbytes,
             flat.ctypes.data, 16, ctypes.byref(ms))
    assert np.array_equal(flat, got.astype(np.float32))
    p1, p2 = np.zeros(2, np.float32), np.zeros(2, np.float32)
    ctx.call("fortai_hip_q8_matvec_host_pair", ctx.h, t2.h, t2.h, q.ctypes.data, q.nbytes, p1.ctypes.data, 8,
             p2.ctypes.data, 8, ctypes.byref(ms))
    assert np.array_equal(p1, p2) and np.array_equal(p1, o2)
    for t in (t1, t2, t3):
        t.free()


def test_ffn_device_and_host(ctx, oracle):
    rng = np.random.default_rng(5)
    H, F = 1024, 3584
    g, u, d = synth.q8_blocks(rng, F, H), synth.q8_blocks(rng, F, H), synth.q8_blocks(rng, H, F)
    x = rng.standard_normal(H).astype(np.float32)
    gate = oracle.matvec(g, F, H, x)
    up = oracle.matvec(u, F, H, x)
    oracle.silu_product(gate, up, F)
    want = oracle.matvec(d, H, F, gate)
    G, U, D = B.Q8Weights(ctx, g, F, H), B.Q8Weights(ctx, u, F, H), B.Q8Weights(ctx, d, H, F)
    dx, out = ctx.upload_array(x), ctx.alloc(H * 4)
    ctx.call("fortai_hip_q8_ffn_device", ctx.h, G.h, U.h, D.h, dx.ptr, H, out.ptr, H)
    got = out.download(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    import ctypes
    q, _ = oracle.quantize(x)
    host = np.zeros(H, np.float32)
    ms = ctypes.c_float()
    ctx.call("fortai_hip_q8_ffn_host", ctx.h, G.h, U.h, D.h, q.ctypes.data, q.nbytes, host.ctypes.data, H * 4,
             ctypes.byref(ms))
    assert np.array_equal(host.view(np.uint32), want.view(np.uint32))
    for t in (G, U, D):
        t.free()


def test_rms_norm_add_copy(ctx, oracle):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(1024) * 30).astype(np.float32)
    w = (1 + 0.05 * rng.standard_normal(1024)).astype(np.float32)
    want = np.zeros_like(x)
    oracle.rms_norm(x, w, np.float32(1e-6), want, 1024)
    dx, dw, do = ctx.upload_array(x), ctx.upload_array(w), ctx.alloc(4096)
    ctx.call("fortai_hip_qwen35_rms_norm_device", ctx.h, dx.ptr, dw.ptr, do.ptr, 1024, 1e-6)
    got = do.download(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ctx.call("fortai_hip_qwen35_add_device", ctx.h, dx.ptr, dw.ptr, do.ptr, 1024)
    assert np.array_equal(do.download(np.float32), x + w)
    ctx.call("fortai_hip_qwen35_copy_device", ctx.h, dw.ptr, do.ptr, 4096)
    assert np.array_equal(do.download(np.float32), w)


def gdn_layer_for_core(ctx, rng, H=1024, heads=16, head=128, kernel=4):
    """A recurrent layer object whose projections are unused by the core step."""
    inner = heads * head
    conv = 2 * head * heads + inner
    mk = lambda rows, width: B.Q8Weights(ctx, synth.q8_blocks(rng, rows, width), rows, width)
    ws = [mk(conv, H), mk(inner, H), mk(heads, H), mk(heads, H), mk(H, inner)]
    conv_w = (rng.standard_normal(conv * kernel) * 0.1).astype(np.float32)
    ssm_a = -np.ones(heads, np.float32)  # decay = exp(-softplus(alpha)) with dt = 0
    ssm_dt = np.zeros(heads, np.float32)
    norm = np.ones(head, np.float32)
    layer = B.Recurrent(ctx, *ws, conv_w, conv, kernel, ssm_a, ssm_dt, norm, head, heads, heads, head, inner, 1e-6)
    return layer, ws, conv_w, ssm_a, ssm_dt, conv


def test_gdn_core_128_steps(ctx, oracle):
    """16 heads x 128, state ~ N(0, 0.02), 128 autoregressive
    steps, through both the per-step entry point (conv1d + SiLU kernel, then the
    delta-rule kernel) and the state-resident one (all 128 steps in one
    launch): every output, the GDN state and the conv windows bit-identical to
    the oracle's."""
    rng = np.random.default_rng(0x35A08B)
    heads, head, kernel, steps = 16, 128, 4, 128
    layer, ws, conv_w, ssm_a, ssm_dt, conv = gdn_layer_for_core(ctx, rng)
    state = (rng.standard_normal(heads * head * head) * 0.02).astype(np.float32)
    cstate = (rng.standard_normal((kernel - 1) * conv) * 0.5).astype(np.float32)
    qkv = rng.standard_normal((steps, conv)).astype(np.float32)
    alpha = rng.standard_normal((steps, heads)).astype(np.float32)
    beta = rng.standard_normal((steps, heads)).astype(np.float32)
    ref_state, ref_conv = state.copy(), cstate.copy()
    work = np.zeros(conv, np.float32)
    want = np.zeros((steps, heads * head), np.float32)
    for t in range(steps):
        oracle.gdn_core_step(qkv[t], alpha[t], beta[t], ssm_a, ssm_dt, conv_w, ref_conv, ref_state, conv, kernel, head,
                             heads, heads, head, np.float32(1e-6), work, want[t])
    bits = lambda a: np.asarray(a, np.float32).view(np.uint32)
    # per step
    layer.set_state(state, cstate)
    dq, da, db, do = ctx.alloc(conv * 4), ctx.alloc(heads * 4), ctx.alloc(heads * 4), ctx.alloc(heads * head * 4)
    for t in range(steps):
        dq.upload(qkv[t]); da.upload(alpha[t]); db.upload(beta[t])
        ctx.call("fortai_hip_qwen35_recurrent_core_device", layer.h, dq.ptr, da.ptr, db.ptr, do.ptr)
        assert np.array_equal(bits(do.download(np.float32)), bits(want[t])), f"per-step output {t}"
    gdn, cst = layer.state()
    assert np.array_equal(bits(cst), bits(ref_conv))
    assert np.array_equal(bits(gdn), bits(ref_state))
    # state-resident: the 128 steps in one launch
    layer.set_state(state, cstate)
    dQ, dA, dB = ctx.upload_array(qkv), ctx.upload_array(alpha), ctx.upload_array(beta)
    dO = ctx.alloc(steps * heads * head * 4)
    ctx.call("fortai_hip_qwen35_recurrent_core_steps_device", layer.h, dQ.ptr, dA.ptr, dB.ptr, steps, dO.ptr)
    got = dO.download(np.float32).reshape(steps, heads * head)
    first = next((t for t in range(steps) if not np.array_equal(bits(got[t]), bits(want[t]))), None)
    assert first is None, f"state-resident output differs from step {first}"
    gdn, cst = layer.state()
    assert np.array_equal(bits(cst), bits(ref_conv))
    assert np.array_equal(bits(gdn), bits(ref_state))
    for b in (dq, da, db, do, dQ, dA, dB, dO):
        b.free()
    layer.free()
    for w in ws:
        w.free()


@pytest.mark.parametrize("L,exact_max,skew", [(1, None, 0), (70, None, 0), (1024, None, 0), (4096, None, 0),
                                              (32768, None, 0), (32768, 1 << 20, 0), (70, 0, 0), (1024, 0, 0),
                                              (4095, 0, 0), (4096, None, 60), (4096, None, 1 << 20),
                                              (8192, None, -90), (8192, None, 0), (5000, None, 0)])
def test_attention_core(ctx, oracle, L, exact_max, skew):
    """8 q / 2 kv heads x 256, fp16 cache, RoPE 1e7, append + attend at position L-1.
    Up to the layer's exact_max positions (default 8192; fortai_hip_qwen35_attention_set_exact_max) the output keeps the reference's two-pass
    summation orders and is bit-exact; beyond it, split-K with an online-softmax merge, within the north
    star's 1e-3 relative.  exact_max None: the default; 1 << 20: exact at 32768; 0: split-K at every L.
    skew: the test option z_skew, which moves the Z candidate windows so that some (60, -90) or all
    (1 << 20) running sums fall outside them and the resolution's own chain runs."""
    rng = np.random.default_rng(L)
    heads, kvh, head, H = 8, 2, 256, 1024
    mk = lambda rows, width: B.Q8Weights(ctx, synth.q8_blocks(rng, rows, width), rows, width)
    ws = [mk(heads * 2 * head, H), mk(kvh * head, H), mk(kvh * head, H), mk(H, heads * head)]
    qn = (1 + 0.05 * rng.standard_normal(head)).astype(np.float32)
    kn = (1 + 0.05 * rng.standard_normal(head)).astype(np.float32)
    maxc = max(L, 64)
    A = B.Attention(ctx, *ws, qn, kn, heads, kvh, head, head, maxc, 64, 1.0e7, 1e-6)
    if exact_max is not None:
        A.set_exact_max(exact_max)
    A.set_test_options(z_skew=skew)
    kc = np.zeros(maxc * kvh * head, np.uint16)
    vc = np.zeros(maxc * kvh * head, np.uint16)
    n = (L - 1) * kvh * head
    kc[:n] = rng.standard_normal(n).astype(np.float16).view(np.uint16)
    vc[:n] = rng.standard_normal(n).astype(np.float16).view(np.uint16)
    A.set_cache(kc, vc, maxc)
    q = rng.standard_normal(heads * 2 * head).astype(np.float32)
    k = rng.standard_normal(kvh * head).astype(np.float32)
    v = rng.standard_normal(kvh * head).astype(np.float32)
    ctx.set_position(L - 1)
    dq, dk, dv, do = ctx.upload_array(q), ctx.upload_array(k), ctx.upload_array(v), ctx.alloc(heads * head * 4)
    ctx.call("fortai_hip_qwen35_attention_core_device", A.h, dq.ptr, dk.ptr, dv.ptr, do.ptr)
    got = do.download(np.float32)
    want = np.zeros(heads * head, np.float32)
    scores = np.zeros(maxc, np.float32)
    qw, kw = q.copy(), k.copy()
    oracle.attention_core_step(qw, kw, v, qn, kn, kc, vc, heads, kvh, head, head, L - 1, 64, np.float32(1e7),
                               np.float32(1e-6), scores, want)
    gk, gv = A.cache(L)
    assert np.array_equal(gk, kc[:L * kvh * head]), "K cache after append must be bit-exact"
    assert np.array_equal(gv, vc[:L * kvh * head]), "V cache after append must be bit-exact"
    limit = 8192 if exact_max is None else exact_max
    if L <= limit:
        # the reference's two-pass softmax with its summation orders: bit-exact
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"max diff {np.max(np.abs(got - want))}"
    else:
        assert rel_err(got, want) <= REL, f"split-K attention off by {rel_err(got, want)}"
        assert not np.array_equal(got, np.zeros_like(got))
    A.free()
    for w in ws:
        w.free()


def same_values(a, b):
    """Bit-identical, NaNs only at the same places (their payloads are not part
    of the reference's arithmetic)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


@pytest.mark.parametrize("L,wide,big", [(70, 0, True), (1024, 0, True), (70, 1, False), (600, 1, False),
                                        (4096, 1, False), (600, 1, True), (4096, 1, True)])
def test_attention_output_kernels(ctx, oracle, L, wide, big):
    """The exact attention output of one sequence through the per-slice kernel
    (wide 0, the decode's) or the batches' wide kernel (wide 1, selected for one
    sequence by the test option force_wide), against the reference step.
    big: exponent-31 halves in value dims 0..19 of kv head 0 at every 7th
    position, which the reference reads as +-huge (gguf_fp16_to_real,
    fortai_gguf_runtime.f90:770-788): those dims of that kv head's heads sum
    terms of ~1e36 (or overflow), and every output, huge or not, must be
    bit-identical through the kernels' flagged instances."""
    rng = np.random.default_rng(L + 7 * wide + big)
    heads, kvh, head, H = 8, 2, 256, 1024
    mk = lambda rows, width: B.Q8Weights(ctx, synth.q8_blocks(rng, rows, width), rows, width)
    ws = [mk(heads * 2 * head, H), mk(kvh * head, H), mk(kvh * head, H), mk(H, heads * head)]
    qn = (1 + 0.05 * rng.standard_normal(head)).astype(np.float32)
    kn = (1 + 0.05 * rng.standard_normal(head)).astype(np.float32)
    maxc = max(L, 64)
    A = B.Attention(ctx, *ws, qn, kn, heads, kvh, head, head, maxc, 64, 1.0e7, 1e-6)
    A.set_test_options(force_wide=bool(wide))
    kc = np.zeros(maxc * kvh * head, np.uint16)
    vc = np.zeros(maxc * kvh * head, np.uint16)
    n = (L - 1) * kvh * head
    kc[:n] = rng.standard_normal(n).astype(np.float16).view(np.uint16)
    vc[:n] = rng.standard_normal(n).astype(np.float16).view(np.uint16)
    if big:
        rows = np.arange(0, L - 1, 7)
        idx = (rows[:, None] * kvh * head + np.arange(20)[None, :]).ravel()
        vc[idx] = (vc[idx] & 0x83ff) | 0x7c00  # exponent 31, the sign and fraction kept
    A.set_cache(kc, vc, maxc)
    q = rng.standard_normal(heads * 2 * head).astype(np.float32)
    k = rng.standard_normal(kvh * head).astype(np.float32)
    v = rng.standard_normal(kvh * head).astype(np.float32)
    ctx.set_position(L - 1)
    dq, dk, dv, do = ctx.upload_array(q), ctx.upload_array(k), ctx.upload_array(v), ctx.alloc(heads * head * 4)
    try:
        ctx.call("fortai_hip_qwen35_attention_core_device", A.h, dq.ptr, dk.ptr, dv.ptr, do.ptr)
        got = do.download(np.float32)
        want = np.zeros(heads * head, np.float32)
        scores = np.zeros(maxc, np.float32)
        oracle.attention_core_step(q.copy(), k.copy(), v, qn, kn, kc, vc, heads, kvh, head, head, L - 1, 64,
                                   np.float32(1e7), np.float32(1e-6), scores, want)
        if big:  # those dims carry the huge terms (|out| ~ 1e36, or beyond: inf / NaN)
            huge = ~np.isfinite(want) | (np.abs(want) > 1e30)
            assert 0 < huge.sum() < heads * head // 2
        assert same_values(got, want), f"{int(np.sum(got.view(np.uint32) != want.view(np.uint32)))} outputs differ"
    finally:
        for b_ in (dq, dk, dv, do):
            b_.free()
        A.free()
        for w in ws:
            w.free()


def test_f16_lm_head_and_argmax(ctx, oracle):
    rng = np.random.default_rng(3)
    rows, width = 248320, 1024
    w = (rng.standard_normal(rows * width, dtype=np.float32) * 0.02).astype(np.float16)
    x = rng.standard_normal(width).astype(np.float32)
    W = B.F16Weights(ctx, w, rows, width)
    dx, do, dt = ctx.upload_array(x), ctx.alloc(rows * 4), ctx.alloc(8)
    ctx.call("fortai_hip_f16_matvec_device", ctx.h, W.h, dx.ptr, width, do.ptr, rows, dt.ptr)
    got = do.download(np.float32)
    # the reference's sequential fp32 chain, evaluated with numpy in the same order
    wt = np.ascontiguousarray(w.reshape(rows, width).T).astype(np.float32)
    acc = np.zeros(rows, np.float32)
    for i in range(width):
        acc = acc + wt[i] * x[i]
    assert np.array_equal(got.view(np.uint32), acc.view(np.uint32))
    assert int(dt.download(np.int64)[0]) == int(np.argmax(acc))
    # standalone argmax with a tie: the first index wins
    vals = np.zeros(100000, np.float32)
    vals[[777, 50000]] = 3.0
    dv = ctx.upload_array(vals)
    ctx.call("fortai_hip_argmax_device", ctx.h, dv.ptr, vals.size, dt.ptr)
    assert int(dt.download(np.int64)[0]) == 777
    # every value NaN: no comparison succeeds and the first index is returned
    # (the oracle's maxloc); the id is always inside the vector
    dn = ctx.upload_array(np.full(100000, np.nan, np.float32))
    ctx.call("fortai_hip_argmax_device", ctx.h, dn.ptr, 100000, dt.ptr)
    assert int(dt.download(np.int64)[0]) == 0
    W.free()
