"""fortai_hip_q8_batch_matvec_noalloc: the batched matvec with its scratch in
the library's fixed per-GPU array (no allocation) against the allocating
entry point, bit for bit, on two calls in a row (the second smaller, so it
runs over what the first left in the array); that it allocates nothing (a
fresh context's on-demand scratch stays empty); that two contexts on one GPU
do not overwrite each other's activations; plus the size limit."""

import ctypes

import numpy as np
import pytest

from fortai_amd import backend as B
from fortai_amd import synth

pytestmark = pytest.mark.gpu


def _run(ctx, entry, w, x, batch, rows, *extra):
    dx = ctx.upload_array(x)
    out = ctx.alloc(batch * rows * 4)
    ctx.call(entry, ctx.h, w.h, dx.ptr, batch, out.ptr, *extra)
    got = out.download(np.float32).reshape(batch, rows)
    dx.free()
    out.free()
    return got


def test_noalloc_matches_allocating_entry_point(ctx):
    rng = np.random.default_rng(11)
    for rows, width, batch in ((3584, 2560, 8), (1024, 1024, 3)):
        w = B.Q8Weights(ctx, synth.q8_blocks(rng, rows, width), rows, width)
        x = rng.standard_normal((batch, width)).astype(np.float32)
        got = _run(ctx, "fortai_hip_q8_batch_matvec_noalloc", w, x, batch, rows)
        want = _run(ctx, "fortai_hip_q8_batch_matvec_device", w, x, batch, rows, None)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{rows}x{width} batch {batch}"
        w.free()


def test_noalloc_allocates_nothing(ctx):
    """On a fresh context the entry point leaves the context's on-demand
    scratch empty; the allocating entry point then fills it."""
    rng = np.random.default_rng(13)
    rows, width, batch = 1024, 2560, 8
    fresh = B.Context(0)
    try:
        w = B.Q8Weights(fresh, synth.q8_blocks(rng, rows, width), rows, width)
        x = rng.standard_normal((batch, width)).astype(np.float32)
        assert fresh.scratch_bytes() == 0
        first = _run(fresh, "fortai_hip_q8_batch_matvec_noalloc", w, x, batch, rows)
        second = _run(fresh, "fortai_hip_q8_batch_matvec_noalloc", w, x[:2], 2, rows)
        assert fresh.scratch_bytes() == 0, "the allocation-free entry point allocated scratch"
        want = _run(fresh, "fortai_hip_q8_batch_matvec_device", w, x, batch, rows, None)
        assert fresh.scratch_bytes() > 0
        assert np.array_equal(first.view(np.uint32), want.view(np.uint32))
        assert np.array_equal(second.view(np.uint32), want[:2].view(np.uint32))
        w.free()
    finally:
        fresh.close()


def test_noalloc_two_contexts_do_not_race(ctx):
    """Calls from two contexts (two streams) on one GPU, queued back to back
    without synchronising: each gets its own activations' outputs."""
    rng = np.random.default_rng(14)
    rows, width = 3584, 4096
    other = B.Context(0)
    try:
        wa = B.Q8Weights(ctx, synth.q8_blocks(rng, rows, width), rows, width)
        wb = B.Q8Weights(other, synth.q8_blocks(rng, rows, width), rows, width)
        xa = rng.standard_normal((8, width)).astype(np.float32)
        xb = rng.standard_normal((8, width)).astype(np.float32)
        want_a = _run(ctx, "fortai_hip_q8_batch_matvec_device", wa, xa, 8, rows, None)
        want_b = _run(other, "fortai_hip_q8_batch_matvec_device", wb, xb, 8, rows, None)
        bufs = []
        for c, w, x in ((ctx, wa, xa), (other, wb, xb), (ctx, wa, xa), (other, wb, xb)):
            dx, out = c.upload_array(x), c.alloc(8 * rows * 4)
            c.synchronize()
            c.call("fortai_hip_q8_batch_matvec_noalloc", c.h, w.h, dx.ptr, 8, out.ptr)
            bufs.append((c, dx, out))
        got = []
        for c, dx, out in bufs:
            c.synchronize()
            got.append(out.download(np.float32).reshape(8, rows))
            dx.free()
            out.free()
        for i, want in enumerate((want_a, want_b, want_a, want_b)):
            assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), f"call {i}"
        wa.free()
        wb.free()
    finally:
        other.close()


def test_noalloc_rejects_beyond_its_limit(ctx):
    rng = np.random.default_rng(12)
    rows, width = 64, 16416  # one 128-wide chunk past the limit at batch 8
    w = B.Q8Weights(ctx, synth.q8_blocks(rng, rows, width), rows, width)
    dx = ctx.alloc(8 * width * 4)
    out = ctx.alloc(8 * rows * 4)
    rc = B.load().fortai_hip_q8_batch_matvec_noalloc(ctx.h, w.h, dx.ptr, 8, out.ptr)
    assert rc == 1  # FORTAI_HIP_INVALID
    assert b"limit" in B.load().fortai_hip_q8_last_error(ctx.h)
    for b in (dx, out):
        b.free()
    w.free()
