"""fortai_hip_q8_batch_matvec_noalloc: the batched matvec with its scratch in
the library's fixed per-GPU array (no allocation) against the allocating
entry point, bit for bit, on two calls in a row (the second smaller, so it
runs over what the first left in the array), plus the size limit."""

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
