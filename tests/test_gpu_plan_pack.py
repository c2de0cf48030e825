"""PlanIR recording of the kernels each decoder launches, and the
repacked-weight cache (survey rank-4 items: src/fortai_plan_ir.f90:7-21,
src/fortai_cache.f90:6-31), through the C ABI."""

import numpy as np
import pytest

from fortai_amd import backend as B
from fortai_amd import synth
from fortai_amd.qwen35 import Qwen35Hip

pytestmark = pytest.mark.gpu


def test_decoder_plans(tiny_model_path):
    m = Qwen35Hip(tiny_model_path, max_context=64, batch=3)
    try:
        d = m.d
        plan = m.decoder.plan()
        # embedding, five launches per layer (three for the mixer, two for the
        # FFN), the LM head with its argmax
        assert len(plan) == 2 + 5 * d.layers
        assert plan[0][0] == "token embedding" and "embedding_kernel" in plan[0][1]
        assert plan[-1][0].startswith("output RMSNorm")
        assert all(b == 1 for _, _, b in plan)
        kernels = " ".join(k for _, k, _ in plan)
        for name in ("q8_matvec_kernel", "gdn_delta_kernel", "attention_scores_kernel", "attention_output_kernel"):
            assert name in kernels
        bplan = m.batch.plan()
        assert bplan and all(b == 3 for _, _, b in bplan)
        assert any("q8_batch" in k for _, k, _ in bplan)
        m.batch.reset()
        m.batch.prefill(np.array([[1, 2, 3]] * 3))
        pplan = m.batch.plan(prefill=True)
        assert any(k.startswith("q8_mmq_exact_kernel") for _, k, _ in pplan)
        assert any("attention_prefill_exact" in k for _, k, _ in pplan)
        assert all(b == 9 for _, _, b in pplan)
    finally:
        m.close()


def test_packed_weights_round_trip(ctx):
    import ctypes
    rng = np.random.default_rng(4)
    rows, width = 1000, 2560
    W = B.Q8Weights(ctx, synth.q8_blocks(rng, rows, width), rows, width)
    planes = W.pack()
    assert planes.nbytes == B.load().fortai_hip_q8_pack_bytes(rows, width)
    W2 = B.Q8Weights.from_packed(ctx, planes, rows, width)
    assert np.array_equal(W2.pack(), planes)
    x = rng.standard_normal((3, width)).astype(np.float32)
    dx = ctx.upload_array(x)
    outs = []
    for w in (W, W2):
        out = ctx.alloc(3 * rows * 4)
        ctx.call("fortai_hip_q8_batch_matvec_device", ctx.h, w.h, dx.ptr, 3, out.ptr, None)
        outs.append(out.download(np.float32))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    W.free()
    W2.free()


def test_model_from_pack_cache(tiny_model_path, tmp_path):
    root = str(tmp_path / "packs")
    traces = []
    for expect_pack in (False, True):
        m = Qwen35Hip(tiny_model_path, max_context=64, pack_cache=root)
        try:
            assert m.loaded_from_pack == expect_pack
            m.reset()
            traces.append(m.generate(9, 24).tolist())
        finally:
            m.close()
    assert traces[0] == traces[1]
