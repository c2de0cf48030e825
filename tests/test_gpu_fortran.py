"""Fortran callers of libfortai_hip.so (GPU).

* fortai_amd/lib/hip_abi_smoke: this repository's iso_c_binding module driven
  from Fortran against the reference's known answers.
* oracle/_ref/ref_dump_hip: the reference's own model sources
  (src/models/qwen35/fortai_qwen35_cpu.f90, unmodified) compiled against
  fortai_amd/fortran/fortai_backend_cuda_on_hip.f90 instead of the CUDA
  binding.  enable_cuda(0) then runs the reference's device pipeline
  (fortai_qwen35_cpu.f90:287-384, 600-800) on this library; its greedy trace
  must equal the compiled reference CPU path's and its logits must be
  bit-identical to it (every per-op entry point keeps the CPU path's
  roundings), at the tiny shapes and at the 0.8B layer shapes.
* oracle/_ref/hip_plan_record: the fused and batched decoders created from
  Fortran over the reference model's own device layers; each step's
  launches recorded into the reference's plan_ir_t (src/fortai_plan_ir.f90)
  through fortai_amd/fortran/fortai_hip_plan.f90 and validated there.
* oracle/_ref/hip_pack_smoke: the Fortran pack cache
  (fortai_amd/fortran/fortai_hip_pack_cache.f90) keyed by the reference's
  pack_key_t / cache_path (src/fortai_cache.f90:6-31).  Matrices uploaded
  from a pack give the same matvec bits as the repacking upload; a pack
  written from Fortran reads in Python (fortai_amd/pack_cache.py) and one
  written from Python reads in Fortran.
"""
from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SMOKE = os.path.join(ROOT, "fortai_amd", "lib", "hip_abi_smoke")
REF_HIP = os.path.join(ROOT, "oracle", "_ref", "ref_dump_hip")
PACK_SMOKE = os.path.join(ROOT, "oracle", "_ref", "hip_pack_smoke")
PLAN_RECORD = os.path.join(ROOT, "oracle", "_ref", "hip_plan_record")
GOLDEN = os.path.join(ROOT, "tests", "golden")

pytestmark = pytest.mark.gpu


def test_fortran_abi_smoke():
    if not os.path.exists(SMOKE):
        pytest.fail("hip_abi_smoke is not built (fortai_amd.build.build())")
    r = subprocess.run([SMOKE], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0
    assert "fortran abi smoke ok" in r.stdout


def golden(stem):
    with np.load(os.path.join(GOLDEN, stem + ".npz")) as z:
        arrays = {k: z[k] for k in z.files}
    with open(os.path.join(GOLDEN, stem + ".json")) as f:
        return arrays, json.load(f)


@pytest.mark.parametrize("stem,graph", [("tiny_model", "0"), ("tiny_q8emb_model", "0"),
                                        ("tiny_q8emb_model", "1"), ("short_q8emb_model", "0"),
                                        ("short_q8emb_model", "1")])
def test_reference_model_on_hip_backend(tmp_path, stem, graph):
    if not os.path.exists(REF_HIP):
        pytest.skip("oracle/_ref/ref_dump_hip not built (needs /root/reference at build time)")
    from fortai_amd import synth
    arrays, meta = golden(stem)
    path = str(tmp_path / "m.gguf")
    synth.write_model(path, synth.CONFIGS[meta["model"]])
    out = tmp_path / "dump"
    out.mkdir()
    env = dict(os.environ, FORTAI_ENABLE_CUDA_GRAPH=graph, OMP_NUM_THREADS="4")
    print(f"ref_dump_hip {meta['model']} graph={graph}", flush=True)
    r = subprocess.run([REF_HIP, path, str(meta["token"]), str(meta["steps"]), str(meta["context"]),
                        str(out), "0", "1"], capture_output=True, text=True, timeout=300, env=env)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    logits = np.fromfile(out / "logits.f32", dtype=np.float32).reshape(meta["steps"], -1)
    tokens = np.fromfile(out / "tokens.i64", dtype=np.int64)
    assert list(tokens) == list(arrays["tokens"])
    for got, want in ((logits[0], arrays["logits_first"]), (logits[-1], arrays["logits_last"])):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            f"logits differ from the reference CPU path (max {float(np.max(np.abs(got - want))):.3e})"


@pytest.mark.parametrize("stem", ["tiny_q8emb_model", "short_q8emb_model"])
def test_plan_recorded_into_reference_plan_ir(tmp_path, stem):
    if not os.path.exists(PLAN_RECORD):
        pytest.skip("oracle/_ref/hip_plan_record not built (needs /root/reference at build time)")
    from fortai_amd import synth
    from fortai_amd.qwen35 import Qwen35Hip
    arrays, meta = golden(stem)
    path = str(tmp_path / "m.gguf")
    synth.write_model(path, synth.CONFIGS[meta["model"]])
    print(f"hip_plan_record {meta['model']}", flush=True)
    r = subprocess.run([PLAN_RECORD, path, str(meta["token"]), str(meta["steps"]), str(meta["context"])],
                       capture_output=True, text=True, timeout=300, env=dict(os.environ, OMP_NUM_THREADS="4"))
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "hip plan record ok" in r.stdout
    lines = r.stdout.splitlines()
    ids = lambda prefix: [int(t) for t in next(x for x in lines if x.startswith(prefix)).split()[len(prefix.split()):]]
    assert ids("trace ") == list(arrays["tokens"])
    assert ids("batch trace ") == list(arrays["tokens"])

    def plan(title):
        i = next(k for k, x in enumerate(lines) if x.startswith(title + " "))
        n = int(lines[i].split()[-1])
        steps = []
        for x in lines[i + 1:i + 1 + n]:
            op, kernel, batch = x.split(" ", 2)[2].split(" | ")
            steps.append((op, kernel, int(batch)))
        return steps

    fortran = plan("decoder plan")
    fbatch = plan("batch plan")
    m = Qwen35Hip(path, max_context=meta["context"], batch=2)
    try:
        # the same launches as the Python-side plan of the same model
        assert fortran == [tuple(s) for s in m.decoder.plan()]
        m.batch.generate([meta["token"]] * 2, [0, 0], 1)
        assert fbatch == [tuple(s) for s in m.batch.plan()]
    finally:
        m.close()
    d = synth.CONFIGS[meta["model"]]
    # the embedding (with the previous argmax finish), 5 steps per layer (an
    # attention layer's scores / softmax / output kernels form one step), the
    # Q8_0 LM head and its argmax
    assert len(fortran) == 1 + 5 * d.layers + 2
    kernels = " ".join(k for _, k, _ in fortran)
    for name in ("step_embedding_kernel", "q8_matvec_kernel", "gdn_delta_kernel", "attention_scores_kernel",
                 "attention_softmax_kernel", "attention_output_kernel"):
        assert name in kernels, name
    assert all(b == 1 for _, _, b in fortran) and all(b == 2 for _, _, b in fbatch)


def test_fortran_pack_cache(tmp_path):
    if not os.path.exists(PACK_SMOKE):
        pytest.skip("oracle/_ref/hip_pack_smoke not built (needs /root/reference at build time)")
    from fortai_amd import pack_cache, synth
    gguf = str(tmp_path / "m.gguf")
    synth.write_model(gguf, synth.CONFIGS["qwen35-tiny"])

    def run(root, mode):
        r = subprocess.run([PACK_SMOKE, gguf, str(root), mode], capture_output=True, text=True, timeout=120)
        print(r.stdout, r.stderr, flush=True)
        assert r.returncode == 0
        assert "fortran pack cache ok" in r.stdout
        return r.stdout.split("pack ", 1)[1].split("\n", 1)[0].strip()

    written = run(tmp_path / "fortran", "write")
    assert written == str(tmp_path / "fortran") + "/packsmoke/hip-gfx950-q8-lanes-abi1.pack"
    records = pack_cache.read(written, pack_cache.gguf_digest(gguf))
    assert records is not None, "the Fortran pack does not read in Python (format or digest differ)"
    assert {k: v[:2] for k, v in records.items()} == {"blk.0.a": (13, 96), "blk.0.bb": (200, 1024),
                                                      "output": (64, 256)}
    # the same records written from Python, read back by the Fortran program
    again = pack_cache.cache_path(str(tmp_path / "python"), pack_cache.PackKey("packsmoke", "hip-gfx950", "q8-lanes", 1))
    pack_cache.write(again, pack_cache.gguf_digest(gguf), records)
    assert open(again, "rb").read() == open(written, "rb").read()
    assert run(tmp_path / "python", "read") == again
