"""Fortran callers of libfortai_hip.so (GPU).

* fortai_amd/lib/hip_abi_smoke: this repository's iso_c_binding module driven
  from Fortran against the reference's known answers.
* oracle/_ref/ref_dump_hip: the reference's own model sources
  (src/models/qwen35/fortai_qwen35_cpu.f90, unmodified) compiled against
  fortai_amd/fortran/fortai_backend_cuda_on_hip.f90 instead of the CUDA
  binding.  enable_cuda(0) then runs the reference's device pipeline
  (fortai_qwen35_cpu.f90:287-384, 600-800) on this library; its greedy trace
  must equal the compiled reference CPU path's and its logits agree within
  1e-3 of the logit range.
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
                                        ("tiny_q8emb_model", "1")])
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
        scale = float(np.max(np.abs(want)))
        assert float(np.max(np.abs(got - want))) <= 1e-3 * scale
