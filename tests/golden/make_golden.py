"""Write the golden vectors the CPU tests pin the oracle with.

Run in a container that has /root/reference (after ``make -C oracle ref``):

    python tests/golden/make_golden.py          # kernels + tiny models (seconds)
    python tests/golden/make_golden.py --full   # + the 0.8B 128-step trace (minutes)
    python tests/golden/make_golden.py --trace4096 [DUMP_DIR]
        # the 0.8B greedy trace over the whole 4096 context (hours on the CPU;
        # DUMP_DIR: an existing ref_dump output of that run to summarize)

Every expected value here comes from the reference's own CPU code compiled
from its sources by oracle/Makefile into oracle/_ref (the AVX2 kernels of
src/backend/cpu/fortai_q8_dot.c and the Fortran decode step of
src/models/qwen35/fortai_qwen35_cpu.f90 driven by oracle/ref_dump.f90).  The
inputs are seeded synthetic data; the tiny model is ``fortai_amd.synth``'s
``qwen35-tiny`` written with its default seed, so the GPU box can regenerate
it without this script.

Outputs (plain arrays, no pickles):
  tests/golden/kernels.npz   float_to_half, quantize, q8_dot, gdn_step, silu
  tests/golden/tiny_model.npz + .json, tiny_q8emb_model.npz + .json
                             (F16 / Q8_0 tied embedding): greedy trace, logits
                             of the first and last step, sha256 of every state
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import tempfile
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from fortai_amd import synth  # noqa: E402
from oracle.oracle import Reference  # noqa: E402

TINY_TOKEN = 17
TINY_STEPS = 24
TINY_CONTEXT = 64


def f2h_inputs(rng) -> np.ndarray:
    """Bit patterns that exercise every branch of the conversion."""
    pats = [rng.integers(0, 1 << 32, 4096, dtype=np.uint64).astype(np.uint32)]
    # every float exponent with fractions around the round bit (bit 12) and the carry
    exps = np.arange(256, dtype=np.uint32) << 23
    fr = np.array([0, 1, 0xfff, 0x1000, 0x1001, 0x1fff, 0x2000, 0x3000, 0x7fefff, 0x7ff000,
                   0x7fffff, 0x400000, 0x401000], dtype=np.uint32)
    grid = (exps[:, None] | fr[None, :]).reshape(-1)
    pats += [grid, grid | 0x80000000]
    return np.concatenate(pats).astype(np.uint32)


def kernels(ref: Reference, rng) -> dict:
    L = ref.lib
    g = {}
    bits = f2h_inputs(rng)
    g["f2h_in"] = bits
    g["f2h_out"] = np.array([L.fortai_float_to_half(float(v)) for v in bits.view(np.float32)],
                            dtype=np.uint16)

    x = (rng.standard_normal(32 * 16) * np.repeat(rng.uniform(0.01, 50, 16), 32)).astype(np.float32)
    x[32:64] = 0.0            # all-zero block: scale 0, quants 0
    x[64] = 1e-30             # tiny amax
    x[96:128] = 1e4           # constant block
    q = np.zeros(16 * 34, dtype=np.int8)
    s = np.zeros(16, dtype=np.float32)
    L.fortai_q8_quantize(x, q, s, x.size)
    g["quant_in"], g["quant_out"], g["quant_scales"] = x, q, s

    rows, nb = 6, 8
    w = rng.integers(-128, 128, (rows, nb, 34), dtype=np.int16).astype(np.int8)
    scales16 = rng.uniform(0.001, 0.1, (rows, nb)).astype(np.float16)
    w[:, :, :2] = scales16.view(np.int8).reshape(rows, nb, 2)
    w[0, 0, 2:] = -128        # vpmaddubsw pair saturation: |-128| * -128 twice
    a = rng.standard_normal(nb * 32).astype(np.float32)
    a[:32] = -5.0
    aq = np.zeros(nb * 34, dtype=np.int8)
    asc = np.zeros(nb, dtype=np.float32)
    L.fortai_q8_quantize(a, aq, asc, a.size)
    dots = np.array([L.fortai_q8_dot(np.ascontiguousarray(w[r]).reshape(-1), aq, asc, nb, 0)
                     for r in range(rows)], dtype=np.float32)
    g["dot_w"], g["dot_aq"], g["dot_as"], g["dot_out"] = w.reshape(-1), aq, asc, dots

    for head in (2, 16, 64):
        st = rng.standard_normal(head * head).astype(np.float32)
        k = rng.standard_normal(head).astype(np.float32)
        k /= np.float32(np.linalg.norm(k))
        v = rng.standard_normal(head).astype(np.float32)
        qv = rng.standard_normal(head).astype(np.float32)
        out = np.zeros(head, dtype=np.float32)
        g[f"gdn{head}_in"] = np.concatenate([st, k, v, qv])
        L.fortai_gdn_step(st, k, v, qv, np.float32(0.93), np.float32(0.4), head,
                          np.float32(1.0 / np.sqrt(head)), out)
        g[f"gdn{head}_state"], g[f"gdn{head}_out"] = st, out

    left = np.linspace(-25, 25, 1001).astype(np.float32)
    right = rng.uniform(0.5, 1.5, left.size).astype(np.float32)
    g["silu_left"], g["silu_right"] = left.copy(), right
    L.fortai_silu_product(left, right, left.size)
    g["silu_out"] = left
    return g


def tiny_model(ref: Reference, config: str) -> tuple[dict, dict]:
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "tiny.gguf")
        synth.write_model(path, synth.CONFIGS[config])
        out = os.path.join(tmp, "dump")
        res = ref.dump(path, TINY_TOKEN, TINY_STEPS, TINY_CONTEXT, out, state=True, threads=1)
        hashes = {}
        for name in sorted(os.listdir(out)):
            if name.startswith("layer"):
                with open(os.path.join(out, name), "rb") as f:
                    hashes[name] = hashlib.sha256(f.read()).hexdigest()
    arrays = {"tokens": res["tokens"], "logits_first": res["logits"][0],
              "logits_last": res["logits"][-1]}
    meta = {"model": config, "seed": "fortai_amd.synth default", "token": TINY_TOKEN,
            "steps": TINY_STEPS, "context": TINY_CONTEXT, "state_sha256": hashes}
    return arrays, meta


FULL_TOKEN = 9419   # greedy 128 steps from token 9419
FULL_STEPS = 128
FULL_CONTEXT = 4096
TOPK = 8


def full_model(ref: Reference, threads: int = 6) -> tuple[dict, dict]:
    """The 0.8B-shaped model of BASELINE config 4 (1.1 GB GGUF, written to a
    temporary directory): the 128-step greedy trace and, per step, the top-8
    logits (index, value) -- the full logits are 1 MB per step."""
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "m.gguf")
        synth.write_model(path, synth.CONFIGS["qwen35-0.8b"])
        res = ref.dump(path, FULL_TOKEN, FULL_STEPS, FULL_CONTEXT, os.path.join(tmp, "out"), threads=threads)
    return summarize_full(res["tokens"], res["logits"])


def summarize_full(tokens, logits):
    top_i = np.argsort(-logits, axis=1, kind="stable")[:, :TOPK].astype(np.int32)
    top_v = np.take_along_axis(logits, top_i, axis=1).astype(np.float32)
    arrays = {"tokens": np.asarray(tokens, dtype=np.int64), "top_index": top_i, "top_value": top_v}
    meta = {"model": "qwen35-0.8b", "seed": "fortai_amd.synth default", "token": FULL_TOKEN,
            "steps": FULL_STEPS, "context": FULL_CONTEXT,
            "min_top2_margin": float(np.min(top_v[:, 0] - top_v[:, 1]))}
    return arrays, meta


TRACE_STEPS = 4096
LAST_TOP = 64  # steps whose top-8 logits are kept


def trace4096(ref: Reference, dump_dir: Optional[str] = None, threads: int = 7) -> tuple[dict, dict]:
    """The 0.8B-shaped model's greedy trace from token 9419 over the whole
    4096-position context (the headline config), run by the compiled
    reference; per step the top-1/top-2 logit margin, and the top-8 logits of
    the last LAST_TOP steps.  The logits (4 GB) are read row by row."""
    with tempfile.TemporaryDirectory() as tmp:
        if dump_dir is None:
            path = os.path.join(tmp, "m.gguf")
            synth.write_model(path, synth.CONFIGS["qwen35-0.8b"])
            dump_dir = os.path.join(tmp, "out")
            ref.dump(path, FULL_TOKEN, TRACE_STEPS, FULL_CONTEXT, dump_dir, threads=threads, keep_logits=True)
        tokens = np.fromfile(os.path.join(dump_dir, "tokens.i64"), dtype=np.int64)
        logits = np.memmap(os.path.join(dump_dir, "logits.f32"), dtype=np.float32, mode="r").reshape(TRACE_STEPS, -1)
        margins = np.zeros(TRACE_STEPS, dtype=np.float32)
        top_i = np.zeros((LAST_TOP, TOPK), dtype=np.int32)
        top_v = np.zeros((LAST_TOP, TOPK), dtype=np.float32)
        for t in range(TRACE_STEPS):
            row = np.asarray(logits[t])
            idx = np.argsort(-row, kind="stable")[:TOPK]
            if int(idx[0]) != int(np.argmax(row)) or int(tokens[t]) != int(np.argmax(row)):
                raise SystemExit(f"step {t}: trace and logits disagree")
            margins[t] = row[idx[0]] - row[idx[1]]
            if t >= TRACE_STEPS - LAST_TOP:
                top_i[t - (TRACE_STEPS - LAST_TOP)] = idx
                top_v[t - (TRACE_STEPS - LAST_TOP)] = row[idx]
    arrays = {"tokens": tokens.astype(np.int64), "margin": margins, "last_top_index": top_i, "last_top_value": top_v}
    meta = {"model": "qwen35-0.8b", "seed": "fortai_amd.synth default", "token": FULL_TOKEN, "steps": TRACE_STEPS,
            "context": FULL_CONTEXT, "positions": f"0..{TRACE_STEPS - 1}",
            "min_top2_margin": float(margins.min()), "argmin_top2_margin": int(np.argmin(margins)),
            "last_top_steps": f"{TRACE_STEPS - LAST_TOP}..{TRACE_STEPS - 1}",
            "reference": "oracle/_ref/ref_dump (the reference's Fortran+C CPU path, -O2 -ffp-contract=off)"}
    return arrays, meta


def main() -> None:
    ref = Reference()
    if not ref.available or not ref.has("ref_dump"):
        sys.exit("oracle/_ref is not built (make -C oracle ref)")
    if "--trace4096" in sys.argv:
        rest = sys.argv[sys.argv.index("--trace4096") + 1:]
        arrays, meta = trace4096(ref, rest[0] if rest else None)
        np.savez_compressed(os.path.join(HERE, "qwen35_0.8b_trace_4096.npz"), **arrays)
        with open(os.path.join(HERE, "qwen35_0.8b_trace_4096.json"), "w") as f:
            json.dump(meta, f, indent=1, sort_keys=True)
        print("wrote the 4096-step trace")
        return
    if "--short-q8emb" in sys.argv:
        # the 0.8B layer shapes with a Q8_0 embedding: the C-ABI boundary test
        # of the reference's own device pipeline at those shapes
        arrays, meta = tiny_model(ref, "qwen35-0.8b-short-q8emb")
        np.savez_compressed(os.path.join(HERE, "short_q8emb_model.npz"), **arrays)
        with open(os.path.join(HERE, "short_q8emb_model.json"), "w") as f:
            json.dump(meta, f, indent=1, sort_keys=True)
        print("wrote short_q8emb_model")
        return
    rng = np.random.default_rng(0x60D)
    np.savez_compressed(os.path.join(HERE, "kernels.npz"), **kernels(ref, rng))
    for config, stem in (("qwen35-tiny", "tiny_model"), ("qwen35-tiny-q8emb", "tiny_q8emb_model")):
        arrays, meta = tiny_model(ref, config)
        np.savez_compressed(os.path.join(HERE, stem + ".npz"), **arrays)
        with open(os.path.join(HERE, stem + ".json"), "w") as f:
            json.dump(meta, f, indent=1, sort_keys=True)
    if "--full" in sys.argv:
        arrays, meta = full_model(ref)
        np.savez_compressed(os.path.join(HERE, "qwen35_0.8b_trace.npz"), **arrays)
        with open(os.path.join(HERE, "qwen35_0.8b_trace.json"), "w") as f:
            json.dump(meta, f, indent=1, sort_keys=True)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
