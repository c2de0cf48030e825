#!/usr/bin/env python3
"""bench.py -- Qwen3.5-0.8B-shaped Q8_0 greedy decode at context 4096 on one MI355X.

Metric: decode tokens/s at batch 1 and context 4096, plus the
Q8_0 matvec HBM GB/s of BASELINE config 1.

A "step" is one greedy decode token of BASELINE config 4 (hidden 1024, 24
layers 3:1 GDN:attention, FFN 3584, vocab 248320, tied fp16 embedding),
synthetic random-init Q8_0 weights from fortai_amd.synth (seeded; no
checkpoint exists offline).  The KV caches are filled by real decoding from
position 0, so the K timed steps run at positions 4096-K .. 4095 and attend
over ~4096 positions.  Each step is one replay of the decoder's HIP graph;
the greedy token and the position advance on the device, so the timed region
holds no host round trip.  All weights are resident in HBM before timing.

The greedy ids of all 4096 positions (cache fill, warm-up, timed steps) are
compared with the compiled reference's 4096-step trace (`trace`).

Also reported:
  roofline      -- the dominant kernel family, every Q8_0 matvec launch of a
                   decode step, timed live with HIP events on the context
                   stream (a graph of exactly those launches);
  roofline_lm_head -- the fp16 LM head + fused argmax (508.6 MB per launch);
  matvec        -- BASELINE config 1 (3584 x 1024 Q8_0, quantize + GEMV) over
                   275 distinct weight copies (1.07 GB, beyond the 256 MB
                   Infinity Cache), as a captured graph of back-to-back launches;
  cpu_baseline  -- the reference CPU path (oracle/_ref/fortai_cpu_run, compiled
                   from the reference's own sources) on this host, bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
START_TOKEN = 9419


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_path(args) -> str:
    from fortai_amd import synth
    path = args.model or os.path.join(os.environ.get("TMPDIR", "/tmp"), "fortai_bench", "qwen35-0.8b.gguf")
    if not os.path.exists(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        log(f"writing the synthetic Qwen3.5-0.8B GGUF to {path}")
        t = time.time()
        synth.write_model(path + ".part", synth.CONFIGS["qwen35-0.8b"])
        os.replace(path + ".part", path)
        log(f"  done in {time.time() - t:.1f}s")
    return path


def bytes_per_token(d, L: int) -> float:
    """Algorithmic HBM bytes of one decode step at context length L: every
    weight once, GDN state read+write, conv window, KV read of L positions."""
    q8 = lambda rows, width: rows * (width // 32) * 34
    ffn = 3 * q8(d.ffn, d.hidden)
    gdn_w = q8(d.conv_size, d.hidden) + q8(d.inner, d.hidden) + 2 * q8(d.value_heads, d.hidden) + q8(d.hidden, d.inner)
    attn_w = q8(2 * d.heads * d.head_size, d.hidden) + 2 * q8(d.kv_heads * d.head_size, d.hidden) + \
        q8(d.hidden, d.heads * d.value_size)
    n_attn = sum(1 for i in range(d.layers) if (i + 1) % d.interval == 0)
    n_gdn = d.layers - n_attn
    gdn_state = 2 * d.value_heads * d.gdn_head ** 2 * 4
    conv = d.conv_size * d.conv_kernel * 4 + (d.conv_kernel - 1) * d.conv_size * 4 * 2
    kv = 2 * L * d.kv_heads * d.head_size * 2
    lm_head = d.vocab * d.hidden * 2
    return d.layers * ffn + n_gdn * (gdn_w + gdn_state + conv) + n_attn * (attn_w + kv) + lm_head + d.hidden * 2


def bench_decode(args, path):
    from fortai_amd.qwen35 import Qwen35Hip
    ctx_len = args.ctx
    log(f"loading {path} onto the GPU (max_context {ctx_len})")
    t = time.time()
    model = Qwen35Hip(path, max_context=ctx_len, direct=DIRECT)
    log(f"  resident in {time.time() - t:.1f}s")
    fill = ctx_len - args.warmup - args.steps
    if fill < 1:
        raise SystemExit("steps + warmup must be below the context length")
    t = time.time()
    model.reset()
    trace = model.generate(START_TOKEN, fill, 0)
    log(f"filled the cache with {fill} real decode steps in {time.time() - t:.2f}s (last token {int(trace[-1])})")
    dec, ctx = model.decoder, model.ctx
    dec.replay(args.warmup)
    ctx.synchronize()
    t0 = time.perf_counter()
    ctx.timer_start()
    dec.replay(args.steps)
    ev_ms = ctx.timer_stop()
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3
    return model, wall_ms, ev_ms, trace_check(dec, ctx_len)


GOLDEN_TRACE = os.path.join(ROOT, "tests", "golden", "qwen35_0.8b_trace_4096.npz")


def trace_check(dec, n: int):
    """The greedy ids of positions 0..n-1 (cache fill, warm-up and timed
    steps) against the compiled reference's trace from token 9419
    (tests/golden/qwen35_0.8b_trace_4096.npz, written by
    tests/golden/make_golden.py --trace4096)."""
    got = dec.trace(0, n)
    out = {"positions": f"0..{n - 1}", "golden": os.path.relpath(GOLDEN_TRACE, ROOT)}
    if not os.path.exists(GOLDEN_TRACE):
        out["trace_matches_reference"] = None
        return out
    import numpy as np
    with np.load(GOLDEN_TRACE) as z:
        want = z["tokens"][:n]
    diff = np.nonzero(got[:len(want)] != want)[0]
    out["compared"] = int(len(want))
    out["trace_matches_reference"] = bool(len(want) == n and diff.size == 0)
    out["first_mismatch"] = int(diff[0]) if diff.size else None
    return out


def lm_head_roofline(model, reps: int = 20):
    """Time the dominant kernel alone: fp16 LM head + fused argmax."""
    import numpy as np
    from fortai_amd import backend as B
    d, ctx = model.d, model.ctx
    x = np.random.default_rng(1).standard_normal(d.hidden).astype(np.float32)
    dx, dlog, dtok = ctx.upload_array(x), ctx.alloc(d.vocab * 4), ctx.alloc(8)
    w = model.output
    launch = lambda: ctx.call("fortai_hip_f16_matvec_device", ctx.h, w.h, dx.ptr, d.hidden, dlog.ptr, d.vocab,
                              dtok.ptr)
    for _ in range(3):
        launch()
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(reps):
        launch()
    ms = ctx.timer_stop() / reps
    algo = d.vocab * d.hidden * 2 + d.hidden * 4 + d.vocab * 4
    achieved = algo / (ms * 1e-3) / 1e9
    for b in (dx, dlog, dtok):
        b.free()
    return {"kernel": "f16_matvec_kernel<false,true> (fp16 LM head 248320x1024 + argmax)",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic_from_profile("lm_head"),
            "algorithmic_bytes": algo, "avg_launch_us": round(ms * 1e3, 2)}


def matvec_family_bytes(d) -> int:
    """Algorithmic bytes of every Q8_0 matvec of one decode step: each
    weight once (34 B per 32 values) plus the activation and output vectors."""
    q8 = lambda rows, width: rows * (width // 32) * 34
    total = 0
    for i in range(d.layers):
        if (i + 1) % d.interval != 0:
            mats = [(d.conv_size + d.inner + 2 * d.value_heads, d.hidden), (d.hidden, d.inner)]
        else:
            mats = [(2 * d.heads * d.head_size + 2 * d.kv_heads * d.head_size, d.hidden),
                    (d.hidden, d.heads * d.value_size)]
        mats += [(2 * d.ffn, d.hidden), (d.hidden, d.ffn)]
        total += sum(q8(r, w) + 4 * (r + w) for r, w in mats)
    return total


def matvec_family_roofline(model, warmup: int = 4, reps: int = 32):
    """The dominant kernel family of the decode step: every Q8_0 matvec launch
    of one step (q8_matvec_kernel, 114 launches at the 0.8B shape), timed live
    with HIP events on the context stream by replaying a graph of exactly those
    launches (a decoder in the FORTAI_HIP_DECODER_MATVEC_ONLY mode: same
    kernels, weights and arguments, the other kernels of the step left out)."""
    from fortai_amd import backend as B
    d = model.d
    dec = B.Decoder(model.ctx, model.recurrent, model.attention,
                    [model.q8[f"blk.{i}.ffn_gate.weight"] for i in range(d.layers)],
                    [model.q8[f"blk.{i}.ffn_up.weight"] for i in range(d.layers)],
                    [model.q8[f"blk.{i}.ffn_down.weight"] for i in range(d.layers)],
                    [n["attn"] for n in model.norms], [n["post"] for n in model.norms], model.output_norm,
                    d.hidden, model.embedding, model.output, 64, d.eps, d.vocab)
    dec.set_mode(matvec_only=True)
    try:
        ctx = model.ctx
        launches = sum(1 for step in dec.plan() if "q8_matvec" in step[1])
        dec.replay(warmup)
        ctx.synchronize()
        ctx.timer_start()
        dec.replay(reps)
        us = ctx.timer_stop() * 1e3 / reps
    finally:
        dec.free()
    algo = matvec_family_bytes(d)
    achieved = algo / (us * 1e-6) / 1e9
    return {"kernel": f"q8_matvec_kernel family: every Q8_0 projection of one decode step ({launches} launches)",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic_from_profile("decode_matvec"),
            "algorithmic_bytes": algo, "us_per_step": round(us, 2), "avg_launch_us": round(us / max(launches, 1), 3)}


def family_breakdown(model, position: int, warmup: int = 4, reps: int = 32):
    """Where the graph-replayed step spends its time, per kernel family: a
    decoder over the same layers in a timing-probe mode enqueues only one
    family's kernels (the Q8_0 projections; the GDN delta rule; the attention
    scores / softmax / output kernels; the embedding with the argmax finish
    and the LM head), captured as a graph and replayed at a fixed position
    (the attention kernels at `position` of the filled cache, so they read
    position + 1 keys and values), timed with HIP events on the context
    stream.  The families run back to back in the full step, so their sum is
    the step's time up to the boundaries between them."""
    from fortai_amd import backend as B
    d, ctx = model.d, model.ctx
    out = {"position": position}
    for fam in ("matvec", "gdn", "attention", "head"):
        dec = B.Decoder(model.ctx, model.recurrent, model.attention,
                        [model.q8[f"blk.{i}.ffn_gate.weight"] for i in range(d.layers)],
                        [model.q8[f"blk.{i}.ffn_up.weight"] for i in range(d.layers)],
                        [model.q8[f"blk.{i}.ffn_down.weight"] for i in range(d.layers)],
                        [n["attn"] for n in model.norms], [n["post"] for n in model.norms], model.output_norm,
                        d.hidden, model.embedding, model.output, model.max_context, d.eps, d.vocab)
        try:
            dec.set_mode(only=[fam])
            launches = len(dec.plan())
            # the head family advances the position itself (from 0 here)
            ctx.set_position(0 if fam == "head" else position)
            dec.replay(warmup)
            ctx.synchronize()
            ctx.timer_start()
            dec.replay(reps)
            us = ctx.timer_stop() * 1e3 / reps
        finally:
            dec.free()
        out[fam] = {"us_per_step": round(us, 2), "plan_steps": launches}
    out["sum_us"] = round(sum(out[f]["us_per_step"] for f in ("matvec", "gdn", "attention", "head")), 2)
    return out


def traffic_from_profile(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    (profiles/<name>_pmc.json, written from a committed profiling run)."""
    path = os.path.join(ROOT, "profiles", f"{name}_pmc.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes_per_launch")


def traffic_probe(reps: int = 5, decode_model: str = None, decode_only: bool = False) -> None:
    """Launches for the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes that
    price each kernel's HBM traffic (direct launches, no graphs, no timing):
    * calibration: fortai_hip_qwen35_add_device over 2^26 floats, algorithmic
      traffic 512 MiB read + 256 MiB written per launch;
    * the fp16 LM head with fused argmax over a random 248320 x 1024 table;
    * the 3584 x 1024 Q8_0 matvec (quantize fused) over 275
      distinct weight copies (1.07 GB, beyond the 256 MB Infinity Cache);
    * BASELINE config 3 at L = 4096: append + scores + exact output kernels;
    * the GDN conv1d + delta-rule step, and the
      state-resident recurrence (128 steps per launch);
    * with decode_model: 8 decode steps of that GGUF with direct launches
      (every matvec, GDN, attention, LM head kernel of the step)."""
    import ctypes as C
    import numpy as np
    from fortai_amd import backend as B
    from fortai_amd import synth
    ctx = B.Context(0)
    n = 1 << 26
    a, b, o = ctx.alloc(4 * n), ctx.alloc(4 * n), ctx.alloc(4 * n)
    for _ in range(reps):
        ctx.call("fortai_hip_qwen35_add_device", ctx.h, a.ptr, b.ptr, o.ptr, n)
    ctx.synchronize()
    for buf in (a, b, o):
        buf.free()
    if decode_only:
        ctx.close()
        return decode_probe(decode_model)
    rows, width = 248320, 1024
    rng = np.random.default_rng(7)
    w = (rng.standard_normal(rows * width, dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    lm = B.F16Weights(ctx, w, rows, width)
    del w
    x = ctx.upload_array(rng.standard_normal(width).astype(np.float32))
    logits, tok = ctx.alloc(rows * 4), ctx.alloc(8)
    for _ in range(reps):
        ctx.call("fortai_hip_f16_matvec_device", ctx.h, lm.h, x.ptr, width, logits.ptr, rows, tok.ptr)
    ctx.synchronize()
    for buf in (x, logits, tok):
        buf.free()
    lm.free()
    log("traffic probe: add (2^26 floats) and LM head launches done")
    # config 1 over rotating copies
    wq, xv = synth.matvec_inputs()
    mats = [B.Q8Weights(ctx, wq, 3584, 1024) for _ in range(275)]
    dx, dout = ctx.upload_array(xv), ctx.alloc(3584 * 4)
    for m in mats:
        ctx.call("fortai_hip_q8_matvec_device_f32", ctx.h, m.h, dx.ptr, 1024, dout.ptr, 3584)
    ctx.synchronize()
    for m in mats:
        m.free()
    dx.free()
    dout.free()
    log("traffic probe: 275 config-1 matvecs done")
    # config 3 at L = 4096
    heads, kvh, head, H, L = 8, 2, 256, 1024, 4096
    ws = [_q8(ctx, rng, heads * 2 * head, H), _q8(ctx, rng, kvh * head, H), _q8(ctx, rng, kvh * head, H),
          _q8(ctx, rng, H, heads * head)]
    A = B.Attention(ctx, *ws, (1 + 0.05 * rng.standard_normal(head)).astype(np.float32),
                    (1 + 0.05 * rng.standard_normal(head)).astype(np.float32), heads, kvh, head, head, L, 64,
                    1.0e7, 1e-6)
    nkv = L * kvh * head
    A.set_cache(rng.standard_normal(nkv).astype(np.float16).view(np.uint16),
                rng.standard_normal(nkv).astype(np.float16).view(np.uint16), L)
    dq = ctx.upload_array(rng.standard_normal(heads * 2 * head).astype(np.float32))
    dk = ctx.upload_array(rng.standard_normal(kvh * head).astype(np.float32))
    dv = ctx.upload_array(rng.standard_normal(kvh * head).astype(np.float32))
    do = ctx.alloc(heads * head * 4)
    ctx.set_position(L - 1)
    for _ in range(reps):
        ctx.call("fortai_hip_qwen35_attention_core_device", A.h, dq.ptr, dk.ptr, dv.ptr, do.ptr)
    ctx.synchronize()
    for buf in (dq, dk, dv, do):
        buf.free()
    A.free()
    for w_ in ws:
        w_.free()
    log("traffic probe: attention at L = 4096 done")
    # config 2
    heads, head, kernel = 16, 128, 4
    inner = heads * head
    conv = 2 * head * heads + inner
    ws = [_q8(ctx, rng, conv, H), _q8(ctx, rng, inner, H), _q8(ctx, rng, heads, H), _q8(ctx, rng, heads, H),
          _q8(ctx, rng, H, inner)]
    layer = B.Recurrent(ctx, *ws, (rng.standard_normal(conv * kernel) * 0.1).astype(np.float32), conv, kernel,
                        -np.exp(rng.standard_normal(heads) * 0.5).astype(np.float32),
                        rng.standard_normal(heads).astype(np.float32), np.ones(head, np.float32), head, heads, heads,
                        head, inner, 1e-6)
    layer.set_state((rng.standard_normal(heads * head * head) * 0.02).astype(np.float32),
                    np.zeros((kernel - 1) * conv, np.float32))
    qkv = ctx.upload_array(rng.standard_normal(conv).astype(np.float32))
    ab = ctx.upload_array(rng.standard_normal(2 * heads).astype(np.float32))
    out = ctx.alloc(inner * 4)
    for _ in range(reps):
        ctx.call("fortai_hip_qwen35_recurrent_core_device", layer.h, qkv.ptr, ab.ptr,
                 C.c_void_p(ab.ptr.value + heads * 4), out.ptr)
    ctx.synchronize()
    # the state-resident form: 128 steps in one launch
    steps = 128
    qkv_s = ctx.upload_array(rng.standard_normal(steps * conv).astype(np.float32))
    alpha_s = ctx.upload_array(rng.standard_normal(steps * heads).astype(np.float32))
    beta_s = ctx.upload_array(rng.standard_normal(steps * heads).astype(np.float32))
    outs = ctx.alloc(steps * inner * 4)
    for _ in range(reps):
        ctx.call("fortai_hip_qwen35_recurrent_core_steps_device", layer.h, qkv_s.ptr, alpha_s.ptr, beta_s.ptr, steps,
                 outs.ptr)
    ctx.synchronize()
    for buf in (qkv, ab, out, qkv_s, alpha_s, beta_s, outs):
        buf.free()
    layer.free()
    for w_ in ws:
        w_.free()
    ctx.close()
    log("traffic probe: GDN step and 128-step recurrence done")
    if decode_model:
        decode_probe(decode_model)


PROBE_STEPS = 8
DIRECT = False  # --no-graph: the decoders enqueue their kernels every step (kernel tracing)


def decode_probe(path: str) -> None:
    """PROBE_STEPS decode steps of the 0.8B model with direct launches."""
    from fortai_amd.qwen35 import Qwen35Hip
    model = Qwen35Hip(path, max_context=256, direct=True)
    model.reset()
    model.generate(START_TOKEN, PROBE_STEPS, 0)
    model.ctx.synchronize()
    model.close()
    log(f"traffic probe: {PROBE_STEPS} direct-launch decode steps done")


def pmc_summary(fetch_dir: str, write_dir: str, family_steps: int = 0) -> None:
    """Per-kernel HBM traffic from the two rocprofv3 --pmc passes of
    --traffic-probe (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each
    scaled by what the same counter reads for the calibration add kernel
    (512 MiB read, 256 MiB written).  Prints a JSON document."""
    import csv
    import glob
    from collections import defaultdict

    def read(directory, counter):
        paths = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
        if not paths:
            raise SystemExit(f"no counter_collection.csv under {directory}")
        per = defaultdict(list)
        with open(paths[0]) as f:
            for r in csv.DictReader(f):
                if r.get("Counter_Name", counter) != counter:
                    continue
                name = r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("fortai_hip::", "")
                name = name.replace("void ", "").replace("(Prologue)", "P").replace("(Epilogue)", "E").split("(")[0]
                per[name].append(float(r["Counter_Value"]))
        return per

    fetch, write = read(fetch_dir, "FETCH_SIZE"), read(write_dir, "WRITE_SIZE")
    cal = [k for k in fetch if k.startswith("add_kernel")][0]
    fscale = 536870912 / (sum(fetch[cal]) / len(fetch[cal]) * 1024)
    wscale = 268435456 / (sum(write[cal]) / len(write[cal]) * 1024)
    kernels = {}
    for k in sorted(fetch):
        f_ = fetch[k]
        w_ = write.get(k, [0.0])
        kernels[k] = {"dispatches": len(f_), "fetch_kib_avg": round(sum(f_) / len(f_), 3),
                      "write_kib_avg": round(sum(w_) / len(w_), 3),
                      "traffic_bytes_avg": int(sum(f_) / len(f_) * 1024 * fscale + sum(w_) / len(w_) * 1024 * wscale)}
    doc = {"calibration": {"kernel": cal, "fetch_scale": round(fscale, 4), "write_scale": round(wscale, 4)},
           "kernels": kernels}
    if family_steps:
        # a decode-only probe: the matvec family's traffic per step
        fam = [k for k in kernels if k.startswith("q8_matvec_kernel")]
        per_step = sum(kernels[k]["traffic_bytes_avg"] * kernels[k]["dispatches"] for k in fam) / family_steps
        doc["matvec_family"] = {"kernels": fam, "steps": family_steps,
                                "launches_per_step": sum(kernels[k]["dispatches"] for k in fam) / family_steps,
                                "traffic_bytes_per_step": int(per_step)}
        doc["traffic_bytes_per_launch"] = int(per_step)  # the family's launches of one step
    print(json.dumps(doc, indent=1))


def bench_matvec(model, copies: int = 275, reps: int = 4):
    """quantize + Q8_0 GEMV, W 3584x1024, x ~ N(0,1)."""
    import numpy as np
    from fortai_amd import backend as B
    from fortai_amd import synth
    ctx = model.ctx
    w, x = synth.matvec_inputs()
    rows, width = 3584, 1024
    mats = [B.Q8Weights(ctx, w, rows, width) for _ in range(copies)]
    dx, dout = ctx.upload_array(x), ctx.alloc(rows * 4)
    ctx.capture_begin()
    for m in mats:
        ctx.call("fortai_hip_q8_matvec_device_f32", ctx.h, m.h, dx.ptr, width, dout.ptr, rows)
    ctx.capture_end()
    ctx.graph_launch()
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(reps):
        ctx.graph_launch()
    ms = ctx.timer_stop() / (reps * copies)
    algo = rows * (width // 32) * 34 + (width // 32) * 34 + width * 4 + rows * 4
    for m in mats:
        m.free()
    dx.free()
    dout.free()
    gbps = algo / (ms * 1e-3) / 1e9
    return {"config": "Q8_0 W 3584x1024 + quantize x, 275 distinct copies (1.07 GB), graph of back-to-back launches",
            "us_per_op": round(ms * 1e3, 3), "algorithmic_bytes": algo, "gbps": round(gbps, 1),
            "frac": round(gbps / HBM_PEAK_GBPS, 4)}


def _q8(ctx, rng, rows, width):
    from fortai_amd import backend as B
    from fortai_amd import synth
    return B.Q8Weights(ctx, synth.q8_blocks(rng, rows, width), rows, width)


def bench_gdn(steps: int = 128, reps: int = 8):
    """one Gated DeltaNet layer (16 heads x 128, conv K=4
    over 6144 channels), state ~ N(0, 0.02), 128 autoregressive steps of
    resident inputs through fortai_hip_qwen35_recurrent_core_device (the
    conv1d+SiLU kernel and the decoder's delta-rule kernel), replayed from a
    captured graph."""
    import ctypes as C
    import numpy as np
    from fortai_amd import backend as B
    ctx = B.Context(0)  # one captured graph per context
    rng = np.random.default_rng(0x35A08B)
    H, heads, head, kernel = 1024, 16, 128, 4
    inner = heads * head
    conv = 2 * head * heads + inner
    ws = [_q8(ctx, rng, conv, H), _q8(ctx, rng, inner, H), _q8(ctx, rng, heads, H), _q8(ctx, rng, heads, H),
          _q8(ctx, rng, H, inner)]
    layer = B.Recurrent(ctx, *ws, (rng.standard_normal(conv * kernel) * 0.1).astype(np.float32), conv, kernel,
                        -np.exp(rng.standard_normal(heads) * 0.5).astype(np.float32),
                        rng.standard_normal(heads).astype(np.float32), np.ones(head, np.float32), head, heads, heads,
                        head, inner, 1e-6)
    layer.set_state((rng.standard_normal(heads * head * head) * 0.02).astype(np.float32),
                    np.zeros((kernel - 1) * conv, np.float32))
    qkv = ctx.upload_array(rng.standard_normal(steps * conv).astype(np.float32))
    ab = ctx.upload_array(rng.standard_normal(steps * 2 * heads).astype(np.float32))
    out = ctx.alloc(inner * 4)
    ctx.capture_begin()
    for t in range(steps):
        at = lambda buf, nbytes: C.c_void_p(buf.ptr.value + nbytes)
        ctx.call("fortai_hip_qwen35_recurrent_core_device", layer.h, at(qkv, t * conv * 4),
                 at(ab, t * 2 * heads * 4), at(ab, (t * 2 + 1) * heads * 4), out.ptr)
    ctx.capture_end()
    ctx.graph_launch()
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(reps):
        ctx.graph_launch()
    us = ctx.timer_stop() * 1e3 / (reps * steps)
    # state r+w + conv state r+w + conv weights + qkv in + o out + alpha/beta (survey section 8(d), config 2)
    algo = 2 * heads * head * head * 4 + 2 * (kernel - 1) * conv * 4 + conv * kernel * 4 + conv * 4 + inner * 4 + 2 * heads * 4
    # state-resident: the same 128 steps in one launch (the state stays in registers)
    alpha_s = ctx.upload_array(rng.standard_normal(steps * heads).astype(np.float32))
    beta_s = ctx.upload_array(rng.standard_normal(steps * heads).astype(np.float32))
    outs = ctx.alloc(steps * inner * 4)
    run = lambda: ctx.call("fortai_hip_qwen35_recurrent_core_steps_device", layer.h, qkv.ptr, alpha_s.ptr, beta_s.ptr,
                           steps, outs.ptr)
    run()
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(reps):
        run()
    us_res = ctx.timer_stop() * 1e3 / (reps * steps)
    # per step: q, k, v inputs, alpha/beta, output; state and windows touch memory once per launch
    algo_res = conv * 4 + inner * 4 + 2 * heads * 4 + (2 * heads * head * head * 4 + 2 * (kernel - 1) * conv * 4 +
                                                       conv * kernel * 4) / steps
    for b in (qkv, ab, out, alpha_s, beta_s, outs):
        b.free()
    layer.free()
    for w in ws:
        w.free()
    ctx.close()
    gbps = algo / (us * 1e-6) / 1e9
    return {"config": f"GDN layer 16x128, conv 4x6144, {steps} autoregressive steps",
            "state_streamed": {"path": "per step: conv1d+SiLU kernel + delta-rule kernel (state read and written "
                                       "every step), graph replay",
                               "us_per_step": round(us, 3), "algorithmic_bytes": algo, "gbps": round(gbps, 1),
                               "frac": round(gbps / HBM_PEAK_GBPS, 4)},
            "state_resident": {"path": "gdn_recurrence_kernel: all steps in one launch, state in registers",
                               "us_per_step": round(us_res, 3), "algorithmic_bytes_per_step": int(algo_res),
                               "gbps": round(algo_res / (us_res * 1e-6) / 1e9, 1),
                               "frac": round(algo_res / (us_res * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                               "note": "latency-bound: a serial chain of 128 dependent steps in 128 workgroups"}}


def bench_attention(cases=((1024, None), (4096, None), (32768, None), (32768, 1 << 20)), calls: int = 16,
                    reps: int = 4):
    """8 q / 2 kv heads x 256, fp16 cache, RoPE 1e7; one K/V
    append at position L-1, then attention over 0..L-1, through
    fortai_hip_qwen35_attention_core_device (scores kernel + exact two-pass
    output kernel up to the layer's exact_max positions, split-K
    beyond), replayed from a captured graph (one context per case).  A case
    is (L, exact_max); exact_max None is the default (8192)."""
    import numpy as np
    from fortai_amd import backend as B
    heads, kvh, head, H = 8, 2, 256, 1024
    results = []
    for L, exact_max in cases:
        ctx = B.Context(0)
        rng = np.random.default_rng(L)
        ws = [_q8(ctx, rng, heads * 2 * head, H), _q8(ctx, rng, kvh * head, H), _q8(ctx, rng, kvh * head, H),
              _q8(ctx, rng, H, heads * head)]
        A = B.Attention(ctx, *ws, (1 + 0.05 * rng.standard_normal(head)).astype(np.float32),
                        (1 + 0.05 * rng.standard_normal(head)).astype(np.float32), heads, kvh, head, head, L, 64,
                        1.0e7, 1e-6)
        if exact_max is not None:
            A.set_exact_max(exact_max)
        path = "exact two-pass" if L <= (8192 if exact_max is None else exact_max) else "split-K (1e-3)"
        n = L * kvh * head
        A.set_cache(rng.standard_normal(n).astype(np.float16).view(np.uint16),
                    rng.standard_normal(n).astype(np.float16).view(np.uint16), L)
        dq = ctx.upload_array(rng.standard_normal(heads * 2 * head).astype(np.float32))
        dk = ctx.upload_array(rng.standard_normal(kvh * head).astype(np.float32))
        dv = ctx.upload_array(rng.standard_normal(kvh * head).astype(np.float32))
        do = ctx.alloc(heads * head * 4)
        ctx.set_position(L - 1)
        ctx.capture_begin()
        for _ in range(calls):
            ctx.call("fortai_hip_qwen35_attention_core_device", A.h, dq.ptr, dk.ptr, dv.ptr, do.ptr)
        ctx.capture_end()
        ctx.graph_launch()
        ctx.synchronize()
        ctx.timer_start()
        for _ in range(reps):
            ctx.graph_launch()
        us = ctx.timer_stop() * 1e3 / (reps * calls)
        # KV read 2048 B per position + the append + q/k/v in and the output (survey section 8(d), config 3)
        algo = 2048 * L + 2048 + (heads * 2 * head + 2 * kvh * head + heads * head) * 4
        gbps = algo / (us * 1e-6) / 1e9
        results.append({"L": L, "path": path, "us_per_step": round(us, 2), "algorithmic_bytes": algo,
                        "gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4)})
        for b in (dq, dk, dv, do):
            b.free()
        A.free()
        for w in ws:
            w.free()
        ctx.close()
    return {"config": "8 q / 2 kv heads x 256, fp16 KV, append + exact attention at position L-1, graph replay",
            "lengths": results}


def host_cpu() -> dict:
    """lscpu model name, physical cores and the CPUs this process may use."""
    info = {"model": None, "physical_cores": None, "cpus_available": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                info["model"] = line.split(":", 1)[1].strip()
        cores = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True, timeout=20).stdout
        info["physical_cores"] = len({ln for ln in cores.splitlines() if ln and not ln.startswith("#")})
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def cpu_baseline(path, ctx_len: int, steps: int, repeats: int = 5):
    """The reference CPU decode on this host (benchmark/README.md:120-135,
    benchmark/tune_qwen35_cpu.sh:18): oracle/_ref/fast/ref_time (the
    reference's sources with its native optimisation flags) runs `steps`
    greedy steps of the same GGUF at the positions the GPU line is timed at
    (ctx-steps .. ctx-1; the cache below them holds zeros, the same work per
    step); first a thread sweep (one run each), then `repeats` runs at the
    fastest thread count, whose median is the value."""
    import statistics
    exe = os.path.join(ROOT, "oracle", "_ref", "fast", "ref_time")
    if not os.path.exists(exe):
        exe = os.path.join(ROOT, "oracle", "_ref", "ref_time")
    if not os.path.exists(exe):
        log("oracle/_ref is not built: no CPU baseline")
        return None
    host = host_cpu()
    limit = min(16, int(os.environ.get("OMP_NUM_THREADS", host["cpus_available"])), host["cpus_available"])
    start = ctx_len - steps

    def run(threads, nsteps, first):
        env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PROC_BIND="spread", OMP_PLACES="cores")
        out = subprocess.run([exe, path, str(START_TOKEN), str(nsteps), str(ctx_len), str(first)], capture_output=True,
                             text=True, env=env, timeout=600)
        m = re.search(r"forward_seconds=\s*([0-9.Ee+-]+)", out.stdout)
        t = re.search(r"last_token=\s*(-?[0-9]+)", out.stdout)
        if out.returncode != 0 or not m or not t:
            raise RuntimeError("reference CPU run failed: " + out.stdout[-300:] + out.stderr[-300:])
        run.last_token = int(t.group(1))
        return nsteps / float(m.group(1))

    sweep = {}
    t = 1
    while t <= limit:
        log(f"CPU baseline: thread sweep, {t} threads")
        sweep[t] = round(run(t, 1, ctx_len - 1), 4)
        t *= 2
    if limit not in sweep:
        sweep[limit] = round(run(limit, 1, ctx_len - 1), 4)
    best = max(sweep, key=sweep.get)
    log(f"CPU baseline: {repeats} runs of {steps} steps at {best} threads")
    vals = [run(best, steps, start) for _ in range(repeats)]
    # the timed build's own output: its greedy trace from position 0 against
    # the golden the GPU trace is checked with (written by the -O2 build)
    check_steps = 16
    run(best, check_steps, 0)
    check = {"steps_from_position_0": check_steps, "last_token": run.last_token}
    if os.path.exists(GOLDEN_TRACE):
        import numpy as np
        with np.load(GOLDEN_TRACE) as z:
            check["golden_token"] = int(z["tokens"][check_steps - 1])
        check["matches_golden"] = check["golden_token"] == run.last_token
    return {"value": round(statistics.median(vals), 4), "unit": "tokens/s", "cores": best, "kind": "reference",
            "output_check": check,
            "sample": f"{steps} greedy decode steps of the same 0.8B GGUF from token {START_TOKEN} at positions "
                      f"{start}..{ctx_len - 1} of a {ctx_len} context (forward + maxloc, load excluded); median of "
                      f"{repeats} runs; the reference's Fortran+C sources built with its native flags "
                      f"(oracle/Makefile ref-fast: -O3 -march=x86-64-v3 -funroll-loops -ffast-math, OpenMP, the "
                      f"AVX2 paths it dispatches)",
            "repeats": [round(v, 4) for v in vals], "min": round(min(vals), 4), "max": round(max(vals), 4),
            "stdev": round(statistics.stdev(vals), 4) if len(vals) > 1 else 0.0,
            "thread_sweep_tokens_per_s": sweep, "host": host}


def bench_config5(steps: int = 32, warmup: int = 4, prompt: int = 512, batch: int = 8, ctx: int = 8192,
                  check: int = 2):
    """Qwen3.5-4B shape (hidden 2560, 32 layers, FFN 9216,
    16 q / 4 kv heads, vocab 248320), batch 8 independent sequences, context
    8192: a 512-token prefill of every sequence, then batch-8 greedy decode
    from the prefilled state.  The default prefill is bit-exact (projections
    in the reference's lane order on the matrix cores, the exact causal
    attention); the 'fast' prefill mode (whole-block dots, fp16 matrix-core
    attention) is timed as a separate variant.  `check` sequences are decoded
    token by token with the single-sequence decoder and compared bit for bit."""
    import ctypes
    import numpy as np
    from fortai_amd import backend as B, synth
    from fortai_amd.qwen35 import Qwen35Hip
    path = os.path.join(os.environ.get("TMPDIR", "/tmp"), "fortai_bench", "qwen35-4b.gguf")
    if not os.path.exists(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        log(f"writing the synthetic Qwen3.5-4B GGUF to {path}")
        t = time.time()
        synth.write_model(path + ".part", synth.CONFIGS["qwen35-4b"])
        os.replace(path + ".part", path)
        log(f"  done in {time.time() - t:.1f}s")
    m = Qwen35Hip(path, max_context=ctx, batch=batch, direct=DIRECT)
    d, ctxh = m.d, m.ctx
    rng = np.random.default_rng(0x51E5)
    prompts = rng.integers(0, d.vocab, size=(batch, prompt))

    def prefill(mode):
        m.batch.set_prefill_mode(mode)
        try:
            m.batch.reset()
            m.batch.prefill(prompts)  # the first call allocates the prefill buffers
            m.batch.reset()
            return m.batch.prefill(prompts)
        finally:
            m.batch.set_prefill_mode("exact")

    _, fast_ms = prefill("fast")
    nxt, prefill_ms = prefill("exact")
    logits = m.batch.logits.copy()
    log(f"config 5 prefill: {batch} x {prompt} tokens in {prefill_ms:.1f} ms (fast variant {fast_ms:.1f} ms)")
    trace = m.batch.generate(nxt, np.full(batch, prompt, dtype=np.int32), 4)
    # decode timing from the prefilled state
    m.batch.reset()
    prefill("exact")
    m.batch.replay(warmup)
    ctxh.synchronize()
    ctxh.timer_start()
    m.batch.replay(steps)
    dec_ms = ctxh.timer_stop()
    step_ms = dec_ms / steps
    # exactness: sequences decoded token by token with the single-sequence decoder
    checked = []
    for s_ in range(check):
        dec = m.decoder
        dec.reset()
        for pos in range(prompt - 1):
            dec.forward(int(prompts[s_, pos]), pos, want_logits=False)
        want_next = dec.forward(int(prompts[s_, -1]), prompt - 1)
        same_logits = bool(np.array_equal(logits[s_].view(np.uint32), dec.logits.view(np.uint32)))
        same_steps = dec.generate(want_next, prompt, 4).tolist() == trace[s_].tolist()
        checked.append(same_logits and int(nxt[s_]) == want_next and same_steps)
    L = prompt + warmup + steps // 2
    q8 = lambda rows, width: rows * (width // 32) * 34
    n_attn = sum(1 for i in range(d.layers) if (i + 1) % d.interval == 0)
    n_gdn = d.layers - n_attn
    weights = d.layers * 3 * q8(d.ffn, d.hidden) + n_gdn * (q8(d.conv_size, d.hidden) + q8(d.inner, d.hidden) +
        2 * q8(d.value_heads, d.hidden) + q8(d.hidden, d.inner)) + n_attn * (q8(2 * d.heads * d.head_size, d.hidden) +
        2 * q8(d.kv_heads * d.head_size, d.hidden) + q8(d.hidden, d.heads * d.value_size)) + d.vocab * d.hidden * 2
    per_seq = n_gdn * (2 * d.value_heads * d.gdn_head ** 2 * 4 + d.conv_size * d.conv_kernel * 4 +
        (d.conv_kernel - 1) * d.conv_size * 8) + n_attn * 2 * L * d.kv_heads * d.head_size * 2 + d.hidden * 2
    step_bytes = weights + batch * per_seq
    # the dominant prefill kernel alone: the FFN gate projection over every prompt token
    w = m.q8["blk.0.ffn_gate.weight"]
    tokens = batch * prompt
    x = rng.standard_normal((tokens, d.hidden)).astype(np.float32)
    dx = ctxh.upload_array(x)
    dq = ctxh.alloc(B.load().fortai_hip_q8_tokens_bytes(tokens, d.hidden))
    out = ctxh.alloc(tokens * d.ffn * 4)
    ctxh.call("fortai_hip_q8_quantize_tokens_device", ctxh.h, dx.ptr, tokens, d.hidden, dq.ptr)
    ms = ctypes.c_float()

    def best_of(entry):
        best = 1e9
        for _ in range(5):
            ctxh.call(entry, ctxh.h, w.h, dq.ptr, tokens, out.ptr, None, ctypes.byref(ms))
            best = min(best, ms.value)
        return best
    exact_best, fast_best = best_of("fortai_hip_q8_mmq_exact_device"), best_of("fortai_hip_q8_mmq_device")
    macs = float(d.ffn) * d.hidden * tokens
    for b_ in (dx, dq, out):
        b_.free()
    m.close()
    tops = 2 * macs / (exact_best * 1e-3) / 1e12
    # vector work of the lane order: per (token, row, block) eight fp32 FMAs and one scale product
    valu_tflops = macs / 32 * 17 / (exact_best * 1e-3) / 1e12
    return {
        "workload": f"Qwen3.5-4B-shaped Q8_0, batch {batch} independent sequences, context {ctx}",
        "prefill": {"tokens": tokens, "prompt_per_sequence": prompt, "ms": round(prefill_ms, 2),
                    "tokens_per_s": round(tokens / (prefill_ms * 1e-3), 1),
                    "path": "projections in the reference's eight-lane fp32 order on v_mfma_f32_16x16x4f16 "
                            "(q8_mmq_exact_kernel); conv1d, delta rule and exact causal attention over time",
                    "fast_variant": {"ms": round(fast_ms, 2), "tokens_per_s": round(tokens / (fast_ms * 1e-3), 1),
                                     "path": "prefill mode fast: whole-block int32 dots on "
                                             "v_mfma_i32_32x32x32_i8, fp16 matrix-core attention (not bit-exact)"}},
        "decode": {"batch": batch, "positions": f"{prompt + warmup}..{prompt + warmup + steps - 1}",
                   "ms_per_step": round(step_ms, 4), "tokens_per_s": round(batch * steps / (dec_ms * 1e-3), 1),
                   "algorithmic_bytes_per_step": int(step_bytes),
                   "gbps": round(step_bytes / (step_ms * 1e-3) / 1e9, 1)},
        "exactness": {"sequences_checked": check, "bit_identical_to_token_by_token_decode": (all(checked) if checked else None),
                      "per_sequence": checked,
                      "what": "last prompt token's logits (bits), greedy next token and the next 4 batched decode "
                              "steps against the single-sequence decoder fed the prompt token by token"},
        "mmq": {"kernel": f"q8_mmq_exact_kernel ({d.ffn} x {d.hidden} FFN gate over {tokens} tokens)",
                "bound": "mfma", "achieved": round(tops, 1), "peak": 2500.0, "unit": "TFLOP/s (fp16 dense)",
                "frac": round(tops / 2500.0, 4), "avg_launch_us": round(exact_best * 1e3, 1),
                "valu": {"achieved": round(valu_tflops, 1), "peak": 157.3, "unit": "TFLOP/s (fp32)",
                         "frac": round(valu_tflops / 157.3, 4)},
                "fast_variant_us": round(fast_best * 1e3, 1)},
    }


def trace_summary(directory: str, steps: int = 64) -> None:
    """Per-kernel time of the last `steps` decode steps of a rocprofv3
    --kernel-trace CSV (a step starts at its embedding kernel)."""
    import csv
    import glob
    from collections import defaultdict
    paths = glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        raise SystemExit(f"no kernel_trace.csv under {directory}")
    rows = []
    with open(paths[0]) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    starts = [i for i, r in enumerate(rows) if "embedding" in r[2]]
    if len(starts) < steps + 1:
        raise SystemExit(f"only {len(starts)} decode steps in the trace")
    sel = rows[starts[-steps - 1]:starts[-1]]
    agg = defaultdict(lambda: [0, 0])
    for s0, s1, name in sel:
        key = name.replace("(anonymous namespace)::", "").replace("fortai_hip::", "").replace("void ", "")
        key = key.replace("(Prologue)", "P").replace("(Epilogue)", "E").split("(")[0]
        agg[key][0] += 1
        agg[key][1] += s1 - s0
    busy = sum(v[1] for v in agg.values()) / steps / 1e3
    print(f"| kernel | calls/step | avg us | us/step | % of busy |")
    print(f"|---|---:|---:|---:|---:|")
    for k, (c, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print(f"| `{k}` | {c / steps:.0f} | {t / c / 1e3:.2f} | {t / steps / 1e3:.1f} | {100 * t / steps / 1e3 / busy:.1f} |")
    print(f"\nkernel busy time per step: {busy:.1f} us over {len(sel) / steps:.0f} dispatches")


def prefill_summary(directory: str) -> None:
    """Per-kernel time per prompt prefill of a rocprofv3 --kernel-trace CSV of
    one or more batch prefills (each starts with one embedding kernel); the
    upload-time kernels (weight repack, fp16 table scan, runtime copies and
    fills) are left out."""
    import csv
    import glob
    from collections import defaultdict
    paths = glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        raise SystemExit(f"no kernel_trace.csv under {directory}")
    agg = defaultdict(lambda: [0, 0])
    with open(paths[0]) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if any(s in name for s in ("q8_repack_kernel", "count_nonfinite_halves_kernel", "__amd_rocclr")):
                continue
            key = name.replace("(anonymous namespace)::", "").replace("fortai_hip::", "").replace("void ", "")
            key = key.replace("(Prologue)", "P").replace("(Epilogue)", "E").split("(")[0]
            agg[key][0] += 1
            agg[key][1] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    n = sum(c for k, (c, _) in agg.items() if "embedding" in k)
    if n == 0:
        raise SystemExit("no prefill (embedding kernel) in the trace")
    busy = sum(v[1] for v in agg.values()) / n / 1e3
    print(f"| kernel | calls/prefill | avg us | us/prefill | % |")
    print(f"|---|---:|---:|---:|---:|")
    for k, (c, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print(f"| `{k}` | {c / n:.0f} | {t / c / 1e3:.1f} | {t / n / 1e3:.0f} | {100 * t / n / 1e3 / busy:.1f} |")
    print(f"\nkernel busy time per prefill: {busy / 1e3:.1f} ms over {n} prefills")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--model", default=None)
    ap.add_argument("--cpu-steps", type=int, default=4)
    ap.add_argument("--cpu-repeats", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-matvec", action="store_true")
    ap.add_argument("--no-kernels", action="store_true", help="skip the config 2 (GDN) and config 3 (attention) figures")
    ap.add_argument("--no-config5", action="store_true", help="skip the config 5 figures (4B shape, batch 8, prefill)")
    ap.add_argument("--config5-only", action="store_true",
                    help="print only the config 5 figures (for kernel tracing of the batch-8 decode)")
    ap.add_argument("--config5-check", type=int, default=2, metavar="N",
                    help="config 5: sequences re-decoded token by token for the exactness check (0 for a kernel "
                         "trace whose last steps are the batched ones)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the kernels the --pmc traffic passes measure (see traffic_probe)")
    ap.add_argument("--probe-decode", action="store_true",
                    help="with --traffic-probe: also run 8 direct-launch decode steps of the 0.8B model")
    ap.add_argument("--probe-decode-only", action="store_true",
                    help="with --traffic-probe: only the calibration and the decode steps; with --pmc-summary: "
                         "also report the matvec family's traffic per decode step")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print per-kernel HBM traffic from the FETCH_SIZE and WRITE_SIZE passes, then exit")
    ap.add_argument("--no-graph", action="store_true",
                    help="enqueue each decode step's kernels directly instead of replaying the HIP graph "
                         "(for kernel tracing)")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="print the per-kernel table of the last --steps decode steps of a rocprofv3 "
                         "--kernel-trace CSV under DIR, then exit")
    ap.add_argument("--prefill-summary", metavar="DIR",
                    help="print the per-kernel table per prompt prefill of a rocprofv3 --kernel-trace CSV under DIR, "
                         "then exit")
    args = ap.parse_args()
    if args.prefill_summary:
        prefill_summary(args.prefill_summary)
        return 0
    if args.trace_summary:
        trace_summary(args.trace_summary, args.steps)
        return 0
    global DIRECT
    DIRECT = bool(args.no_graph)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (the decode step is a batch-1 single-GPU path); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    if args.traffic_probe:
        traffic_probe(decode_model=model_path(args) if (args.probe_decode or args.probe_decode_only) else None,
                      decode_only=args.probe_decode_only)
        return 0
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary, family_steps=PROBE_STEPS if args.probe_decode_only else 0)
        return 0
    if args.config5_only:
        print(json.dumps({"config5": bench_config5(check=args.config5_check)}), flush=True)
        return 0
    path = model_path(args)
    model, wall_ms, ev_ms, trace = bench_decode(args, path)
    tok_s = args.steps / (wall_ms * 1e-3)
    # the timing probes replay graphs of their own; a --no-graph run (kernel
    # tracing, whose profiler cannot follow graph launches) leaves them out
    roof = None if DIRECT else matvec_family_roofline(model)
    roof_lm = None if DIRECT else lm_head_roofline(model)
    families = None if DIRECT else family_breakdown(model, args.ctx - args.steps // 2)
    mv = None if args.no_matvec else bench_matvec(model)
    kernels = None
    if not args.no_kernels:
        kernels = {"gdn_step": bench_gdn(), "attention": bench_attention()}
    d = model.d
    model_cfg5 = None
    decoder = "HIP graph of per-op kernels, replayed once per token"
    step_bytes = bytes_per_token(d, args.ctx - args.steps // 2)
    decode_gbps = step_bytes * tok_s / 1e9
    model.close()
    if not args.no_config5:
        model_cfg5 = bench_config5(check=args.config5_check)
    cpu = None if args.no_cpu_baseline else cpu_baseline(path, args.ctx, args.cpu_steps, args.cpu_repeats)
    line = {
        "metric": "decode tokens/sec (bs=1, ctx 4096) + Q8_0 matvec HBM GB/s, Qwen3.5-0.8B shape",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms / args.steps, 4),
        "ms_per_step_hip_events": round(ev_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0: int8 dot4 -> int32, fp32 accumulate (fp16 LM head, fp32 accumulate)",
        "data": "synthetic (seeded random-init Q8_0 weights of the stated shapes; tied fp16 embedding)",
        "config": {"workload": "Qwen3.5-0.8B-shaped Q8_0 greedy decode, batch 1, positions "
                               f"{args.ctx - args.steps}..{args.ctx - 1} of a {args.ctx}-token context "
                               "(BASELINE config 4)",
                   "hidden": d.hidden, "layers": d.layers, "ffn": d.ffn, "vocab": d.vocab,
                   "context": args.ctx, "batch": 1, "decoder": decoder},
        "decode_hbm": {"algorithmic_bytes_per_token": int(step_bytes), "gbps": round(decode_gbps, 1),
                       "frac_of_8TBps": round(decode_gbps / HBM_PEAK_GBPS, 4)},
        "trace": trace,
        "roofline": roof,
        "roofline_lm_head": roof_lm,
        "step_by_family": families,
        "matvec": mv,
        "kernels": kernels,
        "config5": model_cfg5,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
