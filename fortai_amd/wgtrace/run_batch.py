"""Per-workgroup timeline of the graph-replayed batch-8 decode step (BASELINE
config 5 shape; profiling only).

Loads fortai_amd/wgtrace/libfortai_wgtrace.so (build.sh) in place of the
library, prefills 8 sequences of 512 synthetic tokens on the Qwen3.5-4B-shaped
model, replays four batch steps of the captured graph and prints, for the
last whole step (embedding to embedding): every launch's workgroup count, the
gap from the previous launch's last workgroup end to its first workgroup
start, its span and the median workgroup duration; a per-kernel summary; and
the ring matvec's phase marks (activations in LDS, first group done, half the
groups done, all groups done, end) as median [90th percentile] from the
workgroup's start.  The tracer adds about 0.5 us per launch, so absolute
figures run high; the split between gaps and kernel bodies is what it is for.

usage: python fortai_amd/wgtrace/run_batch.py [GGUF]
"""
import collections
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
os.environ["FORTAI_HIP_LIBRARY"] = os.path.join(HERE, "libfortai_wgtrace.so")
from fortai_amd import backend as B, synth  # noqa: E402
from fortai_amd.qwen35 import Qwen35Hip  # noqa: E402

UNITS = ["q8_kernels", "gdn", "attention", "lm_head"]
KINDS = {3: "att_scores", 4: "att_softmax", 8: "ring_matvec", 9: "pair_matvec", 10: "q8l_prep",
         11: "gdn_delta_gated", 12: "att_output_wide", 14: "batch_output_norm",
         15: "embedding", 5: "att_output", 1: "q8_matvec", 2: "gdn_delta", 6: "step_embedding", 7: "lm_head"}
REC = np.dtype([("t0", "<u8"), ("t1", "<u8"), ("kind", "<u4"), ("block", "<u4"), ("mark", "<u4", (4,))])


def main():
    path = sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.environ.get("TMPDIR", "/tmp"), "fortai_bench",
                                                              "qwen35-4b.gguf")
    if not os.path.exists(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        synth.write_model(path, synth.CONFIGS["qwen35-4b"])
    lib = B.load()
    m = Qwen35Hip(path, max_context=8192, fused=False, batch=8)
    toks = np.random.default_rng(0x51E5).integers(0, m.d.vocab, size=(8, 512))
    m.batch.reset()
    m.batch.prefill(toks)
    m.batch.replay(2)
    m.ctx.synchronize()
    for u in UNITS:
        getattr(lib, "fortai_wgtrace_" + u)(None, 1)
    m.batch.replay(4)
    m.ctx.synchronize()
    recs = []
    for u in UNITS:
        buf = np.zeros(8 * 1024 * 512, REC)
        getattr(lib, "fortai_wgtrace_" + u)(C.c_void_p(buf.ctypes.data), 0)
        recs.append(buf[buf["t1"] > 0])
    r = np.concatenate(recs)
    # a ring slot overwritten while it was being read back can pair one
    # launch's start with another's end: keep records of 0..10 ms
    dur = r["t1"].astype(np.int64) - r["t0"].astype(np.int64)
    r = r[(dur >= 0) & (dur < 1_000_000)]
    r = r[np.argsort(r["t0"], kind="stable")]
    launches, cur = [], None
    for x in r:
        kind = int(x["kind"]) & 0xFF
        if cur is None or kind != cur["kind"] or x["t0"] > cur["end"]:
            cur = {"kind": kind, "start": int(x["t0"]), "end": int(x["t1"]), "n": 0, "durs": [], "marks": []}
            launches.append(cur)
        cur["end"] = max(cur["end"], int(x["t1"]))
        cur["n"] += 1
        cur["durs"].append(int(x["t1"]) - int(x["t0"]))
        lo = int(x["t0"]) & 0xFFFFFFFF
        cur["marks"].append([(int(v) - lo) & 0xFFFFFFFF for v in x["mark"]] + [int(x["t1"]) - int(x["t0"])])
    emb = [i for i, l in enumerate(launches) if l["kind"] == 15]
    step = launches[emb[-2]:emb[-1]]
    total = (launches[emb[-1]]["start"] - launches[emb[-2]]["start"]) / 100
    print(f"batch 8: one step = {len(step)} traced launches, {total:.1f} us (traced build)\n")
    print("| # | kernel | workgroups | gap us | span us | median workgroup us |")
    print("|---:|---|---:|---:|---:|---:|")
    rows, prev = [], None
    for i, l in enumerate(step):
        gap = (l["start"] - prev) / 100 if prev else 0.0
        prev = l["end"]
        rows.append((KINDS.get(l["kind"], str(l["kind"])), l["n"], gap, (l["end"] - l["start"]) / 100,
                     np.median(l["durs"]) / 100, i))
        if i < 24:
            print(f"| {i} | {rows[-1][0]} | {rows[-1][1]} | {gap:.2f} | {rows[-1][3]:.2f} | {rows[-1][4]:.2f} |")
    print("\n| kernel | workgroups | launches | gaps us | spans us | mean span us | mean median workgroup us "
          "| mean longest workgroup us |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|")
    agg = collections.defaultdict(lambda: [0, 0.0, 0.0, 0.0, 0.0])
    for (name, n, gap, span, med, i) in rows:
        a = agg[(name, n)]
        a[0] += 1
        a[1] += gap
        a[2] += span
        a[3] += med
        a[4] += max(step[i]["durs"]) / 100
    for (name, n), a in sorted(agg.items(), key=lambda kv: -kv[1][2]):
        print(f"| {name} | {n} | {a[0]} | {a[1]:.1f} | {a[2]:.1f} | {a[2] / a[0]:.2f} | {a[3] / a[0]:.2f} "
              f"| {a[4] / a[0]:.2f} |")
    print(f"| all | | {len(rows)} | {sum(x[2] for x in rows):.1f} | {sum(x[3] for x in rows):.1f} | | | |")
    print("\nring matvec phase marks, us from the workgroup's start, median [90th percentile]:\n")
    print("| # | workgroups | activations in LDS | first group | half the groups | all groups | end |")
    print("|---:|---:|---|---|---|---|---|")
    for i, l in enumerate(step[:24]):
        if l["kind"] != 8:
            continue
        a = np.array(l["marks"]) / 100
        cells = " | ".join(f"{np.median(a[:, j]):.2f} [{np.percentile(a[:, j], 90):.2f}]" for j in range(5))
        print(f"| {i} | {l['n']} | {cells} |")
    print("\nring matvec workgroup durations:\n")
    for i, l in enumerate(step[:24]):
        if l["kind"] != 8:
            continue
        print(f"launch {i}: {l['n']} workgroups, median workgroup {np.median(l['durs']) / 100:.2f} us, "
              f"90th percentile {np.percentile(l['durs'], 90) / 100:.2f} us, max {max(l['durs']) / 100:.2f} us")


if __name__ == "__main__":
    main()
