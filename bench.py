"""Benchmark of the encoder forward (BertModel.ForwardBatch) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one forward of the whole batch (embeddings -> 12 layers -> pooled
vectors) with token ids already resident in HBM.  Prints one JSON line:
throughput in embeddings/s, the roofline of the dominant kernel (measured with
HIP events on the library's stream inside the timed steps), the overall MFMA
utilisation, and the CPU baseline (the oracle, a C restatement of the
reference CPU path over OpenBLAS) timed on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import hashlib
import importlib.util
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
METRIC = "embeddings/sec/GPU (Nomic-style, b256 s512, fp16) + MFMA util %"
PEAK_MFMA_TFLOPS = {0: 157.3, 1: 2500.0, 2: 2500.0}  # MI355X dense fp32 / fp16 / bf16
PEAK_HBM_GBS = 8000.0


def _package():
    name = "longbow_fletcher_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = ROOT / "longbow-fletcher_amd"
    spec = importlib.util.spec_from_file_location(name, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def kernel_work(cfg, lengths, esz, synth):
    """Algorithmic work per launch of each kernel class: (flops, hbm bytes)."""
    T = int(lengths.sum())
    H, I = cfg.hidden, cfg.intermediate
    Ni = cfg.inter_cols
    sq = float((lengths.astype(np.float64) ** 2).sum())
    # Embedding: gather the word rows (+ the position rows of absolute
    # models; RoPE models have none), write the normalised rows, read the ids
    # (+ positions).  The type-0 row and LayerNorm parameters stay cached.
    gathers = 1 if cfg.position == synth.POS_ROPE else 2
    return {
        "embed": (0.0, T * H * esz * (gathers + 1) + T * 4 * gathers),
        "qkv_gemm": (2.0 * T * H * 3 * H, (T * H + 3 * H * H + T * 3 * H) * esz),
        "attention": (4.0 * sq * H, (T * 3 * H + T * H) * esz),
        "o_gemm": (2.0 * T * H * H, (T * H * 2 + H * H) * esz),
        "add_layernorm": (0.0, 3 * T * H * esz),
        "ffn_up_gemm": (2.0 * T * H * Ni, (T * H + Ni * H + T * I) * esz),
        "ffn_down_gemm": (2.0 * T * I * H, (T * I + I * H + T * H) * esz),
        "pool": (0.0, T * H * esz + len(lengths) * H * 4),
    }


def kernel_source_sha():
    """Hash of the device code (csrc/*.hip, *.hpp, *.inc): a traffic profile
    describes the kernels it was measured on only while this matches."""
    h = hashlib.sha256()
    for f in sorted((ROOT / "longbow-fletcher_amd" / "csrc").iterdir()):
        if f.suffix in (".hip", ".hpp", ".inc"):
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()[:16]


def counters_summary(fetch_dir, write_dir, workload, out_path):
    """Per-launch HBM bytes of each kernel class from two rocprofv3 passes of
    `bench.py --calibrate --no-profile` (FETCH_SIZE, then WRITE_SIZE; KiB per
    dispatch), scaled by what the same counters read for the calibration
    copy (read 256 MiB, write 256 MiB)."""
    def load(d, counter):
        rows = []
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(path)):
                if r["Counter_Name"] == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
        rows.sort()
        return rows

    def classes(rows):
        """Dispatch -> class: the calibration copy first, then the forwards'
        kernels by name; of the two plain-store GEMMs of a layer the first is
        the O projection, the second FFN-down."""
        out, calib, plain = [], None, 0
        for did, name, val in rows:
            if calib is None and "cast_kernelIDF16_DF16_" in name:
                # The calibration copy: cast_kernel<fp16, fp16> over 256 MiB
                # (weight loading runs cast_kernel<fp32, fp16> before it).
                calib = val
                continue
            if "embed_ln" in name or "embed_rows" in name:
                cls = "embed"
            elif "attn_" in name:
                cls = "attention"
            elif "layernorm" in name:
                cls = "add_layernorm"
            elif "pool_" in name:
                cls = "pool"
            elif "gemm_w4" in name:
                epi = name.split("kernelIDF16_Li")[1][0] if "kernelIDF16_Li" in name else "?"
                if epi == "4":
                    cls = "qkv_gemm"
                elif epi == "3":
                    cls = "ffn_up_gemm"
                else:
                    cls = "o_gemm" if plain % 2 == 0 else "ffn_down_gemm"
                    plain += 1
            else:
                continue
            out.append((cls, name, val))
        return calib, out

    def launches(rows):
        """Consecutive dispatches of one class are one launch of it (the
        pool's partial and final kernels), as in the bench's timing."""
        out = []
        for cls, name, v in rows:
            if out and out[-1][0] == cls and cls == "pool":
                out[-1] = (cls, out[-1][1], out[-1][2] + v)
            else:
                out.append((cls, name, v))
        return out

    fcal, frows = classes(load(fetch_dir, "FETCH_SIZE"))
    wcal, wrows = classes(load(write_dir, "WRITE_SIZE"))
    frows, wrows = launches(frows), launches(wrows)
    moved_kib = 256 * 1024.0
    ff, wf = moved_kib / fcal, moved_kib / wcal
    agg = collections.defaultdict(lambda: {"fetch": [], "write": [], "kernel": None})
    for cls, name, v in frows:
        agg[cls]["fetch"].append(v * ff * 1024)
        agg[cls]["kernel"] = name
    for cls, name, v in wrows:
        agg[cls]["write"].append(v * wf * 1024)
    per = {c: {"fetch_bytes": int(np.mean(a["fetch"])), "write_bytes": int(np.mean(a["write"])),
               "kernel": a["kernel"]} for c, a in agg.items() if a["fetch"] and a["write"]}
    doc = {"workload": workload, "csrc_sha": kernel_source_sha(),
           "calibration_factor_fetch": ff, "calibration_factor_write": wf, "per_launch": per}
    pathlib.Path(out_path).write_text(json.dumps(doc, indent=1) + "\n")
    return doc


def cpu_baseline(fl, cfg, weights, lengths, ids, budget_s):
    """Times the oracle on whole sequences of the workload until ~budget_s;
    returns the baseline and the oracle's outputs for those sequences (rows
    0 .. n-1), which the parity check compares with the GPU's."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    cores = max(1, min(int(cores or 1), 64))
    oracle.set_threads(cores)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])

    def run(rows):
        sub = np.concatenate([ids[starts[r]:starts[r] + lengths[r]] for r in rows])
        t0 = time.perf_counter()
        out = oracle.forward(cfg, weights, sub, lengths[rows])
        return time.perf_counter() - t0, out

    t1, first = run([0])
    n = int(max(1, min(len(lengths), budget_s / max(t1, 1e-3))))
    rows = list(range(n))
    t, outs = run(rows) if n > 1 else (t1, first)
    return {"value": round(n / t, 3), "unit": "embeddings/s", "cores": cores, "kind": "port",
            "sample": f"{n} of {len(lengths)} sequences of the same workload "
                      f"(lengths {int(lengths[rows].min())}-{int(lengths[rows].max())}), "
                      f"oracle fp32 reference math, OpenBLAS threads = {cores}, {t:.1f} s"}, outs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="nomic-b256-s512-f16")
    ap.add_argument("--cpu-seconds", type=float, default=25.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the end-to-end (host ids in, pooled vectors out) measurement")
    ap.add_argument("--calibrate", action="store_true",
                    help="run one plain 256 MiB fp16 copy kernel first (reference for HBM counters)")
    ap.add_argument("--no-per-op", action="store_true",
                    help="skip the per-op path (bert.go op by op through the C ABI)")
    ap.add_argument("--counters-summary", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "OUT_JSON"),
                    help="write the per-launch HBM traffic JSON from two rocprofv3 counter "
                         "passes (FETCH_SIZE, WRITE_SIZE) of this script with --calibrate")
    a = ap.parse_args()
    if a.counters_summary:
        doc = counters_summary(*a.counters_summary[:2], a.workload, a.counters_summary[2])
        print(json.dumps(doc, indent=1))
        return
    if a.gpus != 1:
        print(json.dumps({"error": "this backend is measured on one GPU; multi-GPU serving is "
                                   "one independent model replica per device with a host-side "
                                   "split of the sequences, --gpus must be 1"}))
        sys.exit(2)

    fl = _package()
    if not fl.LIB_PATH.exists():
        spec = importlib.util.spec_from_file_location("_b", ROOT / "longbow-fletcher_amd/build.py")
        b = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(b)
        b.build()
    synth = fl.synth
    w = synth.WORKLOADS[a.workload]
    cfg, lengths = w.cfg, w.lengths()
    ids = synth.make_ids(lengths)
    log(f"workload {w.name}: B={len(lengths)} tokens={int(lengths.sum())}")
    t0 = time.time()
    weights = synth.make_weights(cfg)
    log(f"weights generated in {time.time() - t0:.1f}s")

    ctx = fl.Context(0)
    model = fl.Model(ctx, cfg, dtype=w.dtype,
                     math=fl.MATH_REFERENCE if w.dtype == fl.F32 else fl.MATH_EXACT)
    model.load(weights)
    d_ids = ctx.int32(ids)
    d_out = ctx.empty((len(lengths), cfg.hidden))
    ctx.synchronize()

    if a.calibrate:
        # A copy of known size (read 256 MiB, write 256 MiB) whose FETCH_SIZE /
        # WRITE_SIZE calibrate the counters read for the encoder's kernels.
        src = ctx.empty((128 * 1024 * 1024,), fl.F16)
        dst = ctx.cast(src, fl.F16)
        ctx.synchronize()
        src.free()
        dst.free()
    for i in range(a.warmup):
        model.forward_device(d_ids, lengths, d_out)
    ctx.synchronize()
    log("warmup done")

    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        model.forward_device(d_ids, lengths, d_out)
    ctx.synchronize()
    total = time.perf_counter() - t0
    ms_step = total * 1000.0 / a.steps
    value = len(lengths) * a.steps / total
    log(f"timed {a.steps} steps: {ms_step:.3f} ms/step, {value:.1f} emb/s")
    nan, bad = model.status()

    out_gpu = d_out.numpy()  # the timed run's last output, checked against the oracle below
    esz = 4 if w.dtype == fl.F32 else 2
    work = kernel_work(cfg, lengths, esz, synth)
    total_flops = cfg.layers * sum(work[k][0] for k in
                                   ("qkv_gemm", "attention", "o_gemm", "ffn_up_gemm",
                                    "ffn_down_gemm"))
    peak = PEAK_MFMA_TFLOPS[w.dtype]
    mfma_util = total_flops / (ms_step * 1e-3) / (peak * 1e12)

    roofline, kernels = None, {}
    if not a.no_profile:
        model.set_profiling(True)
        ctx.synchronize()
        for _ in range(a.steps):
            model.forward_device(d_ids, lengths, d_out)
        prof = model.profile()
        model.set_profiling(False)
        for name, (ms, cnt) in prof.items():
            if cnt:
                avg = ms / cnt
                fl_, by = work[name]
                kernels[name] = {"avg_ms": round(avg, 4), "launches": cnt,
                                 "share": None,
                                 "tflops": round(fl_ / (avg * 1e-3) / 1e12, 1) if fl_ else None,
                                 "gbs": round(by / (avg * 1e-3) / 1e9, 1)}
        tot = sum(prof[n][0] for n in kernels)
        for n in kernels:
            kernels[n]["share"] = round(prof[n][0] / tot, 4)
        dom = max(kernels, key=lambda n: prof[n][0])
        fl_, by = work[dom]
        avg_s = kernels[dom]["avg_ms"] * 1e-3
        traffic, traffic_note = None, "no counter profile for this workload"
        tfile = ROOT / "profiles" / f"encoder_forward_{w.name.replace('-', '_')}_traffic.json"
        if tfile.exists():
            # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE /
            # WRITE_SIZE passes over this workload (see the profile summary),
            # used only while the kernels are the ones it was measured on.
            doc = json.loads(tfile.read_text())
            t = doc["per_launch"].get(dom)
            if doc.get("csrc_sha") != kernel_source_sha():
                traffic_note = "counter profile predates the current kernel sources"
            elif t:
                traffic = t["fetch_bytes"] + t["write_bytes"]
                traffic_note = f"rocprofv3 FETCH_SIZE + WRITE_SIZE, {tfile.name}"
        if fl_:
            ach = fl_ / avg_s / 1e12
            roofline = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 1), "peak": peak,
                        "unit": "TFLOP/s", "frac": round(ach / peak, 4), "traffic": traffic,
                        "algorithmic_bytes": by, "traffic_source": traffic_note}
        else:
            ach = by / avg_s / 1e9
            roofline = {"kernel": dom, "bound": "hbm", "achieved": round(ach, 1),
                        "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBS, 4),
                        "traffic": traffic, "traffic_source": traffic_note}
        log(json.dumps(kernels))

    e2e = None
    if not a.no_e2e:
        # Host int64 ids in, host fp32 vectors out (PCIe included), with the
        # reference's Linux GPU batching defaults: the pipelined entry point
        # against one synchronous forward per batch of the same plan.
        ms_, mt_ = 512, 16384
        plan = fl.plan_batches(lengths, ms_, mt_)
        starts = np.concatenate([[0], np.cumsum(lengths)])
        model.embed(ids, lengths, ms_, mt_)
        reps = max(1, min(5, a.steps))
        t0 = time.perf_counter()
        for _ in range(reps):
            _o, _n, nb = model.embed(ids, lengths, ms_, mt_)
        pipe_s = (time.perf_counter() - t0) / reps
        t0 = time.perf_counter()
        for _ in range(reps):
            for first, count in plan:
                model.forward(ids[starts[first]:starts[first + count]], lengths[first:first + count])
        seq_s = (time.perf_counter() - t0) / reps
        # Untimed first call: the fp16 cast kernel's first launch loads it.
        model.embed(ids, lengths, ms_, mt_, out_dtype=fl.F16)
        t0 = time.perf_counter()
        for _ in range(reps):
            model.embed(ids, lengths, ms_, mt_, out_dtype=fl.F16)
        pipe16_s = (time.perf_counter() - t0) / reps
        e2e = {"max_seqs": ms_, "max_tokens": mt_, "batches": nb,
               "pipelined_embeddings_per_s": round(len(lengths) / pipe_s, 1),
               "pipelined_f16_out_embeddings_per_s": round(len(lengths) / pipe16_s, 1),
               "sequential_embeddings_per_s": round(len(lengths) / seq_s, 1)}
        # The same with one batch per call (a budget as large as the workload;
        # 288 GB of HBM holds it easily).
        big = int(lengths.sum())
        model.embed(ids, lengths, len(lengths), big)
        t0 = time.perf_counter()
        for _ in range(reps):
            model.embed(ids, lengths, len(lengths), big)
        e2e["whole_batch_embeddings_per_s"] = round(len(lengths) * reps / (time.perf_counter() - t0), 1)
        # Latency of a short request (one sequence, host ids in, host vector
        # out): the few-row GEMM path.
        short = {}
        for n_tok in (16, 128):
            sl = np.array([min(n_tok, int(lengths[0]))], np.int64)
            sid = ids[:int(sl[0])]
            for _ in range(3):
                model.forward(sid, sl)
            t0 = time.perf_counter()
            for _ in range(20):
                model.forward(sid, sl)
            short[f"ms_per_call_{int(sl[0])}_tokens"] = round((time.perf_counter() - t0) / 20 * 1e3, 3)
        e2e["short_request"] = short
        log(f"end to end: {e2e}")

    per_op = None
    if not a.no_per_op:
        # The per-op path: bert.go's ForwardBatch op by op through the C ABI,
        # the path the unchanged Go model takes (perop.py: the Tensor calls of
        # bert.go on the binding's backend, fp32 master stream included),
        # same batch.
        from importlib import import_module
        perop = import_module(fl.__name__ + ".perop")
        dev = import_module(fl.__name__ + ".device")
        be = dev.RocmBackend(0, w.dtype, rope_base=cfg.rope_base)
        pm = perop.PerOpModel(be, cfg, weights)
        be.PutTensor(pm.forward_device(ids, lengths))
        be.Synchronize()
        reps = 3
        t0 = time.perf_counter()
        for _ in range(reps):
            be.PutTensor(pm.forward_device(ids, lengths))
        be.Synchronize()
        dt = (time.perf_counter() - t0) / reps
        pm.close()
        be.close()
        per_op = {"embeddings_per_s": round(len(lengths) / dt, 1), "ms_per_step": round(dt * 1e3, 3),
                  "steps": reps}
        log(f"per-op path: {per_op}")

    cpu, parity = None, None
    if not a.no_cpu_baseline:
        log("cpu baseline ...")
        cpu, want = cpu_baseline(fl, cfg, weights, lengths, ids, a.cpu_seconds)
        log(f"cpu baseline {cpu}")
        # Parity of the timed run's output with the oracle on the same rows.
        got = out_gpu[:len(want)].astype(np.float64)
        wd = want.astype(np.float64)
        cos = (got * wd).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(wd, axis=1))
        parity = {"rows": int(len(want)), "min_cos": round(float(cos.min()), 7),
                  "max_abs": float(np.abs(got - wd).max()),
                  "against": "oracle (reference CPU path restated, fp32, reference math)",
                  "bar_cos": 0.99999 if w.dtype == fl.F32 else 0.999}
        log(f"parity {parity}")

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "embeddings/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": {0: "fp32", 1: "fp16", 2: "bf16"}[w.dtype],
        "data": "synthetic (seeded N(0,0.02) weights, uniform ids in [1000,30000) framed 101/102)",
        "config": {"workload": w.name, "model": cfg.name, "layers": cfg.layers,
                   "hidden": cfg.hidden, "heads": cfg.heads, "global_batch": len(lengths),
                   "seq_len": int(lengths.max()), "tokens": int(lengths.sum()),
                   "parallelism": "single GPU"},
        "mfma_util": round(mfma_util, 4),
        "algorithmic_tflops": round(total_flops / (ms_step * 1e-3) / 1e12, 1),
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": cpu,
        "parity": parity,
        "end_to_end": e2e,
        "per_op_path": per_op,
        "output_nan": nan, "bad_ids": bad,
    }
    print(json.dumps(out), flush=True)
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
