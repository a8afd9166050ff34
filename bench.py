#!/usr/bin/env python3
"""Benchmark of the MI355X quantized linear-projection path (one GPU).

Step (the default workload): the batch=1 decode matvec
set of a Qwen2.5-0.5B-shaped i4 HQQ@64 model -- 24 layers of independent
seeded weights, each q 896x896, k 128x896, v 128x896, o 896x896, gate 4864x896,
up 4864x896, down 896x4864, plus lm_head 151936x896: 169 i4 matvec launches on
one stream, inputs resident in HBM.

Printed (one JSON line on stdout):
  value        algorithmic GB/s of the whole step; bytes per matvec are the
               reference's own definition weight_bytes + 4*(M+K)
               (benchmarks/bench_kernels.cpp:487), i.e. 280,664,064 B per step
  us_per_layer_set  time of one layer's 7 matvecs (the 24-layer part / 24)
  headline     BASELINE configs[2] lm_head 151936x2560 alone, rotated over
               3 copies (657 MB > 2x the 256 MB MALL) so reads come from HBM
  roofline     the dominant kernel (the i4 MFMA matvec instance used for
               in_dim=896) over the step's launches: HIP-event duration of its
               launches back to back on the launch stream, against 8 TB/s
  cpu_baseline the compiled reference's `ref` matvec (oracle/_ref, tiny-llm's
               kernels/matvec/matvec_i4_ref.cpp built unmodified), row-split
               over host threads, on the same step; the C++ restatement is
               used when the compiled reference is absent
Progress goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes
import importlib.util
import json
import os
import sys
import threading
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
PEAK_GBS = 8000.0
METRIC = "i4 matvec achieved HBM GB/s (% of MI355X peak); µs per layer matvec set"
G = 64
HIDDEN, INTER, VOCAB = 896, 4864, 151936
LAYER = [("q", 896, HIDDEN), ("k", 128, HIDDEN), ("v", 128, HIDDEN), ("o", 896, HIDDEN),
         ("gate", INTER, HIDDEN), ("up", INTER, HIDDEN), ("down", HIDDEN, INTER)]
N_LAYERS = 24


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_pkg():
    spec = importlib.util.spec_from_file_location("tiny_llm_amd", os.path.join(REPO, "tiny-llm_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["tiny_llm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def algo_bytes(M, K):
    return M * ((K + G - 1) // G) * (4 + G // 2) + 4 * (M + K)


class Workload:
    """All matrices of the step, generated on the host once and uploaded."""

    def __init__(self, tq):
        self.tq = tq
        self.host = []   # (name, M, K, w_host, x_host) kept for the CPU baseline
        self.ops = []
        self.bufs = []
        t0 = time.time()
        for layer in range(N_LAYERS):
            xs = {}
            for name, M, K in LAYER:
                # q/k/v share the attention input, gate/up share the MLP input
                key = {"q": "attn", "k": "attn", "v": "attn", "gate": "mlp", "up": "mlp"}.get(name, name)
                if key not in xs:
                    xs[key] = tq.synth_normal(K, seed=tq.synth_seed(0, layer, "x_" + key))
                self._add(f"L{layer}.{name}", M, K, tq.synth_i4(M, K, G, seed=tq.synth_seed(0, layer, name)), xs[key])
        self._add("lm_head", VOCAB, HIDDEN, tq.synth_i4(VOCAB, HIDDEN, G, seed=tq.synth_seed(0, -1, "lm_head")),
                  tq.synth_normal(HIDDEN, seed=tq.synth_seed(0, -1, "x_final")))
        log(f"[bench] workload: {len(self.ops)} matvecs, {self.bytes / 1e6:.1f} MB algorithmic per step, "
            f"generated+uploaded in {time.time() - t0:.1f}s")

    def _add(self, name, M, K, w, x):
        tq = self.tq
        dw, dx, dy = tq.DeviceBuffer.from_array(w), tq.DeviceBuffer.from_array(x), tq.DeviceBuffer(4 * M)
        self.bufs += [dw, dx, dy]
        self.host.append((name, M, K, w, x))
        self.ops.append(tq.Op(tq.OP_I4_MATVEC, dw.ptr, dx.ptr, dy.ptr, M, K, 1, G))

    @property
    def bytes(self):
        return sum(algo_bytes(M, K) for _, M, K, _, _ in self.host)


def time_ops(tq, ops, reps, warmup, stream):
    tq.run_ops(ops, warmup, stream)
    stream.synchronize()
    e0, e1 = tq.Event(), tq.Event()
    e0.record(stream)
    tq.run_ops(ops, reps, stream)
    e1.record(stream)
    return e0.elapsed_ms(e1) / reps


def headline(tq, stream, reps=60):
    """configs[2] lm_head 151936x2560, 3 rotated copies (657 MB)."""
    M, K = VOCAB, 2560
    w = tq.synth_i4(M, K, G, seed=tq.synth_seed(0, -1, "lm_head_2560"))
    x = tq.synth_normal(K, seed=tq.synth_seed(0, -1, "x_2560"))
    copies = [tq.DeviceBuffer.from_array(w) for _ in range(3)]
    dx, dy = tq.DeviceBuffer.from_array(x), tq.DeviceBuffer(4 * M)
    ops = [tq.Op(tq.OP_I4_MATVEC, c.ptr, dx.ptr, dy.ptr, M, K, 1, G) for c in copies]
    ms = time_ops(tq, ops, reps, 5, stream) / len(ops)
    gbs = algo_bytes(M, K) / (ms * 1e-3) / 1e9
    for c in copies:
        c.free()
    return {"shape": "151936x2560 G64 (BASELINE configs[2] lm_head)", "us": round(ms * 1e3, 2),
            "gbs": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4), "bytes": algo_bytes(M, K),
            "rotation": "3 copies, 657 MB"}


def cpu_baseline(work, budget_s=12.0):
    """The reference's ref matvec (or the restatement) over the same step, row-split across threads."""
    sys.path.insert(0, REPO)
    import oracle  # the checker; used here only as the CPU baseline
    ref = oracle.ref_lib()
    kind = "reference" if ref is not None else "port"
    fn = ref.tqref_matvec_i4 if ref is not None else oracle.lib().orc_matvec_i4
    threads = max(1, min(16, os.cpu_count() or 1))
    outs = [np.empty(M, np.float32) for _, M, _, _, _ in work.host]

    def run_step():
        jobs = []
        for (name, M, K, w, x), y in zip(work.host, outs):
            rb = w.size // M
            parts = min(threads, M)
            for p in range(parts):
                a, b = M * p // parts, M * (p + 1) // parts
                if b > a:
                    jobs.append((w.ctypes.data + a * rb, x.ctypes.data, y.ctypes.data + 4 * a, b - a, K))
        # each worker walks its share of the jobs; ctypes releases the GIL in the call
        def worker(i):
            for j in range(i, len(jobs), threads):
                wp, xp, yp, m, k = jobs[j]
                fn(wp, xp, yp, m, k, G)
        ts = [threading.Thread(target=worker, args=(i,)) for i in range(threads)]
        for t in ts:
            t.start()
        for t in ts:
            t.join()

    run_step()  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        run_step()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 50:
            break
    ms = el / n * 1e3
    cpu = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(work.bytes / (ms * 1e-3) / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "ms_per_step": round(ms, 2), "cpu": cpu,
            "sample": f"{n} full steps (all 169 matvecs, {work.bytes / 1e6:.0f} MB), rows split over {threads} threads"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU reference timing")
    ap.add_argument("--no-headline", action="store_true", help="skip the 151936x2560 rotated headline")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the matvec would shard by "
              "output rows with one all-gather of y; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    tq = load_pkg()
    if tq.device_count() < 1:
        print("no HIP device visible", file=sys.stderr)
        sys.exit(1)
    log(f"[bench] device: {tq.device_name()}")
    stream = tq.Stream()
    work = Workload(tq)

    # whole step
    tq.synchronize()
    ms_step = time_ops(tq, work.ops, args.steps, args.warmup, stream)
    value = work.bytes / (ms_step * 1e-3) / 1e9
    log(f"[bench] step: {ms_step * 1e3:.1f} us, {value:.1f} GB/s")
    # the 24 layers alone
    layer_ops = work.ops[:-1]
    ms_layers = time_ops(tq, layer_ops, args.steps, 2, stream)
    us_layer = ms_layers * 1e3 / N_LAYERS
    log(f"[bench] layer set: {us_layer:.2f} us per layer")
    # dominant kernel: the in_dim=896 launches (q,k,v,o,gate,up x 24 + lm_head) back to back
    dom = [op for op in work.ops if op.in_dim == HIDDEN]
    dom_bytes = sum(algo_bytes(op.out_dim, op.in_dim) for op in dom)
    ms_dom = time_ops(tq, dom, args.steps, 2, stream)
    per_launch_us = ms_dom * 1e3 / len(dom)
    achieved = dom_bytes / len(dom) / (per_launch_us * 1e-6) / 1e9
    log(f"[bench] dominant kernel: {len(dom)} launches/step, {per_launch_us:.2f} us avg, {achieved:.1f} GB/s")

    head = None if args.no_headline else headline(tq, stream)
    if head:
        log(f"[bench] headline 151936x2560: {head['us']} us, {head['gbs']} GB/s ({100 * head['frac']:.1f}% of 8 TB/s)")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(work)
        log(f"[bench] cpu baseline ({cpu['kind']}, {cpu['cores']} threads): {cpu['ms_per_step']} ms/step, "
            f"{cpu['value']} GB/s")

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "i8xi8->i32 MFMA, f32 epilogue", "data": "synthetic",
        "pct_of_peak": round(100 * value / PEAK_GBS, 2),
        "us_per_layer_set": round(us_layer, 2),
        "config": {"workload": "BASELINE configs[1]: Qwen2.5-0.5B-shaped i4 HQQ@64 decode matvec set, batch=1, "
                               "24 layers x (q,k,v,o 896/128x896; gate,up 4864x896; down 896x4864) + lm_head "
                               "151936x896, independent seeded weights",
                   "bytes_per_step": work.bytes, "launches_per_step": len(work.ops), "group_size": G},
        "roofline": {"bound": "hbm", "kernel": "i4_matvec_mfma<1> (in_dim 896 launches)",
                     "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": None,
                     "launches": len(dom), "bytes_per_launch": dom_bytes // len(dom),
                     "avg_launch_us": round(per_launch_us, 3)},
        "headline": head,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
