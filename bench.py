#!/usr/bin/env python3
"""Benchmark of the MI355X quantized linear-projection path (one GPU).

Step (the default workload): the batch=1 decode matvec
set of a Qwen2.5-0.5B-shaped i4 HQQ@64 model -- 24 layers of independent
seeded weights, each q 896x896, k 128x896, v 128x896, o 896x896, gate 4864x896,
up 4864x896, down 896x4864, plus lm_head 151936x896 -- with each layer's
matvec set as ONE launch (tqhip_matvec_i4_set_dev: the seven matrices and their
four activation vectors) and the lm_head as another: 25 launches on one stream,
inputs resident in HBM, issued eagerly. Every step reads weights cold: the
steps rotate over three copies of all weights (3 x 280.7 MB, more than twice
the 256 MB MALL). The same matvecs issued the way the reference runtime calls
them (qwen_forward_token: mv_qkv, mv o, mv_pair gate/up, mv down per layer, then
matvec_i4 lm_head; 97 launches) are timed the same way under "step_runtime_order".

Printed (one JSON line on stdout):
  value        algorithmic GB/s of the whole step; bytes per matvec are the
               reference's own definition weight_bytes + 4*(M+K)
               (benchmarks/bench_kernels.cpp:487): 280,664,064 B per step
  us_per_layer_set  time of one layer's 7 matvecs as one set launch, over the
               72 distinct layer sets of the three copies (cold)
  layer_set    that figure, the same launches replayed from a HIP graph, and the
               layer's dependency-ordered 4-launch form (qkv, o, gate/up, down)
  step_runtime_order  the 97-launch step in the reference runtime's call order
  step_dependent  the 25-launch step with every layer set reading the previous
               one's outputs (each set waits for the whole set before it)
  graph        the 25-launch step captured into a HIP graph and replayed
  roofline     the kernel with the largest share of the step's time: the set
               kernel (24 of the 25 launches), its 72 cold launches timed back
               to back with HIP events on the launch stream, against 8 TB/s;
               traffic = HBM bytes per launch from the committed rocprofv3
               FETCH_SIZE/WRITE_SIZE summary, when present
  ceilings     measured on the same GPU in the same run: a cold stream read
               (1 GiB), the back-to-back empty-kernel launch floor, and the dense
               fp16 MFMA rate (v_mfma_f32_32x32x16_f16 from registers)
  headline     BASELINE configs[2] lm_head 151936x2560 alone, rotated over
               3 copies (657 MB > 2x the 256 MB MALL) so reads come from HBM
  configs2     BASELINE configs[2] gate/up 9728x2560, down 2560x9728, attention
               4096x2560 and 2560x4096, each rotated over > 512 MB of copies
  prefill      BASELINE configs[4] dequant-GEMM 9728x2560 at 32/128/512
               tokens: us, TFLOP/s and fraction of the dense fp16 MFMA peak
  vq2          BASELINE configs[3] VQ2 matvec 3072x1024 and VQ2 151936x896,
               rotated copies, us and GB/s
  host_call    the reference-signature host-pointer entry point (x H2D,
               kernel, y D2H; weights cached in HBM), PCIe-inclusive us
  engine       the device-resident decode engine (tqhip_decode_*) on a
               Qwen2.5-0.5B-shaped dense i4 HQQ@64 model (24 layers, 14/2 heads,
               tied i4 embedding, q/k/v biases, random weights): ms per token
               and tokens/s of step() (one graph replay, token in and next
               token out), over --steps tokens after --warmup tokens; the same
               for a BiIP-rotated VQ2 file of that shape (vq2_rotated)
  cpu_baseline the compiled reference's `ref` matvec (oracle/_ref, tiny-llm's
               kernels/matvec/matvec_i4_ref.cpp built unmodified), row-split
               over host threads, on the same step; the C++ restatement is
               used when the compiled reference is absent
  verify       the correctness gate (as the reference's bench_kernels checks
               every variant against `ref` before it reports a time,
               benchmarks/bench_kernels.cpp:255-259, 472-481): outside the timed
               regions each section keeps the outputs of its last timed launch,
               and the CPU-baseline leg checks them -- the step's 169 outputs
               against the reference outputs the CPU baseline computed on the
               same inputs, the headline, configs[0]/[2] and VQ2 outputs against
               the CPU checker, prefill on every 97th row (every row at 32
               tokens), the decode engines' logits against the reference's own
               CPU decode of the same file. Each section gets
               verify: {rel_l2, max_rel, verdict}; a section that fails has its
               figures reported as null (value too, for the step)
Progress goes to stderr, with each section's wall-clock seconds.
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
PEAK_MFMA_TFLOPS = 2500.0  # dense fp16/bf16
METRIC = "i4 matvec achieved HBM GB/s (% of MI355X peak); µs per layer matvec set"
G = 64
HIDDEN, INTER, VOCAB = 896, 4864, 151936
LAYER = [("q", 896, HIDDEN), ("k", 128, HIDDEN), ("v", 128, HIDDEN), ("o", 896, HIDDEN),
         ("gate", INTER, HIDDEN), ("up", INTER, HIDDEN), ("down", HIDDEN, INTER)]
N_LAYERS = 24
N_COPIES = 3  # weight copies the steps rotate over: 3 x 280.7 MB > 2 x the 256 MB MALL


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


LAYER_BYTES = sum(algo_bytes(M, K) for _, M, K in LAYER)  # 8,478,208


class Workload:
    """All matrices of the step, generated on the host once (seeded) and uploaded N_COPIES
    times at different addresses, so consecutive steps read cold weights."""

    def __init__(self, tq):
        self.tq = tq
        self.host = []   # (name, M, K, w_host, x_host) per matrix, kept for the CPU baseline
        self.bufs = []
        self.keep = []   # tqhip_i4_mat arrays the set ops point at
        t0 = time.time()
        weights, acts = {}, {}
        for layer in range(N_LAYERS):
            for name, M, K in LAYER:
                # q/k/v share the attention input, gate/up share the MLP input
                key = {"q": "attn", "k": "attn", "v": "attn", "gate": "mlp", "up": "mlp"}.get(name, name)
                if (layer, key) not in acts:
                    acts[(layer, key)] = tq.synth_normal(K, seed=tq.synth_seed(0, layer, "x_" + key))
                weights[(layer, name)] = tq.synth_i4(M, K, G, seed=tq.synth_seed(0, layer, name))
                self.host.append((f"L{layer}.{name}", M, K, weights[(layer, name)], acts[(layer, key)]))
        w_lm = tq.synth_i4(VOCAB, HIDDEN, G, seed=tq.synth_seed(0, -1, "lm_head"))
        x_lm = tq.synth_normal(HIDDEN, seed=tq.synth_seed(0, -1, "x_final"))
        self.host.append(("lm_head", VOCAB, HIDDEN, w_lm, x_lm))
        # activations and outputs once (small; re-read from L2 either way), weights per copy
        dx = {k: self._dev(v) for k, v in acts.items()}
        dy = {(layer, name): self._dev(None, 4 * M) for layer in range(N_LAYERS) for name, M, _ in LAYER}
        dx_lm, dy_lm = self._dev(x_lm), self._dev(None, 4 * VOCAB)
        # every copy writes the same outputs (the copies hold the same weights): one output buffer
        # per matrix, in the order of self.host, read back for the correctness gate
        self.outputs = [dy[(layer, name)] for layer in range(N_LAYERS) for name, _, _ in LAYER] + [dy_lm]
        self.set_steps, self.rt_steps = [], []  # per copy: the 25-launch and the 97-launch step
        wdev, wlm = {}, []  # the copies' weight buffers
        for c in range(N_COPIES):
            set_ops, rt_ops = [], []
            for layer in range(N_LAYERS):
                m = {}
                for name, M, K in LAYER:
                    key = {"q": "attn", "k": "attn", "v": "attn", "gate": "mlp", "up": "mlp"}.get(name, name)
                    wdev[(c, layer, name)] = self._dev(weights[(layer, name)])
                    m[name] = (wdev[(c, layer, name)], dx[(layer, key)], dy[(layer, name)], M, K)
                arr = tq.i4_set([m[name] for name, _, _ in LAYER])
                self.keep.append(arr)
                set_ops.append(tq.set_op(arr, G))
                q, k, v, o, g, u, d = (m[name] for name, _, _ in LAYER)
                rt_ops += [tq.Op(tq.OP_I4_QKV, q[0].ptr, q[1].ptr, q[2].ptr, q[3], HIDDEN, 1, G,
                                 k[0].ptr, v[0].ptr, k[2].ptr, v[2].ptr, k[3]),
                           tq.Op(tq.OP_I4_MATVEC, o[0].ptr, o[1].ptr, o[2].ptr, o[3], o[4], 1, G),
                           tq.Op(tq.OP_I4_PAIR, g[0].ptr, g[1].ptr, g[2].ptr, g[3], HIDDEN, 1, G,
                                 u[0].ptr, None, u[2].ptr, None, 0),
                           tq.Op(tq.OP_I4_MATVEC, d[0].ptr, d[1].ptr, d[2].ptr, d[3], d[4], 1, G)]
            wlm.append(self._dev(w_lm))
            lm = tq.Op(tq.OP_I4_MATVEC, wlm[c].ptr, dx_lm.ptr, dy_lm.ptr, VOCAB, HIDDEN, 1, G)
            self.set_steps.append(set_ops + [lm])
            self.rt_steps.append(rt_ops + [lm])
        # The dependent step: the same 25 launches of the same weight copies, but every input of
        # layer l > 0 is an output of layer l - 1 (attention input <- down, MLP input <- o,
        # o input <- q, down input <- gate; the lm_head reads the last down output), so each
        # layer set waits for the whole previous one, as a decode token's layers do. Its own
        # output buffers (the gate above checks the independent step's).
        self.dep_steps = []
        ydep = {(layer, name): self._dev(None, 4 * M) for layer in range(N_LAYERS) for name, M, _ in LAYER}
        dy_lm_dep = self._dev(None, 4 * VOCAB)
        feed = {"attn": "down", "mlp": "o", "o": "q", "down": "gate"}
        for c in range(N_COPIES):
            dep_ops = []
            for layer in range(N_LAYERS):
                m = {}
                for name, M, K in LAYER:
                    key = {"q": "attn", "k": "attn", "v": "attn", "gate": "mlp", "up": "mlp"}.get(name, name)
                    xin = dx[(layer, key)] if layer == 0 else ydep[(layer - 1, feed[key])]
                    m[name] = (wdev[(c, layer, name)], xin, ydep[(layer, name)], M, K)
                arr = tq.i4_set([m[name] for name, _, _ in LAYER])
                self.keep.append(arr)
                dep_ops.append(tq.set_op(arr, G))
            dep_ops.append(tq.Op(tq.OP_I4_MATVEC, wlm[c].ptr, ydep[(N_LAYERS - 1, "down")].ptr, dy_lm_dep.ptr, VOCAB,
                                 HIDDEN, 1, G))
            self.dep_steps.append(dep_ops)
        self.bytes = N_LAYERS * LAYER_BYTES + algo_bytes(VOCAB, HIDDEN)
        log(f"[bench] workload: {len(self.host)} matvecs per step, {len(self.set_steps[0])} launches as layer sets "
            f"({len(self.rt_steps[0])} in runtime order), {self.bytes / 1e6:.1f} MB algorithmic per step, "
            f"{N_COPIES} weight copies ({N_COPIES * self.bytes / 1e6:.0f} MB), built in {time.time() - t0:.1f}s")

    def _dev(self, host, nbytes=None):
        b = self.tq.DeviceBuffer(nbytes) if host is None else self.tq.DeviceBuffer.from_array(host)
        self.bufs.append(b)
        return b

    def steps(self, n, runtime_order=False, dependent=False):
        """The op list of n consecutive steps, rotating over the weight copies."""
        src = self.rt_steps if runtime_order else self.dep_steps if dependent else self.set_steps
        return [op for i in range(n) for op in src[i % N_COPIES]]

    def layer_sets(self):
        """The 72 layer-set launches of the three copies (no lm_head)."""
        return [op for c in range(N_COPIES) for op in self.set_steps[c][:-1]]

    def layer_runtime_order(self):
        return [op for c in range(N_COPIES) for op in self.rt_steps[c][:-1]]

    def download_outputs(self):
        """The step's 169 outputs as its last launches left them (after a synchronisation)."""
        self.tq.synchronize()
        return [b.download(np.float32, M) for b, (_, M, _, _, _) in zip(self.outputs, self.host)]


# ---- correctness gate -------------------------------------------------------------------------
# Outputs of the timed sections, checked after all timing by the CPU-baseline leg (gate()).
PENDING = []
MATVEC_BAR, PREFILL_BAR, ENGINE_BAR = 1e-5, 2e-3, 1e-4  # rel L2 bars (north star; engine: decode tests)
FIGURES = ("us", "gbs", "frac", "tflops", "mfma_frac", "us_batch_min", "us_batch_max", "ms_per_token",
           "tokens_per_s", "value")


def compare(got, want, l2_bar, max_bar=1e-3):
    """rel L2 and max|err| / max|want|, the bars of the parity tests; a non-finite output where the
    reference is finite (or the reverse) fails."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    fin = np.isfinite(want)
    if not np.array_equal(np.isfinite(got), fin):
        return {"rel_l2": None, "max_rel": None, "verdict": "FAIL", "why": "finiteness differs"}
    d = got[fin] - want[fin]
    den = np.linalg.norm(want[fin])
    l2 = float(np.linalg.norm(d) / (den if den > 0 else 1.0))
    sc = float(np.max(np.abs(want[fin]))) if fin.any() else 0.0
    mx = float(np.max(np.abs(d)) / (sc if sc > 0 else 1.0)) if d.size else 0.0
    return {"rel_l2": float(f"{l2:.3e}"), "max_rel": float(f"{mx:.3e}"),
            "verdict": "PASS" if l2 <= l2_bar and mx <= max_bar else "FAIL", "bar": f"rel L2 <= {l2_bar:g}, "
            f"max|err| <= {max_bar:g} max|y|"}


def worst(checks):
    """One verify record for several outputs: the largest figures, FAIL if any failed."""
    out = {"rel_l2": None, "max_rel": None, "verdict": "PASS", "outputs": len(checks)}
    for c in checks:
        for k in ("rel_l2", "max_rel"):
            if c[k] is not None and (out[k] is None or c[k] > out[k]):
                out[k] = c[k]
        if c["verdict"] != "PASS":
            out["verdict"] = "FAIL"
        if "bar" in c:
            out["bar"] = c["bar"]
    return out


def settle(rec, check):
    """Attaches a verify record; a failing section reports its figures as null."""
    rec["verify"] = check
    if check["verdict"] != "PASS":
        for k in FIGURES:
            if k in rec:
                rec[k] = None


def time_ops(tq, ops, reps, warmup, stream, batches=1):
    """ms per pass over `ops`: HIP events around `reps` back-to-back passes on
    `stream`; with batches > 1, the median over that many such measurements."""
    tq.run_ops(ops, warmup, stream)
    stream.synchronize()
    out = []
    for _ in range(batches):
        e0, e1 = tq.Event(), tq.Event()
        e0.record(stream)
        tq.run_ops(ops, reps, stream)
        e1.record(stream)
        out.append(e0.elapsed_ms(e1) / reps)
    return float(np.median(out))


def time_graph(tq, ops, reps, warmup, stream, batches=1):
    """ms per pass over `ops` captured once into a HIP graph (tq.OpsGraph) and
    replayed: HIP events around `reps` back-to-back replays on `stream`; with
    batches > 1, the median over that many such measurements. Every kernel of
    the list runs in every replay; the graph only removes the per-launch host
    and dispatch cost."""
    graph = tq.OpsGraph(ops, stream)
    try:
        for _ in range(warmup):
            graph.launch()
        stream.synchronize()
        out = []
        for _ in range(batches):
            e0, e1 = tq.Event(), tq.Event()
            e0.record(stream)
            for _ in range(reps):
                graph.launch()
            e1.record(stream)
            out.append(e0.elapsed_ms(e1) / reps)
        return float(np.median(out))
    finally:
        graph.close()


def layer_set(tq, work, stream, reps):
    """Per-layer figures over the 72 distinct (cold) layers of the three copies: one set
    launch per layer eagerly, the same launches replayed from a HIP graph, and the layer's
    dependency-ordered 4-launch form."""
    sets = work.layer_sets()
    us = time_ops(tq, sets, reps, 2, stream, batches=5) * 1e3 / len(sets)
    us_graph = time_graph(tq, sets, reps, 2, stream, batches=5) * 1e3 / len(sets)
    rt = work.layer_runtime_order()
    us_rt = time_ops(tq, rt, reps, 2, stream, batches=5) * 1e3 / len(sets)
    return {"us": round(us, 2), "us_graph": round(us_graph, 2), "us_4launch": round(us_rt, 2),
            "layers_timed": len(sets), "bytes": LAYER_BYTES,
            "kernel": "i4_matvec_set (one launch: q, k, v, o, gate, up, down; four activation vectors)",
            "4launch": "mv_qkv, mv o, mv_pair gate/up, mv down (qwen_forward_token.cpp:401, 458, 639, 658)"}


TRAFFIC_FILE = os.path.join(REPO, "profiles", "i4_matvec_set_layer_traffic.json")


def roofline(us_set):
    """The set kernel: algorithmic bytes of a layer set over its mean launch time (the 72
    cold launches of layer_set, back to back, HIP events on the launch stream)."""
    achieved = LAYER_BYTES / (us_set * 1e-6) / 1e9
    traffic = None
    try:
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        pass
    return {"bound": "hbm", "kernel": "i4_matvec_set<SMAX, R> (every layer's set launch, 24 of the step's 25)",
            "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4),
            "traffic": traffic, "launches": N_LAYERS, "bytes_per_launch": LAYER_BYTES,
            "avg_launch_us": round(us_set, 3)}


CEIL_LIB = os.path.join(REPO, "tiny-llm_amd", "libtqceil.so")


def ceilings(tq, stream):
    """What this GPU sustains, measured in the same run: a cold 1 GiB stream read (4x the
    MALL; 16-byte loads, grid-stride), the back-to-back launch floor of an empty kernel, and
    dense fp16 MFMA from registers."""
    lib = ctypes.CDLL(CEIL_LIB)
    lib.tqceil_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_void_p]
    lib.tqceil_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.tqceil_mfma_f16.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.tqceil_shared_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_void_p]
    sp = ctypes.c_void_p(stream.ptr)

    def timed(fn, reps=1, batches=5):
        fn()
        stream.synchronize()
        out = []
        for _ in range(batches):
            e0, e1 = tq.Event(), tq.Event()
            e0.record(stream)
            for _ in range(reps):
                fn()
            e1.record(stream)
            out.append(e0.elapsed_ms(e1) / reps)
        return float(np.median(out))

    nb = 1 << 30
    buf, out = tq.DeviceBuffer(nb), tq.DeviceBuffer(4 * 8192)
    tq.lib().tqhip_memset(buf.ptr, 1, nb)
    read = {}
    names = ("4 loads", "8 loads", "8 nt loads")
    for variant in range(3):
        for blocks in (2048, 4096, 8192):
            ms = timed(lambda: lib.tqceil_stream_read(buf.ptr, nb, out.ptr, blocks, variant, sp))
            read[f"{names[variant]}, {blocks} wg"] = nb / (ms * 1e-3) / 1e9
    # cold reads of one matrix's size (configs[0], the layer set, the configs[2] and VQ2 shapes, the
    # i4 lm_head 151936x896), one launch each at offsets rotating through the 1 GiB buffer, back to
    # back: the floor a single matvec launch of that many bytes can reach here (launch cost and the
    # ramp to full bandwidth included)
    sized = {}
    for size in (804864, 2474496, 5924864, 8478208, 14057472, 34647040, 77187072):
        step = (size + 4095) // 4096 * 4096
        offs = [(i * step) % (nb - step) for i in range(60)]
        best_s = None
        for variant in (1, 2):
            for blocks in (256, 512, 1024, 2048):
                def batch():
                    for o in offs:
                        lib.tqceil_stream_read(buf.ptr + o, size // 16 * 16, out.ptr, blocks, variant, sp)
                ms = timed(batch, 1, batches=5) / len(offs)
                if best_s is None or ms < best_s[0]:
                    best_s = (ms, variant, blocks)
        sized[str(size)] = {"us": round(best_s[0] * 1e3, 2), "gbs": round(size / (best_s[0] * 1e-3) / 1e9, 1),
                            "frac": round(size / (best_s[0] * 1e-3) / 1e9 / PEAK_GBS, 4),
                            "best": f"{names[best_s[1]]}, {best_s[2]} wg"}
    buf.free()
    best = max(read, key=read.get)
    # one L2-resident buffer (32 tokens x 2560 fp32, the few-token GEMM's X) read whole by every workgroup
    sb = 32 * 2560 * 4
    sbuf = tq.DeviceBuffer(sb)
    tq.lib().tqhip_memset(sbuf.ptr, 1, sb)
    shared = {}
    for blocks, threads in ((256, 1024), (256, 512), (512, 512), (1024, 256)):
        ms = timed(lambda: lib.tqceil_shared_read(sbuf.ptr, sb, out.ptr, blocks, threads, sp))
        shared[f"{blocks}x{threads}"] = {"us": round(ms * 1e3, 2), "gbs_per_cu": round(blocks * sb / 256 / (ms * 1e-3) / 1e9, 1)}
    sbuf.free()
    empty = {}
    for blocks, threads in ((1, 64), (1024, 256)):
        empty[f"{blocks}x{threads}"] = round(timed(lambda: lib.tqceil_empty(blocks, threads, 200, sp), 1) * 1e3 / 200, 3)
    mf = {}
    for variant, name in ((0, "32x32x16"), (1, "16x16x32")):
        for blocks in (1024, 2048):
            iters = 4096000 // blocks
            ms = timed(lambda: lib.tqceil_mfma_f16(blocks, iters, variant, out.ptr, sp), batches=3)
            mf[f"{name}, {blocks} wg"] = blocks * 4 * 4 * iters * 32768 / (ms * 1e-3) / 1e12
    best_mf = max(mf, key=mf.get)
    tflops = mf[best_mf]
    return {"stream_read_gbs": round(read[best], 1), "stream_read_frac": round(read[best] / PEAK_GBS, 4),
            "stream_read": {"bytes": nb, "best": best, "gbs": {k: round(v, 1) for k, v in read.items()}},
            "empty_launch_us": empty,
            "cold_read_one_launch": {"note": "one launch reading N cold bytes, back to back (bytes -> us)",
                                     "sizes": sized},
            "shared_read": {"bytes": sb, "note": "every workgroup reads the same buffer; GB/s per CU of 256",
                            "runs": shared},
            "mfma_f16_tflops": round(tflops, 1), "mfma_f16_frac": round(tflops / PEAK_MFMA_TFLOPS, 4),
            "mfma": {"best": best_mf, "tflops": {k: round(v, 1) for k, v in mf.items()}}}


def headline(tq, stream, reps=20):
    """configs[2] lm_head 151936x2560, 3 rotated copies (657 MB): median of 15
    batches of 20 rotations (60 launches each). Batch medians drift by up to
    15% over a run on the same box (kernel traces show stretches of slower
    launches that recover), so many batches are taken; the fastest and
    slowest batch are reported beside the median."""
    M, K = VOCAB, 2560
    w = tq.synth_i4(M, K, G, seed=tq.synth_seed(0, -1, "lm_head_2560"))
    x = tq.synth_normal(K, seed=tq.synth_seed(0, -1, "x_2560"))
    copies = [tq.DeviceBuffer.from_array(w) for _ in range(3)]
    dx, dy = tq.DeviceBuffer.from_array(x), tq.DeviceBuffer(4 * M)
    ops = [tq.Op(tq.OP_I4_MATVEC, c.ptr, dx.ptr, dy.ptr, M, K, 1, G) for c in copies]
    tq.run_ops(ops, 5, stream)
    stream.synchronize()
    per = []
    for _ in range(15):
        per.append(time_ops(tq, ops, reps, 0, stream) / len(ops))
    ms = float(np.median(per))
    gbs = algo_bytes(M, K) / (ms * 1e-3) / 1e9
    stream.synchronize()
    y = dy.download(np.float32, M)
    for c in copies:
        c.free()
    rec = {"shape": "151936x2560 G64 (BASELINE configs[2] lm_head)", "us": round(ms * 1e3, 2),
           "gbs": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4), "bytes": algo_bytes(M, K),
           "us_batch_min": round(min(per) * 1e3, 2), "us_batch_max": round(max(per) * 1e3, 2),
           "rotation": "3 copies, 657 MB"}
    PENDING.append((rec, "i4", (w, x, M, K), y))
    return rec


def prefill(tq, stream, reps=30):
    """W 9728x2560 i4 HQQ@64 times X of 32/128/512 tokens. W is rotated over enough
    copies to exceed 2x the 256 MB MALL (every call reads its W cold from HBM); X, an
    activation, is one buffer."""
    M, K = 9728, 2560
    w = tq.synth_i4(M, K, G, seed=tq.synth_seed(0, -1, "prefill_w"))
    ncopy = (512 << 20) // (M * (K // G) * (4 + G // 2)) + 1
    dws = [tq.DeviceBuffer.from_array(w) for _ in range(ncopy)]
    rows = []
    for n in (32, 128, 512):
        x = tq.synth_normal(K * n, seed=tq.synth_seed(0, n, "prefill_x"))
        dx, dy = tq.DeviceBuffer.from_array(x), tq.DeviceBuffer(4 * M * n)
        ops = [tq.Op(tq.OP_I4_MATMUL, dw.ptr, dx.ptr, dy.ptr, M, K, n, G) for dw in dws]
        ms = time_ops(tq, ops, max(1, reps // 10), 1, stream, batches=5) / len(ops)
        fl = 2.0 * M * K * n
        tf = fl / (ms * 1e-3) / 1e12
        rec = {"tokens": n, "us": round(ms * 1e3, 2), "tflops": round(tf, 1),
               "mfma_frac": round(tf / PEAK_MFMA_TFLOPS, 4),
               "gbs": round((M * (K // G) * (4 + G // 2) + 4 * (K + M) * n) / (ms * 1e-3) / 1e9, 1)}
        rows.append(rec)
        stream.synchronize()
        PENDING.append((rec, "matmul", (w, x, M, K, n), dy.download(np.float32, M * n)))
        dx.free()
        dy.free()
    for dw in dws:
        dw.free()
    return {"shape": "W 9728x2560 G64, X 2560 x tokens (BASELINE configs[4])",
            "mfma": "v_mfma_f32_32x32x16_f16, fp32 accumulate", "w_copies": ncopy, "tokens": rows}


CONFIGS2 = ((9728, 2560, "gate/up"), (2560, 9728, "down"), (4096, 2560, "attn in"), (2560, 4096, "attn out"))


def cold_matvec(tq, stream, M, K, tag):
    """One i4 matvec M x K G64 per launch, device-resident, rotated over enough weight copies to
    exceed 2x the 256 MB MALL (cold reads); median of 7 batches of at least 60 launches."""
    w = tq.synth_i4(M, K, G, seed=tq.synth_seed(0, -4, f"{tag}_{M}x{K}"))
    x = tq.synth_normal(K, seed=tq.synth_seed(0, -4, f"{tag}x_{K}"))
    b = algo_bytes(M, K)
    ncopy = (512 << 20) // (M * ((K + G - 1) // G) * (4 + G // 2)) + 1
    copies = [tq.DeviceBuffer.from_array(w) for _ in range(ncopy)]
    dx, dy = tq.DeviceBuffer.from_array(x), tq.DeviceBuffer(4 * M)
    ops = [tq.Op(tq.OP_I4_MATVEC, c.ptr, dx.ptr, dy.ptr, M, K, 1, G) for c in copies]
    ms = time_ops(tq, ops, max(1, 60 // ncopy), 1, stream, batches=7) / len(ops)
    stream.synchronize()
    y = dy.download(np.float32, M)
    for c in copies:
        c.free()
    dx.free()
    dy.free()
    rec = {"shape": f"{M}x{K}", "us": round(ms * 1e3, 2), "gbs": round(b / (ms * 1e-3) / 1e9, 1),
           "frac": round(b / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes": b, "copies": ncopy}
    PENDING.append((rec, "i4", (w, x, M, K), y))
    return rec


def configs0(tq, stream):
    """the single i4 matvec 4864x896 (the reference's CPU-runnable case) on
    the GPU, one launch, cold. Launch-bound: compare with the one-launch floor for its bytes."""
    return cold_matvec(tq, stream, 4864, HIDDEN, "c0")


def configs2(tq, stream):
    """BASELINE configs[2] (Qwen3.5-4B scale) matvecs other than the lm_head:
    gate/up 9728x2560, down 2560x9728, attention 4096x2560 and 2560x4096, each
    rotated over enough copies to exceed 2x the 256 MB MALL (cold reads);
    median of 7 batches of at least 60 launches."""
    rows = []
    for M, K, role in CONFIGS2:
        r = cold_matvec(tq, stream, M, K, "c2")
        r["role"] = role  # the same dict the gate fills in
        rows.append(r)
    return rows


def vq2(tq, stream, reps=20):
    """VQ2 matvec: BASELINE configs[3] 3072x1024 and the reference's VQ2 lm_head
    shape 151936x896 (kernels_baseline.csv:32), rotated over enough copies to
    exceed 2x the 256 MB MALL; median of 7 batches."""
    rows = []
    for M, K, ncopy in ((3072, 1024, 700), (151936, 896, 16)):
        w = tq.synth_vq2(M, K, seed=tq.synth_seed(0, -3, f"vq2_{M}"))
        x = tq.synth_normal(K, seed=tq.synth_seed(0, -3, f"vq2x_{M}"))
        copies = [tq.DeviceBuffer.from_array(w) for _ in range(ncopy)]
        dx, dy = tq.DeviceBuffer.from_array(x), tq.DeviceBuffer(4 * M)
        ops = [tq.Op(tq.OP_VQ2_MATVEC, c.ptr, dx.ptr, dy.ptr, M, K, 1, 0) for c in copies]
        ms = time_ops(tq, ops, max(1, reps * 3 // ncopy), 1, stream, batches=7) / len(ops)
        b = 2048 + M * (K // 4) + 4 * (M + K)
        rec = {"shape": f"{M}x{K}", "us": round(ms * 1e3, 2), "gbs": round(b / (ms * 1e-3) / 1e9, 1),
               "frac": round(b / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes": b, "copies": ncopy}
        rows.append(rec)
        stream.synchronize()
        PENDING.append((rec, "vq2", (w, x, M, K), dy.download(np.float32, M)))
        for c in copies:
            c.free()
        dx.free()
        dy.free()
    return rows


def host_call(tq, reps=50):
    """The reference-signature entry point (tqhip_matvec_i4: host x in, host y out,
    weights cached in HBM after the first call): PCIe-inclusive latency per call (median of
    reps wall-clock calls), then the same calls with HIP events around the x upload, the
    kernel and the y download (tqhip_host_timing), medians of each."""
    rows = []
    lib = tq.lib()
    for M, K in ((4864, HIDDEN), (VOCAB, 2560)):
        w = tq.synth_i4(M, K, G, seed=tq.synth_seed(0, -2, f"host_{M}"))
        x = tq.synth_normal(K, seed=tq.synth_seed(0, -2, f"hostx_{M}"))
        y = np.empty(M, np.float32)
        f = lib.tqhip_matvec_i4
        args = (w.ctypes.data, x.ctypes.data, y.ctypes.data, M, K, G)
        for _ in range(3):
            f(*args)
        wall = []
        for _ in range(reps):
            t0 = time.perf_counter()
            f(*args)
            wall.append(time.perf_counter() - t0)
        us = float(np.median(wall)) * 1e6
        lib.tqhip_host_timing(1)
        split = []
        a, b, c = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
        for _ in range(reps):
            f(*args)
            lib.tqhip_host_timing_last(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
            split.append((a.value, b.value, c.value))
        lib.tqhip_host_timing(0)
        med = np.median(np.array(split), axis=0) * 1e3
        rows.append({"shape": f"{M}x{K}", "us": round(us, 2), "gbs": round(algo_bytes(M, K) / (us * 1e-6) / 1e9, 1),
                     "split_us": {"x_upload": round(float(med[0]), 2), "kernel": round(float(med[1]), 2),
                                  "y_download": round(float(med[2]), 2)}})
    lib.tqhip_release_weights()
    return rows


def engine(tq, steps, warmup):
    """Decode engine tokens/s on a synthetic Qwen2.5-0.5B-shaped dense i4 model held in memory."""
    img, cfg, _ = tq.tqwen_synth.dense_i4_model(hidden=HIDDEN, n_heads=14, n_kv_heads=2, head_dim=64, inter=INTER,
                                             vocab=VOCAB, layers=N_LAYERS, group_size=G, seed=11,
                                             max_seq_len=4096)
    m = tq.ModelFile.from_image(img)
    t0 = time.perf_counter()
    m.upload()
    upload_s = time.perf_counter() - t0
    eng = tq.DecodeEngine(m, warmup + steps + 1)
    tok = 1
    for _ in range(warmup):
        tok = eng.step(tok)
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = eng.step(tok)
    dt = (time.perf_counter() - t0) / steps
    got = replay(eng, ENGINE_CHECK_TOKENS)  # outside the timed region, for the correctness gate
    eng.close()
    m.close()
    # the reference's own CPU decode (QwenModel::forward_token, `ref` kernels) on the same file: its
    # time per token (a CPU baseline) and its logits for the gate
    cpu, want = ref_decode(img, ENGINE_CHECK_TOKENS, timed=3)
    # the same shape as a BiIP-rotated VQ2 file (VQ2 projections, fp16 vectors, compact-i4 embedding)
    img2, _, _ = tq.tqwen_synth.dense_i4_model(hidden=HIDDEN, n_heads=14, n_kv_heads=2, head_dim=64, inter=INTER,
                                            vocab=VOCAB, layers=N_LAYERS, group_size=G, seed=12, max_seq_len=4096,
                                            vq2=True, rotated=True)
    m2 = tq.ModelFile.from_image(img2)
    eng2 = tq.DecodeEngine(m2, warmup + steps + 1)
    tok = 1
    for _ in range(warmup):
        tok = eng2.step(tok)
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = eng2.step(tok)
    dt2 = (time.perf_counter() - t0) / steps
    got2 = replay(eng2, ENGINE_CHECK_TOKENS[:2])
    eng2.close()
    m2.close()
    _, want2 = ref_decode(img2, ENGINE_CHECK_TOKENS[:2], timed=0)
    vq2 = {"model": "the same shape as a BiIP-rotated VQ2 file", "file_bytes": len(img2),
           "ms_per_token": round(dt2 * 1e3, 4), "tokens_per_s": round(1.0 / dt2, 1)}
    rec = {"model": "Qwen2.5-0.5B-shaped dense i4 HQQ@64 (24 layers, hidden 896, 14/2 heads, inter 4864, "
                    "vocab 151936, tied i4 embedding), random weights", "vq2_rotated": vq2,
           "file_bytes": len(img), "upload_s": round(upload_s, 3), "positions": f"{warmup}..{warmup + steps - 1}",
           "ms_per_token": round(dt * 1e3, 4), "tokens_per_s": round(1.0 / dt, 1), "cpu_reference": cpu}
    if want is not None:
        settle(rec, check_logits(got, want))
    if want2 is not None:
        settle(vq2, check_logits(got2, want2))
    return rec


ENGINE_CHECK_TOKENS = (1, 2, 3, 4)


def replay(eng, tokens):
    """The engine from position 0 again on a fixed token sequence: (next token, logits) per step."""
    eng.reset()
    out = []
    for t in tokens:
        nxt = eng.step(t)
        out.append((nxt, eng.logits().copy()))
    return out


def ref_decode(img, tokens, timed):
    """The reference's own CPU decode (oracle/_ref: QwenModel::forward_token with the `ref` kernels,
    one thread) of a model image on a token sequence: its ms per token over the last `timed`
    steps (None when timed is 0), and its logits per step. (None, None) when the compiled reference
    is absent."""
    sys.path.insert(0, REPO)
    import oracle  # the CPU baseline and checker
    ref = oracle.ref_lib()
    if ref is None:
        return None, None
    import tempfile
    logits, t0 = [], None
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "bench.tqwen")
        with open(path, "wb") as f:
            f.write(img)
        err = ctypes.create_string_buffer(512)
        if not ref.tqref_decode_create(path.encode(), 16, err, len(err)):
            log(f"[bench] reference decode unavailable: {err.value.decode(errors='replace')}")
            return None, None
        for i, t in enumerate(tokens):
            if i == len(tokens) - timed:
                t0 = time.perf_counter()
            ref.tqref_decode_step(t)
            lg = np.empty(VOCAB, np.float32)
            ref.tqref_decode_logits(lg.ctypes.data, VOCAB)
            logits.append(lg)
        el = time.perf_counter() - t0 if timed else 0.0
    cpu = None
    if timed:
        cpu = {"ms_per_token": round(el / timed * 1e3, 1), "tokens": timed, "cores": 1, "kind": "reference"}
    return cpu, logits


def check_logits(got, want):
    """Engine logits per step against the reference decode's: rel L2 <= 1e-4 (the decode tests' bar:
    fp32 sums where the reference sums in double, a two-pass softmax), and the same next token
    wherever the reference's top two logits are more than 1e-3 of the logit scale apart."""
    checks = []
    for (tok, g), w in zip(got, want):
        c = compare(g, w, ENGINE_BAR, max_bar=1e-2)
        top = np.sort(w)[-2:]
        if top[1] - top[0] > 1e-3 * np.max(np.abs(w)) and tok != int(np.argmax(w)):
            c["verdict"] = "FAIL"
        checks.append(c)
    out = worst(checks)
    out["tokens"] = len(checks)
    out["bar"] = f"rel L2 <= {ENGINE_BAR:g} per step, same greedy token where the top-2 gap > 1e-3 of the scale"
    return out


def cpu_baseline(work, budget_s=12.0):
    """The reference's ref matvec (or the restatement) over the same step, row-split across threads."""
    sys.path.insert(0, REPO)
    import oracle  # the checker; used here only as the CPU baseline
    ref = oracle.ref_lib()
    kind = "reference" if ref is not None else "port"
    fn = ref.tqref_matvec_i4 if ref is not None else oracle.lib().orc_matvec_i4
    # Every host CPU the process may use, up to 16: the GPU box gives one GPU's job a share
    # of 16 threads whatever nproc shows (worker pools are sized to that share there).
    host_cpus = os.cpu_count() or 1
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = host_cpus
    threads = max(1, min(16, usable))
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
            "ms_per_step": round(ms, 2), "cpu": cpu, "host_cpus": host_cpus, "usable_cpus": usable,
            "threads_why": "all usable CPUs up to the 16-thread share a one-GPU job has on the GPU box",
            "sample": f"{n} full steps (all 169 matvecs, {work.bytes / 1e6:.0f} MB), rows split over {threads} threads"}, outs


def gate(pending, threads=16):
    """The correctness gate over the outputs the timed sections kept: each against the CPU checker
    (the restatement of the reference's ref kernels, pinned bit for bit to the compiled reference;
    row-split over threads). i4 and VQ2 matvecs at the matvec bar, the prefill GEMM at the prefill
    bar on every 97th row (every row at 32 tokens)."""
    sys.path.insert(0, REPO)
    import oracle  # the checker
    for rec, kind, args, got in pending:
        if kind == "i4":
            w, x, M, K = args
            c = compare(got, oracle.matvec_i4(w, x, M, K, G, threads=threads), MATVEC_BAR)
        elif kind == "vq2":
            w, x, M, K = args
            c = compare(got, oracle.matvec_vq2(w, x, M, K, threads=threads), MATVEC_BAR)
        else:
            w, x, M, K, n = args
            rows = np.arange(M) if n <= 32 else np.arange(0, M, 97)
            rb = w.size // M
            want = oracle.matmul_i4(np.ascontiguousarray(w.reshape(M, rb)[rows]).ravel(), x, rows.size, K, n, G,
                                    threads=threads)
            c = compare(got.reshape(n, M)[:, rows], want, PREFILL_BAR)
            c["rows_checked"] = int(rows.size)
        settle(rec, c)


def check_step(work, ref_outs):
    """The step's 169 outputs (as its last timed launches left them) against the reference outputs
    the CPU baseline computed on the same inputs."""
    got = work.download_outputs()
    return worst([compare(g, w, MATVEC_BAR) for g, w in zip(got, ref_outs)])


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=60)
    ap.add_argument("--warmup", type=int, default=6)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU reference timing")
    ap.add_argument("--no-headline", action="store_true", help="skip the 151936x2560 rotated headline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill dequant-GEMM timings")
    ap.add_argument("--no-host-call", action="store_true", help="skip the host-pointer (PCIe-inclusive) timing")
    ap.add_argument("--no-vq2", action="store_true", help="skip the VQ2 matvec timings")
    ap.add_argument("--no-engine", action="store_true", help="skip the device-resident decode engine timing")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay of the step")
    ap.add_argument("--no-configs2", action="store_true",
                    help="skip the configs[0] matvec and the configs[2] gate/up, down and attention matvecs")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the stream-read / launch / MFMA ceilings")
    ap.add_argument("--only", choices=("prefill", "vq2", "headline", "configs0", "configs2", "ceilings", "engine"),
                    help="run just this section and print its JSON (for profiler runs; not the contract line)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MB",
                    help="first run one device-to-device copy of MB MiB (a known-size kernel for counter runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the matvec would shard by "
              "output rows, each GPU holding whole 16-row tiles and the full x, with one all-gather of y). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    tq = load_pkg()
    t_section = [time.perf_counter()]

    def took(name):  # wall-clock seconds of each section, on stderr
        now = time.perf_counter()
        log(f"[bench] ({name}: {now - t_section[0]:.1f} s)")
        t_section[0] = now

    if tq.device_count() < 1:
        print("no HIP device visible", file=sys.stderr)
        sys.exit(1)
    log(f"[bench] device: {tq.device_name()}")
    stream = tq.Stream()
    if args.copy_calibration > 0:
        nb = args.copy_calibration << 20
        a, b = tq.DeviceBuffer(nb), tq.DeviceBuffer(nb)
        tq.lib().tqhip_memset(a.ptr, 1, nb)
        tq.synchronize()
        tq.lib().tqhip_memcpy_d2d(b.ptr, a.ptr, nb)
        tq.synchronize()
        log(f"[bench] calibration copy: {nb} bytes device to device")
        a.free()
        b.free()
    if args.only:
        if args.only == "engine":
            print(json.dumps({"engine": engine(tq, args.steps, args.warmup)}), flush=True)
            return
        fn = {"prefill": prefill, "vq2": vq2, "headline": headline, "configs2": configs2, "ceilings": ceilings,
              "configs0": configs0}[args.only]
        print(json.dumps({args.only: fn(tq, stream)}), flush=True)
        return
    work = Workload(tq)

    # whole step: --warmup untimed steps, then exactly --steps timed steps, rotating over the copies
    tq.run_ops(work.steps(args.warmup), 1, stream)
    tq.synchronize()
    ms_step = time_ops(tq, work.steps(args.steps), 1, 0, stream) / args.steps
    value = work.bytes / (ms_step * 1e-3) / 1e9
    log(f"[bench] step (one set launch per layer + lm_head): {ms_step * 1e3:.1f} us, {value:.1f} GB/s")
    ms_rt = time_ops(tq, work.steps(args.steps, runtime_order=True), 1, 1, stream) / args.steps
    rt = {"ms_per_step": round(ms_rt, 4), "value": round(work.bytes / (ms_rt * 1e-3) / 1e9, 1),
          "launches_per_step": len(work.rt_steps[0])}
    log(f"[bench] step in the runtime's call order ({rt['launches_per_step']} launches): {ms_rt * 1e3:.1f} us, "
        f"{rt['value']} GB/s")
    ms_dep = time_ops(tq, work.steps(args.steps, dependent=True), 1, 1, stream) / args.steps
    dep = {"ms_per_step": round(ms_dep, 4), "value": round(work.bytes / (ms_dep * 1e-3) / 1e9, 1),
           "launches_per_step": len(work.dep_steps[0]),
           "chain": "layer l > 0 reads layer l - 1's outputs (attention in <- down, MLP in <- o, o in <- q, "
                    "down in <- gate); the lm_head reads the last down output"}
    log(f"[bench] dependent step (each layer set reads the previous one's outputs): {ms_dep * 1e3:.1f} us, "
        f"{dep['value']} GB/s")
    took("steps")
    ls = layer_set(tq, work, stream, max(2, args.steps // N_COPIES))
    log(f"[bench] layer set: {ls['us']} us as one launch ({ls['us_graph']} us from a HIP graph), "
        f"{ls['us_4launch']} us as 4 dependency-ordered launches")
    took("layer set")
    step_outputs = work.download_outputs()  # the outputs of the set launches just timed, for the gate
    graph = None
    if not args.no_graph:  # the step captured into one HIP graph (three steps, one per copy) and replayed
        ms_graph = time_graph(tq, work.steps(N_COPIES), max(1, args.steps // N_COPIES), 1, stream) / N_COPIES
        graph = {"ms_per_step": round(ms_graph, 4), "value": round(work.bytes / (ms_graph * 1e-3) / 1e9, 1)}
        log(f"[bench] step as a HIP graph replay: {ms_graph * 1e3:.1f} us, {graph['value']} GB/s")
    # The host-pointer call before the sections that allocate and free hundreds of weight copies:
    # measured after them (the VQ2 section's 716), its 4864x896 call once took 132 us against
    # 25-27 us in a fresh process, with the same HIP-event split (not reproduced in isolation).
    host = None if args.no_host_call else host_call(tq)
    if host:
        log(f"[bench] host-pointer call (x H2D + kernel + y D2H, weights cached): " +
            ", ".join(f"{r['shape']} {r['us']} us (upload {r['split_us']['x_upload']}, kernel "
                      f"{r['split_us']['kernel']}, download {r['split_us']['y_download']})" for r in host))
        took("host call")
    roof = roofline(ls["us"])
    log(f"[bench] dominant kernel (set): {roof['avg_launch_us']} us per launch, {roof['achieved']} GB/s "
        f"({100 * roof['frac']:.1f}% of 8 TB/s)")
    ceil = None if args.no_ceilings else ceilings(tq, stream)
    if ceil:
        log(f"[bench] ceilings: stream read {ceil['stream_read_gbs']} GB/s, empty launch {ceil['empty_launch_us']} us, "
            f"fp16 MFMA {ceil['mfma_f16_tflops']} TFLOP/s")
        took("ceilings")

    head = None if args.no_headline else headline(tq, stream)
    if head:
        log(f"[bench] headline 151936x2560: {head['us']} us, {head['gbs']} GB/s ({100 * head['frac']:.1f}% of 8 TB/s)")
        took("headline")
    c0 = None if args.no_configs2 else configs0(tq, stream)
    if c0:
        log(f"[bench] configs[0] matvec {c0['shape']}: {c0['us']} us, {c0['gbs']} GB/s (one cold launch)")
    c2 = None if args.no_configs2 else configs2(tq, stream)
    if c2:
        log("[bench] configs[2] matvecs: " + ", ".join(f"{r['shape']} {r['us']} us {r['gbs']} GB/s" for r in c2))
        took("configs0/2")
    pre = None if args.no_prefill else prefill(tq, stream)
    if pre:
        for r in pre["tokens"]:
            log(f"[bench] prefill 9728x2560 x{r['tokens']}: {r['us']} us, {r['tflops']} TFLOP/s "
                f"({100 * r['mfma_frac']:.1f}% of dense fp16 MFMA)")
        took("prefill")

    v = None if args.no_vq2 else vq2(tq, stream)
    if v:
        log("[bench] vq2 matvec: " + ", ".join(f"{r['shape']} {r['us']} us {r['gbs']} GB/s" for r in v))
        took("vq2")

    eng = None if args.no_engine else engine(tq, args.steps, args.warmup)
    if eng:
        log(f"[bench] decode engine: {eng['ms_per_token']} ms/token, {eng['tokens_per_s']} tokens/s "
            f"(positions {eng['positions']}); rotated VQ2 file: {eng['vq2_rotated']['ms_per_token']} ms/token")
        took("engine")

    # The CPU leg: the reference's own kernels timed on the host (the CPU baseline), then the
    # correctness gate with the reference outputs and the checker.
    cpu, verify = None, None
    if not args.no_cpu_baseline:
        cpu, ref_outs = cpu_baseline(work)
        log(f"[bench] cpu baseline ({cpu['kind']}, {cpu['cores']} threads of {cpu['host_cpus']}): "
            f"{cpu['ms_per_step']} ms/step, {cpu['value']} GB/s")
        took("cpu baseline")
        step_check = worst([compare(g, w, MATVEC_BAR) for g, w in zip(step_outputs, ref_outs)])
        gate(PENDING)
        verify = {"step": step_check}
        for name, sec in (("headline", head), ("configs0", c0)):
            if sec:
                verify[name] = sec["verify"]
        if c2:
            verify["configs2"] = worst([r["verify"] for r in c2])
        if pre:
            verify["prefill"] = worst([r["verify"] for r in pre["tokens"]])
        if v:
            verify["vq2"] = worst([r["verify"] for r in v])
        if eng and "verify" in eng:
            verify["engine"] = eng["verify"]
        if eng and "verify" in eng["vq2_rotated"]:
            verify["engine_vq2_rotated"] = eng["vq2_rotated"]["verify"]
        for name, c in verify.items():
            log(f"[bench] verify {name}: {c['verdict']} (rel L2 {c['rel_l2']}, max rel {c['max_rel']})")
        took("gate")
        if step_check["verdict"] != "PASS":  # a step whose outputs fail the gate has no figure
            value, ms_step = None, None

    out = {
        "metric": METRIC, "value": None if value is None else round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": None if ms_step is None else round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4 codes x f32 activations (i8 digit planes of the activations, exact integer "
                 "dot products, f32 epilogue)",
        "data": "synthetic (BASELINE distributions, seeded); weights read cold (3 rotated copies)",
        "pct_of_peak": None if value is None else round(100 * value / PEAK_GBS, 2),
        "us_per_layer_set": ls["us"],
        "layer_set": ls,
        "step_runtime_order": rt,
        "step_dependent": dep,
        "graph": graph,
        "config": {"workload": "BASELINE configs[1]: Qwen2.5-0.5B-shaped i4 HQQ@64 decode matvec set, batch=1, "
                               "24 layers x (q 896x896, k/v 128x896, o 896x896, gate/up 4864x896, down 896x4864) "
                               "+ lm_head 151936x896, independent seeded weights; one set launch per layer",
                   "bytes_per_step": work.bytes, "matvecs_per_step": len(work.host),
                   "launches_per_step": len(work.set_steps[0]), "group_size": G, "weight_copies": N_COPIES},
        "roofline": roof,
        "ceilings": ceil,
        "headline": head,
        "configs0": c0,
        "configs2": c2,
        "prefill": pre,
        "vq2": v,
        "host_call": host,
        "engine": eng,
        "cpu_baseline": cpu,
        "verify": verify,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
