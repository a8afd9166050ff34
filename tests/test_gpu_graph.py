"""An op list captured into a HIP graph (tqhip_ops_graph_create) and replayed.

Every replay must equal an eager run of the same list on the same inputs, bit for
bit (the same kernels run), with eager work and host synchronisations between
the replays and new activations written before each one: the replay reads the
buffers at replay time, and the split-K tile counters come back to zero after
every replay. The list covers every kernel family the step uses: the
register-path matvec (single, qkv, pair), split-K, the wave-private DMA ring,
VQ2 and the prefill GEMM. The eager result is also checked against the oracle.
"""
import numpy as np
import pytest

from conftest import max_abs_rel, rel_l2

pytestmark = pytest.mark.gpu

G = 64


def test_graph_replays_match_eager_runs(gpu, orc):
    K = 896
    mats = {"single": (4864, K), "q": (896, K), "k": (128, K), "v": (128, K), "gate": (4864, K), "up": (4864, K),
            "down": (896, 4864), "ring": (40000, 2560), "mm": (300, K)}
    ws = {n: gpu.synth_i4(m, k, G, seed=300 + i) for i, (n, (m, k)) in enumerate(mats.items())}
    wv = gpu.synth_vq2(3072, 1024, seed=400)
    dw = {n: gpu.DeviceBuffer.from_array(w) for n, w in ws.items()}
    dwv = gpu.DeviceBuffer.from_array(wv)
    NT = 7  # prefill tokens
    xk = {K: gpu.DeviceBuffer(4 * K), 4864: gpu.DeviceBuffer(4 * 4864), 2560: gpu.DeviceBuffer(4 * 2560),
          1024: gpu.DeviceBuffer(4 * 1024), "mm": gpu.DeviceBuffer(4 * K * NT)}
    dy = {n: gpu.DeviceBuffer(4 * m * (NT if n == "mm" else 1)) for n, (m, _) in mats.items()}
    dyv = gpu.DeviceBuffer(4 * 3072)
    Op = gpu.Op
    ops = [
        Op(gpu.OP_I4_MATVEC, dw["single"].ptr, xk[K].ptr, dy["single"].ptr, 4864, K, 1, G, None, None, None, None, 0),
        Op(gpu.OP_I4_QKV, dw["q"].ptr, xk[K].ptr, dy["q"].ptr, 896, K, 1, G, dw["k"].ptr, dw["v"].ptr, dy["k"].ptr,
           dy["v"].ptr, 128),
        Op(gpu.OP_I4_PAIR, dw["gate"].ptr, xk[K].ptr, dy["gate"].ptr, 4864, K, 1, G, dw["up"].ptr, None, dy["up"].ptr,
           None, 0),
        Op(gpu.OP_I4_MATVEC, dw["down"].ptr, xk[4864].ptr, dy["down"].ptr, 896, 4864, 1, G, None, None, None, None, 0),
        Op(gpu.OP_I4_MATVEC, dw["ring"].ptr, xk[2560].ptr, dy["ring"].ptr, 40000, 2560, 1, G, None, None, None, None,
           0),
        Op(gpu.OP_VQ2_MATVEC, dwv.ptr, xk[1024].ptr, dyv.ptr, 3072, 1024, 1, 0, None, None, None, None, 0),
        Op(gpu.OP_I4_MATMUL, dw["mm"].ptr, xk["mm"].ptr, dy["mm"].ptr, 300, K, NT, G, None, None, None, None, 0),
    ]
    outs = list(dy.items()) + [("vq2", dyv)]
    sizes = {n: m * (NT if n == "mm" else 1) for n, (m, _) in mats.items()}
    sizes["vq2"] = 3072

    def set_inputs(seed):
        xs = {}
        for key, buf in xk.items():
            n = K * NT if key == "mm" else key
            xs[key] = gpu.synth_normal(n, seed=seed + (n % 1000))
            gpu.lib().tqhip_memcpy_h2d(buf.ptr, xs[key].ctypes.data, 4 * n)
        return xs

    def read_all():
        return {n: b.download(np.float32, sizes[n]) for n, b in outs}

    stream = gpu.Stream()
    set_inputs(1)
    graph = gpu.OpsGraph(ops, stream)
    try:
        for rep in range(3):
            xs = set_inputs(10 + rep)
            gpu.run_ops(ops, 1, stream)  # eager run of the same list on the same inputs
            stream.synchronize()
            want = read_all()
            for n, b in outs:  # the replay must write every output itself
                gpu.lib().tqhip_memset(b.ptr, 0xFF, 4 * sizes[n])
            graph.launch()
            stream.synchronize()
            got = read_all()
            for n in want:
                assert np.array_equal(got[n], want[n]), f"replay {rep}: {n} differs from the eager run"
        # the eager results of the last inputs against the oracle
        checks = [("single", ws["single"], xs[K], 4864, K), ("q", ws["q"], xs[K], 896, K),
                  ("down", ws["down"], xs[4864], 896, 4864), ("ring", ws["ring"], xs[2560], 40000, 2560)]
        for n, w, x, m, k in checks:
            ref = orc.matvec_i4(w, x, m, k, G, threads=16)
            assert rel_l2(want[n], ref) <= 1e-5 and max_abs_rel(want[n], ref) <= 1e-3, n
        ref = orc.matvec_vq2(wv, xs[1024], 3072, 1024)
        assert rel_l2(want["vq2"], ref) <= 1e-5, "vq2"
    finally:
        graph.close()
