"""An op list captured into a HIP graph (tqhip_ops_graph_create) and replayed.

Every replay must equal an eager run of the same list on the same inputs, bit for
bit (the same kernels run), with eager work and host synchronisations between
the replays and new activations written before each one: the replay reads the
buffers at replay time, and the split-K tile counters come back to zero after
every replay. The list covers every kernel family the step uses: the
register-path matvec (single, qkv, pair), split-K, the wave-private DMA ring,
VQ2 (one wave per row, and the dot-product table kernel with its 128 KB of static LDS) and
the prefill GEMM. The eager result is also checked against the oracle.
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
    MT = 151936  # VQ2 lm_head rows: the table kernel
    wvt = gpu.synth_vq2(MT, K, seed=401)
    dw = {n: gpu.DeviceBuffer.from_array(w) for n, w in ws.items()}
    dwv, dwvt = gpu.DeviceBuffer.from_array(wv), gpu.DeviceBuffer.from_array(wvt)
    NT = 7  # prefill tokens
    xk = {K: gpu.DeviceBuffer(4 * K), 4864: gpu.DeviceBuffer(4 * 4864), 2560: gpu.DeviceBuffer(4 * 2560),
          1024: gpu.DeviceBuffer(4 * 1024), "mm": gpu.DeviceBuffer(4 * K * NT)}
    dy = {n: gpu.DeviceBuffer(4 * m * (NT if n == "mm" else 1)) for n, (m, _) in mats.items()}
    dyv, dyvt = gpu.DeviceBuffer(4 * 3072), gpu.DeviceBuffer(4 * MT)
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
        Op(gpu.OP_VQ2_MATVEC, dwvt.ptr, xk[K].ptr, dyvt.ptr, MT, K, 1, 0, None, None, None, None, 0),
        Op(gpu.OP_I4_MATMUL, dw["mm"].ptr, xk["mm"].ptr, dy["mm"].ptr, 300, K, NT, G, None, None, None, None, 0),
    ]
    outs = list(dy.items()) + [("vq2", dyv), ("vq2_table", dyvt)]
    sizes = {n: m * (NT if n == "mm" else 1) for n, (m, _) in mats.items()}
    sizes["vq2"] = 3072
    sizes["vq2_table"] = MT

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
        ref = orc.matvec_vq2(wvt, xs[K], MT, K, threads=8)
        assert rel_l2(want["vq2_table"], ref) <= 1e-5 and max_abs_rel(want["vq2_table"], ref) <= 1e-3, "vq2_table"
    finally:
        graph.close()


def test_graph_scratch_survives_larger_eager_calls(gpu, orc):
    """A graph owns its scratch: after it is captured, eager calls that grow the stream's
    own scratch (a 512-token prefill, split-K matvecs) on the capture stream and on
    another stream cannot move or free what the replay uses. Every replay, on the capture
    stream or on another one, equals the eager run before it bit for bit."""
    K, NT = 896, 7
    w_mm = gpu.synth_i4(300, K, G, seed=500)
    w_sp = gpu.synth_i4(2560, 4096, G, seed=501)  # split-K over two parts
    d_mm, d_sp = gpu.DeviceBuffer.from_array(w_mm), gpu.DeviceBuffer.from_array(w_sp)
    x_mm = gpu.synth_normal(K * NT, seed=502)
    x_sp = gpu.synth_normal(4096, seed=503)
    dx_mm, dx_sp = gpu.DeviceBuffer.from_array(x_mm), gpu.DeviceBuffer.from_array(x_sp)
    dy_mm, dy_sp = gpu.DeviceBuffer(4 * 300 * NT), gpu.DeviceBuffer(4 * 2560)
    Op = gpu.Op
    ops = [Op(gpu.OP_I4_MATMUL, d_mm.ptr, dx_mm.ptr, dy_mm.ptr, 300, K, NT, G, None, None, None, None, 0),
           Op(gpu.OP_I4_MATVEC, d_sp.ptr, dx_sp.ptr, dy_sp.ptr, 2560, 4096, 1, G, None, None, None, None, 0)]
    # large eager work: a 512-token prefill (2.6 MB of X scratch) and a wider split-K matvec
    Mb, Kb, Nb = 9728, 2560, 512
    w_big = gpu.synth_i4(Mb, Kb, G, seed=504)
    d_big = gpu.DeviceBuffer.from_array(w_big)
    dx_big = gpu.DeviceBuffer.from_array(gpu.synth_normal(Kb * Nb, seed=505))
    dy_big = gpu.DeviceBuffer(4 * Mb * Nb)
    w_sp2 = gpu.synth_i4(4096, 9728, G, seed=506)
    d_sp2 = gpu.DeviceBuffer.from_array(w_sp2)
    dx_sp2, dy_sp2 = gpu.DeviceBuffer.from_array(gpu.synth_normal(9728, seed=507)), gpu.DeviceBuffer(4 * 4096)
    big = [Op(gpu.OP_I4_MATMUL, d_big.ptr, dx_big.ptr, dy_big.ptr, Mb, Kb, Nb, G, None, None, None, None, 0),
           Op(gpu.OP_I4_MATVEC, d_sp2.ptr, dx_sp2.ptr, dy_sp2.ptr, 4096, 9728, 1, G, None, None, None, None, 0)]

    s1, s2 = gpu.Stream(), gpu.Stream()
    graph = gpu.OpsGraph(ops, s1)
    try:
        gpu.run_ops(ops, 1, s1)
        s1.synchronize()
        want_mm, want_sp = dy_mm.download(np.float32, 300 * NT), dy_sp.download(np.float32, 2560)
        ref = orc.matmul_i4(w_mm, x_mm, 300, K, NT, G, threads=16)
        assert rel_l2(want_mm, ref) <= 2e-3 and max_abs_rel(want_mm, ref) <= 1e-3
        ref = orc.matvec_i4(w_sp, x_sp, 2560, 4096, G, threads=16)
        assert rel_l2(want_sp, ref) <= 1e-5 and max_abs_rel(want_sp, ref) <= 1e-3
        for rep, stream in enumerate((s1, s2, s1)):
            gpu.run_ops(big, 1, s1)  # grows the capture stream's own scratch
            gpu.run_ops(big, 1, s2)
            s1.synchronize()
            s2.synchronize()
            for b, n in ((dy_mm, 300 * NT), (dy_sp, 2560)):
                gpu.lib().tqhip_memset(b.ptr, 0xFF, 4 * n)
            graph.launch(stream)
            stream.synchronize()
            assert np.array_equal(dy_mm.download(np.float32, 300 * NT), want_mm), f"replay {rep}: prefill"
            assert np.array_equal(dy_sp.download(np.float32, 2560), want_sp), f"replay {rep}: split-K"
    finally:
        graph.close()


def test_prefill_on_two_streams_at_once(gpu, orc):
    """Two prefill GEMMs in flight together on two streams: each stream has its own fp16
    copy of X, so neither sees the other's activations."""
    G_ = 64
    cases = [(512, 896, 40, 600), (384, 640, 24, 601)]
    streams = [gpu.Stream(), gpu.Stream()]
    bufs = []
    for (M, K, N, seed), s in zip(cases, streams):
        w = gpu.synth_i4(M, K, G_, seed=seed)
        x = gpu.synth_normal(K * N, seed=seed + 50)
        dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M * N)
        bufs.append((w, x, dw, dx, dy))
    for rep in range(3):
        for (M, K, N, _), (w, x, dw, dx, dy), s in zip(cases, bufs, streams):
            gpu.matmul_i4_dev(dw, dx, dy, M, K, N, G_, stream=s)  # no synchronisation between the two
        for s in streams:
            s.synchronize()
        for (M, K, N, _), (w, x, dw, dx, dy) in zip(cases, bufs):
            got = dy.download(np.float32, M * N)
            ref = orc.matmul_i4(w, x, M, K, N, G_, threads=16)
            assert rel_l2(got, ref) <= 2e-3 and max_abs_rel(got, ref) <= 1e-3, (rep, M, K, N)
