"""One launch over a set of i4 matvecs with their own activations (tqhip_matvec_i4_set_dev).

Every output of the set is held to the matvec bar (rel L2 <= 1e-5, max|err| <= 1e-3 of
max|y|) against the oracle, and where tqhip_matvec_i4_dev runs the set kernel on the
same matrix alone (every decode-size launch of the layer), the set output must have
the same bits. Cases: the Qwen2.5-0.5B layer set, the
Qwen3.5-4B layer shapes, the golden fixtures of the reference in one set,
ragged shapes, more than eight matrices, matrices the set kernel does not take
(G != 64, K % 4 != 0, misaligned x, K > 10240), error codes, and a captured op list.
"""
import numpy as np
import pytest

from conftest import golden, golden_names, max_abs_rel, rel_l2

pytestmark = pytest.mark.gpu

QWEN25_LAYER = [("q", 896, 896, "attn"), ("k", 128, 896, "attn"), ("v", 128, 896, "attn"), ("o", 896, 896, "o"),
                ("gate", 4864, 896, "mlp"), ("up", 4864, 896, "mlp"), ("down", 896, 4864, "down")]


def assert_close(got, want, what):
    l2, mx = rel_l2(got, want), max_abs_rel(got, want)
    assert l2 <= 1e-5 and mx <= 1e-3, f"{what}: rel_l2={l2:.3e} max_rel={mx:.3e}"


def assert_close_rows(got, want, orc, w, x, M, K, what):
    """For outputs of a few rows, where one near-cancelled row dominates the relative L2:
    each row within 1e-5 of the size of its own terms, sum_k |w_mk * x_k| (an fp32 dot
    product of K terms stays well inside that), plus the usual bar where M >= 16."""
    wd = orc.dequant_i4_matrix_f64(w, M, K, 64)
    bound = 1e-5 * (np.abs(wd) @ np.abs(x.astype(np.float64)))
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= bound), f"{what}: worst row err/bound = {float(np.max(err / bound)):.3f}"
    if M >= 16:
        assert_close(got, want, what)


def build(gpu, spec, G, seed):
    """spec: (name, M, K, x key); matrices sharing a key share the activation vector."""
    xs, mats = {}, []
    for i, (name, M, K, key) in enumerate(spec):
        if key not in xs:
            x = gpu.synth_normal(K, seed=seed + 1000 + len(xs))
            xs[key] = (x, gpu.DeviceBuffer.from_array(x))
        w = gpu.synth_i4(M, K, G, seed=seed + i)
        mats.append((name, M, K, w, xs[key], gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer(4 * M)))
    return mats


def run_set(gpu, mats, G):
    arr = gpu.i4_set([(dw, x[1], dy, M, K) for _, M, K, _, x, dw, dy in mats])
    for _, M, _, _, _, _, dy in mats:
        gpu.lib().tqhip_memset(dy.ptr, 0xFF, 4 * M)  # every output must be written by the set
    gpu.matvec_i4_set_dev(arr, G)
    gpu.synchronize()
    return [dy.download(np.float32, M) for _, M, _, _, _, _, dy in mats]


def singles(gpu, mats, G):
    out = []
    for _, M, K, _, x, dw, _ in mats:
        dy = gpu.DeviceBuffer(4 * M)
        gpu.matvec_i4_dev(dw, x[1], dy, M, K, G)
        gpu.synchronize()
        out.append(dy.download(np.float32, M))
    return out


def test_qwen25_layer_set(gpu, orc):
    mats = build(gpu, QWEN25_LAYER, 64, seed=40)
    got = run_set(gpu, mats, 64)
    alone = singles(gpu, mats, 64)
    for (name, M, K, w, x, _, _), g, a in zip(mats, got, alone):
        assert_close(g, orc.matvec_i4(w, x[0], M, K, 64, threads=16), name)
        assert np.array_equal(g, a), f"{name}: set output differs from the single launch (the same kernel)"
    # the same set again: bit-identical (deterministic)
    again = run_set(gpu, mats, 64)
    for (name, *_), g, h in zip(mats, got, again):
        assert np.array_equal(g, h), name


def test_qwen35_4b_layer_shapes(gpu, orc):
    """every long-row matrix has >= 2048 rows, so each wave takes two rows. With a
    896x4864 matrix added, the set runs one long row per wave; the rows of a matrix get the same
    bits either way, and the same bits as its single launch."""
    spec = [("qkv_in", 4096, 2560, "attn"), ("o", 2560, 4096, "o"), ("gate", 9728, 2560, "mlp"),
            ("up", 9728, 2560, "mlp"), ("down", 2560, 9728, "down")]
    mats = build(gpu, spec, 64, seed=60)
    got = run_set(gpu, mats, 64)
    alone = singles(gpu, mats, 64)
    for (name, M, K, w, x, _, _), g, a in zip(mats, got, alone):
        assert_close(g, orc.matvec_i4(w, x[0], M, K, 64, threads=16), name)
        assert np.array_equal(g, a), f"{name}: set output differs from the single launch"
    small = build(gpu, [("small_down", 896, 4864, "s")], 64, seed=70)
    mixed = run_set(gpu, mats + small, 64)
    for (name, *_), g, m in zip(mats, got, mixed):
        assert np.array_equal(g, m), f"{name}: two long rows per wave vs one differ"
    _, M, K, w, x, _, _ = small[0]
    assert_close(mixed[-1], orc.matvec_i4(w, x[0], M, K, 64, threads=16), "small_down")


def test_golden_fixtures_in_one_set(gpu):
    """The reference's outputs (tests/golden, written by its compiled ref kernel) for every
    G = 64 fixture, all in one set launch: special fp16 headers and partial groups included."""
    names = [n for n in golden_names("i4_") if n.endswith("_g64") and "pair" not in n and "qkv" not in n]
    assert len(names) >= 6
    mats, wants = [], []
    for n in names:
        f = golden(n)
        M, K, G = (int(v) for v in f["dims"])
        x = np.ascontiguousarray(f["x"], np.float32)
        mats.append((n, M, K, f["w"], (x, gpu.DeviceBuffer.from_array(x)), gpu.DeviceBuffer.from_array(f["w"]),
                     gpu.DeviceBuffer(4 * M)))
        wants.append(f["y"])
    got = run_set(gpu, mats, 64)
    for (n, *_), g, y in zip(mats, got, wants):
        assert_close(g, y, n)


def test_ragged_and_more_than_eight(gpu, orc):
    # rows not a multiple of a workgroup's rows, partial last groups, K just over 1024 (one
    # wave-row slot) and over 2048 (two), single rows; 11 matrices = two launches
    spec = [("a", 1, 64, "a"), ("b", 3, 200, "b"), ("c", 9, 1028, "c"), ("d", 17, 2052, "d"), ("e", 333, 964, "e"),
            ("f", 5, 4, "f"), ("g", 100, 10240, "g"), ("h", 7, 6144, "h"), ("i", 250, 36, "i"), ("j", 13, 1024, "j"),
            ("k", 2, 8196, "k")]
    mats = build(gpu, spec, 64, seed=80)
    got = run_set(gpu, mats, 64)
    for (name, M, K, w, x, _, _), g in zip(mats, got):
        assert_close_rows(g, orc.matvec_i4(w, x[0], M, K, 64, threads=16), orc, w, x[0], M, K, f"{name} {M}x{K}")


def test_matrices_the_set_kernel_does_not_take(gpu, orc):
    """G = 128 (the whole call), K % 4 != 0, K > 10240 and a misaligned x go through the
    single-matrix kernels; the rest of the set still runs."""
    mats = build(gpu, [("odd_k", 40, 70, "a"), ("wide", 24, 12288, "b"), ("ok", 300, 896, "c")], 64, seed=90)
    # a misaligned activation pointer: x offset by one float inside a larger buffer
    K = 896
    xb = gpu.synth_normal(K + 1, seed=95)
    dxb = gpu.DeviceBuffer.from_array(xb)
    w = gpu.synth_i4(64, K, 64, seed=96)
    mats.append(("misaligned", 64, K, w, (xb[1:].copy(), dxb.ptr + 4), gpu.DeviceBuffer.from_array(w),
                 gpu.DeviceBuffer(4 * 64)))
    got = run_set(gpu, mats, 64)
    for (name, M, K, w, x, _, _), g in zip(mats, got):
        assert_close(g, orc.matvec_i4(w, x[0], M, K, 64, threads=16), name)
    mats = build(gpu, [("g128a", 100, 1024, "a"), ("g128b", 33, 640, "b")], 128, seed=97)
    got = run_set(gpu, mats, 128)
    for (name, M, K, w, x, _, _), g in zip(mats, got):
        assert_close(g, orc.matvec_i4(w, x[0], M, K, 128, threads=16), name)


def test_error_codes(gpu):
    lib = gpu.lib()
    arr = gpu.i4_set([(0, 0, 0, 0, 64)])
    assert lib.tqhip_matvec_i4_set_dev(gpu.ctypes.addressof(arr), 1, 64, None) == gpu.EBADSHAPE
    arr = gpu.i4_set([(0, 0, 0, 4, 64)])
    assert lib.tqhip_matvec_i4_set_dev(gpu.ctypes.addressof(arr), 1, 3, None) == gpu.EBADGROUP
    assert lib.tqhip_matvec_i4_set_dev(None, 1, 64, None) == gpu.EBADSHAPE
    assert lib.tqhip_matvec_i4_set_dev(None, 0, 64, None) == gpu.OK  # an empty set launches nothing


def test_set_op_in_a_captured_graph(gpu, orc):
    """TQHIP_OP_I4_SET in an op list: eager run and graph replays agree bit for bit, with new
    activations written before each replay (the replay reads them at replay time)."""
    mats = build(gpu, QWEN25_LAYER, 64, seed=120)
    arr = gpu.i4_set([(dw, x[1], dy, M, K) for _, M, K, _, x, dw, dy in mats])
    ops = [gpu.set_op(arr, 64)]
    stream = gpu.Stream()
    graph = gpu.OpsGraph(ops, stream)
    keys = {}
    for _, _, K, _, x, _, _ in mats:
        keys[id(x)] = (x, K)
    try:
        for rep in range(3):
            for i, (x, K) in enumerate(keys.values()):
                v = gpu.synth_normal(K, seed=130 + 10 * rep + i)
                x[1].upload(v)
                x[0][:] = v
            gpu.run_ops(ops, 1, stream)
            stream.synchronize()
            want = [dy.download(np.float32, M) for _, M, _, _, _, _, dy in mats]
            for _, M, _, _, _, _, dy in mats:
                gpu.lib().tqhip_memset(dy.ptr, 0xFF, 4 * M)
            graph.launch()
            stream.synchronize()
            for (name, M, K, w, x, _, dy), wv in zip(mats, want):
                assert np.array_equal(dy.download(np.float32, M), wv), f"replay {rep}: {name}"
        for (name, M, K, w, x, _, _), wv in zip(mats, want):
            assert_close(wv, orc.matvec_i4(w, x[0], M, K, 64, threads=16), name)
    finally:
        graph.close()


def test_non_finite_activation_stays_in_its_matrix(gpu, orc):
    """A NaN in one activation vector of a set (up's x): every output of the matrices that read it
    is non-finite, as in the reference, and the matrices with other activation vectors are finite
    and unchanged (each workgroup converts only its own matrix's activations)."""
    mats = build(gpu, QWEN25_LAYER, 64, seed=70)
    clean = run_set(gpu, mats, 64)
    x_mlp, dx_mlp = next(m[4] for m in mats if m[0] == "gate")
    poisoned = x_mlp.copy()
    poisoned[100] = np.nan
    dx_mlp.upload(poisoned)
    got = run_set(gpu, mats, 64)
    for (name, M, K, w, x, _, _), g, c in zip(mats, got, clean):
        if name in ("gate", "up"):
            assert not np.any(np.isfinite(orc.matvec_i4(w, poisoned, M, K, 64, threads=16)))
            assert not np.any(np.isfinite(g)), f"{name}: finite outputs from a NaN activation"
        else:
            assert np.array_equal(g, c), f"{name}: changed by another matrix's NaN activation"
