"""i4 HQQ matvec on the GPU against the oracle (and the reference's golden outputs).

Tolerance: rel L2 <= 1e-5 and max|err| <= 1e-3 * max|y_ref|.
"""
import numpy as np
import pytest

from conftest import golden, golden_names, max_abs_rel, rel_l2

pytestmark = pytest.mark.gpu

REL_L2 = 1e-5
MAX_REL = 1e-3


def assert_close(got, want, what=""):
    l2, mx = rel_l2(got, want), max_abs_rel(got, want)
    assert l2 <= REL_L2 and mx <= MAX_REL, f"{what}: rel_l2={l2:.3e} max_rel={mx:.3e}"


@pytest.mark.parametrize("name", [n for n in golden_names("i4_") if "qkv" not in n and "pair" not in n])
def test_golden_through_registry(gpu, name):
    f = golden(name)
    M, K, G = (int(v) for v in f["dims"])
    assert gpu.set_matvec_i4_impl_by_name("hip")
    got = gpu.matvec_i4(f["w"], f["x"], M, K, G)
    assert_close(got, f["y"], name)
    if name == "i4_kat_1x4_g4":
        assert abs(got[0] - 28.0) < 1e-5  # tests/test_matvec_i4.cpp:212


def test_golden_pair_and_qkv(gpu):
    f = golden("i4_pair_16x256_g64")
    M, K, G = (int(v) for v in f["dims"])
    y1, y2 = gpu.matvec_pair_i4(f["w1"], f["w2"], f["x"], M, K, G)
    assert_close(y1, f["y1"], "pair y1")
    assert_close(y2, f["y2"], "pair y2")
    f = golden("i4_qkv_48_16x256_g64")
    q, kv, K, G = (int(v) for v in f["dims"])
    yq, yk, yv = gpu.matvec_qkv_i4(f["wq"], f["wk"], f["wv"], f["x"], q, kv, K, G)
    assert_close(yq, f["yq"], "qkv q")
    assert_close(yk, f["yk"], "qkv k")
    assert_close(yv, f["yv"], "qkv v")


SHAPES = [
    (1, 64, 64), (15, 896, 64), (16, 896, 64), (17, 896, 64), (128, 896, 64), (896, 896, 64),
    (4864, 896, 64), (896, 4864, 64), (300, 2560, 64), (2560, 9728, 64), (333, 200, 64),
    (257, 1024, 128), (100, 520, 40), (64, 4096, 256), (50, 100, 32), (7, 70, 6), (41, 1000, 48),
    # register-path kernel over many tiles per workgroup (one, two and three
    # windows per wave, run-time group size); the wave-private DMA ring (three
    # windows: one and two workgroups per CU, rows of more than 24 windows,
    # more tiles than the register path has workgroups); the register path
    # with one three-window tile per workgroup
    (151936, 896, 64), (16384, 1536, 64), (20000, 2560, 64), (40000, 520, 40), (60000, 2560, 64),
    (20000, 4096, 64), (9728, 2560, 64), (4096, 2560, 64),
    # the set kernel (G = 64, K % 4 == 0, x 16-byte aligned, small grids): every
    # lane of a half-wave live (K = 1024), a partial last group (K = 964), rows
    # shorter than a group, one and two rows per half-wave
    (40, 1024, 64), (3000, 964, 64), (9, 36, 64), (16000, 512, 64),
]


@pytest.mark.parametrize("M,K,G", SHAPES)
def test_device_api_matches_oracle(gpu, orc, M, K, G):
    w = gpu.synth_i4(M, K, G, seed=M * 131 + K)
    x = gpu.synth_normal(K, seed=K + 7)
    want = orc.matvec_i4(w, x, M, K, G, threads=8)
    dw, dx = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x)
    dy = gpu.DeviceBuffer(4 * M)
    gpu.matvec_i4_dev(dw, dx, dy, M, K, G)
    got = dy.download(np.float32, M)
    assert_close(got, want, f"fast {M}x{K} G{G}")
    gpu.matvec_i4_generic_dev(dw, dx, dy, M, K, G)
    assert_close(dy.download(np.float32, M), want, f"generic {M}x{K} G{G}")


def test_activation_extremes_per_group(gpu, orc):
    # one huge and one tiny activation per group: the per-group exponent must keep precision
    M, K, G = 64, 2560, 64
    w = gpu.synth_i4(M, K, G, seed=99)
    x = gpu.synth_normal(K, seed=98)
    x[::64] *= 1e4
    x[1::64] *= 1e-6
    x[5 * 64:6 * 64] = 0.0
    want = orc.matvec_i4(w, x, M, K, G)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M)
    gpu.matvec_i4_dev(dw, dx, dy, M, K, G)
    assert_close(dy.download(np.float32, M), want, "extremes")


def test_headline_lm_head_shape_and_determinism(gpu, orc):
    M, K, G = 151936, 2560, 64
    w = gpu.synth_i4(M, K, G, seed=gpu.synth_seed(0, 0, "lm_head"))
    x = gpu.synth_normal(K, seed=gpu.synth_seed(0, 0, "x"))
    want = orc.matvec_i4(w, x, M, K, G, threads=16)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M)
    gpu.matvec_i4_dev(dw, dx, dy, M, K, G)
    y1 = dy.download(np.float32, M)
    assert_close(y1, want, "lm_head 151936x2560")
    gpu.matvec_i4_dev(dw, dx, dy, M, K, G)
    assert np.array_equal(dy.download(np.float32, M), y1)  # fixed reduction order


def test_bad_shapes_return_codes(gpu):
    lib = gpu.lib()
    assert lib.tqhip_matvec_i4_dev(None, None, None, 0, 64, 64, None) == gpu.EBADSHAPE
    assert lib.tqhip_matvec_i4_dev(None, None, None, 4, 0, 64, None) == gpu.EBADSHAPE
    assert lib.tqhip_matvec_i4_dev(None, None, None, 4, 64, 63, None) == gpu.EBADGROUP
    assert lib.tqhip_matvec_i4_dev(None, None, None, 4, 64, 0, None) == gpu.EBADGROUP
    assert lib.tqhip_matvec_vq2_dev(None, None, None, 4, 6, None) == gpu.EBADSHAPE
    assert lib.tqhip_matmul_i4_dev(None, None, None, 4, 64, 0, 64, None) == gpu.EBADSHAPE


def test_misaligned_activations_take_another_kernel(gpu, orc):
    """x 4 bytes past a 16-byte boundary: the set kernel needs 16-byte aligned
    activations, so this launch goes to the MFMA register path; same results as
    the oracle either way."""
    M, K, G = 896, 896, 64
    w = gpu.synth_i4(M, K, G, seed=77)
    x = gpu.synth_normal(K + 4, seed=78)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M)
    st = gpu.lib().tqhip_matvec_i4_dev(dw.ptr, dx.ptr + 4, dy.ptr, M, K, G, None)
    assert st == 0
    gpu.synchronize()
    assert_close(dy.download(np.float32, M), orc.matvec_i4(w, x[1:K + 1], M, K, G, threads=16), "misaligned x")


# qkv / pair on device buffers: one launch over all the matrices or one per
# matrix (group sizes the fused kernels do not cover). Each output must meet the
# bar against the oracle and equal the single-matrix launch: bit for bit where
# both launches run the same kernel ("exact" below: the kernel is chosen by row
# length and tile count, and a row's sum does not depend on where in the grid
# it is computed), else within 1e-6 of the output scale (the fused launch has
# more tiles than the single one and can take another kernel, which adds the
# same terms in another order: e.g. 19456 fused rows at K = 2560 run the MFMA
# kernels, a single 9728-row matrix the set kernel).
def same_as_single(got, single, exact):
    if exact:
        return np.array_equal(got, single)
    return float(np.max(np.abs(got - single))) <= 1e-6 * max(float(np.max(np.abs(single))), 1e-30)


@pytest.mark.parametrize("q,kv,K,G,exact", [(896, 128, 896, 64, True), (4096, 1024, 2560, 64, True),
                                            (100, 17, 520, 40, True), (64, 16, 4864, 64, True),
                                            (40, 8, 1000, 128, True), (24, 24, 200, 6, True)])
def test_qkv_dev_one_launch_matches_single_and_oracle(gpu, orc, q, kv, K, G, exact):
    ws = [gpu.synth_i4(m, K, G, seed=1000 + i) for i, m in enumerate((q, kv, kv))]
    x = gpu.synth_normal(K, seed=7)
    dws = [gpu.DeviceBuffer.from_array(w) for w in ws]
    dx = gpu.DeviceBuffer.from_array(x)
    dys = [gpu.DeviceBuffer(4 * m) for m in (q, kv, kv)]
    gpu.matvec_qkv_i4_dev(*dws, dx, *dys, q, kv, K, G)
    got = [d.download(np.float32, m) for d, m in zip(dys, (q, kv, kv))]
    for i, (w, m) in enumerate(zip(ws, (q, kv, kv))):
        single = gpu.DeviceBuffer(4 * m)
        gpu.matvec_i4_dev(dws[i], dx, single, m, K, G)
        assert same_as_single(got[i], single.download(np.float32, m), exact), f"qkv matrix {i} vs its own launch"
        assert_close(got[i], orc.matvec_i4(w, x, m, K, G, threads=16), f"qkv {i}")


@pytest.mark.parametrize("M,K,G,exact", [(4864, 896, 64, True), (9728, 2560, 64, False), (33, 130, 64, True),
                                         (300, 4864, 64, True)])
def test_pair_dev_one_launch_matches_single_and_oracle(gpu, orc, M, K, G, exact):
    w1, w2 = gpu.synth_i4(M, K, G, seed=21), gpu.synth_i4(M, K, G, seed=22)
    x = gpu.synth_normal(K, seed=23)
    d1, d2, dx = gpu.DeviceBuffer.from_array(w1), gpu.DeviceBuffer.from_array(w2), gpu.DeviceBuffer.from_array(x)
    y1, y2 = gpu.DeviceBuffer(4 * M), gpu.DeviceBuffer(4 * M)
    gpu.matvec_pair_i4_dev(d1, d2, dx, y1, y2, M, K, G)
    for w, dw, dy in ((w1, d1, y1), (w2, d2, y2)):
        single = gpu.DeviceBuffer(4 * M)
        gpu.matvec_i4_dev(dw, dx, single, M, K, G)
        got = dy.download(np.float32, M)
        assert same_as_single(got, single.download(np.float32, M), exact)
        assert_close(got, orc.matvec_i4(w, x, M, K, G, threads=16), "pair")


def test_run_ops_pair_and_qkv_kinds(gpu, orc):
    """The op-list runner's PAIR and QKV kinds give the same outputs as the entry points."""
    K, G, q, kv = 896, 64, 896, 128
    ws = [gpu.synth_i4(m, K, G, seed=50 + i) for i, m in enumerate((q, kv, kv, 4864, 4864))]
    x = gpu.synth_normal(K, seed=51)
    dws = [gpu.DeviceBuffer.from_array(w) for w in ws]
    dx = gpu.DeviceBuffer.from_array(x)
    dys = [gpu.DeviceBuffer(4 * m) for m in (q, kv, kv, 4864, 4864)]
    ops = [gpu.Op(gpu.OP_I4_QKV, dws[0].ptr, dx.ptr, dys[0].ptr, q, K, 1, G, dws[1].ptr, dws[2].ptr, dys[1].ptr,
                  dys[2].ptr, kv),
           gpu.Op(gpu.OP_I4_PAIR, dws[3].ptr, dx.ptr, dys[3].ptr, 4864, K, 1, G, dws[4].ptr, None, dys[4].ptr, None, 0)]
    gpu.run_ops(ops, 2)
    gpu.synchronize()
    for w, d, m in zip(ws, dys, (q, kv, kv, 4864, 4864)):
        assert_close(d.download(np.float32, m), orc.matvec_i4(w, x, m, K, G, threads=16), "run_ops")


# Split-K path (long rows, few tiles; rows a multiple of 16 bytes): several
# workgroups per 16-row tile, partial sums meeting in exchange slots that every
# launch leaves empty. At G = 64 the set kernel takes these shapes when x is
# 16-byte aligned, so each runs twice: aligned (set kernel) and with x 4 bytes
# off (1600x4864, 2560x4096, 2560x9728 and 1030x2688 then run split-K, the
# smaller ones the MFMA kernels); G = 128 runs split-K either way.
@pytest.mark.parametrize("M,K,G", [(896, 4864, 64), (1600, 4864, 64), (2560, 9728, 64), (2560, 4096, 64),
                                   (100, 4864, 64), (300, 8192, 128), (17, 1792, 64), (64, 3072, 128),
                                   (1030, 2688, 64)])
def test_split_k_matches_oracle_and_repeats(gpu, orc, M, K, G):
    w = gpu.synth_i4(M, K, G, seed=M * 7 + K)
    x = gpu.synth_normal(K + 4, seed=K)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M)
    for off in (0, 1):  # x at a 16-byte boundary, then 4 bytes past one
        xs = x[off:off + K]
        outs = []
        for _ in range(3):  # the tile counters must come back to zero after every launch
            assert gpu.lib().tqhip_matvec_i4_dev(dw.ptr, dx.ptr + 4 * off, dy.ptr, M, K, G, None) == 0
            gpu.synchronize()
            outs.append(dy.download(np.float32, M))
        assert all(np.array_equal(outs[0], o) for o in outs[1:]), "result changed between launches"
        assert_close(outs[0], orc.matvec_i4(w, np.ascontiguousarray(xs), M, K, G, threads=16),
                     f"{M}x{K} G{G} x offset {4 * off}")


def test_split_k_on_two_streams(gpu, orc):
    """Launches on different streams use different scratch buffers."""
    M, K, G = 1600, 4864, 128  # split-K (100 tiles), with its per-stream scratch
    ws = [gpu.synth_i4(M, K, G, seed=s) for s in (1, 2)]
    xs = [gpu.synth_normal(K, seed=s) for s in (3, 4)]
    dws = [gpu.DeviceBuffer.from_array(w) for w in ws]
    dxs = [gpu.DeviceBuffer.from_array(x) for x in xs]
    dys = [gpu.DeviceBuffer(4 * M) for _ in range(2)]
    streams = [gpu.Stream(), gpu.Stream()]
    for _ in range(20):
        for i in range(2):
            gpu.matvec_i4_dev(dws[i], dxs[i], dys[i], M, K, G, stream=streams[i])
    for st in streams:
        st.synchronize()
    for i in range(2):
        assert_close(dys[i].download(np.float32, M), orc.matvec_i4(ws[i], xs[i], M, K, G, threads=16), f"stream {i}")
