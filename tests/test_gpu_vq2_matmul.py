"""VQ2 matvec and i4 matmul on the GPU against the oracle and the golden outputs.

VQ2 tolerance: rel L2 <= 1e-5 and max|err| <= 1e-3 * max|y_ref| (north star matvec bar).
matmul_i4 tolerance: rel L2 <= 2e-3 and max|err| <= 1e-3 * max|y_ref| (north star prefill bar).
"""
import numpy as np
import pytest

from conftest import fp16_operand_bound_ok, golden, golden_names, max_abs_rel, rel_l2

pytestmark = pytest.mark.gpu


def assert_close(got, want, l2_tol, what=""):
    l2, mx = rel_l2(got, want), max_abs_rel(got, want)
    assert l2 <= l2_tol and mx <= 1e-3, f"{what}: rel_l2={l2:.3e} max_rel={mx:.3e}"


@pytest.mark.parametrize("name", golden_names("vq2_"))
def test_vq2_golden_through_registry(gpu, name):
    f = golden(name)
    M, K = (int(v) for v in f["dims"])
    assert gpu.set_matvec_vq2_impl_by_name("hip")
    got = gpu.matvec_vq2(f["w"], f["x"], M, K)
    assert_close(got, f["y"], 1e-5, name)
    if name == "vq2_kat_1x4":
        assert abs(got[0] - 20.0) < 1e-5  # tests/test_matvec_vq2.cpp:163


def test_matmul_vq2_golden_decomposes(gpu):
    f = golden("mm_vq2_48x192x5")
    M, K, N = (int(v) for v in f["dims"])
    assert_close(gpu.matmul_vq2(f["w"], f["x"], M, K, N), f["y"], 1e-5, "matmul_vq2")


# aligned index rows (in_dim % 16 == 0): one wave per row up to 4M lookups, then the
# conflict-free replica kernel with one chunk per row, several, a partial last chunk and many
# tiles per wave (151936x896: the table kernel); the rest: the byte-load kernel
@pytest.mark.parametrize("M,K", [(3072, 1024), (1, 4), (513, 896), (4864, 896), (100, 52), (77, 1000), (16384, 2048),
                                 (2001, 3056), (151936, 896), (3, 16)])
def test_vq2_device_api_matches_oracle(gpu, orc, M, K):
    w = gpu.synth_vq2(M, K, seed=M + K)
    x = gpu.synth_normal(K, seed=K)
    want = orc.matvec_vq2(w, x, M, K, threads=8)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M)
    gpu.matvec_vq2_dev(dw, dx, dy, M, K)
    assert_close(dy.download(np.float32, M), want, 1e-5, f"vq2 {M}x{K}")


# at least 256 rows per CU, in_dim % 64 == 0 and <= 1024: the dot-product table kernel.
# Rows per workgroup not a multiple of a wave's 16-row batch (65869 rows: 258 per workgroup,
# two batches on some waves), four batches on some waves (200000 rows: 782 per workgroup),
# more workgroups than CUs (300001 rows: 293 workgroups of up to 1024 rows), a full 64-dword
# row (1024), rows of 40 dwords (640), 16 (256) and one dword (64).
@pytest.mark.parametrize("M,K", [(65869, 896), (131072, 1024), (200000, 640), (70001, 64), (300001, 256)])
def test_vq2_table_kernel_matches_oracle(gpu, orc, M, K):
    w = gpu.synth_vq2(M, K, seed=M + 7 * K)
    x = gpu.synth_normal(K, seed=K + 5)
    want = orc.matvec_vq2(w, x, M, K, threads=8)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M)
    gpu.lib().tqhip_memset(dy.ptr, 0xFF, 4 * M)  # every row must be written
    gpu.matvec_vq2_dev(dw, dx, dy, M, K)
    assert_close(dy.download(np.float32, M), want, 1e-5, f"vq2 {M}x{K}")


@pytest.mark.parametrize("M,K", [(3072, 1024), (32768, 896), (151936, 896), (2001, 3052)])
def test_vq2_non_finite_codebook_entry(gpu, orc, M, K):
    """Codebook entry 0 set to +inf: a row is non-finite exactly where the oracle's is (the rows
    that use entry 0), so positions past the row end (padding lanes, table columns) contribute
    exactly 0 whatever the entries hold. One shape per kernel, each with a padded last chunk:
    one wave per row, replica (224-byte rows), table, byte loads (in_dim % 16 != 0)."""
    w = gpu.synth_vq2(M, K, seed=M + 11 * K)
    w[0:8] = np.frombuffer(np.full(4, np.inf, np.float16).tobytes(), np.uint8)
    x = gpu.synth_normal(K, seed=K + 9)
    want = orc.matvec_vq2(w, x, M, K, threads=8)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M)
    gpu.matvec_vq2_dev(dw, dx, dy, M, K)
    got = dy.download(np.float32, M)
    fin = np.isfinite(want)
    assert 0 < np.count_nonzero(~fin) < M, "the case needs rows with and without entry 0"
    assert np.array_equal(np.isfinite(got), fin), f"{np.count_nonzero(np.isfinite(got) != fin)} rows differ in finiteness"
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert_close(got[fin], want[fin], 1e-5, f"vq2 {M}x{K} finite rows")


@pytest.mark.parametrize("M,K", [(896, 896), (4864, 896), (16384, 2048), (65869, 896)])
def test_vq2_activations_at_any_float_offset(gpu, orc, M, K):
    """x 4 bytes past a 16-byte boundary: the one-wave-per-row kernel (up to 4M lookups) then
    loads the activations one float at a time; the replica kernel never needs the alignment."""
    w = gpu.synth_vq2(M, K, seed=M + 3 * K)
    x = gpu.synth_normal(K, seed=K + 1)
    xb = np.zeros(K + 4, np.float32)
    xb[1:K + 1] = x
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(xb), gpu.DeviceBuffer(4 * M)
    assert gpu.lib().tqhip_matvec_vq2_dev(dw.ptr, dx.ptr + 4, dy.ptr, M, K, None) == 0
    gpu.synchronize()
    assert_close(dy.download(np.float32, M), orc.matvec_vq2(w, x, M, K, threads=8), 1e-5, f"vq2 {M}x{K} x+4")


@pytest.mark.parametrize("name", golden_names("mm_i4_"))
def test_matmul_i4_golden_through_registry(gpu, name):
    f = golden(name)
    M, K, N, G = (int(v) for v in f["dims"])
    assert gpu.set_matmul_i4_impl_by_name("hip")
    assert_close(gpu.matmul_i4(f["w"], f["x"], M, K, N, G), f["y"], 2e-3, name)


# Tile configurations: N <= 32, N <= 64 and larger; ragged M/N/K; group sizes
# 32, 96, 128 (MFMA path) and 40 (not a multiple of 32: per-column matvec path).
@pytest.mark.parametrize("M,K,N,G", [(9728, 2560, 32, 64), (300, 896, 7, 64), (1000, 640, 48, 128),
                                     (520, 2560, 130, 64), (129, 100, 65, 32), (200, 384, 70, 96),
                                     (64, 200, 40, 40), (1, 64, 1, 64), (33, 1000, 129, 64)])
def test_matmul_i4_device_api_matches_oracle(gpu, orc, M, K, N, G):
    w = gpu.synth_i4(M, K, G, seed=M + N)
    x = gpu.synth_normal(K * N, seed=N)
    want = orc.matmul_i4(w, x, M, K, N, G, threads=16)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M * N)
    gpu.matmul_i4_dev(dw, dx, dy, M, K, N, G)
    got = dy.download(np.float32, M * N)
    if M * N < 16:  # one near-cancelled output decides the relative measures
        assert fp16_operand_bound_ok(got, want, orc, w, x, M, K, N, G), f"matmul {M}x{K}x{N}"
    else:
        assert_close(got, want, 2e-3, f"matmul {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(512, 2560, 64), (300, 1000, 40)])
def test_matmul_i4_x_conversion_paths_same_bits(gpu, orc, M, K, N):
    """X 16-byte aligned (16-byte loads and stores in the fp16 conversion) and X 4 bytes past an
    alignment (one float per load): the same fp16 X, so the same output bits (above 32 tokens
    both go through the MFMA GEMM)."""
    w = gpu.synth_i4(M, K, 64, seed=M + K + N)
    x = gpu.synth_normal(K * N, seed=N + 3)
    x[5 * K:6 * K] *= 1e-20  # a token far below the others: its own exponent
    dw, dy_a, dy_u = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer(4 * M * N), gpu.DeviceBuffer(4 * M * N)
    xb = np.zeros(K * N + 8, np.float32)
    xb[4:4 + K * N] = x  # 16-byte aligned copy at float 4
    xb_u = np.zeros(K * N + 8, np.float32)
    xb_u[1:1 + K * N] = x  # misaligned copy at float 1
    da, du = gpu.DeviceBuffer.from_array(xb), gpu.DeviceBuffer.from_array(xb_u)
    lib = gpu.lib()
    assert lib.tqhip_matmul_i4_dev(dw.ptr, da.ptr + 16, dy_a.ptr, M, K, N, 64, None) == 0
    assert lib.tqhip_matmul_i4_dev(dw.ptr, du.ptr + 4, dy_u.ptr, M, K, N, 64, None) == 0
    gpu.synchronize()
    ya, yu = dy_a.download(np.float32, M * N), dy_u.download(np.float32, M * N)
    assert np.array_equal(ya.view(np.uint32), yu.view(np.uint32))
    assert_close(ya, orc.matmul_i4(w, x, M, K, N, 64, threads=16), 2e-3, f"matmul {M}x{K}x{N}")


def test_matmul_i4_per_token_scale_extremes(gpu, orc):
    """Token columns of very different magnitude (1e30, 1e-30, 0, N(0,1)) each
    keep the bar on their own: the fp16 staging scales every column by its own
    power of two."""
    M, K, N, G = 256, 640, 40, 64
    w = gpu.synth_i4(M, K, G, seed=5)
    x = gpu.synth_normal(K * N, seed=6).reshape(N, K).copy()
    x[1] *= 1e30
    x[2] *= 1e-30
    x[3] = 0.0
    x[4, ::7] = 0.0
    x = x.reshape(-1)
    want = orc.matmul_i4(w, x, M, K, N, G, threads=16).reshape(N, M)
    got = gpu.matmul_i4(w, x, M, K, N, G).reshape(N, M)
    assert np.all(got[3] == 0.0)
    for n in range(N):
        if n == 3:
            continue
        assert_close(got[n], want[n], 2e-3, f"column {n}")


def test_matmul_i4_prefill_shape_every_output(gpu, orc):
    """The prefill configuration (9728 weight rows, K 2560, 512 tokens) in
    one launch, every one of its 5.0M outputs against the oracle (a few seconds on 16 threads)."""
    M, K, N, G = 9728, 2560, 512, 64
    w = gpu.synth_i4(M, K, G, seed=11)
    x = gpu.synth_normal(K * N, seed=12)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M * N)
    gpu.matmul_i4_dev(dw, dx, dy, M, K, N, G)
    want = orc.matmul_i4(w, x, M, K, N, G, threads=16)
    assert_close(dy.download(np.float32, M * N), want, 2e-3, "9728x2560x512")


def test_matmul_i4_prefill_rows_full_shape_128_tokens(gpu, orc):
    """The prefill weight shape with 128 tokens, every output against the oracle."""
    M, K, N, G = 9728, 2560, 128, 64
    w = gpu.synth_i4(M, K, G, seed=13)
    x = gpu.synth_normal(K * N, seed=14)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M * N)
    gpu.matmul_i4_dev(dw, dx, dy, M, K, N, G)
    want = orc.matmul_i4(w, x, M, K, N, G, threads=16)
    assert_close(dy.download(np.float32, M * N), want, 2e-3, "9728x2560x128")


# tqhip_matvec_vq2_set_dev: a VQ2 layer's projections with their own activations in one launch of
# the one-wave-per-row kernel. Every output within the matvec bar of the oracle and bit-identical
# to tqhip_matvec_vq2_dev on the same matrix. Cases: the Qwen2.5-0.5B layer (q/k/v sharing x,
# gate/up sharing x, o and down with their own), more than eight matrices (two launches), a launch
# closed at 8M lookups, matrices that run alone (in_dim % 16 != 0, above 4M lookups), x at a
# 4-byte offset (the scalar activation loads for the whole launch), and the error codes.
def _vq2_set_case(gpu, orc, spec, seed, x_offset=0):
    xs, mats = {}, []
    for i, (M, K, key) in enumerate(spec):
        if key not in xs:
            x = gpu.synth_normal(K, seed=seed + 100 + len(xs))
            xb = np.zeros(K + 4, np.float32)
            xb[x_offset // 4:x_offset // 4 + K] = x
            xs[key] = (x, gpu.DeviceBuffer.from_array(xb))
        w = gpu.synth_vq2(M, K, seed=seed + i)
        mats.append((M, K, w, xs[key], gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer(4 * M)))
    arr = gpu.i4_set([(dw, x[1].ptr + x_offset, dy, M, K) for M, K, _, x, dw, dy in mats])
    for M, _, _, _, _, dy in mats:
        gpu.lib().tqhip_memset(dy.ptr, 0xFF, 4 * M)  # every output must be written by the set
    gpu.matvec_vq2_set_dev(arr)
    gpu.synchronize()
    for i, (M, K, w, x, dw, dy) in enumerate(mats):
        got = dy.download(np.float32, M)
        assert_close(got, orc.matvec_vq2(w, x[0], M, K, threads=8), 1e-5, f"set matrix {i} {M}x{K}")
        alone = gpu.DeviceBuffer(4 * M)
        assert gpu.lib().tqhip_matvec_vq2_dev(dw.ptr, x[1].ptr + x_offset, alone.ptr, M, K, None) == 0
        gpu.synchronize()
        assert np.array_equal(got.view(np.uint32), alone.download(np.float32, M).view(np.uint32)), \
            f"set matrix {i} {M}x{K}: differs from the single launch"


def test_vq2_set_qwen25_layer(gpu, orc):
    _vq2_set_case(gpu, orc, [(896, 896, "a"), (128, 896, "a"), (128, 896, "a"), (896, 896, "o"),
                             (4864, 896, "m"), (4864, 896, "m"), (896, 4864, "d")], seed=3)


def test_vq2_set_many_mixed_and_offset(gpu, orc):
    spec = [(300 + 37 * i, 64 * (1 + i % 5), "k%d" % (i % 5)) for i in range(10)]  # ten: two launches
    spec += [(2001, 3052, "odd"),        # in_dim % 16 != 0: alone (byte kernel)
             (20000, 1024, "big"),       # 5.1M lookups: alone (replica kernel)
             (16384, 1024, "c1"), (16384, 1024, "c1")]  # 4M lookups each: the second opens a new launch
    _vq2_set_case(gpu, orc, spec, seed=11)
    _vq2_set_case(gpu, orc, [(896, 896, "a"), (128, 896, "a"), (4864, 896, "m")], seed=5, x_offset=4)


def test_vq2_set_errors(gpu):
    lib = gpu.lib()
    w, x, y = gpu.DeviceBuffer(4096), gpu.DeviceBuffer(4096), gpu.DeviceBuffer(4096)
    assert lib.tqhip_matvec_vq2_set_dev(None, 1, None) == gpu.EBADSHAPE
    assert lib.tqhip_matvec_vq2_set_dev(None, 0, None) == gpu.OK  # an empty set launches nothing
    arr = gpu.i4_set([(w, x, y, 4, 6)])  # in_dim not a multiple of 4
    assert lib.tqhip_matvec_vq2_set_dev(gpu.ctypes.addressof(arr), 1, None) == gpu.EBADSHAPE
    arr = gpu.i4_set([(w, x, y, 0, 64)])
    assert lib.tqhip_matvec_vq2_set_dev(gpu.ctypes.addressof(arr), 1, None) == gpu.EBADSHAPE


def test_vq2_set_op_in_a_captured_graph(gpu, orc):
    """TQHIP_OP_VQ2_SET in an op list: eager run and graph replays agree bit for bit with new
    activations written before each replay, and with the single-matrix launches."""
    spec = [(896, 896, "a"), (128, 896, "a"), (128, 896, "a"), (4864, 896, "m"), (4864, 896, "m")]
    xs, mats = {}, []
    for i, (M, K, key) in enumerate(spec):
        if key not in xs:
            xs[key] = (np.zeros(K, np.float32), gpu.DeviceBuffer(4 * K), K)
        w = gpu.synth_vq2(M, K, seed=200 + i)
        mats.append((M, K, w, xs[key], gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer(4 * M)))
    arr = gpu.i4_set([(dw, x[1], dy, M, K) for M, K, _, x, dw, dy in mats])
    ops = [gpu.vq2_set_op(arr)]
    stream = gpu.Stream()
    graph = gpu.OpsGraph(ops, stream)
    try:
        for rep in range(3):
            for i, (xv, xd, K) in enumerate(xs.values()):
                xv[:] = gpu.synth_normal(K, seed=210 + 10 * rep + i)
                xd.upload(xv)
            gpu.run_ops(ops, 1, stream)
            stream.synchronize()
            want = [dy.download(np.float32, M) for M, _, _, _, _, dy in mats]
            for M, _, _, _, _, dy in mats:
                gpu.lib().tqhip_memset(dy.ptr, 0xFF, 4 * M)
            graph.launch()
            stream.synchronize()
            for i, ((M, K, w, x, dw, dy), wv) in enumerate(zip(mats, want)):
                assert np.array_equal(dy.download(np.float32, M).view(np.uint32), wv.view(np.uint32)), (rep, i)
                alone = gpu.DeviceBuffer(4 * M)
                assert gpu.lib().tqhip_matvec_vq2_dev(dw.ptr, x[1].ptr, alone.ptr, M, K, None) == 0
                gpu.synchronize()
                assert np.array_equal(alone.download(np.float32, M).view(np.uint32), wv.view(np.uint32)), (rep, i)
        for (M, K, w, x, _, _), wv in zip(mats, want):
            assert_close(wv, orc.matvec_vq2(w, x[0], M, K, threads=8), 1e-5, f"{M}x{K}")
    finally:
        graph.close()
