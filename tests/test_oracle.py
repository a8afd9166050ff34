"""Pins the CPU oracle (oracle/oracle.cpp) before anything is checked against it.

Each check is chosen so that a plausible slip in the restatement fails it:
  * golden fixtures written by the compiled reference (bit-exact outputs);
  * the reference tests' known answers (y=28, y=20, dequant rows);
  * an independent numpy decode of the layout followed by a float64 GEMV
    (catches swapped nibbles, swapped scale/zero, a wrong sign of zero);
  * brute force over every code with special fp16 scales/zeros;
  * invariants: row permutation, column decomposition of matmul, VQ2
    pair/qkv/matmul decomposition, zero rows, group additivity;
  * the compiled reference itself on random inputs, where it was built.
"""
import numpy as np
import pytest

from conftest import golden, golden_names


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- golden fixtures (compiled reference)

@pytest.mark.parametrize("name", golden_names("i4_") )
def test_matvec_i4_matches_reference_fixture(orc, name):
    f = golden(name)
    if "wq" in f:
        q_dim, kv_dim, K, G = (int(v) for v in f["dims"])
        assert np.array_equal(bits(orc.matvec_i4(f["wq"], f["x"], q_dim, K, G)), bits(f["yq"]))
        assert np.array_equal(bits(orc.matvec_i4(f["wk"], f["x"], kv_dim, K, G)), bits(f["yk"]))
        assert np.array_equal(bits(orc.matvec_i4(f["wv"], f["x"], kv_dim, K, G)), bits(f["yv"]))
        return
    if "w1" in f:
        M, K, G = (int(v) for v in f["dims"])
        assert np.array_equal(bits(orc.matvec_i4(f["w1"], f["x"], M, K, G)), bits(f["y1"]))
        assert np.array_equal(bits(orc.matvec_i4(f["w2"], f["x"], M, K, G)), bits(f["y2"]))
        return
    M, K, G = (int(v) for v in f["dims"])
    assert np.array_equal(bits(orc.matvec_i4(f["w"], f["x"], M, K, G)), bits(f["y"]))


@pytest.mark.parametrize("name", golden_names("mm_i4_"))
def test_matmul_i4_matches_reference_fixture(orc, name):
    f = golden(name)
    M, K, N, G = (int(v) for v in f["dims"])
    assert np.array_equal(bits(orc.matmul_i4(f["w"], f["x"], M, K, N, G)), bits(f["y"]))
    assert np.array_equal(bits(orc.matmul_i4(f["w"], f["x"], M, K, N, G, threads=3)), bits(f["y"]))


@pytest.mark.parametrize("name", golden_names("vq2_"))
def test_matvec_vq2_matches_reference_fixture(orc, name):
    f = golden(name)
    M, K = (int(v) for v in f["dims"])
    assert np.array_equal(bits(orc.matvec_vq2(f["w"], f["x"], M, K)), bits(f["y"]))


def test_matmul_vq2_fixture_is_columnwise_matvec(orc):
    f = golden("mm_vq2_48x192x5")
    M, K, N = (int(v) for v in f["dims"])
    cols = [orc.matvec_vq2(f["w"], f["x"][n * K:(n + 1) * K], M, K) for n in range(N)]
    assert np.array_equal(bits(np.concatenate(cols)), bits(f["y"]))


def test_half_to_float_all_patterns(orc):
    f = golden("fp16_conversions")
    got = orc.halves_to_floats(f["half_bits"])
    assert np.array_equal(bits(got), bits(f["half_to_float"]))
    # and against numpy's IEEE conversion, NaN payloads aside
    npv = f["half_bits"].view(np.float16).astype(np.float32)
    finite = ~np.isnan(npv)
    assert np.array_equal(bits(got[finite]), bits(npv[finite]))
    assert np.all(np.isnan(got[~finite]))


def test_float_to_half_matches_reference_and_numpy(orc):
    f = golden("fp16_conversions")
    got = orc.floats_to_halves(f["floats"])
    assert np.array_equal(got, f["float_to_half"])
    # numpy rounds to nearest even; the reference flushes |f| < 2^-24 to zero (ref_ops.h:94)
    x = f["floats"]
    npv = x.astype(np.float16).view(np.uint16)
    keep = ~np.isnan(x) & ((np.abs(x) >= 2.0 ** -24) | (x == 0))
    assert np.array_equal(got[keep], npv[keep])
    tiny = (np.abs(x) < 2.0 ** -24) & (x != 0)
    assert np.all((got[tiny] & 0x7FFF) == 0)


def test_dequant_i4_row_known_answers(orc):
    f = golden("dequant_i4_row")
    out = orc.dequant_i4_row(f["kat_embed"], 0, 8, 4)
    assert np.array_equal(out, np.array([-4, 0, 3.5, -2.5, 0, 0, 0, 0], np.float32))  # test_quant_ops.cpp:87
    assert np.array_equal(out, f["kat_out"])
    rows, dim, G = (int(v) for v in f["dims"])
    for r in range(rows):
        assert np.array_equal(bits(orc.dequant_i4_row(f["table"], r, dim, G)), bits(f["table_rows"][r]))


def test_dequant_i4_row_partial_tail_of_fives(orc):
    # tests/test_quant_ops.cpp:94-112: dim 6, gs 4, scale 1, zero 0, every code 5.
    row = np.zeros(12, dtype=np.uint8)
    for g in range(2):
        row[6 * g:6 * g + 2] = np.array([1.0], np.float16).view(np.uint8)
        row[6 * g + 2:6 * g + 4] = np.array([0.0], np.float16).view(np.uint8)
        row[6 * g + 4] = row[6 * g + 5] = (5 << 4) | 5
    assert np.array_equal(orc.dequant_i4_row(row, 0, 6, 4), np.full(6, 5.0, np.float32))


# ---------------------------------------------------------------- known answers, closed forms, invariants

def test_known_answer_i4_y28(orc):
    f = golden("i4_kat_1x4_g4")
    assert orc.matvec_i4(f["w"], f["x"], 1, 4, 4)[0] == 28.0


def test_known_answer_vq2_y20(orc):
    f = golden("vq2_kat_1x4")
    assert orc.matvec_vq2(f["w"], f["x"], 1, 4)[0] == 20.0


@pytest.mark.parametrize("M,K,G", [(64, 256, 64), (32, 200, 64), (17, 520, 40), (5, 100, 32), (3, 70, 6), (9, 1000, 256)])
def test_matvec_i4_equals_numpy_float64_gemv(tqa, orc, M, K, G):
    w = tqa.synth_i4(M, K, G, seed=1000 + M)
    x = tqa.synth_normal(K, seed=2000 + K)
    deq = orc.dequant_i4_matrix_f64(w, M, K, G)
    want = (deq @ x.astype(np.float64)).astype(np.float32)
    got = orc.matvec_i4(w, x, M, K, G)
    # same products, different double summation order: equal to within one float ulp
    assert np.all(np.abs(got - want) <= np.spacing(np.abs(want)) + 1e-30)


@pytest.mark.parametrize("M,K", [(32, 128), (33, 200), (100, 52)])
def test_matvec_vq2_equals_numpy_float64_gemv(tqa, orc, M, K):
    w = tqa.synth_vq2(M, K, seed=77 + M, cb_std=1.0)
    x = tqa.synth_normal(K, seed=78)
    cb = w[:2048].view(np.float16).astype(np.float64).reshape(256, 4)
    idx = w[2048:].reshape(M, K // 4)
    dense = cb[idx].reshape(M, K)
    want = (dense @ x.astype(np.float64)).astype(np.float32)
    got = orc.matvec_vq2(w, x, M, K)
    assert np.all(np.abs(got - want) <= np.spacing(np.abs(want)) + 1e-30)


def test_brute_force_every_code_with_special_scales(orc):
    specials = np.array([0.0, -0.0, 5.96e-8, 6.1e-5, 0.002, 0.02, 1.0, -2.5, 65504.0], dtype=np.float16)
    zeros = np.array([0.0, 15.0, 7.25, -1.0, 0.5], dtype=np.float16)
    G = 16
    for s in specials:
        for z in zeros:
            w = np.zeros(4 + G // 2, dtype=np.uint8)
            w[0:2] = np.array([s]).view(np.uint8)
            w[2:4] = np.array([z]).view(np.uint8)
            codes = np.arange(16, dtype=np.uint8)
            w[4:] = codes[0::2] | (codes[1::2] << 4)
            for k in range(G):
                x = np.zeros(G, dtype=np.float32)
                x[k] = 1.0
                y = orc.matvec_i4(w, x, 1, G, G)[0]
                want = (np.float32(k) - np.float32(z)) * np.float32(s)
                assert np.float32(y) == np.float32(want) or (np.isnan(y) and np.isnan(want)), (s, z, k)


def test_zero_point_equal_to_code_gives_zero(orc):
    G, K = 64, 192
    groups = K // G
    w = np.zeros(groups * (4 + G // 2), dtype=np.uint8).reshape(groups, -1)
    w[:, 0:2] = np.array([0.0137], np.float16).view(np.uint8)
    w[:, 2:4] = np.array([9.0], np.float16).view(np.uint8)
    w[:, 4:] = 9 | (9 << 4)
    x = np.random.default_rng(0).standard_normal(K).astype(np.float32)
    assert orc.matvec_i4(w.reshape(-1), x, 1, K, G)[0] == 0.0


def test_row_permutation_commutes(tqa, orc):
    M, K, G = 40, 320, 64
    w = tqa.synth_i4(M, K, G, seed=5)
    x = tqa.synth_normal(K, seed=6)
    rb = orc.i4_row_bytes(K, G)
    perm = np.random.default_rng(1).permutation(M)
    wp = w.reshape(M, rb)[perm].reshape(-1).copy()
    assert np.array_equal(orc.matvec_i4(wp, x, M, K, G), orc.matvec_i4(w, x, M, K, G)[perm])


def test_group_split_is_additive(tqa, orc):
    M, K, G = 24, 512, 64
    w = tqa.synth_i4(M, K, G, seed=8)
    x = tqa.synth_normal(K, seed=9)
    gb = 4 + G // 2
    a = 3  # groups in the first half
    w2 = w.reshape(M, K // G, gb)
    y1 = orc.matvec_i4(w2[:, :a].reshape(-1).copy(), x[:a * G].copy(), M, a * G, G).astype(np.float64)
    y2 = orc.matvec_i4(w2[:, a:].reshape(-1).copy(), x[a * G:].copy(), M, K - a * G, G).astype(np.float64)
    y = orc.matvec_i4(w, x, M, K, G).astype(np.float64)
    assert np.allclose(y1 + y2, y, rtol=1e-6, atol=1e-6)


def test_matmul_columns_are_matvecs(tqa, orc):
    M, K, N, G = 48, 128, 3, 64  # tests/test_matvec_i4.cpp:514-536
    w = tqa.synth_i4(M, K, G, seed=11)
    x = tqa.synth_normal(K * N, seed=12)
    y = orc.matmul_i4(w, x, M, K, N, G)
    for n in range(N):
        assert np.array_equal(y[n * M:(n + 1) * M], orc.matvec_i4(w, x[n * K:(n + 1) * K].copy(), M, K, G))


def test_multithreaded_oracle_is_bit_identical(tqa, orc):
    M, K, G = 513, 896, 64
    w = tqa.synth_i4(M, K, G, seed=13)
    x = tqa.synth_normal(K, seed=14)
    assert np.array_equal(orc.matvec_i4(w, x, M, K, G, threads=7), orc.matvec_i4(w, x, M, K, G))
    v = tqa.synth_vq2(M, K, seed=15)
    assert np.array_equal(orc.matvec_vq2(v, x, M, K, threads=5), orc.matvec_vq2(v, x, M, K))


def test_byte_accounting_known_values(orc):
    # tests/test_quantization.cpp:66-78 and runtime/tiny_format.h:73-78, 100-103
    assert orc.quantized_size(0, 128, 256, 0) == 131072
    assert orc.quantized_size(1, 128, 256, 0) == 65536
    assert orc.quantized_size(3, 128, 256, 64) == 18432
    assert orc.quantized_size(4, 3072, 1024, 0) == 788480
    assert orc.i4_row_bytes(896, 64) == 504
    assert orc.i4_row_bytes(2560, 64) == 1440
    assert orc.i4_row_bytes(4864, 64) == 2736
    assert orc.i4_row_bytes(9728, 64) == 5472
    assert orc.i4_row_bytes(200, 64) == 144
    assert orc.vq2_tensor_bytes(3072, 1024) == 788480
    assert 151936 * orc.i4_row_bytes(2560, 64) == 218787840


# ---------------------------------------------------------------- the compiled reference itself

@pytest.mark.parametrize("seed", [0, 1, 2])
def test_oracle_equals_compiled_reference_on_random_inputs(tqa, orc, seed):
    r = orc.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref not built here (it needs the reference tree)")
    rng = np.random.default_rng(seed)
    for M, K, G in [(37, 448, 64), (11, 390, 128), (5, 96, 32), (8, 1000, 40)]:
        w = tqa.synth_i4(M, K, G, seed=int(rng.integers(1 << 30)), zero=(-2.0, 17.0))
        x = (rng.standard_normal(K) * 10.0).astype(np.float32)
        y_ref = np.empty(M, np.float32)
        r.tqref_matvec_i4(w.ctypes.data, x.ctypes.data, y_ref.ctypes.data, M, K, G)
        assert np.array_equal(bits(orc.matvec_i4(w, x, M, K, G)), bits(y_ref))
    for M, K in [(41, 256), (7, 12)]:
        v = tqa.synth_vq2(M, K, seed=int(rng.integers(1 << 30)), cb_std=1.0)
        x = rng.standard_normal(K).astype(np.float32)
        y_ref = np.empty(M, np.float32)
        r.tqref_matvec_vq2(v.ctypes.data, x.ctypes.data, y_ref.ctypes.data, M, K)
        assert np.array_equal(bits(orc.matvec_vq2(v, x, M, K)), bits(y_ref))
    assert r.tqref_unknown_i4_name_rejected() == 1


# ---------------------------------------------------------------- BiIP activation rotation

BIIP_CASES = [(896, 128, True), (896, 128, False), (4864, 256, True), (256, 64, True), (128, 128, True),
              (256, 4, True), (256, 2, True), (1024, 256, False), (3072, 256, True), (7, 1, True)]


def biip_inputs(dim, with_scale, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(dim) * 3.0).astype(np.float32)
    scale = rng.uniform(0.25, 4.0, dim).astype(np.float32) if with_scale else None
    sign = np.where(rng.random(dim) < 0.5, -1.0, 1.0).astype(np.float32)
    return x, scale, sign


def sylvester(n):
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


@pytest.mark.parametrize("dim,bs,with_scale", BIIP_CASES)
def test_biip_rotate_equals_compiled_reference(orc, dim, bs, with_scale):
    r = orc.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref not built here (it needs the reference tree)")
    x, scale, sign = biip_inputs(dim, with_scale, dim + bs)
    want = np.empty(dim, np.float32)
    r.tqref_biip_rotate(x.ctypes.data, want.ctypes.data, dim, None if scale is None else scale.ctypes.data,
                        sign.ctypes.data, bs)
    assert np.array_equal(bits(orc.biip_rotate(x, scale, sign, bs)), bits(want))


@pytest.mark.parametrize("dim,bs,with_scale", BIIP_CASES)
def test_biip_rotate_equals_dense_hadamard(orc, dim, bs, with_scale):
    """blockHadamard((x / scale) * sign) with the Sylvester matrix H / sqrt(bs) in float64
    (the mathematics the butterfly computes; tests/test_biip_rotate.cpp:40-62 checks the
    same against a naive Hadamard)."""
    x, scale, sign = biip_inputs(dim, with_scale, 3 * dim + bs)
    v = x.astype(np.float64) * sign
    if scale is not None:
        v = x.astype(np.float64) / scale * sign
    H = sylvester(bs) / np.sqrt(bs)
    want = (v.reshape(-1, bs) @ H.T).reshape(-1)
    got = orc.biip_rotate(x, scale, sign, bs).astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-5 * max(np.max(np.abs(want)), 1.0)


def test_biip_rotate_is_orthogonal_and_in_place_safe(orc):
    x, _, sign = biip_inputs(2048, False, 5)
    y = orc.biip_rotate(x, None, sign, 256)
    assert abs(np.linalg.norm(y.astype(np.float64)) / np.linalg.norm(x.astype(np.float64)) - 1.0) < 1e-6
    z = x.copy()
    orc.lib().orc_biip_rotate(z.ctypes.data, z.ctypes.data, z.size, None, sign.ctypes.data, 256)
    assert np.array_equal(bits(z), bits(y))
