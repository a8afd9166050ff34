"""Wide-range activations and special fp16 group headers on every i4 matvec kernel family.

The exact-integer kernels scale each group of 64 activations by its own power of two; the
checks here put that scaling under stress -- one activation per group 1e4 times larger and one
1e6 times smaller than the rest, and a group of zeros -- and feed headers with subnormal,
negative and zero scales and out-of-range zeros (finite values; the reference decodes them with
half_to_float, kernels/ref_ops.h:51-74). Each shape is chosen for the kernel it runs
(launch_i4_matvec's routing; x is offset by 4 bytes where a case must avoid the set kernel,
which needs 16-byte aligned activations):

    set kernel     4864x896, 896x4864, 2560x9728       (x aligned; rows of 1, 3 and 5 slots)
    DMA ring       151936x2560                          (i4_matvec_dma)
    register path  151936x896                           (i4_matvec_pipe)
    wave ring      9728x2560, x + 4 bytes               (i4_matvec_seg)
    split-K        2560x9728, x + 4 bytes               (i4_matvec_split)
    reg kernel     8192x6144, x + 4 bytes               (i4_matvec_reg: rows of 54 windows)

Bar (north star): rel L2 <= 1e-5 and max|err| <= 1e-3 of max|y| against the oracle.
"""
import numpy as np
import pytest

from conftest import extreme_x, max_abs_rel, rel_l2, special_headers

pytestmark = pytest.mark.gpu

G = 64
CASES = [("set, 1 row per half-wave", 4864, 896, 0), ("set, 3 slots", 896, 4864, 0), ("set, 5 slots", 2560, 9728, 0),
         ("dma ring", 151936, 2560, 0), ("register path", 151936, 896, 0), ("wave ring", 9728, 2560, 1),
         ("split-K", 2560, 9728, 1), ("reg kernel", 8192, 6144, 1)]


def run(gpu, w, x, M, K, off):
    xb = np.zeros(K + 4, np.float32)
    xb[off:off + K] = x
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(xb), gpu.DeviceBuffer(4 * M)
    assert gpu.lib().tqhip_matvec_i4_dev(dw.ptr, dx.ptr + 4 * off, dy.ptr, M, K, G, None) == 0
    gpu.synchronize()
    return dy.download(np.float32, M)


def check(got, want, what):
    l2, mx = rel_l2(got, want), max_abs_rel(got, want)
    assert l2 <= 1e-5 and mx <= 1e-3, f"{what}: rel_l2={l2:.3e} max_rel={mx:.3e}"


@pytest.mark.parametrize("name,M,K,off", CASES, ids=[c[0] for c in CASES])
def test_wide_range_activations(gpu, orc, name, M, K, off):
    print(f"[extremes] activations {name} {M}x{K} offset {4 * off}", flush=True)
    w = gpu.synth_i4(M, K, G, seed=M + 3 * K)
    x = extreme_x(K, seed=K + 1)
    check(run(gpu, w, x, M, K, off), orc.matvec_i4(w, x, M, K, G, threads=16), f"{name} activations")


@pytest.mark.parametrize("name,M,K,off", CASES, ids=[c[0] for c in CASES])
def test_special_fp16_headers(gpu, orc, name, M, K, off):
    print(f"[extremes] headers {name} {M}x{K} offset {4 * off}", flush=True)
    w = special_headers(gpu.synth_i4(M, K, G, seed=M + 5 * K), M, K, seed=M)
    x = gpu.synth_normal(K, seed=K + 2)
    check(run(gpu, w, x, M, K, off), orc.matvec_i4(w, x, M, K, G, threads=16), f"{name} headers")


@pytest.mark.parametrize("name,M,K,off", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("where", ["one group", "whole vector"])
def test_tiny_activations(gpu, orc, name, M, K, off, where):
    """|x| ~ 1e-35: the group's power of two 2^f then has f >= 128, past the largest finite float,
    so a kernel must scale each value (ldexpf(x, f)) rather than form 2^f alone; the whole-vector
    case leaves every output near 1e-35, still a normal float in the reference's float cast."""
    print(f"[extremes] tiny activations ({where}) {name} {M}x{K} offset {4 * off}", flush=True)
    w = gpu.synth_i4(M, K, G, seed=M + 7 * K)
    x = gpu.synth_normal(K, seed=K + 3)
    if where == "whole vector":
        x = (x * np.float32(1e-35)).astype(np.float32)
    else:
        x[64:128] *= np.float32(1e-35)
    want = orc.matvec_i4(w, x, M, K, G, threads=16)
    assert np.all(np.isfinite(want)) and np.max(np.abs(want)) > 0
    check(run(gpu, w, x, M, K, off), want, f"{name} tiny activations ({where})")


@pytest.mark.parametrize("name,M,K,off", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("kind", ["nan", "inf", "-inf"])
def test_non_finite_activation(gpu, orc, name, M, K, off, kind):
    """One non-finite activation: the reference's double sum of w * x is then inf or NaN in every
    row (inf * w is +-inf, or NaN for w = 0; NaN * w is NaN), so every output must be non-finite.
    The exact-integer kernels would otherwise drop a NaN from the group maximum and saturate an
    inf in the integer conversion, and return finite values."""
    print(f"[extremes] non-finite activation ({kind}) {name} {M}x{K} offset {4 * off}", flush=True)
    w = gpu.synth_i4(M, K, G, seed=M + 11 * K)
    x = gpu.synth_normal(K, seed=K + 4)
    x[K // 3] = np.float32(kind)
    want = orc.matvec_i4(w, x, M, K, G, threads=16)
    got = run(gpu, w, x, M, K, off)
    assert not np.any(np.isfinite(want))
    bad = np.count_nonzero(np.isfinite(got))
    assert bad == 0, f"{name} {kind}: {bad} of {M} outputs finite where the oracle's are not"


@pytest.mark.parametrize("M,K", [(3072, 1024), (32768, 896), (151936, 896), (2001, 3052)])
@pytest.mark.parametrize("kind", ["nan", "inf"])
def test_vq2_non_finite_activation(gpu, orc, M, K, kind):
    """The same on every VQ2 kernel (one wave per row, replica, table, byte loads): fp32 products of
    the codebook entries, so a non-finite activation reaches every row (and entry * inf with a zero
    entry component is NaN, as in the reference)."""
    print(f"[extremes] vq2 non-finite activation ({kind}) {M}x{K}", flush=True)
    w = gpu.synth_vq2(M, K, seed=M + 13 * K)
    x = gpu.synth_normal(K, seed=K + 6)
    x[K // 2 + 1] = np.float32(kind)
    want = orc.matvec_vq2(w, x, M, K, threads=16)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M)
    gpu.matvec_vq2_dev(dw, dx, dy, M, K)
    got = dy.download(np.float32, M)
    assert np.array_equal(np.isfinite(got), np.isfinite(want)), \
        f"vq2 {M}x{K} {kind}: {np.count_nonzero(np.isfinite(got) != np.isfinite(want))} rows differ in finiteness"


@pytest.mark.parametrize("M,K,N", [(9728, 2560, 32), (9728, 2560, 5), (9728, 2560, 128), (1000, 640, 48)])
@pytest.mark.parametrize("kind", ["nan", "inf"])
def test_prefill_non_finite_activation(gpu, orc, M, K, N, kind):
    """matmul_i4 with one non-finite activation in token 1: every output of that token is inf or NaN
    in the reference and must be non-finite here; every other token stays finite and within the
    prefill bar. Covers the few-token kernel (N <= 32) and the fp16-staged MFMA GEMM (N > 32)."""
    print(f"[extremes] prefill non-finite activation ({kind}) {M}x{K}x{N}", flush=True)
    w = gpu.synth_i4(M, K, G, seed=M + K + N)
    x = gpu.synth_normal(K * N, seed=K + N + 7)
    x[1 * K + K // 5] = np.float32(kind)
    want = orc.matmul_i4(w, x, M, K, N, G, threads=16).reshape(N, M)
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * M * N)
    gpu.matmul_i4_dev(dw, dx, dy, M, K, N, G)
    got = dy.download(np.float32, M * N).reshape(N, M)
    assert not np.any(np.isfinite(want[1]))
    assert not np.any(np.isfinite(got[1])), f"token 1: {np.count_nonzero(np.isfinite(got[1]))} outputs finite"
    rest = np.ones(N, bool)
    rest[1] = False
    assert np.all(np.isfinite(got[rest]))
    l2, mx = rel_l2(got[rest], want[rest]), max_abs_rel(got[rest], want[rest])
    assert l2 <= 2e-3 and mx <= 1e-3, f"other tokens: rel_l2={l2:.3e} max_rel={mx:.3e}"
