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
