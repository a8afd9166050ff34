"""The few-token prefill kernel (up to 32 tokens at G = 64: one launch that converts X itself
and adds the K-slice partials of each 128-row tile in slice order) against the oracle.

The cases cover the slice geometry launch_i4_matmul picks (about 2.4 workgroups per CU, at
most 8 steps per slice; the figures are for 256 CUs):

    9728x2560     76 tiles x  8 slices of 5 steps   (the prefill configuration)
    2560x9728     20 tiles x 31 slices of 4-5 steps (long rows)
    4096x2560     32 tiles x 19 slices of 2-3 steps
    38912x2560   304 tiles x  5 slices of 8 steps   (most steps per slice)
    896x4864       7 tiles x 76 slices of 1 step    (one slice per step)
    130x2500       2 tiles x 40 slices; K % 64 = 4, the last tile 2 rows
    100x96, 1x64   a tile of fewer rows than a wave, K = 1.5 groups / 1 slice (no partials)

An X that is not 16-byte aligned goes to the fp16-staging kernel instead, so one case runs at
an offset of 4 bytes as a cross-check of the two paths. Bar (north star prefill): rel L2 <=
2e-3 and max|err| <= 1e-3 of max|y| against the oracle.
"""
import numpy as np
import pytest

from conftest import extreme_x, fp16_operand_bound_ok, max_abs_rel, rel_l2, special_headers

pytestmark = pytest.mark.gpu

G = 64
CASES = [(9728, 2560, 32), (9728, 2560, 1), (2560, 9728, 17), (4096, 2560, 32), (38912, 2560, 3), (896, 4864, 5),
         (130, 2500, 31), (100, 96, 3), (1, 64, 1)]


def assert_close(got, want, what):
    l2, mx = rel_l2(got, want), max_abs_rel(got, want)
    assert l2 <= 2e-3 and mx <= 1e-3, f"{what}: rel_l2={l2:.3e} max_rel={mx:.3e}"


def run(gpu, w, x, M, K, N, off=0):
    xb = np.zeros(K * N + 4, np.float32)
    xb[off:off + K * N] = x
    dw, dx, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(xb), gpu.DeviceBuffer(4 * M * N)
    gpu.lib().tqhip_memset(dy.ptr, 0xFF, 4 * M * N)  # every output must be written
    assert gpu.lib().tqhip_matmul_i4_dev(dw.ptr, dx.ptr + 4 * off, dy.ptr, M, K, N, G, None) == 0
    gpu.synchronize()
    return dy.download(np.float32, M * N)


@pytest.mark.parametrize("M,K,N", CASES, ids=[f"{m}x{k}x{n}" for m, k, n in CASES])
def test_few_tokens_match_oracle(gpu, orc, M, K, N):
    print(f"[few] {M}x{K} N={N}", flush=True)
    w = gpu.synth_i4(M, K, G, seed=M + 7 * K + N)
    x = gpu.synth_normal(K * N, seed=K + N)
    got, want = run(gpu, w, x, M, K, N), orc.matmul_i4(w, x, M, K, N, G, threads=16)
    if M * N < 16:  # one near-cancelled output decides the relative measures
        assert fp16_operand_bound_ok(got, want, orc, w, x, M, K, N, G), f"{M}x{K}x{N}"
    else:
        assert_close(got, want, f"{M}x{K}x{N}")


def test_repeated_calls_are_bit_identical_and_leave_counters_clear(gpu):
    """The partials meet in slice order whatever order the workgroups finish in, and every
    launch leaves the tile counters at zero: three calls of one shape with a different shape
    in between give the same bits."""
    M, K, N = 9728, 2560, 32
    w = gpu.synth_i4(M, K, G, seed=3)
    x = gpu.synth_normal(K * N, seed=4)
    first = run(gpu, w, x, M, K, N)
    w2 = gpu.synth_i4(4096, 2560, G, seed=5)
    run(gpu, w2, gpu.synth_normal(2560 * 7, seed=6), 4096, 2560, 7)
    for _ in range(2):
        assert np.array_equal(run(gpu, w, x, M, K, N).view(np.uint32), first.view(np.uint32))


def test_unaligned_x_takes_the_staging_kernel_and_agrees(gpu, orc):
    M, K, N = 2560, 2560, 12
    w = gpu.synth_i4(M, K, G, seed=8)
    x = gpu.synth_normal(K * N, seed=9)
    want = orc.matmul_i4(w, x, M, K, N, G, threads=16)
    assert_close(run(gpu, w, x, M, K, N, off=1), want, "x + 4 bytes")
    assert_close(run(gpu, w, x, M, K, N, off=0), want, "aligned x")


def test_per_token_and_per_group_extremes(gpu, orc):
    """Token columns 1e30, 1e-30, zero and N(0,1), and within every group one activation 1e4
    times larger and one 1e6 times smaller than the rest: each column keeps the bar on its own
    (every slice of every token gets its own power-of-two scale)."""
    M, K, N = 4096, 2560, 8
    w = gpu.synth_i4(M, K, G, seed=21)
    x = np.stack([extreme_x(K, seed=30 + n) for n in range(N)])
    x[1] *= 1e30
    x[2] *= 1e-30
    x[3] = 0.0
    x[5] = gpu.synth_normal(K, seed=40)
    x = x.reshape(-1)
    want = orc.matmul_i4(w, x, M, K, N, G, threads=16).reshape(N, M)
    got = run(gpu, w, x, M, K, N).reshape(N, M)
    assert np.all(got[3] == 0.0)
    for n in range(N):
        if n != 3:
            assert_close(got[n], want[n], f"column {n}")


def test_special_fp16_headers(gpu, orc):
    M, K, N = 2560, 9728, 9
    w = special_headers(gpu.synth_i4(M, K, G, seed=51), M, K, seed=52)
    x = gpu.synth_normal(K * N, seed=53)
    assert_close(run(gpu, w, x, M, K, N), orc.matmul_i4(w, x, M, K, N, G, threads=16), "special headers")
