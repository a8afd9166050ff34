"""The allocation-free prefill entry point (tqhip_matmul_i4_noalloc_dev) against
tqhip_matmul_i4_dev, through the C ABI.

Both run the same kernels; the only difference is where their scratch lives (the
library's static device array instead of a stream's grow-only buffers), so the
outputs must agree bit for bit, call after call, with the second call of each
pair smaller than the first (the array keeps the previous call's contents). The
results are also held to the prefill bar against the oracle, and a call that
needs more than the static array is refused before anything is launched.
"""
import numpy as np
import pytest

from conftest import max_abs_rel, rel_l2

pytestmark = pytest.mark.gpu


def run_pair(gpu, w, x, M, K, N, G, stream):
    dw, dx = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x)
    ya, yb = gpu.DeviceBuffer(4 * M * N), gpu.DeviceBuffer(4 * M * N)
    gpu.lib().tqhip_memset(yb.ptr, 0xFF, 4 * M * N)  # the no-alloc call must write every output
    gpu.matmul_i4_dev(dw, dx, ya, M, K, N, G, stream=stream)
    st = gpu.matmul_i4_noalloc_dev(dw, dx, yb, M, K, N, G, stream=stream)
    assert st == gpu.OK, st
    stream.synchronize()
    return ya.download(np.float32, M * N), yb.download(np.float32, M * N)


# G = 64 above 32 tokens: the MFMA GEMM (512 tokens at K = 2560 uses 10.5 MB of the 16 MiB), then
# a smaller call over the same array. G = 64 up to 32 tokens: the few-token kernel (partial
# products in the array, tile counters in its last 64 KiB, which every launch must leave at
# zero for the next: 32 tokens, a smaller call with fewer tiles, 32 tokens again). G = 40: one
# matvec per token column, no scratch.
NOALLOC_CASES = {
    "gemm": (64, [(9728, 2560, 512), (896, 896, 40)]),
    "few-token": (64, [(9728, 2560, 32), (4096, 2560, 7), (9728, 2560, 32)]),
    "per-column": (40, [(640, 520, 9), (200, 280, 3)]),
}


@pytest.mark.parametrize("kind", list(NOALLOC_CASES))
def test_noalloc_matches_dev_entry_point(gpu, orc, kind):
    stream = gpu.Stream()
    G, cases = NOALLOC_CASES[kind]
    for i, (M, K, N) in enumerate(cases):
        print(f"[no-alloc] {kind} call {i}: M={M} K={K} N={N} G={G}", flush=True)
        w = gpu.synth_i4(M, K, G, seed=700 + 10 * i + G)
        x = gpu.synth_normal(K * N, seed=701 + 10 * i + G)
        want, got = run_pair(gpu, w, x, M, K, N, G, stream)
        assert np.array_equal(got, want), f"call {i}: no-alloc result differs from tqhip_matmul_i4_dev"
        if M * N <= 9728 * 32:  # the oracle at sizes it finishes in seconds
            ref = orc.matmul_i4(w, x, M, K, N, G, threads=16)
        else:  # sampled rows of the 9728x2560x512 call
            rows = np.arange(0, M, 97)
            rb = gpu.i4_row_bytes(K, G)
            wr = w.reshape(M, rb)[rows].ravel()
            ref = orc.matmul_i4(wr, x, rows.size, K, N, G, threads=16)
            got = got.reshape(N, M)[:, rows].ravel()
        assert rel_l2(got, ref) <= 2e-3 and max_abs_rel(got, ref) <= 1e-3, i


def test_noalloc_refuses_calls_beyond_the_static_array(gpu):
    """Refusals come before any launch. The operands are real device buffers of the call's size
    (uninitialised), so a call that were wrongly launched would compute, not touch a null pointer."""
    def call(M, K, N):
        dw = gpu.DeviceBuffer(M * gpu.i4_row_bytes(K, 64))
        dx, dy = gpu.DeviceBuffer(4 * K * N), gpu.DeviceBuffer(4 * M * N)
        st = gpu.matmul_i4_noalloc_dev(dw, dx, dy, M, K, N, 64)
        gpu.synchronize()
        for b in (dw, dx, dy):
            b.free()
        return st

    assert call(9728, 2560, 3262) == gpu.ENOSCRATCH  # the fp16 copy: 16 MiB - 64 KiB hold 3261 tokens at K 2560
    # few tokens whose partial products do not fit (1187 tiles x 2 K slices x 16 KiB = 38.9 MB):
    # refused, not rerouted to the MFMA GEMM, whose bits differ from tqhip_matmul_i4_dev's
    assert call(151936, 896, 8) == gpu.ENOSCRATCH
    # shape and operand checks (nothing to launch on)
    assert gpu.matmul_i4_noalloc_dev(None, None, None, 0, 2560, 8, 64) == gpu.EBADSHAPE
    dw, dx, dy = gpu.DeviceBuffer(896 * gpu.i4_row_bytes(896, 64)), gpu.DeviceBuffer(4 * 896 * 8), gpu.DeviceBuffer(4 * 896 * 8)
    assert gpu.matmul_i4_noalloc_dev(dw, None, dy, 896, 896, 8, 64) == gpu.EBADSHAPE
    assert gpu.matmul_i4_noalloc_dev(dw, dx, None, 896, 896, 40, 64) == gpu.EBADSHAPE
