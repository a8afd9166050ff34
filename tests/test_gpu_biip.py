"""BiIP activation rotation on the GPU (tqhip_biip_rotate*) against the oracle.

The oracle's rotation is pinned bit for bit to the compiled reference
(kernels/biip/biip_rotate.cpp) and to a dense float64 Hadamard in
tests/test_oracle.py. The HIP kernel performs the same fp32 operations in the
same order for every element, so the bar here is bit-exact.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (dim, block_size, with_scale): the reference test's shapes (tests/test_biip_rotate.cpp:104-161),
# deployment shapes (in_dim 1024/2048/3072 at block 256), several workgroups (9728), block 1
CASES = [(896, 128, True), (896, 128, False), (4864, 256, True), (256, 64, True), (128, 128, True),
         (256, 4, True), (256, 2, True), (1024, 256, True), (2048, 256, False), (3072, 256, True),
         (9728, 256, True), (7, 1, True), (4096, 2048, True)]


def inputs(dim, with_scale, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(dim) * 3.0).astype(np.float32)
    scale = rng.uniform(0.25, 4.0, dim).astype(np.float32) if with_scale else None
    sign = np.where(rng.random(dim) < 0.5, -1.0, 1.0).astype(np.float32)
    return x, scale, sign


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("dim,bs,with_scale", CASES)
def test_biip_rotate_matches_oracle_bit_for_bit(gpu, orc, dim, bs, with_scale):
    x, scale, sign = inputs(dim, with_scale, dim * 3 + bs)
    want = orc.biip_rotate(x, scale, sign, bs)
    assert gpu.lib().tqhip_set_ops_impl_by_name(b"hip") == 1
    got = gpu.biip_rotate(x, scale, sign, bs)  # host pointers, through the ops registry
    assert np.array_equal(bits(got), bits(want)), "registry entry"
    dx, dy, dsg = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * dim), gpu.DeviceBuffer.from_array(sign)
    dsc = gpu.DeviceBuffer.from_array(scale) if scale is not None else None
    gpu.biip_rotate_dev(dx, dy, dim, dsc, dsg, bs)
    assert np.array_equal(bits(dy.download(np.float32, dim)), bits(want)), "device entry"
    gpu.biip_rotate_dev(dx, dx, dim, dsc, dsg, bs)  # in place
    assert np.array_equal(bits(dx.download(np.float32, dim)), bits(want)), "in place"


def test_biip_rotate_then_matvec_in_one_op_list(gpu, orc):
    """The rotated-matvec sequence of the reference runtime (QwenModel::mv_rot,
    runtime/qwen_model.cpp:229-238): rotate x, then matvec the rotated x, as two
    ops of one list on one stream."""
    dim, bs, M, G = 1024, 256, 3072, 64
    x, scale, sign = inputs(dim, True, 11)
    w = gpu.synth_i4(M, dim, G, seed=12)
    dx, dxr, dsc, dsg = (gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * dim),
                         gpu.DeviceBuffer.from_array(scale), gpu.DeviceBuffer.from_array(sign))
    dw, dy = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer(4 * M)
    ops = [gpu.Op(gpu.OP_BIIP_ROTATE, None, dx.ptr, dxr.ptr, 0, dim, 1, bs, dsc.ptr, dsg.ptr, None, None, 0),
           gpu.Op(gpu.OP_I4_MATVEC, dw.ptr, dxr.ptr, dy.ptr, M, dim, 1, G)]
    gpu.run_ops(ops, 1)
    gpu.synchronize()
    xr = orc.biip_rotate(x, scale, sign, bs)
    assert np.array_equal(bits(dxr.download(np.float32, dim)), bits(xr))
    want = orc.matvec_i4(w, xr, M, dim, G, threads=8)
    got = dy.download(np.float32, M)
    assert np.linalg.norm(got - want) <= 1e-5 * np.linalg.norm(want)


def test_biip_rotate_bad_shapes_return_codes(gpu):
    lib = gpu.lib()
    assert lib.tqhip_biip_rotate_dev(None, None, 100, None, None, 64, None) == gpu.EBADSHAPE  # 64 does not divide 100
    assert lib.tqhip_biip_rotate_dev(None, None, 96, None, None, 12, None) == gpu.EBADSHAPE   # not a power of two
    assert lib.tqhip_biip_rotate_dev(None, None, 0, None, None, 1, None) == gpu.EBADSHAPE
    assert gpu.lib().tqhip_set_ops_impl_by_name(b"ref") == 0  # no CPU path in this library
    assert gpu.lib().tqhip_set_ops_impl_by_name(b"hip") == 1
    assert gpu.lib().tqhip_ops_impl_name() == b"hip"
