// biip_rotate.hip -- BiIP activation rotation for gfx950.
//
// y = blockHadamard((x / scale) * sign), the contract of the reference's
// biip_rotate_activation (kernels/dispatch.h:220-231; scalar reference
// kernels/biip/biip_rotate.cpp:37-68): scale == nullptr skips the division;
// every block of block_size elements (a power of two) goes through the
// unnormalised Walsh-Hadamard butterfly, stage h = 1, 2, 4, ... replacing
// (a, c) at (j, j + h) by (a + c, a - c), and is then scaled by
// 1 / sqrt(block_size). It runs ahead of every matvec of a rotated model.
//
// One workgroup takes a chunk of whole blocks (up to 2048 elements) into LDS,
// runs the butterfly stages there, two per barrier, and writes the
// scaled result. Every element goes through the same fp32 operations in the
// same order as the scalar reference (one correctly rounded division, the
// sign product, the adds and subtracts of each stage, the final product), so
// the result is bit-identical to it. y may alias x: a workgroup reads its
// whole chunk before it writes any of it, and chunks are disjoint.

#include "tq_common.h"

#include <cmath>

namespace tqhip {
namespace {

constexpr int kBiipThreads = 256;
constexpr int kBiipChunk = 2048;  // elements per workgroup: whole blocks (block_size divides it)

// Up to three rotations of one x (their own sign / scale / output), one per
// grid row: the q / k / v or gate / up projections of a rotated layer.
struct RotSets {
    const float *scale[3];
    const float *sign[3];
    float *y[3];
};

__device__ void rotate_chunk(float *v, const float *x, float *y, int dim, const float *__restrict__ scale,
                             const float *__restrict__ sign, int lg_bs, float inv_sqrt);

__global__ __launch_bounds__(kBiipThreads) void biip_rotate_kernel(const float *x, float *y, int dim,
                                                                   const float *__restrict__ scale,
                                                                   const float *__restrict__ sign, int lg_bs,
                                                                   float inv_sqrt) {
    __shared__ float v[kBiipChunk];
    rotate_chunk(v, x, y, dim, scale, sign, lg_bs, inv_sqrt);
}

__global__ __launch_bounds__(kBiipThreads) void biip_rotate_sets(const float *x, RotSets rs, int dim, int lg_bs,
                                                                 float inv_sqrt) {
    __shared__ float v[kBiipChunk];
    const int k = blockIdx.y;
    rotate_chunk(v, x, rs.y[k], dim, rs.scale[k], rs.sign[k], lg_bs, inv_sqrt);
}

__device__ void rotate_chunk(float *v, const float *x, float *y, int dim, const float *__restrict__ scale,
                             const float *__restrict__ sign, int lg_bs, float inv_sqrt) {
    const int base = blockIdx.x * kBiipChunk;
    const int n = min(kBiipChunk, dim - base);  // a whole number of blocks
    for (int i = threadIdx.x; i < n; i += kBiipThreads) {
        const int j = base + i;
        v[i] = scale ? (x[j] / scale[j]) * sign[j] : x[j] * sign[j];
    }
    // stages h = 2^lg and 2h together on the four elements j + {0, h, 2h, 3h} of a block: each
    // element gets the adds and subtracts of the two stages in their order, one barrier for both
    int lg = 0;
    for (; lg + 1 < lg_bs; lg += 2) {
        __syncthreads();
        const int h = 1 << lg;
        for (int p = threadIdx.x; p < n / 4; p += kBiipThreads) {
            const int j = ((p >> lg) << (lg + 2)) + (p & (h - 1));
            const float x0 = v[j], x1 = v[j + h], x2 = v[j + 2 * h], x3 = v[j + 3 * h];
            const float y0 = x0 + x1, y1 = x0 - x1, y2 = x2 + x3, y3 = x2 - x3;
            v[j] = y0 + y2;
            v[j + h] = y1 + y3;
            v[j + 2 * h] = y0 - y2;
            v[j + 3 * h] = y1 - y3;
        }
    }
    if (lg < lg_bs) {  // a last single stage h = 2^lg
        __syncthreads();
        const int h = 1 << lg;
        for (int p = threadIdx.x; p < n / 2; p += kBiipThreads) {
            const int j = ((p >> lg) << (lg + 1)) + (p & (h - 1));  // pair (j, j + h) within its block
            const float a = v[j], c = v[j + h];
            v[j] = a + c;
            v[j + h] = a - c;
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kBiipThreads) y[base + i] = v[i] * inv_sqrt;
}

}  // namespace

int launch_biip_rotate(const float *x, float *y, int dim, const float *scale, const float *sign, int block_size,
                       hipStream_t stream) {
    if (dim < 1 || block_size < 1 || (block_size & (block_size - 1)) || block_size > kBiipChunk ||
        dim % block_size)
        return kBadShape;
    if (!x || !y || !sign) return kBadShape;  // nothing is launched on a null operand (scale may be null)
    int lg = 0;
    while ((1 << lg) < block_size) ++lg;
    // computed on the host exactly as the reference does (float sqrt, then 1.0f / it)
    const float inv_sqrt = 1.0f / std::sqrt(static_cast<float>(block_size));
    const int grid = (dim + kBiipChunk - 1) / kBiipChunk;
    hipLaunchKernelGGL(biip_rotate_kernel, dim3(grid), dim3(kBiipThreads), 0, stream, x, y, dim, scale, sign, lg,
                       inv_sqrt);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

int launch_biip_rotate_n(int n, const float *x, float *const *y, int dim, const float *const *scale,
                         const float *const *sign, int block_size, hipStream_t stream) {
    if (n < 1 || n > 3 || dim < 1 || block_size < 1 || (block_size & (block_size - 1)) || block_size > kBiipChunk ||
        dim % block_size)
        return kBadShape;
    if (!x) return kBadShape;
    int lg = 0;
    while ((1 << lg) < block_size) ++lg;
    const float inv_sqrt = 1.0f / std::sqrt(static_cast<float>(block_size));
    RotSets rs{};
    for (int k = 0; k < n; ++k) {
        if (!sign[k] || !y[k]) return kBadShape;
        rs.scale[k] = scale[k];
        rs.sign[k] = sign[k];
        rs.y[k] = y[k];
    }
    const int grid = (dim + kBiipChunk - 1) / kBiipChunk;
    hipLaunchKernelGGL(biip_rotate_sets, dim3(grid, n), dim3(kBiipThreads), 0, stream, x, rs, dim, lg, inv_sqrt);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

}  // namespace tqhip
