// vq2_matvec.hip -- batch=1 VQ2 (d=4, 256-entry fp16 codebook) matvec for gfx950.
//
// Computes y[o] = sum_b codebook[idx[o][b]] . x[4b : 4b+4], the contract of the
// reference's matvec_vq2_ref (kernels/matvec/matvec_vq2_ref.cpp:52-81), on the
// layout [codebook 256 x 4 fp16 = 2048 B][out_dim x in_dim/4 uint8 indices].
//
// Design: the codebook is decoded once per workgroup into LDS as fp32 rows of
// 16 bytes (one ds_read_b128 per index). A wave owns a tile of kRows rows and
// sweeps the row in steps of 64 lanes x 4 indices; each lane keeps the 16
// activations of its 4 indices in VGPRs and reuses them for all kRows rows, so
// x is read once per tile. Partial sums are reduced across the wave at the end
// of the tile. fp32 accumulation.

#include "tq_common.h"

#include <algorithm>

namespace tqhip {
namespace {

constexpr int kRows = 8;  // rows per wave tile
constexpr int kWavesPerBlock = 4;
constexpr int kBufferFlags = 0x00020000;

__device__ inline float half_bits(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xFFFFu)));
}

// ALIGNED: the index rows start on 4-byte boundaries (in_dim % 16 == 0), so a
// lane's 4 indices are one dword load; otherwise bytes are loaded one by one.
template <bool ALIGNED>
__global__ __launch_bounds__(256) void vq2_matvec_kernel(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                         float *__restrict__ y, int M, int K) {
    __shared__ float4 cb[kVq2Entries];
    for (int e = threadIdx.x; e < kVq2Entries; e += blockDim.x) {
        const uint16_t *h = reinterpret_cast<const uint16_t *>(w) + kVq2Dim * e;
        cb[e] = make_float4(half_bits(h[0]), half_bits(h[1]), half_bits(h[2]), half_bits(h[3]));
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nb = K / kVq2Dim;  // index bytes per row
    const uint8_t *idx = w + kVq2CodebookBytes;
    const int tiles = (M + kRows - 1) / kRows;
    const int gw = blockIdx.x * kWavesPerBlock + wave;
    const int nw = gridDim.x * kWavesPerBlock;

    for (int tile = gw; tile < tiles; tile += nw) {
        const int row0 = tile * kRows;
        const size_t rem = static_cast<size_t>(M - row0) * nb;
        const int nrec = rem > 0xFFFFFFFFull ? -1 : static_cast<int>(static_cast<unsigned>(rem));
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(idx) + static_cast<size_t>(row0) * nb, static_cast<short>(0), nrec, kBufferFlags);
        float acc[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) acc[r] = 0.f;
        for (int b = 4 * lane; b < nb; b += 256) {
            // activations of this lane's (up to) 4 blocks, reused for all rows
            float4 xv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float *xp = x + 4 * (b + j);
                xv[j] = (b + j < nb) ? make_float4(xp[0], xp[1], xp[2], xp[3]) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                unsigned q;
                if (ALIGNED) {
                    q = __builtin_amdgcn_raw_buffer_load_b32(rs, r * nb + b, 0, 0);
                } else {
                    q = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (b + j < nb) q |= static_cast<unsigned>(__builtin_amdgcn_raw_buffer_load_b8(rs, r * nb + b + j, 0, 0)) << (8 * j);
                }
                float a = acc[r];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 c = cb[(q >> (8 * j)) & 0xFFu];
                    a = fmaf(c.x, xv[j].x, a);
                    a = fmaf(c.y, xv[j].y, a);
                    a = fmaf(c.z, xv[j].z, a);
                    a = fmaf(c.w, xv[j].w, a);
                }
                acc[r] = a;
            }
        }
        // Rows past M read zeros (buffer range check) and are not stored.
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            float v = acc[r];
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0 && row0 + r < M) y[row0 + r] = v;
        }
    }
}

int device_cus_vq2() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        TQ_HIP_CHECK(hipGetDevice(&dev));
        TQ_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        if (cus < 1) cus = 1;
    }
    return cus;
}

}  // namespace

int launch_vq2_matvec(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, hipStream_t stream) {
    if (out_dim < 1 || in_dim < kVq2Dim || in_dim % kVq2Dim) return kBadShape;
    const int tiles = (out_dim + kRows - 1) / kRows;
    const int grid = std::max(1, std::min((tiles + kWavesPerBlock - 1) / kWavesPerBlock, device_cus_vq2() * 8));
    const bool aligned = (in_dim % 16) == 0 && (reinterpret_cast<uintptr_t>(w) % 4) == 0;
    if (aligned)
        hipLaunchKernelGGL(vq2_matvec_kernel<true>, dim3(grid), dim3(64 * kWavesPerBlock), 0, stream, w, x, y,
                           out_dim, in_dim);
    else
        hipLaunchKernelGGL(vq2_matvec_kernel<false>, dim3(grid), dim3(64 * kWavesPerBlock), 0, stream, w, x, y,
                           out_dim, in_dim);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

}  // namespace tqhip
