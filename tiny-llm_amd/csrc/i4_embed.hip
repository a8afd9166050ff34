// i4_embed.hip -- compact-i4 embedding rows for gfx950.
//
// out[t][k] = (q - zero) * scale of row rows[t] of an i4-packed table, the
// contract of the reference's dequant_i4_row (kernels/ref_ops.h:183-205), which
// its prefill calls once per token for the embedding lookup
// (runtime/qwen_forward_prefill.cpp:180). Rows are [scale fp16 | zero fp16 |
// G/2 code bytes] groups, low nibble first; a partial last group decodes only
// its first dim - col elements. Each element is one fp32 subtraction and one
// product, as in the reference (no fused multiply-add), so the result is
// bit-identical to it.
//
// One workgroup per token row; 256 threads sweep the row's elements, each
// reading its group header and its code byte (the row's bytes are contiguous,
// so a wave's reads coalesce).

#include "tq_common.h"

namespace tqhip {
namespace {

__device__ inline float half_f(unsigned h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xFFFFu)));
}

__global__ __launch_bounds__(256) void i4_embed_rows_kernel(const uint8_t *__restrict__ embed,
                                                            const int *__restrict__ rows, int dim, int group_size,
                                                            float *__restrict__ out) {
    const int t = blockIdx.x;
    const int groups = (dim + group_size - 1) / group_size;
    const int gbytes = kI4Header + group_size / 2;
    const uint8_t *r = embed + static_cast<size_t>(rows[t]) * groups * gbytes;
    float *o = out + static_cast<size_t>(t) * dim;
    for (int k = threadIdx.x; k < dim; k += blockDim.x) {
        const int g = k / group_size, i = k - g * group_size;
        const uint8_t *gp = r + static_cast<size_t>(g) * gbytes;
        const float scale = half_f(gp[0] | (gp[1] << 8));
        const float zero = half_f(gp[2] | (gp[3] << 8));
        const uint8_t b = gp[kI4Header + (i >> 1)];
        const int q = (i & 1) ? (b >> 4) : (b & 0x0F);
        o[k] = (static_cast<float>(q) - zero) * scale;
    }
}

}  // namespace

int launch_i4_embed_rows(const uint8_t *embed, const int *rows, int n, int dim, int group_size, float *out,
                         hipStream_t stream) {
    if (n < 1 || dim < 1 || group_size < 2 || (group_size & 1)) return kBadShape;
    if (!embed || !rows || !out) return kBadShape;
    hipLaunchKernelGGL(i4_embed_rows_kernel, dim3(n), dim3(256), 0, stream, embed, rows, dim, group_size, out);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

}  // namespace tqhip
