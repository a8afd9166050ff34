// i4_lane.h -- device helpers shared by the i4 matvec kernels (i4_matvec.hip, i4_set.hip):
// fp16 header decode, buffer resources over matrix rows, and a store that keeps the global
// address space (the DPP and row-swap reductions are in lane_sum.h).
#pragma once

#include "lane_sum.h"
#include "tq_common.h"

namespace tqhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr unsigned kNibbles = 0x0F0F0F0Fu;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family word 3)

__device__ inline float half_bits(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xFFFFu)));
}

// The power of two 2^f that puts a group's largest |x| m into [2^21, 2^22): the exact-integer
// kernels convert the group to X = rint(x * 2^f), |X| <= 2^22. f <= 149, so ldexpf(x, f) (one
// v_ldexp_f32, exact for every finite x of the group) must scale the value itself: 2^f alone
// is not a finite float for f >= 128. Zero and non-finite maxima give 0.
__device__ inline int group_exponent(float m) {
    if (!(m > 0.f && m <= 3.40282347e38f)) return 0;
    int e;
    frexpf(m, &e);  // m in [2^(e-1), 2^e)
    return min(22 - e, 149);
}

// |v|, or +inf when v is an infinity or a NaN: a group maximum taken over these with fmaxf is
// +inf exactly when the group holds a non-finite activation (fmaxf alone drops a NaN).
__device__ inline float abs_or_inf(float v) {
    const float a = fabsf(v);
    return a <= 3.40282347e38f ? a : __builtin_inff();
}

// The epilogue's 2^-f for a group with maximum m, or NaN when the group holds a non-finite
// activation (m = +inf): every row's sum then takes the NaN, so each output is non-finite where
// the reference's double sum of w * x is (an inf or NaN x gives inf or NaN products, w = 0
// included), instead of a finite value from saturated integer conversions.
__device__ inline float group_unscale(float m, int f) {
    return m <= 3.40282347e38f ? ldexpf(1.f, -f) : __builtin_nanf("");
}

// A store of one output through a global-memory pointer. A pointer rebuilt
// from an integer has lost its address space, and a plain store through it
// becomes a flat store, which also counts against the LDS wait counter: every
// later LDS barrier would then wait for the store to complete.
__device__ inline void store_y(float *p, float v) { *(__attribute__((address_space(1))) float *)p = v; }

// Buffer resource over rows row0 .. M-1 of a matrix of row_bytes-byte rows:
// loads past the last row read 0.
__device__ inline __amdgpu_buffer_rsrc_t rows_rsrc(const uint8_t *w, int M, int row_bytes, int row0) {
    const size_t rem = row0 < M ? static_cast<size_t>(M - row0) * row_bytes : 0;  // past the end: every load reads 0
    const int nrec = rem > 0xFFFFFFFFull ? -1 : static_cast<int>(static_cast<unsigned>(rem));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w) + static_cast<size_t>(row0) * row_bytes,
                                             static_cast<short>(0), nrec, kBufferFlags);
}

}  // namespace
}  // namespace tqhip
