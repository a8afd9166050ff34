// i4_lane.h -- device helpers shared by the i4 matvec kernels (i4_matvec.hip, i4_set.hip):
// fp16 header decode, DPP and row-swap reductions in a fixed order, buffer resources over
// matrix rows, and a store that keeps the global address space.
#pragma once

#include "tq_common.h"

namespace tqhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr unsigned kNibbles = 0x0F0F0F0Fu;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family word 3)

// DPP controls (gfx9): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror,
// row_ror:8, row_shr:n.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140, kDppRor8 = 0x128;
constexpr int kDppShr1 = 0x111, kDppShr2 = 0x112, kDppShr4 = 0x114, kDppShr8 = 0x118;

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

template <int CTRL>
__device__ inline float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ inline int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// a[l] + a[l^16], then + the same of lane l^32: the four 16-lane rows of the
// wave summed in every lane, in the order of two xor-shuffle steps (16, then
// 32). gfx950's row swaps move the values in registers, where a shuffle is an
// LDS permute round trip. v_permlane16_swap(d, s) exchanges the odd rows of d
// with the even rows of s, so with d = s = a the two results hold rows
// (0,0,2,2) and (1,1,3,3) and their sum is a[l] + a[l^16] in every lane (fp
// addition commutes); v_permlane32_swap does the same for the wave halves.
__device__ __forceinline__ float sum_rows4(float a) {
    const unsigned u = __builtin_bit_cast(unsigned, a);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float b = __builtin_bit_cast(float, static_cast<unsigned>(p[0])) +
                    __builtin_bit_cast(float, static_cast<unsigned>(p[1]));
    const unsigned v = __builtin_bit_cast(unsigned, b);
    const auto q = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __builtin_bit_cast(float, static_cast<unsigned>(q[0])) +
           __builtin_bit_cast(float, static_cast<unsigned>(q[1]));
}

// Sum of the 16 lanes of each row (DPP, fixed order), left in every lane of the row.
__device__ __forceinline__ float sum_row16(float p) {
    p += dpp_f<kDppXor1>(p);
    p += dpp_f<kDppXor2>(p);
    p += dpp_f<kDppHalfMirror>(p);
    p += dpp_f<kDppMirror>(p);
    return p;
}

// Sum of the 32 lanes of each half-wave, in every lane of it.
__device__ __forceinline__ float sum_half_wave(float p) {
    p = sum_row16(p);
    const unsigned pu = __builtin_bit_cast(unsigned, p);
    const auto sw = __builtin_amdgcn_permlane16_swap(pu, pu, false, false);  // rows (0,0,2,2) and (1,1,3,3)
    return __builtin_bit_cast(float, static_cast<unsigned>(sw[0])) +
           __builtin_bit_cast(float, static_cast<unsigned>(sw[1]));
}

// Sum of the 64 lanes of the wave, in every lane.
__device__ __forceinline__ float sum_wave(float p) { return sum_rows4(sum_row16(p)); }

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
