// lane_sum.h -- exchanges and sums between the lanes of a wave in registers (DPP, gfx950's
// row swaps), in a fixed order: shared by the i4 kernels (i4_matvec.hip, i4_set.hip) and the
// VQ2 kernels (vq2_matvec.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace tqhip {
namespace {

// DPP controls (gfx9): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror,
// row_ror:8, row_shr:n.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140, kDppRor8 = 0x128;
constexpr int kDppShr1 = 0x111, kDppShr2 = 0x112, kDppShr4 = 0x114, kDppShr8 = 0x118;

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

// The value of lane l ^ DL (DL a power of two up to 32), in registers: quad_perm for 1 and 2,
// row shifts within the 16-lane row for 4 and 8 (lanes with the bit clear read l + DL, the
// others l - DL), the row swaps for 16 and 32 (with d = s = v, v_permlane16_swap leaves rows
// (0, 0, 2, 2) in its first result and (1, 1, 3, 3) in its second).
template <int DL>
__device__ __forceinline__ float lane_xor(float v, int lane) {
    if constexpr (DL == 1) {
        return dpp_f<kDppXor1>(v);
    } else if constexpr (DL == 2) {
        return dpp_f<kDppXor2>(v);
    } else if constexpr (DL == 4 || DL == 8) {
        const float up = dpp_f<0x100 + DL>(v);  // row_shl:DL (lane l reads l + DL)
        const float dn = dpp_f<0x110 + DL>(v);  // row_shr:DL (lane l reads l - DL)
        return (lane & DL) ? dn : up;
    } else {
        static_assert(DL == 16 || DL == 32, "lane distance");
        const unsigned u = __builtin_bit_cast(unsigned, v);
        if constexpr (DL == 16) {
            const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
            return __builtin_bit_cast(float, static_cast<unsigned>((lane & 16) ? p[0] : p[1]));
        } else {
            const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
            return __builtin_bit_cast(float, static_cast<unsigned>((lane & 32) ? p[0] : p[1]));
        }
    }
}

// The value of lane l ^ DL for a double: both 32-bit halves moved by lane_xor (moves only).
template <int DL>
__device__ __forceinline__ double lane_xor_d(double v, int lane) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const float lo = lane_xor<DL>(__builtin_bit_cast(float, static_cast<unsigned>(b)), lane);
    const float hi = lane_xor<DL>(__builtin_bit_cast(float, static_cast<unsigned>(b >> 32)), lane);
    return __builtin_bit_cast(double, (static_cast<unsigned long long>(__builtin_bit_cast(unsigned, hi)) << 32) |
                                          __builtin_bit_cast(unsigned, lo));
}

// for (o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o): the same additions in the same order (each
// lane adds the value of lane l ^ o), with the exchanges in registers instead of LDS permutes.
__device__ __forceinline__ float xor_sum_wave(float v) {
    const int lane = threadIdx.x & 63;
    v += lane_xor<32>(v, lane);
    v += lane_xor<16>(v, lane);
    v += lane_xor<8>(v, lane);
    v += lane_xor<4>(v, lane);
    v += lane_xor<2>(v, lane);
    v += lane_xor<1>(v, lane);
    return v;
}

// The largest of the wave's 64 values, in every lane.
__device__ __forceinline__ float xor_max_wave(float v) {
    const int lane = threadIdx.x & 63;
    v = fmaxf(v, lane_xor<32>(v, lane));
    v = fmaxf(v, lane_xor<16>(v, lane));
    v = fmaxf(v, lane_xor<8>(v, lane));
    v = fmaxf(v, lane_xor<4>(v, lane));
    v = fmaxf(v, lane_xor<2>(v, lane));
    v = fmaxf(v, lane_xor<1>(v, lane));
    return v;
}

__device__ __forceinline__ double xor_sum_wave(double v) {
    const int lane = threadIdx.x & 63;
    v += lane_xor_d<32>(v, lane);
    v += lane_xor_d<16>(v, lane);
    v += lane_xor_d<8>(v, lane);
    v += lane_xor_d<4>(v, lane);
    v += lane_xor_d<2>(v, lane);
    v += lane_xor_d<1>(v, lane);
    return v;
}

}  // namespace
}  // namespace tqhip
