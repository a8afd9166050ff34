// i4_set_core.h -- the per-row machinery of the i4 matvec set kernel (i4_set.hip), shared with
// the data-flow decode kernel (decode_flow.hip) so that a row gives the same bits in both: the
// activations as exact integers in LDS (stage_x), the per-half-group v_dot4 arithmetic
// (half_group_int), the fixed-order workgroup sum, and the prologue arithmetic (SwiGLU,
// RMSNorm).
#pragma once

#include "i4_lane.h"

namespace tqhip {
namespace {

#ifndef TQ_SET_WAVES
#define TQ_SET_WAVES 8
#endif
constexpr int kSetWaves = TQ_SET_WAVES;     // waves per workgroup
constexpr int kSetThreads = 64 * kSetWaves;
constexpr int kSetMaxSlots = 5;   // wave-per-row slots of 64 half-groups: K <= 5 * 64 * 32

// ---- activations as exact integers -------------------------------------------------------
// Every group of 64 activations is scaled by its own power of two 2^f (its largest |x|
// lands in [2^21, 2^22)) and rounded to the nearest integer: X = x * 2^f rounded,
// |X| <= 2^22, the only rounding before the epilogue. X's two's-complement bytes are its
// digits, X = b0 + 256 b1 + 65536 s2 with b0, b1 unsigned and s2 the signed third byte
// (exact while |X| < 2^23). They go to LDS as the byte operands of v_dot4: per 8-element
// block six dwords [byte p][even | odd], "even" holding elements 0, 2, 4, 6 and "odd" 1,
// 3, 5, 7 -- the order in which a code dword's low and high nibbles present the weights.
// Per half-group (32 elements) LDS also holds sum(X) (as a float) and 2^-f.
constexpr int kBlockBytes = 24;  // one 8-element block: 3 digit planes x (even, odd) dwords

// Round to nearest (ties upward: floor(v + 0.5)), one instruction.
__device__ inline int round_int(float v) {
    int r;
    asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// Thread t converts 16-byte chunk c = t + kSetThreads i (elements 4c .. 4c + 3) of every chunk
// the rows read (c < C): the 16 chunks of a group are one DPP row (16 lanes), the 8
// chunks of a half-group half of one.
__device__ __forceinline__ void stage_x(float4 q, int c, int Kc, int C, unsigned char *xp, float2 *hs) {
    if (c >= Kc) q = make_float4(0.f, 0.f, 0.f, 0.f);  // past K: zeros
    float m = fmaxf(fmaxf(abs_or_inf(q.x), abs_or_inf(q.y)), fmaxf(abs_or_inf(q.z), abs_or_inf(q.w)));
    m = fmaxf(m, dpp_f<kDppXor1>(m));
    m = fmaxf(m, dpp_f<kDppXor2>(m));
    m = fmaxf(m, dpp_f<kDppHalfMirror>(m));
    m = fmaxf(m, dpp_f<kDppMirror>(m));  // the group's largest |x| (inf if any is not finite), in all 16 lanes
    const int f = group_exponent(m);
    // the value itself is scaled (2^f is not a finite float for f >= 128; x * 2^f is exact)
    const unsigned X0 = round_int(ldexpf(q.x, f)), X1 = round_int(ldexpf(q.y, f));
    const unsigned X2 = round_int(ldexpf(q.z, f)), X3 = round_int(ldexpf(q.w, f));
    int sum = static_cast<int>(X0 + X1 + X2 + X3);
    sum += dpp_i<kDppXor1>(sum);
    sum += dpp_i<kDppXor2>(sum);
    sum += dpp_i<kDppHalfMirror>(sum);  // the half-group's sum(X), in its 8 lanes
    if (c >= C) return;
    // elements 4c + 0, 2 are "even" bytes 2 (c & 1) + 0, 1 of the block; 4c + 1, 3 "odd"
    unsigned char *blk = xp + (c >> 1) * kBlockBytes + 2 * (c & 1);
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        const unsigned sel = 0x0C0C0000u | ((4u + p) << 8) | p;  // byte p of the second, byte p of the first
        *reinterpret_cast<unsigned short *>(blk + 8 * p) = static_cast<unsigned short>(__builtin_amdgcn_perm(X2, X0, sel));
        *reinterpret_cast<unsigned short *>(blk + 8 * p + 4) =
            static_cast<unsigned short>(__builtin_amdgcn_perm(X3, X1, sel));
    }
    if ((c & 7) == 0) hs[c >> 3] = make_float2(static_cast<float>(sum), group_unscale(m, f));
}

// scale * 2^-f * (sum(q * X) - zero * sum(X)) over one half-group: the 16 code bytes cd,
// the group header hd, the half-group's 24 operand dwords xv (4 blocks) and its
// (sum(X), 2^-f). The digit sums are exact integers (v_dot4: unsigned for b0 and b1,
// signed for s2); sum(q * X) = (a0 + 256 a1) + 65536 a2 is formed in fp32.
__device__ __forceinline__ float half_group_int(const v4i &cd, unsigned hd, const unsigned (&xv)[24], float2 hs) {
    unsigned a0 = 0, a1 = 0;
    int a2 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned d = static_cast<unsigned>(cd[j]);
        const unsigned lo = d & kNibbles, hi = (d >> 4) & kNibbles;
        a0 = __builtin_amdgcn_udot4(lo, xv[6 * j + 0], a0, false);
        a0 = __builtin_amdgcn_udot4(hi, xv[6 * j + 1], a0, false);
        a1 = __builtin_amdgcn_udot4(lo, xv[6 * j + 2], a1, false);
        a1 = __builtin_amdgcn_udot4(hi, xv[6 * j + 3], a1, false);
        a2 = __builtin_amdgcn_sdot4(static_cast<int>(lo), static_cast<int>(xv[6 * j + 4]), a2, false);
        a2 = __builtin_amdgcn_sdot4(static_cast<int>(hi), static_cast<int>(xv[6 * j + 5]), a2, false);
    }
    const float V = fmaf(static_cast<float>(a2), 65536.f, static_cast<float>(a0 + a1 * 256u));
    const float sc = half_bits(hd), z = half_bits(hd >> 16);
    // 2^-f times the exact integer sum first: for tiny activations (f > 126) 2^-f is subnormal and
    // sc * 2^-f could lose its digits, while 2^-f * (...) is still a normal float; for normal
    // products both orders round once and give the same bits.
    return sc * (hs.y * fmaf(-z, hs.x, V));
}

// Rows of at most 32 half-groups (S = 0): R rows per half-wave, 2R per wave, 8R per
// workgroup. Rows of more: R per wave over S slots, kSetWaves R per workgroup.
// Sum of v over the workgroup, in double, in a fixed order (each wave by shuffles, then the
// kSetWaves wave sums in wave order).
__device__ inline double set_block_sum(double v) {
    v = xor_sum_wave(v);
    __shared__ double red[kSetWaves];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = red[0];
#pragma unroll
    for (int w = 1; w < kSetWaves; ++w) t += red[w];
    return t;
}

__device__ inline float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// ---- activation prologues ----------------------------------------------------------------
// The arithmetic the set kernel's prologues apply to each 16-byte chunk of activations, shared
// with the data-flow decode kernel so both give the same bits.

// swiglu_ref (kernels/silu/swiglu_ref.cpp): silu(g) * u.
__device__ __forceinline__ float swiglu1(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

__device__ __forceinline__ float4 swiglu4(float4 g, float4 u) {
    return make_float4(swiglu1(g.x, u.x), swiglu1(g.y, u.y), swiglu1(g.z, u.z), swiglu1(g.w, u.w));
}

// One chunk's share of rmsnorm_ref's double sum of squares (kernels/rmsnorm/rmsnorm_ref.cpp).
__device__ __forceinline__ double sq4(float4 h) {
    return static_cast<double>(h.x) * h.x + static_cast<double>(h.y) * h.y + static_cast<double>(h.z) * h.z +
           static_cast<double>(h.w) * h.w;
}

// 1 / sqrt(mean + eps) from the workgroup's double sum of squares over K elements.
__device__ __forceinline__ float rms_scale(double ss, int K, float eps) {
    const float mean_sq = static_cast<float>(ss / K);
    return 1.0f / sqrtf(mean_sq + eps);
}

// (x * scale) * w per element.
__device__ __forceinline__ float4 rms_apply(float4 x, float scale, float4 w) {
    return make_float4((x.x * scale) * w.x, (x.y * scale) * w.y, (x.z * scale) * w.z, (x.w * scale) * w.w);
}

}  // namespace
}  // namespace tqhip
