// i4_matmul.hip -- batched-prefill i4 dequant-GEMM for gfx950.
//
// Y[M,N] = W_i4[M,K] * X[K,N] with X and Y column-major (x[n*K+k], y[n*M+m]),
// the contract of the reference's matmul_i4_ref (kernels/matvec/matmul_i4_ref.cpp:53-114):
// W row m, element k dequantizes to (q - zero) * scale of its group, in fp32.
//
// MFMA path (group size a multiple of 32):
//   1. x_to_f16: every token column n of X is scaled by an exact power of two
//      2^e_n (its largest |x| lands in [2^14, 2^15)) and rounded to fp16,
//      zero-padded to a multiple of 64 along K. The scale keeps fp16 clear of
//      overflow and gives every token the full 11-bit significand; 2^-e_n is
//      applied exactly in the epilogue.
//   2. i4_matmul_mfma: workgroup tiles of BM weight rows x BN tokens, 64 K
//      elements per step. Global -> LDS DMA brings each step's raw W slice
//      (group headers + packed codes) and fp16 X slice into a ring of 2-4
//      stages, issued stages - 1 steps ahead. Each wave dequantizes its W
//      operands from the raw codes in LDS straight into registers as
//      q * scale - zero * scale with one rounding to fp16 (v_fma_mix), and
//      contracts with v_mfma_f32_32x32x16_f16 (fp32 accumulation).
//      fp16 and bf16 MFMA run at the same rate on gfx950; fp16 keeps 8x
//      finer rounding of both operands.
// Up to 32 tokens at G = 64 (16-byte aligned X, K % 4 == 0): one launch that converts X
// itself and splits K over workgroups (section 5 below).
// Other group sizes: one i4 matvec per token column.

#include "i4_lane.h"
#include "tq_common.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace tqhip {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));

constexpr int kStepK = 64;             // K elements per main-loop step
constexpr int kThreads = 256;

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void *base, size_t bytes) {
    const int nrec = bytes > 0xFFFFFFFFull ? -1 : static_cast<int>(static_cast<unsigned>(bytes));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), nrec, kBufferFlags);
}

// q * s + nzs in fp32 is exact (q has 4 bits, s and the zero 11: q * s and nzs = -zero * s
// are exact products and their sum needs at most 24 bits), so rounding it to fp16 with
// v_cvt_pk_f16_f32 (round to nearest even) rounds once, as v_fma_mix would; measured on
// MI355X v_fma_mix issues at a third to a quarter of the rate of v_fma_f32.
// (asm: left to itself the compiler folds the fp32 FMA and the conversion back into v_fma_mix)
__device__ inline unsigned pair_f16(float a, float b) {
    unsigned r;
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// ---- 1. X (fp32, column n = token) -> fp16 * 2^e_n, rows padded to Kp.
// One workgroup per token; the column is read once into registers (Kp <= 256 *
// kXRegs), its max taken, then converted and stored. Longer columns: two passes.
// PERM: within every 8 elements, element e goes to position ((e & 3) << 1) | (e >> 2), the
// k-slot order in which the packed-fp16 dequantization leaves a code dword's elements.
__device__ __forceinline__ int x_pos(int k, bool perm) {
    return perm ? (k & ~7) | ((k & 3) << 1) | ((k >> 2) & 1) : k;
}
constexpr int kXRegs = 16;
template <bool PERM>
__global__ __launch_bounds__(256) void x_to_f16(const float *__restrict__ x, int K, int Kp, _Float16 *__restrict__ xh,
                                                  float *__restrict__ xinv) {
    const int n = blockIdx.x;
    const float *xc = x + static_cast<size_t>(n) * K;
    float v[kXRegs];
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < kXRegs; ++i) {
        const int k = threadIdx.x + i * 256;
        v[i] = k < K ? xc[k] : 0.f;
        m = fmaxf(m, fabsf(v[i]));
    }
    m = xor_max_wave(m);
    __shared__ float wm[4];
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    int e = 0;
    if (m > 0.f && m <= 3.0e38f) {  // finite, nonzero: max * 2^e in [2^14, 2^15)
        int E;
        frexpf(m, &E);
        e = min(max(15 - E, -120), 120);
    }
    _Float16 *hc = xh + static_cast<size_t>(n) * Kp;
#pragma unroll
    for (int i = 0; i < kXRegs; ++i) {
        const int k = threadIdx.x + i * 256;
        if (k < Kp) hc[x_pos(k, PERM)] = static_cast<_Float16>(ldexpf(v[i], e));
    }
    if (threadIdx.x == 0) xinv[n] = ldexpf(1.f, -e);
}

// x_to_f16 for K % 4 == 0 and x 16-byte aligned: thread t takes 8-element chunks t and t + 256
// (two 16-byte loads each) and stores each chunk's 8 fp16 values, in the chunk's slot order,
// with one 16-byte store. The same exponent and the same per-element rounding as x_to_f16.
template <bool PERM>
__global__ __launch_bounds__(256) void x_to_f16_vec(const float *__restrict__ x, int K, int Kp,
                                                      _Float16 *__restrict__ xh, float *__restrict__ xinv) {
    constexpr int kChunks = kXRegs / 8;  // 8-element chunks per thread (Kp <= 256 * kXRegs)
    const int n = blockIdx.x;
    const float4 *xc = reinterpret_cast<const float4 *>(x + static_cast<size_t>(n) * K);
    float v[kChunks][8];
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int c = threadIdx.x + 256 * i;  // elements 8c .. 8c + 7
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool ok = 8 * c + 4 * h < K;  // K % 4 == 0: a float4 is all in or all out
            const float4 q = ok ? xc[2 * c + h] : make_float4(0.f, 0.f, 0.f, 0.f);
            v[i][4 * h] = q.x;
            v[i][4 * h + 1] = q.y;
            v[i][4 * h + 2] = q.z;
            v[i][4 * h + 3] = q.w;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[i][e]));
    }
    m = xor_max_wave(m);
    __shared__ float wm[4];
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    int e = 0;
    if (m > 0.f && m <= 3.0e38f) {  // finite, nonzero: max * 2^e in [2^14, 2^15)
        int E;
        frexpf(m, &E);
        e = min(max(15 - E, -120), 120);
    }
    uint4 *hc = reinterpret_cast<uint4 *>(xh + static_cast<size_t>(n) * Kp);
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int c = threadIdx.x + 256 * i;
        if (8 * c >= Kp) continue;
        unsigned short o[8];
#pragma unroll
        for (int el = 0; el < 8; ++el)
            o[x_pos(el, PERM)] = __builtin_bit_cast(unsigned short, static_cast<_Float16>(ldexpf(v[i][el], e)));
        hc[c] = make_uint4(o[0] | (static_cast<unsigned>(o[1]) << 16), o[2] | (static_cast<unsigned>(o[3]) << 16),
                           o[4] | (static_cast<unsigned>(o[5]) << 16), o[6] | (static_cast<unsigned>(o[7]) << 16));
    }
    if (threadIdx.x == 0) xinv[n] = ldexpf(1.f, -e);
}

template <bool PERM>
__global__ __launch_bounds__(256) void x_to_f16_long(const float *__restrict__ x, int K, int Kp,
                                                       _Float16 *__restrict__ xh, float *__restrict__ xinv) {
    const int n = blockIdx.x;
    const float *xc = x + static_cast<size_t>(n) * K;
    float m = 0.f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) m = fmaxf(m, fabsf(xc[k]));
    m = xor_max_wave(m);
    __shared__ float wm[4];
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    int e = 0;
    if (m > 0.f && m <= 3.0e38f) {
        int E;
        frexpf(m, &E);
        e = min(max(15 - E, -120), 120);
    }
    _Float16 *hc = xh + static_cast<size_t>(n) * Kp;
    for (int k = threadIdx.x; k < Kp; k += blockDim.x)
        hc[x_pos(k, PERM)] = static_cast<_Float16>(k < K ? ldexpf(xc[k], e) : 0.f);
    if (threadIdx.x == 0) xinv[n] = ldexpf(1.f, -e);
}

__device__ inline float half_bits_f(unsigned h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h & 0xFFFFu)));
}

// 8 consecutive elements (one code dword, low nibble first) of one group as
// the fp16 MFMA operand: q * scale - zero * scale, rounded once (within one
// fp16 rounding of the reference's fp32 (q - zero) * scale).
// Byte b of v as a float (v_cvt_f32_ubyte{b}: no separate extract).
template <int B>
__device__ inline float ubyte_f(unsigned v) {
    float f;
    if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(v));
    if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(v));
    if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(v));
    if constexpr (B == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(v));
    return f;
}

// The group's scale and -zero * scale as plain fp32 registers: the compiler would otherwise fold
// their fp16 -> fp32 conversion into every FMA as a v_fma_mix_f32 (the slow mixed-precision
// form).
__device__ inline void opaque_f32(float &s, float &nzs) { asm("" : "+v"(s), "+v"(nzs)); }

__device__ inline h8 dequant8(unsigned c, float s, float nzs) {
    const unsigned lo = c & 0x0F0F0F0Fu;         // elements 0, 2, 4, 6
    const unsigned hi = (c >> 4) & 0x0F0F0F0Fu;  // elements 1, 3, 5, 7
    u4v pk;
    pk[0] = pair_f16(fmaf(ubyte_f<0>(lo), s, nzs), fmaf(ubyte_f<0>(hi), s, nzs));
    pk[1] = pair_f16(fmaf(ubyte_f<1>(lo), s, nzs), fmaf(ubyte_f<1>(hi), s, nzs));
    pk[2] = pair_f16(fmaf(ubyte_f<2>(lo), s, nzs), fmaf(ubyte_f<2>(hi), s, nzs));
    pk[3] = pair_f16(fmaf(ubyte_f<3>(lo), s, nzs), fmaf(ubyte_f<3>(hi), s, nzs));
    return __builtin_bit_cast(h8, pk);
}

// ---- packed-fp16 dequantization (the G = 64 GEMM)
// A nibble q OR-ed into the mantissa of a fixed fp16 exponent reads as 1024 + q (bits 0..3 under
// exponent 2^10) or 64 + q (bits 4..7 under 2^6), both exact; subtracting 1024 or 64 gives q
// exactly, and fma(q, s, fp16(-z s)) rounds once. Eight elements cost 13 instructions (one shift,
// four v_and_or_b32, four v_pk_add_f16, four v_pk_fma_f16) against 23 for the fp32 form. The
// halves come out in the k-slot order (0, 4, 1, 5, 2, 6, 3, 7) of the code dword's elements, so
// X is stored in that order within every 8 elements (x_to_f16 with kPermute).
typedef _Float16 hf2 __attribute__((ext_vector_type(2)));
__device__ inline hf2 as_h2(unsigned u) { return __builtin_bit_cast(hf2, u); }
__device__ inline unsigned as_u(hf2 h) { return __builtin_bit_cast(unsigned, h); }
// (v_and_or_b32 is a VOP3 instruction: its two constants cannot both be literals, so the magic
// exponent comes in a VGPR and the mask in an SGPR)
__device__ inline unsigned and_or(unsigned c, unsigned mask, unsigned magic) {
    unsigned r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(c), "s"(mask), "v"(magic));
    return r;
}
// element e of the code dword sits at k-slot ((e & 3) << 1) | (e >> 2)
__device__ __host__ constexpr int pk_slot(int e) { return ((e & 3) << 1) | (e >> 2); }
struct PkConst {
    unsigned k64, k54;  // the two magic exponents, held in VGPRs
};
__device__ inline PkConst pk_const() {
    PkConst k{0x64006400u, 0x54005400u};
    asm volatile("" : "+v"(k.k64), "+v"(k.k54));
    return k;
}
// The group's (s, s) and (-z s, -z s) from its header dword [scale | zero].
__device__ inline void pk_header(unsigned hd, hf2 &s2, hf2 &c2) {
    s2 = as_h2(__builtin_amdgcn_perm(hd, hd, 0x01000100u));
    const hf2 z2 = as_h2(__builtin_amdgcn_perm(hd, hd, 0x03020302u));
    c2 = -(z2 * s2);
}
__device__ inline h8 dequant8_pk(unsigned c, hf2 s2, hf2 c2, PkConst k) {
    const hf2 m1024 = {static_cast<_Float16>(-1024.f), static_cast<_Float16>(-1024.f)};
    const hf2 m64 = {static_cast<_Float16>(-64.f), static_cast<_Float16>(-64.f)};
    const unsigned c8 = c >> 8;
    const hf2 q0 = as_h2(and_or(c, 0x000F000Fu, k.k64)) + m1024;   // elements 0, 4
    const hf2 q1 = as_h2(and_or(c, 0x00F000F0u, k.k54)) + m64;     // 1, 5
    const hf2 q2 = as_h2(and_or(c8, 0x000F000Fu, k.k64)) + m1024;  // 2, 6
    const hf2 q3 = as_h2(and_or(c8, 0x00F000F0u, k.k54)) + m64;    // 3, 7
    u4v pk;
    pk[0] = as_u(__builtin_elementwise_fma(q0, s2, c2));
    pk[1] = as_u(__builtin_elementwise_fma(q1, s2, c2));
    pk[2] = as_u(__builtin_elementwise_fma(q2, s2, c2));
    pk[3] = as_u(__builtin_elementwise_fma(q3, s2, c2));
    return __builtin_bit_cast(h8, pk);
}

// s_waitcnt vmcnt(n), expcnt / lgkmcnt untouched (gfx9 encoding). The count assumes the loads
// issued before it in program order: the sched_barriers keep the machine scheduler from
// moving a load across it (scheduling groups would otherwise carry a step's interleaved loads
// past the next step's wait, and vmcnt(n) would then let that step's own loads still be in
// flight).
__device__ __forceinline__ void wait_vm(int n) {
    __builtin_amdgcn_sched_barrier(0);
    switch (n) {
#define TQ_VMWAIT(N) case N: __builtin_amdgcn_s_waitcnt(((N) & 15) | (7 << 4) | (15 << 8) | (((N) >> 4) << 14)); break;
        TQ_VMWAIT(0) TQ_VMWAIT(1) TQ_VMWAIT(2) TQ_VMWAIT(3) TQ_VMWAIT(4) TQ_VMWAIT(5) TQ_VMWAIT(6) TQ_VMWAIT(7)
        TQ_VMWAIT(8) TQ_VMWAIT(9) TQ_VMWAIT(10) TQ_VMWAIT(11) TQ_VMWAIT(12) TQ_VMWAIT(13) TQ_VMWAIT(14)
        TQ_VMWAIT(15) TQ_VMWAIT(16) TQ_VMWAIT(17) TQ_VMWAIT(18) TQ_VMWAIT(19) TQ_VMWAIT(20) TQ_VMWAIT(21)
        TQ_VMWAIT(22) TQ_VMWAIT(23) TQ_VMWAIT(24) TQ_VMWAIT(25) TQ_VMWAIT(26) TQ_VMWAIT(27) TQ_VMWAIT(28)
        TQ_VMWAIT(32)
#undef TQ_VMWAIT
        default: __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); break;
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Workgroup barrier that waits for this wave's LDS operations only (global ->
// LDS transfers of later steps stay in flight). The sched_barriers keep the machine
// scheduler from moving anything across it (a memory clobber binds only the compiler's
// IR passes: scheduling groups would otherwise hoist the step's LDS reads above it).
__device__ inline void lds_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

constexpr int kWDwords = 10;                    // per row and step
constexpr int kWStage1 = 128 * kWDwords * 4;    // bytes of W per step and 128 rows
constexpr int kWDma1 = 128 * kWDwords / 64 / 4; // dword DMAs per wave per step and 128 rows (= 5)

// Byte offsets, within a row, of one step's W data: per 32-element half t the
// group header and the first of its 16 code bytes (each half lies in one group
// as G % 32 == 0). Uniform across the workgroup (scalar arithmetic).
struct StepOffsets {
    int hdr[2], code[2];
    bool valid[2];
};
template <int GT>
__device__ __forceinline__ StepOffsets step_offsets(int s, int Grt, int gb, int groups) {
    const int G = GT ? GT : Grt;  // a compile-time group size turns the divisions into shifts
    StepOffsets o;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int k = s * kStepK + 32 * t;
        const int g = k / G;
        o.valid[t] = g < groups;
        const int gc = min(g, groups - 1);  // past the last group: any valid bytes, masked later
        o.hdr[t] = gc * gb;
        o.code[t] = gc * gb + 4 + (k - gc * G) / 2;
    }
    return o;
}

// One step's global -> LDS DMAs of one wave (nw dword DMAs of W, nx 16-byte
// DMAs of X, the X part starting xbase bytes into the stage); every lane of
// every DMA is live, so the count per wave and step is fixed. Per lane only a
// select and an add depend on the step. (Not a lambda in the kernel: HIP
// compiles those for the host too, where the DMA builtin does not exist.)
__device__ __forceinline__ void issue_step(__amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t xr, unsigned char *st,
                                           const int *wrow, const int *wsel, int nw, const int *xoff, int nx,
                                           int xbase, int wave, int s, const StepOffsets &o) {
#pragma unroll
    for (int q = 0; q < nw; ++q) {
        // wsel: slot 0/1 -> header of half 0/1; slot 2+4t+i -> code dword i of half t
        const int sl = wsel[q];
        const int t = sl < 2 ? sl : (sl - 2) >> 2;
        const int base = sl < 2 ? (t ? o.hdr[1] : o.hdr[0]) : (t ? o.code[1] : o.code[0]) + 4 * ((sl - 2) & 3);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            wr, (__attribute__((address_space(3))) void *)(st + 256 * (wave * nw + q)), 4, wrow[q] + base, 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < nx; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xr, (__attribute__((address_space(3))) void *)(st + xbase + 1024 * (wave * nx + q)), 16,
            xoff[q] + s * kStepK * 2, 0, 0, 0);
}

// ---- 2. MFMA tile kernel
//   4 waves; wave w owns weight rows 32*WM*w .. +32*WM of the workgroup's
//   BM = 128 * WM and all BN = 32 * WN tokens. Per 64-element K step,
//   global -> LDS DMA brings
//     W: per row 10 dwords [header of half 0, header of half 1, 8 code dwords]
//        (each 32-element half lies in one group as G % 32 == 0);
//     X: BN rows x 128 B of fp16, 16-byte chunks XOR-swizzled by row (c ^ (r & 7))
//   into a ring of S stages issued S - 1 steps ahead. Each wave dequantizes its
//   A operands from the raw codes in LDS straight into registers; every X (B)
//   operand read from LDS feeds WM MFMAs.
template <int WM, int WN, int GT>
__global__ __launch_bounds__(kThreads) void i4_matmul_mfma(const uint8_t *__restrict__ w,
                                                           const _Float16 *__restrict__ xh,
                                                           const float *__restrict__ xinv, float *__restrict__ y,
                                                           int M, int N, int K, int Kp, int G, int row_bytes, int S) {
    constexpr int BM = 128 * WM;
    constexpr int BN = 32 * WN;
    constexpr int WStage = kWStage1 * WM;
    constexpr int WDma = kWDma1 * WM;
    constexpr int XStage = BN * 128;
    constexpr int P = WDma + WN;  // DMAs per wave per step
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    if constexpr (GT != 0) G = GT;
    const int gb = 4 + G / 2;
    const int groups = (K + G - 1) / G;
    const int steps = Kp / kStepK;
    const int stage_bytes = WStage + XStage;

    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + static_cast<size_t>(m0) * row_bytes,
                                                static_cast<size_t>(M - m0) * row_bytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(xh + static_cast<size_t>(n0) * Kp,
                                                static_cast<size_t>(N - n0) * Kp * 2);

    // this wave's W DMAs: dword d = 64 * (wave * WDma + q) + lane of the stage
    int wrow[WDma], wslot[WDma];
#pragma unroll
    for (int q = 0; q < WDma; ++q) {
        const int d = 64 * (wave * WDma + q) + lane;
        wrow[q] = (d / kWDwords) * row_bytes;
        wslot[q] = d % kWDwords;
    }
    // this wave's X DMAs: 16-byte position p = 64 * (wave * WN + q) + lane
    int xoff[WN];
#pragma unroll
    for (int q = 0; q < WN; ++q) {
        const int p = 64 * (wave * WN + q) + lane;
        const int r = p >> 3, c = (p & 7) ^ (r & 7);
        xoff[q] = r * Kp * 2 + 16 * c;
    }
    auto issue = [&](int s, int slot) {
        issue_step(wr, xr, smem + slot * stage_bytes, wrow, wslot, WDma, xoff, WN, WStage, wave, s,
                   step_offsets<GT>(s, G, gb, groups));
    };

    f16x acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = f16x{};

    const int li = lane & 31, kq = lane >> 5;
    int issued = 0;
    for (; issued < S - 1 && issued < steps; ++issued) issue(issued, issued);
    int slot = 0, islot = issued == S ? 0 : issued;  // ring slots of step s and of the next issue
    for (int s = 0; s < steps; ++s) {
        wait_vm((issued - s - 1) * P);  // this wave's part of step s has landed
        lds_barrier();                  // every wave's part has; step s - 1's slot is free
        if (issued < steps) {
            issue(issued, islot);
            ++issued;
            islot = islot == S - 1 ? 0 : islot + 1;
        }
        const unsigned char *st = smem + slot * stage_bytes;
        const StepOffsets so = step_offsets<GT>(s, G, gb, groups);
        // all of the step's LDS operands first, so their latencies overlap
        unsigned hd[WM][2], c[WM][4];
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const unsigned *wrw = reinterpret_cast<const unsigned *>(st) + (32 * (WM * wave + i) + li) * kWDwords;
            hd[i][0] = wrw[0];
            hd[i][1] = wrw[1];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) c[i][kk] = wrw[2 + 2 * kk + kq];
        }
        const unsigned char *sx = st + WStage;
        h8 b[4][WN];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int r = 32 * j + li;
                b[kk][j] = *reinterpret_cast<const h8 *>(sx + r * 128 + 16 * ((2 * kk + kq) ^ (r & 7)));
            }
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const float s0 = so.valid[0] ? half_bits_f(hd[i][0]) : 0.f;
            const float s1 = so.valid[1] ? half_bits_f(hd[i][1]) : 0.f;
            const float z0 = so.valid[0] ? -(half_bits_f(hd[i][0] >> 16) * s0) : 0.f;
            const float z1 = so.valid[1] ? -(half_bits_f(hd[i][1] >> 16) * s1) : 0.f;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const h8 a = kk < 2 ? dequant8(c[i][kk], s0, z0) : dequant8(c[i][kk], s1, z1);
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b[kk][j], acc[i][j], 0, 0, 0);
            }
        }
        slot = slot == S - 1 ? 0 : slot + 1;
    }
    wait_vm(0);

    // epilogue: lane holds rows (r/4)*8 + (lane/32)*4 + r%4 of column lane%32
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        const int n = n0 + 32 * j + li;
        if (n >= N) continue;
        const float sc = xinv[n];
        float *yc = y + static_cast<size_t>(n) * M;
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int m = m0 + 32 * (WM * wave + i) + 8 * r4 + 4 * kq;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (m + q < M) yc[m + q] = acc[i][j][4 * r4 + q] * sc;
            }
    }
}

// ---- 3. MFMA tile kernel, slot-major staging
//   The same tile, dequantization and MFMA as i4_matmul_mfma, with the per-step
//   overhead taken out of the loop:
//   - W is staged slot-major, [10 slots][128 rows] dwords (slot 0/1: group
//     header of half 0/1 of the step; slot 2 + 4t + i: code dword i of half t).
//     One DMA instruction moves one slot of 64 rows: its per-lane source is
//     row * row_bytes, fixed for the whole loop, and the step enters only
//     through the scalar offset of the slot (SALU), so no per-lane selects.
//     Reading a slot back, 32 consecutive lanes read 32 consecutive dwords.
//   - X rows are 128 B; 16-byte chunk c of token row r is stored at position
//     c ^ ((r >> 1) & 7). A ds_read_b128 is served 16 lanes at a time, one
//     256-byte bank sweep: the 16 rows a group reads differ in (r & 1, chunk),
//     so they cover the sweep once (no bank conflicts).
//   - Every step issues the same DMAs, also past the last step (reads past a
//     row or the end of the buffer land in a slot that is never consumed), so
//     the wait before each step is one constant s_waitcnt.
constexpr int kWSlots = 10;
constexpr int kBM = 128;

// Byte offset within a row of the step-s dword of W slot `slot` (scalar).
template <int GT>
__device__ __forceinline__ int w_slot_offset(int slot, int s, int G, int gb, int groups) {
    const int t = slot < 2 ? slot : (slot - 2) >> 2;
    const int k = s * kStepK + 32 * t;
    const int g = min(k / (GT ? GT : G), groups - 1);  // past the last group: in-row bytes, masked later
    const int base = g * gb;
    return slot < 2 ? base : base + 4 + (k - g * (GT ? GT : G)) / 2 + 4 * ((slot - 2) & 3);
}

// One step's DMAs of one wave: 5 W slot DMAs (instruction i = 5 * wave + q:
// slot i >> 1, rows 64 (i & 1) + lane) and nx X DMAs of 16 bytes per lane.
// (Not a template and not a lambda: the DMA builtin exists for the device only.)
__device__ __forceinline__ void issue_step2(__amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t xr, unsigned char *st,
                                            const int *wvo, const int *wso, const int *xvo, int nx, int xso,
                                            int wstage, int wave) {
#pragma unroll
    for (int q = 0; q < 5; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            wr, (__attribute__((address_space(3))) void *)(st + 256 * (5 * wave + q)), 4, wvo[q], wso[q], 0, 0);
#pragma unroll
    for (int q = 0; q < nx; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xr, (__attribute__((address_space(3))) void *)(st + wstage + 1024 * (nx * wave + q)), 16, xvo[q], xso, 0,
            0);
}

template <int WN, int GT, int S>
__global__ __launch_bounds__(kThreads) void i4_matmul_mfma2(const uint8_t *__restrict__ w,
                                                            const _Float16 *__restrict__ xh,
                                                            const float *__restrict__ xinv, float *__restrict__ y,
                                                            int M, int N, int K, int Kp, int G, int row_bytes) {
    constexpr int BN = 32 * WN;
    constexpr int WStage = kWSlots * kBM * 4;
    constexpr int StageBytes = WStage + BN * 128;
    constexpr int P = 5 + WN;  // DMAs per wave per step
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m0 = blockIdx.x * kBM, n0 = blockIdx.y * BN;
    if constexpr (GT != 0) G = GT;
    const int gb = 4 + G / 2;
    const int groups = (K + G - 1) / G;
    const int steps = Kp / kStepK;

    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + static_cast<size_t>(m0) * row_bytes,
                                                static_cast<size_t>(M - m0) * row_bytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(xh + static_cast<size_t>(n0) * Kp,
                                                static_cast<size_t>(N - n0) * Kp * 2);
    int wvo[5], wslot[5];
#pragma unroll
    for (int q = 0; q < 5; ++q) {
        const int i = 5 * wave + q;
        wslot[q] = i >> 1;
        wvo[q] = (64 * (i & 1) + lane) * row_bytes;
    }
    int xvo[WN];
#pragma unroll
    for (int q = 0; q < WN; ++q) {
        const int p = 64 * (WN * wave + q) + lane;
        const int r = p >> 3, c = (p & 7) ^ ((r >> 1) & 7);
        xvo[q] = r * Kp * 2 + 16 * c;
    }
    // G = 64: both halves of step s lie in group s, so a slot's offset is
    // 36 * s plus a constant of the slot
    int wconst[5];
#pragma unroll
    for (int q = 0; q < 5; ++q) wconst[q] = w_slot_offset<GT>(wslot[q], 0, G, gb, groups);
    auto issue = [&](int s) {
        int wso[5];
        if constexpr (GT == 64) {
            const int base = gb * min(s, groups - 1);
#pragma unroll
            for (int q = 0; q < 5; ++q) wso[q] = base + wconst[q];
        } else {
#pragma unroll
            for (int q = 0; q < 5; ++q) wso[q] = w_slot_offset<GT>(wslot[q], s, G, gb, groups);
        }
        issue_step2(wr, xr, smem + (s % S) * StageBytes, wvo, wso, xvo, WN, s * kStepK * 2, WStage, wave);
    };

    f16x acc[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[j] = f16x{};
    const int li = lane & 31, kq = lane >> 5;
    const int row = 32 * wave + li;
    // LDS read offsets within a stage (bytes)
    int xro[4][WN];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int r = 32 * j + li;
            xro[kk][j] = WStage + 16 * (8 * r + ((2 * kk + kq) ^ ((r >> 1) & 7)));
        }

#pragma unroll
    for (int s = 0; s < S - 1; ++s) issue(s);
    for (int s = 0; s < steps; ++s) {
        wait_vm((S - 2) * P);  // this wave's part of step s has landed
        lds_barrier();         // every wave's part has; step s - 1's slot is free
        issue(s + S - 1);      // (past the last step: never consumed)
        const unsigned char *st = smem + (s % S) * StageBytes;
        const unsigned *ws = reinterpret_cast<const unsigned *>(st);
        const unsigned hd0 = ws[row], hd1 = ws[kBM + row];
        unsigned c[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) c[kk] = ws[(2 + 4 * (kk >> 1) + 2 * (kk & 1) + kq) * kBM + row];
        h8 b[4][WN];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int j = 0; j < WN; ++j) b[kk][j] = *reinterpret_cast<const h8 *>(st + xro[kk][j]);
        const bool v0 = (s * kStepK) / G < groups, v1 = (s * kStepK + 32) / G < groups;
        const float s0 = v0 ? half_bits_f(hd0) : 0.f;
        const float s1 = v1 ? half_bits_f(hd1) : 0.f;
        const float z0 = v0 ? -(half_bits_f(hd0 >> 16) * s0) : 0.f;
        const float z1 = v1 ? -(half_bits_f(hd1 >> 16) * s1) : 0.f;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const h8 a = kk < 2 ? dequant8(c[kk], s0, z0) : dequant8(c[kk], s1, z1);
#pragma unroll
            for (int j = 0; j < WN; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b[kk][j], acc[j], 0, 0, 0);
        }
    }
    wait_vm(0);

    // epilogue: lane holds rows (r/4)*8 + (lane/32)*4 + r%4 of column lane%32
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        const int n = n0 + 32 * j + li;
        if (n >= N) continue;
        const float sc = xinv[n];
        float *yc = y + static_cast<size_t>(n) * M;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int m = m0 + 32 * wave + 8 * r4 + 4 * kq;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (m + q < M) yc[m + q] = acc[j][4 * r4 + q] * sc;
        }
    }
}

// ---- 4. G = 64: W straight into registers
//   At G = 64 a step's 64 elements of a row are one group: 36 contiguous bytes
//   [scale | zero | 32 code bytes] at 36 s. Lane (row, half h) loads the group
//   header and the 16 code bytes of its half into VGPRs, S - 1 steps ahead, so W
//   never passes through LDS (measured: the dword-granular W staging of
//   i4_matmul_mfma2 was 40% of its time). X is staged as in i4_matmul_mfma2.
//   The loop is unrolled by S so that every register slot index is a
//   constant; steps past the last are loaded (never consumed) and not
//   computed, which keeps every wait one constant s_waitcnt.
//   The A operands are dequantized with packed fp16 arithmetic (dequant8_pk), which
//   leaves a code dword's elements in k-slot order (0, 4, 1, 5, 2, 6, 3, 7); X comes
//   from x_to_f16<true> in the same order, so both operands agree slot for slot.
//   Y leaves in 16-byte stores (4 rows of a token) where M % 4 == 0 and y is 16-byte
//   aligned: four times fewer store instructions than one float each, which took
//   the 512-token call from 48 to 39 us on MI355X (the output is 20 MB there).
//   Measured on MI355X at 512 tokens with copies of this kernel that skip parts of
//   the work: without the MFMAs or without the dequantization the time hardly
//   changes; without the loads of W and X it drops by three quarters. The loop is
//   bound by the time each workgroup's loads take to arrive, not by arithmetic.
// The X DMAs d0 .. d0 + nx - 1 of a step (1 KB each, at byte 1024 d of the stage); nx <= ND.
template <int ND>
__device__ __forceinline__ void issue_x(__amdgpu_buffer_rsrc_t xr, unsigned char *st, const int *xvo, int nx, int d0,
                                        int xso) {
#pragma unroll
    for (int q = 0; q < ND; ++q)
        if (q < nx)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void *)(st + 1024 * (d0 + q)), 16, xvo[q], xso, 0, 0);
}

template <int WN, int S, int NWV>
__global__ __launch_bounds__(64 * NWV) void i4_matmul_g64(const uint8_t *__restrict__ w,
                                                          const _Float16 *__restrict__ xh,
                                                          const float *__restrict__ xinv, float *__restrict__ y, int M,
                                                          int N, int K, int Kp, int row_bytes, int vec_y) {
    constexpr int BN = 32 * WN;
    constexpr int BM = 32 * NWV;
    constexpr int XStage = BN * 128;
    // The step's 4 WN X DMAs (1 KB each) are dealt out in order: waves below XR issue XA + 1 of
    // them, the others XA. P: this wave's loads per step (W 4 + 16 bytes, its X DMAs).
    constexpr int XA = 4 * WN / NWV, XR = 4 * WN % NWV;
    constexpr int XD = XA + (XR ? 1 : 0);
    constexpr int kGroupBytes = 36;
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    const int groups = (K + 63) / 64;
    const int steps = Kp / kStepK;  // = groups

    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + static_cast<size_t>(m0) * row_bytes,
                                                static_cast<size_t>(M - m0) * row_bytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(xh + static_cast<size_t>(n0) * Kp,
                                                static_cast<size_t>(N - n0) * Kp * 2);
    // Lane (row li, half h) takes elements 32 h .. 32 h + 31 of every step: the group header
    // and code bytes 16 h .. 16 h + 15; MFMA k-slot 8 h + p of k-block kk holds element
    // 32 h + 8 kk + e, p = pk_slot(e), on the A (W) and the B (X) side.
    const int li = lane & 31, h = lane >> 5;
    const int wvo = (32 * wave + li) * row_bytes;
    const int nx = XA + (wave < XR ? 1 : 0), d0 = XA * wave + min(wave, XR);
    int xvo[XD > 0 ? XD : 1];
#pragma unroll
    for (int q = 0; q < XD; ++q) {
        const int p = 64 * min(d0 + q, 4 * WN - 1) + lane;
        const int r = p >> 3, c = (p & 7) ^ ((r >> 1) & 7);
        xvo[q] = r * Kp * 2 + 16 * c;
    }
    int xro[4][WN];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int r = 32 * j + li;
            xro[kk][j] = 16 * (8 * r + ((4 * h + kk) ^ ((r >> 1) & 7)));
        }

    const PkConst pkc = pk_const();
    unsigned hd[S];
    u4v cd[S];
    auto issue = [&](auto uc, int s) {  // step s into register slot and X stage u = s % S
        constexpr int u = decltype(uc)::value;
        const int so = kGroupBytes * min(s, groups - 1);  // (past the last step: in-row bytes, never used)
        hd[u] = __builtin_amdgcn_raw_buffer_load_b32(wr, wvo, so, 0);
        cd[u] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(wr, wvo + 4 + 16 * h, so, 0));
        issue_x<XD>(xr, smem + u * XStage, xvo, nx, d0, s * kStepK * 2);
    };
    f16x acc[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[j] = f16x{};
    // k-blocks k0 .. k1 - 1 of the step in register slot and X stage u
    auto compute = [&](auto uc, int k0, int k1) {
        constexpr int u = decltype(uc)::value;
        const unsigned char *st = smem + u * XStage;
        hf2 s2, c2;
        pk_header(hd[u], s2, c2);
#pragma unroll
        for (int kk = k0; kk < k1; ++kk) {
            h8 b[WN];
#pragma unroll
            for (int j = 0; j < WN; ++j) b[j] = *reinterpret_cast<const h8 *>(st + xro[kk][j]);
            const h8 a = dequant8_pk(cd[u][kk], s2, c2, pkc);
#pragma unroll
            for (int j = 0; j < WN; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b[j], acc[j], 0, 0, 0);
        }
    };
    // full: the step is below `steps`. Its loads of step s + S - 1 go in between the first and
    // the last two k-blocks' MFMAs (program order; no branch), so that a wave stalled on a full
    // memory pipeline has MFMAs in flight.
    auto round_step = [&](auto uc, int s, auto full) {
        constexpr int u = decltype(uc)::value;
        if (XR == 0 || wave < XR)  // this wave's loads of step s have landed
            wait_vm((S - 2) * (2 + XD));
        else
            wait_vm((S - 2) * (2 + XA));
        lds_barrier();  // every wave's X part has; step s - 1's stage is free
        if constexpr (decltype(full)::value) {
            compute(uc, 0, 2);
            issue(std::integral_constant<int, (u + S - 1) % S>{}, s + S - 1);
            compute(uc, 2, 4);
        } else {
            issue(std::integral_constant<int, (u + S - 1) % S>{}, s + S - 1);
            if (s < steps) compute(uc, 0, 4);
        }
    };

    issue(std::integral_constant<int, 0>{}, 0);
    if constexpr (S > 2) issue(std::integral_constant<int, 1>{}, 1);
    if constexpr (S > 3) issue(std::integral_constant<int, 2>{}, 2);
    static_assert(S >= 2 && S <= 4, "register slots 0..3");
    const std::true_type full;
    const std::false_type tail;
    int s0 = 0;
    for (; s0 + S <= steps; s0 += S) {
        round_step(std::integral_constant<int, 0>{}, s0, full);
        round_step(std::integral_constant<int, 1>{}, s0 + 1, full);
        if constexpr (S > 2) round_step(std::integral_constant<int, 2>{}, s0 + 2, full);
        if constexpr (S > 3) round_step(std::integral_constant<int, 3>{}, s0 + 3, full);
    }
    if (s0 < steps) {
        round_step(std::integral_constant<int, 0>{}, s0, tail);
        round_step(std::integral_constant<int, 1>{}, s0 + 1, tail);
        if constexpr (S > 2) round_step(std::integral_constant<int, 2>{}, s0 + 2, tail);
        if constexpr (S > 3) round_step(std::integral_constant<int, 3>{}, s0 + 3, tail);
    }
    wait_vm(0);

    // epilogue: lane holds rows (r/4)*8 + (lane/32)*4 + r%4 of column lane%32
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        const int n = n0 + 32 * j + li;
        if (n >= N) continue;
        const float sc = xinv[n];
        float *yc = y + static_cast<size_t>(n) * M;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int m = m0 + 32 * wave + 8 * r4 + 4 * h;
            if (vec_y && m + 3 < M) {
                *reinterpret_cast<float4 *>(yc + m) = make_float4(acc[j][4 * r4] * sc, acc[j][4 * r4 + 1] * sc,
                                                                  acc[j][4 * r4 + 2] * sc, acc[j][4 * r4 + 3] * sc);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (m + q < M) yc[m + q] = acc[j][4 * r4 + q] * sc;
            }
        }
    }
}

// ---- 5. Few tokens (N <= 32, G = 64): one launch
//   A kernel launch costs a few microseconds on this GPU whatever it does, so at a few
//   tokens a separate X conversion pass would cost as much as the GEMM. Here every
//   workgroup converts the X it needs itself. The grid is (128-row tile) x (K slice):
//   workgroup (tile, ks) forms the partial product of its 128 rows over the slice's
//   steps for all tokens; the last workgroup of a tile to finish adds the KS partials in
//   slice order (fixed, whatever the arrival order) and stores Y. One CU reads only some
//   50-90 GB/s from L2, so the fp32 X of a whole row of K per workgroup would take
//   several microseconds: the slices spread it over the CUs.
//   - X: the slice of the 32 token rows is read once (fp32, 16-byte loads), scaled per
//     token by the power of two that puts the token's largest |x| in the slice into
//     [2^13, 2^14), and stored to LDS as fp16, [step][token][64 elements] with the
//     16-byte chunks of token n at positions c ^ ((n >> 1) & 7): the 16 rows a
//     ds_read_b128 pass serves cover one 256-byte bank sweep exactly (rows n and n + 8 on
//     the same chunk, as c ^ (n & 7) had them, share banks). Within a chunk the 8 elements
//     are in the k-slot order of the packed-fp16 dequantization (dequant8_pk).
//   - W: each row's slice (9 dwords a step, contiguous) comes in with one DMA into LDS at
//     an odd dword pitch. (A load per lane and row touches a cache line per lane; the
//     DMA touches the 2-3 lines the slice spans.) Wave w then takes rows 32 w .. 32 w + 31:
//     lane (row r, half h) reads the group header and code dwords 1 + 4 h .. 4 + 4 h of each
//     step, so MFMA k-slot 8 h + p of k-block j holds element 32 h + 8 j + p of the step,
//     on the A (W) and on the B (X) side.
//   - Partials: [tile][slice][4 waves x 4 float4 x 64 lanes] fp32 (the MFMA's register
//     order: every store and load instruction moves 1 KB in one piece), written at device
//     scope. The slices of a tile are 8 workgroups apart and workgroups are dealt to the 8
//     XCDs in turn, so a tile normally stays on one XCD and the last arrival reads the
//     other partials from that XCD's L2; the arrival counter (zero between launches: the
//     last arrival resets it) carries each writer's XCD, so a partial written elsewhere is
//     read at device scope instead.
constexpr int kSkRows = 128;
constexpr int kDeviceScope = 16;  // buffer cache policy: sc1 (device-scope coherent)
constexpr int kL1Bypass = 1;      // buffer cache policy: sc0 (misses in the CU's L1, served by the XCD's L2)
constexpr int kSkXccSlots = 14;   // slices whose writer's XCD the arrival counter carries
constexpr int kSkReduceBatch = 6; // partials the last arrival has in flight at once
typedef float f4v __attribute__((ext_vector_type(4)));
constexpr int kSkTile = kSkRows * 32;  // floats of one partial
constexpr int kSkMaxSteps = 7;  // a row's slice (9 dwords a step) within one 64-lane DMA

template <int SMAX>
__global__ __launch_bounds__(256) void i4_matmul_skinny(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                        float *__restrict__ y, int M, int K, int N, int row_bytes,
                                                        int T, int KS, float *__restrict__ part,
                                                        unsigned long long *__restrict__ arrivals, int vec_y) {
    __shared__ __align__(16) unsigned char xs[SMAX * 4096];
    __shared__ __align__(16) unsigned char ws_lds[kSkRows * (9 * SMAX + 1) * 4];
    __shared__ float inv_s[32];
    __shared__ int last_s;
    __shared__ unsigned long long writers_s;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // workgroup b -> tile 8 (b / (8 KS)) + b % 8, slice (b / 8) % KS: the slices of a tile are
    // 8 workgroups apart, so with workgroups dealt to the 8 XCDs in turn they share one XCD
    const int tile = (blockIdx.x / (8 * KS)) * 8 + (blockIdx.x & 7), ks = (blockIdx.x >> 3) % KS;
    const int m0 = tile * kSkRows;
    if (m0 >= M) return;  // a padding tile (the tile count rounded up to 8)
    const int s0 = (ks * T) / KS, ns = ((ks + 1) * T) / KS - s0;  // steps [s0, s0 + ns), 1 <= ns <= SMAX

    // 1. X: thread t takes token n = t / 8 and float4s (t % 8) + 8 q of the token's slice
    const int n = threadIdx.x >> 3, sub = threadIdx.x & 7;
    const int k0 = 64 * s0;
    const float4 *xr = reinterpret_cast<const float4 *>(x + static_cast<size_t>(n < N ? n : 0) * K + k0);
    float4 xv[2 * SMAX];
    unsigned okm = 0;  // bit q: float4 q lies in the matrix (masked to zero after the loads land)
#pragma unroll
    for (int q = 0; q < 2 * SMAX; ++q) {
        const int f = sub + 8 * q;
        const bool ok = n < N && q < 2 * ns && k0 + 4 * f < K;  // K % 4 == 0: a float4 is all in or all out
        okm |= static_cast<unsigned>(ok) << q;
        xv[q] = xr[ok ? f : 0];
    }
    // (the X loads stay ahead of the W DMAs in the instruction stream: step 3 counts on it)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // 2. W: the slice of each of the tile's 128 rows is 9 ns contiguous dwords; one DMA per row
    //    (wave w: rows 32 w .. 32 w + 31, lane i: dword i) lands it at LDS dword r * P, with
    //    the odd pitch P = 9 ns | 1, so the 32 rows a wave reads in step j (dword r P + 9 j + c)
    //    fall in 32 different banks
    const int P = (9 * ns) | 1;
    const int li = lane & 31, h = lane >> 5;
    if (lane < 9 * ns) {  // only the slice's lanes: a DMA lane writes LDS dword (base + lane), and
                          // lanes past 9 ns would land in the next row's dwords
        const __amdgpu_buffer_rsrc_t wr = rows_rsrc(w, M, row_bytes, m0);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int r = 32 * wave + i;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                wr, (__attribute__((address_space(3))) void *)(ws_lds + 4 * r * P), 4, r * row_bytes + 4 * lane,
                36 * s0, 0, 0);
        }
    }

    // 3. the slice's X to fp16 in LDS, scaled per token, while the W rows are in flight: the
    //    wave's 32 row DMAs were issued after its X loads, so vmcnt(32) is the X loads alone
    static_assert(kSkRows / 4 == 32, "32 row DMAs per wave");
    wait_vm(32);
#pragma unroll
    for (int q = 0; q < 2 * SMAX; ++q) {
        const bool ok = (okm >> q) & 1u;
        xv[q].x = ok ? xv[q].x : 0.f;
        xv[q].y = ok ? xv[q].y : 0.f;
        xv[q].z = ok ? xv[q].z : 0.f;
        xv[q].w = ok ? xv[q].w : 0.f;
    }
    float m = 0.f;
#pragma unroll
    for (int q = 0; q < 2 * SMAX; ++q)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[q].x), fabsf(xv[q].y)), fmaxf(fabsf(xv[q].z), fabsf(xv[q].w))));
    m = fmaxf(m, dpp_f<kDppXor1>(m));
    m = fmaxf(m, dpp_f<kDppXor2>(m));
    m = fmaxf(m, dpp_f<kDppHalfMirror>(m));  // the 8 lanes of token n
    int e = 0;  // zero or non-finite: unscaled (inf and NaN carry through)
    if (m > 0.f && m <= 3.0e38f) e = min(14 - __builtin_amdgcn_frexp_expf(m), 126);
    const float sc = ldexpf(1.f, e);
    if (sub == 0) inv_s[n] = ldexpf(1.f, -e);
    // Within each 8 elements the chunk holds them in the packed dequantization's k-slot order
    // (0, 4, 1, 5, 2, 6, 3, 7): the even thread of a pair (elements 0..3 of the 8) takes 4, 5
    // from the odd one and writes slots 0..3; the odd thread takes 2, 3 and writes slots 4..7.
    const bool odd = sub & 1;
#pragma unroll
    for (int q = 0; q < 2 * SMAX; ++q) {
        const int c = (sub >> 1) + 4 * (q & 1);  // 16-byte chunk of step q / 2
        const float a0 = xv[q].x * sc, a1 = xv[q].y * sc, a2 = xv[q].z * sc, a3 = xv[q].w * sc;  // exact scaling
        const float r0 = dpp_f<kDppXor1>(odd ? a0 : a2), r1 = dpp_f<kDppXor1>(odd ? a1 : a3);
        uint2 pk;
        pk.x = odd ? pair_f16(r0, a2) : pair_f16(a0, r0);  // one rounding each
        pk.y = odd ? pair_f16(r1, a3) : pair_f16(a1, r1);
        *reinterpret_cast<uint2 *>(xs + 4096 * (q >> 1) + 128 * n + 16 * (c ^ ((n >> 1) & 7)) + 8 * (sub & 1)) = pk;
    }
    wait_vm(0);  // this wave's W rows have landed in LDS
    lds_barrier();

    // 4. the slice's steps: lane (row 32 w + li, half h) takes the header and code dwords
    //    1 + 4 h .. 4 + 4 h of the step's group
    const PkConst pkc = pk_const();
    f16x acc = {};
    const unsigned *wl = reinterpret_cast<const unsigned *>(ws_lds) + (32 * wave + li) * P;
#pragma unroll
    for (int j = 0; j < SMAX; ++j) {
        if (j < ns) {
            const unsigned hd = wl[9 * j];
            unsigned cd[4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) cd[kk] = wl[9 * j + 1 + 4 * h + kk];
            hf2 s2, c2;
            pk_header(hd, s2, c2);
            h8 b[4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                b[kk] = *reinterpret_cast<const h8 *>(xs + 4096 * j + 128 * li + 16 * ((4 * h + kk) ^ ((li >> 1) & 7)));
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(dequant8_pk(cd[kk], s2, c2, pkc), b[kk], acc, 0, 0, 0);
        }
    }

    // 5. the partial, stored as the MFMA leaves it: float4 r4 of lane l of wave w at index
    //    (4 w + r4) * 64 + l (rows 32 w + 8 r4 + 4 h + 0..3 of token l % 32, h = l / 32), so
    //    every store and load instruction moves 1 KB in one piece. Partials are stored at
    //    device scope (sc1: written through this XCD's L2 to the level where all XCDs meet),
    //    so a store that has completed is visible everywhere and the counter needs no cache
    //    write-back or invalidation (both act on a whole L2). The counter add carries the
    //    writer's XCD (slices < kSkXccSlots): the last arrival reads a partial written on its
    //    own XCD from that L2 (which the write went through) and any other one at device
    //    scope (its own L2 may hold an older copy of the line).
    const float iv = inv_s[li];
    const int xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 7;  // HW_REG_XCC_ID bits 0..3
    f4v own[4];
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
        own[r4] = f4v{acc[4 * r4] * iv, acc[4 * r4 + 1] * iv, acc[4 * r4 + 2] * iv, acc[4 * r4 + 3] * iv};
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(part + static_cast<size_t>(tile) * KS * kSkTile,
                                                static_cast<size_t>(KS) * kSkTile * sizeof(float));
    const int lo = 16 * (256 * wave + lane);  // byte offset of the lane's float4 r4 = 0 in a partial
    if (KS > 1) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, own[r4]), pr,
                                                   lo + 4 * (ks * kSkTile) + 1024 * r4, 0, kDeviceScope);
        wait_vm(0);       // this wave's partial stores have completed
        __syncthreads();  // and every other wave's
        if (threadIdx.x == 0) {
            // bits 56..63: arrivals; bits 4 p .. 4 p + 3: 1 + the XCD of slice p's writer
            const unsigned long long mine =
                (1ull << 56) | (ks < kSkXccSlots ? static_cast<unsigned long long>(xcc + 1) << (4 * ks) : 0ull);
            const unsigned long long prev =
                __hip_atomic_fetch_add(arrivals + tile, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = (prev >> 56) == static_cast<unsigned long long>(KS - 1);
            if (last) __hip_atomic_store(arrivals + tile, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_s = last;
            writers_s = prev;
        }
        __syncthreads();
        if (!last_s) return;
    }
    const unsigned long long writers = writers_s;

    // 6. the last arrival: Y = the KS partials added in slice order (its own from registers,
    //    the others loaded kSkReduceBatch at a time)
    f4v sum[4] = {};
    for (int p0 = 0; p0 < KS; p0 += kSkReduceBatch) {
        f4v v[kSkReduceBatch][4];
#pragma unroll
        for (int u = 0; u < kSkReduceBatch; ++u) {
            const int p = min(p0 + u, KS - 1);
            if (p == ks) continue;
            const bool here = p < kSkXccSlots && ((writers >> (4 * p)) & 15) == static_cast<unsigned>(xcc + 1);
            if (here) {
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    v[u][r4] = __builtin_bit_cast(
                        f4v, __builtin_amdgcn_raw_buffer_load_b128(pr, lo + 4 * (p * kSkTile) + 1024 * r4, 0, kL1Bypass));
            } else {
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    v[u][r4] = __builtin_bit_cast(
                        f4v, __builtin_amdgcn_raw_buffer_load_b128(pr, lo + 4 * (p * kSkTile) + 1024 * r4, 0, kDeviceScope));
            }
        }
#pragma unroll
        for (int u = 0; u < kSkReduceBatch; ++u) {
            if (p0 + u >= KS) break;
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const f4v t = p0 + u == ks ? own[r4] : v[u][r4];
                sum[r4][0] += t[0];
                sum[r4][1] += t[1];
                sum[r4][2] += t[2];
                sum[r4][3] += t[3];
            }
        }
    }
    if (li >= N) return;
    float *yc = y + static_cast<size_t>(li) * M;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
        const int m = m0 + 32 * wave + 8 * r4 + 4 * h;
        if (vec_y && m + 3 < M) {
            *reinterpret_cast<float4 *>(yc + m) = make_float4(sum[r4][0], sum[r4][1], sum[r4][2], sum[r4][3]);
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (m + c < M) yc[m + c] = sum[r4][c];
        }
    }
}

// Raises fn's dynamic-LDS limit to what the CU's 160 KB leaves beside its static LDS
// (once per kernel; `limit` caches the figure).
int raise_lds_limit(const void *fn, size_t &limit) {
    hipFuncAttributes attr{};
    if (hipFuncGetAttributes(&attr, fn) != hipSuccess || attr.sharedSizeBytes >= 160 * 1024) return kLaunchFailed;
    const size_t cap = 160 * 1024 - attr.sharedSizeBytes;
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(cap)) != hipSuccess)
        return kLaunchFailed;
    limit = cap;
    return kOk;
}

template <int WM, int WN, int GT>
int launch_tiles(const uint8_t *w, const _Float16 *xh, const float *xinv, float *y, int M, int N, int K, int Kp, int G,
                 int rb, hipStream_t stream) {
    constexpr int BM = 128 * WM, BN = 32 * WN;
    constexpr int stage = kWStage1 * WM + BN * 128;
    const int S = std::max(2, std::min(4, (80 * 1024) / stage));  // ring depth within 80 KB of LDS
    const size_t lds = static_cast<size_t>(S) * stage;
    static size_t limit = 0;  // dynamic LDS the kernel may take (0: not raised from the default 64 KB yet)
    if (lds > 64 * 1024 && limit == 0) {
        // what the CU's 160 KB leaves beside the kernel's static LDS
        const void *fn = reinterpret_cast<const void *>(i4_matmul_mfma<WM, WN, GT>);
        if (raise_lds_limit(fn, limit) != kOk) return kLaunchFailed;
    }
    if (lds > 64 * 1024 && lds > limit) return kTooLarge;
    const dim3 grid((M + BM - 1) / BM, (N + BN - 1) / BN);
    hipLaunchKernelGGL((i4_matmul_mfma<WM, WN, GT>), grid, dim3(kThreads), lds, stream, w, xh, xinv, y, M, N, K, Kp, G,
                       rb, S);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

template <int WN, int GT, int S>
int launch_tiles2(const uint8_t *w, const _Float16 *xh, const float *xinv, float *y, int M, int N, int K, int Kp, int G,
                  int rb, hipStream_t stream) {
    constexpr int BN = 32 * WN;
    const size_t lds = static_cast<size_t>(S) * (kWSlots * kBM * 4 + BN * 128);
    static size_t limit = 0;
    if (lds > 64 * 1024 && limit == 0) {
        const void *fn = reinterpret_cast<const void *>(i4_matmul_mfma2<WN, GT, S>);
        if (raise_lds_limit(fn, limit) != kOk) return kLaunchFailed;
    }
    if (lds > 64 * 1024 && lds > limit) return kTooLarge;
    // row offsets of the 128 staged rows and token-row offsets must fit the 32-bit DMA offsets
    if (static_cast<size_t>(kBM) * rb + static_cast<size_t>(Kp) * 2 >= (1ull << 31)) return kTooLarge;
    const dim3 grid((M + kBM - 1) / kBM, (N + BN - 1) / BN);
    hipLaunchKernelGGL((i4_matmul_mfma2<WN, GT, S>), grid, dim3(kThreads), lds, stream, w, xh, xinv, y, M, N, K, Kp, G,
                       rb);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

template <int WN, int S, int NWV>
int launch_g64(const uint8_t *w, const _Float16 *xh, const float *xinv, float *y, int M, int N, int K, int Kp, int rb,
               hipStream_t stream) {
    constexpr int BN = 32 * WN, BM = 32 * NWV;
    const size_t lds = static_cast<size_t>(S) * BN * 128;
    static size_t limit = 0;
    if (lds > 64 * 1024 && limit == 0) {
        const void *fn = reinterpret_cast<const void *>(i4_matmul_g64<WN, S, NWV>);
        if (raise_lds_limit(fn, limit) != kOk) return kLaunchFailed;
    }
    if (lds > 64 * 1024 && lds > limit) return kTooLarge;
    if (static_cast<size_t>(BM) * rb + static_cast<size_t>(Kp) * 2 * BN >= (1ull << 31)) return kTooLarge;
    const dim3 grid((M + BM - 1) / BM, (N + BN - 1) / BN);
    const int vec_y = M % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    hipLaunchKernelGGL((i4_matmul_g64<WN, S, NWV>), grid, dim3(64 * NWV), lds, stream, w, xh, xinv, y, M, N, K, Kp,
                       rb, vec_y);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

// The few-token kernel applies: G = 64, at most 32 tokens, whole 16-byte X loads (K % 4 == 0,
// X 16-byte aligned) and the byte offsets of 128 rows within 31 bits.
bool skinny_applies(const float *x, int K, int N, int group_size) {
    return group_size == 64 && N <= 32 && K % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
           static_cast<size_t>(kSkRows) * i4_row_bytes(K, 64) < (1ull << 31);
}

struct SkinnyGeom {
    int tiles, T, KS, smax;
    size_t part_bytes;  // the partial products
};

// About 1.9 workgroups per CU (all resident at once; measured on MI355X at 9728x2560x32: 6
// slices of 6-7 steps beat 8 of 5, the reduction of fewer partials outweighing the longer
// slices), at most kSkMaxSteps steps per slice and at most one slice per step.
SkinnyGeom skinny_geom(int M, int K) {
    SkinnyGeom g;
    g.tiles = (M + kSkRows - 1) / kSkRows;
    g.T = (K + 63) / 64;
    const int cus = device_cu_count();
    const int ks = std::max((19 * cus + 5 * g.tiles) / (10 * g.tiles), (g.T + kSkMaxSteps - 1) / kSkMaxSteps);
    g.KS = std::max(1, std::min(ks, g.T));
    g.smax = (g.T + g.KS - 1) / g.KS;
    g.part_bytes = static_cast<size_t>(g.tiles) * g.KS * kSkTile * sizeof(float);
    return g;
}

int launch_skinny(const uint8_t *w, const float *x, float *y, int M, int K, int N, const SkinnyGeom &g, float *part,
                  unsigned long long *arrivals, hipStream_t stream) {
    const int rb = static_cast<int>(i4_row_bytes(K, 64));
    const int vec_y = M % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;  // 16-byte Y stores
    const dim3 grid((g.tiles + 7) / 8 * 8 * g.KS), block(256);
    switch (g.smax) {
#define TQ_SKINNY(S)                                                                                             \
    case S:                                                                                                      \
        hipLaunchKernelGGL(i4_matmul_skinny<S>, grid, block, 0, stream, w, x, y, M, K, N, rb, g.T, g.KS, part, \
                           arrivals, vec_y);                                                                     \
        break;
        TQ_SKINNY(1) TQ_SKINNY(2) TQ_SKINNY(3) TQ_SKINNY(4) TQ_SKINNY(5) TQ_SKINNY(6) TQ_SKINNY(7)
#undef TQ_SKINNY
        default:
            return kBadShape;
    }
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

// Token blocks of 32 per wave (WN). Measured on MI355X at 9728x2560: one
// block for <= 32 tokens, two for <= 128 (30.6 vs 38.2 us at 128 tokens),
// three above (128-token tiles and two row blocks per wave were slower: fewer
// workgroups, more registers).
int pick_wn(int N) { return N <= 32 ? 1 : N <= 128 ? 2 : 3; }

// The MFMA path applies: a group size that is a multiple of 32 and byte offsets within 31 bits.
bool mfma_applies(int M, int K, int N, int group_size) {
    const size_t Kp = (static_cast<size_t>(K) + kStepK - 1) / kStepK * kStepK;
    return group_size % 32 == 0 && i4_row_bytes(K, group_size) * static_cast<size_t>(M) < (1ull << 31) &&
           Kp * 2 * static_cast<size_t>(N) < (1ull << 31);
}

// Other shapes: one matvec per token column.
int matmul_by_columns(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                      hipStream_t stream) {
    for (int n = 0; n < N; ++n) {
        const int st = launch_i4_matvec(w, x + static_cast<size_t>(n) * K, y + static_cast<size_t>(n) * M, M, K,
                                        group_size, stream);
        if (st != kOk) return st;
    }
    return kOk;
}

// The MFMA path with X's fp16 copy and per-token scales at ws (prefill_scratch_bytes(K, N) bytes).
int matmul_mfma(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size, unsigned char *ws,
                hipStream_t stream) {
    const size_t rb = i4_row_bytes(K, group_size);
    const size_t Kp = (static_cast<size_t>(K) + kStepK - 1) / kStepK * kStepK;
    const size_t xh_bytes = (Kp * 2 * N + 255) / 256 * 256;
    _Float16 *xh = reinterpret_cast<_Float16 *>(ws);
    float *xinv = reinterpret_cast<float *>(ws + xh_bytes);
    const int ikp = static_cast<int>(Kp), irb = static_cast<int>(rb);
    const int wn = pick_wn(N);
    // The G = 64 kernel (packed-fp16 dequantization) takes X in its k-slot order; the other
    // kernels in natural order. Its workgroups address 32 NWV rows and 32 WN token rows of X
    // with 32-bit offsets.
    const int g64_bm = wn == 1 ? 32 : wn == 2 ? 128 : 256;
    const bool g64 = group_size == 64 && static_cast<size_t>(g64_bm) * rb + Kp * 2 * 32 * wn < (1ull << 31);
    const bool lng = Kp > static_cast<size_t>(256 * kXRegs);
    const bool vec = !lng && K % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;  // 16-byte loads
    if (g64)
        hipLaunchKernelGGL(lng ? x_to_f16_long<true> : vec ? x_to_f16_vec<true> : x_to_f16<true>, dim3(N), dim3(256), 0,
                           stream, x, K, ikp, xh, xinv);
    else
        hipLaunchKernelGGL(lng ? x_to_f16_long<false> : vec ? x_to_f16_vec<false> : x_to_f16<false>, dim3(N), dim3(256),
                           0, stream, x, K, ikp, xh, xinv);
    if (hipGetLastError() != hipSuccess) return kLaunchFailed;
    int st;
    if (g64) {
        // one-wave workgroups of 32 rows for a single token block: four times
        // the workgroups (304 at 9728 rows), each with a wave-private X ring
        // Tiles measured on MI355X at 9728x2560 (512 / 128 tokens): 128 x 96 52.9 / 33.0 us,
        // 128 x 64 57.9 / 27.7, 128 x 128 58.7 / 38.9; two or more row blocks per wave
        // (256 x 96, 256 x 64, 128 x 96 over 2 waves, ...) 66-82 / 40-72; and staging W
        // through LDS in 3-step chunks did not beat the loads straight into registers.
        // (At 512 tokens, 128 x 160 tiles with 1 wave per SIMD, 256 x 128 tiles of 8 waves and
        // W staged through LDS in 4-step chunks by 16-byte DMAs were no faster either.)
        // Above 128 tokens: 256 x 96 tiles of 8 waves (one 32-row block each, W in registers)
        // with a 3-step ring, 228 workgroups at 9728 x 512: 44.6-45.1 us per call against
        // 46.3-47.2 for 128 x 96 tiles of 4 waves with a 4-step ring (a 4-step ring with 8 waves:
        // 45.7-46.4; a 2-step ring: 60; the token tiles of a row tile on one XCD: no change).
        // At 128 tokens the 4-step ring of 4 waves stays (3 steps: 26.2 us, 2: 41.1, 128 x 32
        // tiles: 25.2, 256 x 32 tiles of 8 waves: 34.3, against 24.0).
        return wn == 1   ? launch_g64<1, 4, 1>(w, xh, xinv, y, M, N, K, ikp, irb, stream)
               : wn == 2 ? launch_g64<2, 4, 4>(w, xh, xinv, y, M, N, K, ikp, irb, stream)
                         : launch_g64<3, 3, 8>(w, xh, xinv, y, M, N, K, ikp, irb, stream);
    }
    if (group_size == 64) {
        st = wn == 1   ? launch_tiles2<1, 64, 4>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream)
             : wn == 2 ? launch_tiles2<2, 64, 4>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream)
                       : launch_tiles2<3, 64, 4>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
    } else {
        st = wn == 1   ? launch_tiles2<1, 0, 4>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream)
             : wn == 2 ? launch_tiles2<2, 0, 4>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream)
                       : launch_tiles2<3, 0, 4>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
    }
    if (st != kTooLarge) return st;
    if (group_size == 64) {
        if (wn == 1) return launch_tiles<1, 1, 64>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
        if (wn == 2) return launch_tiles<1, 2, 64>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
        return launch_tiles<1, 3, 64>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
    }
    if (wn == 1) return launch_tiles<1, 1, 0>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
    if (wn == 2) return launch_tiles<1, 2, 0>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
    return launch_tiles<1, 3, 0>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
}

// ---- allocation-free variant --------------------------------------------------------------
// `scratch` holds X's fp16 copy and the per-token scales for callers that cannot
// allocate (code under graph capture, serving loops). Every GPU the library runs on
// holds its own copy for the life of the process; all calls on one GPU share it, so
// calls that overlap on one GPU race. Nothing in it has to start at zero: x_to_f16
// writes every byte the GEMM reads (the padding columns included).
// The last kNoAllocArrivalBytes are the few-token kernel's arrival counters: zero when the
// code object is loaded and after every launch, and never written by anything else.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr size_t kNoAllocArrivalBytes = size_t{64} << 10;
constexpr size_t kNoAllocWorkBytes = kNoAllocScratchBytes - kNoAllocArrivalBytes;

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, once looked up

// The device address of `scratch` on the current device. The host-side name is only a
// handle for the lookup; kernels get this address.
int noalloc_scratch(unsigned char **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return kHipFailed;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return kHipFailed;
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<unsigned char *>(g_scratch_ptr[dev]);
    return kOk;
}

}  // namespace

int launch_i4_matmul_noalloc(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                             hipStream_t stream) {
    if (M < 1 || K < 1 || N < 1 || group_size < 2 || (group_size & 1)) return kBadShape;
    // (the size checks below come first, so a call's ENOSCRATCH does not depend on its pointers;
    // every launch below is preceded by the null check)
    const bool operands = w && x && y;
    if (skinny_applies(x, K, N, group_size)) {
        // launch_i4_matmul runs the few-token kernel here; another kernel would give other
        // bits, so a call whose partials do not fit is refused rather than rerouted
        // (e.g. 151936x896 at up to 32 tokens: 1187 tiles x 2 slices x 16 KiB).
        const SkinnyGeom g = skinny_geom(M, K);
        if (g.part_bytes > kNoAllocWorkBytes || static_cast<size_t>(g.tiles) * 8 > kNoAllocArrivalBytes)
            return kNoScratch;
        if (!operands) return kBadShape;
        unsigned char *ws = nullptr;
        const int st = noalloc_scratch(&ws);
        if (st != kOk) return st;
        return launch_skinny(w, x, y, M, K, N, g, reinterpret_cast<float *>(ws),
                             reinterpret_cast<unsigned long long *>(ws + kNoAllocWorkBytes), stream);
    }
    const bool mfma = mfma_applies(M, K, N, group_size);
    if (mfma && prefill_scratch_bytes(K, N) > kNoAllocWorkBytes) return kNoScratch;
    if (!operands) return kBadShape;
    unsigned char *ws = nullptr;
    if (mfma) {
        const int st = noalloc_scratch(&ws);
        if (st != kOk) return st;
        return matmul_mfma(w, x, y, M, K, N, group_size, ws, stream);
    }
    // One matvec per token column under a scratch set with no buffers: a kernel that would
    // need split-K slots is not chosen, and nothing is allocated.
    static ScratchSet *none = scratch_set_fixed(nullptr, 0);
    ScratchScope scope(none);
    return matmul_by_columns(w, x, y, M, K, N, group_size, stream);
}

int launch_i4_matmul(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                     hipStream_t stream) {
    if (M < 1 || K < 1 || N < 1 || group_size < 2 || (group_size & 1)) return kBadShape;
    if (!w || !x || !y) return kBadShape;  // nothing is launched on a null operand
    if (skinny_applies(x, K, N, group_size)) {
        const SkinnyGeom g = skinny_geom(M, K);
        unsigned long long *slots = nullptr;  // zero between launches: the arrival counters
        int st = scratch_split_slots(stream, static_cast<size_t>(g.tiles), &slots);
        if (st != kOk) return st;
        void *part = nullptr;
        st = scratch_prefill(stream, g.part_bytes, &part);
        if (st != kOk) return st;
        return launch_skinny(w, x, y, M, K, N, g, static_cast<float *>(part), slots, stream);
    }
    if (!mfma_applies(M, K, N, group_size)) return matmul_by_columns(w, x, y, M, K, N, group_size, stream);
    void *ws = nullptr;
    const int st = scratch_prefill(stream, prefill_scratch_bytes(K, N), &ws);  // the stream's (or scope's) buffer
    if (st != kOk) return st;
    return matmul_mfma(w, x, y, M, K, N, group_size, static_cast<unsigned char *>(ws), stream);
}

}  // namespace tqhip
