// i4_matvec.hip -- batch=1 i4 HQQ (asymmetric uint4, fp16 scale/zero per group) matvec for gfx950.
//
// Computes y[o] = sum_g sum_i (q[o,g,i] - zero[o,g]) * scale[o,g] * x[g*G + i], the
// contract of the reference's matvec_i4_ref (kernels/matvec/matvec_i4_ref.cpp:45-103),
// on the reference's interleaved layout: every row is ceil(K/G) groups of
// [scale fp16 | zero fp16 | G/2 bytes of codes], low nibble = even element.
//
// Fast path (G % 8 == 0, G >= 40): integer MFMA.
//   * Activations are turned, once per workgroup, into exact integers
//     X = rint(x * 2^f_g) with one power-of-two exponent per group (|X| <= 2^22),
//     split into three signed base-256 digits ("planes") d0 + 256*d1 + 65536*d2.
//   * The weight codes are used as they are: each packed dword is split into its
//     even and odd nibbles with two AND masks, giving 8 int8 values 0..15.
//   * v_mfma_i32_16x16x64_i8 contracts 16 weight rows against a 16-row
//     activation operand whose rows are (group slot h, plane p), so one MFMA
//     pair yields the exact integer sums sum(q*X) per plane and per group for
//     a 64-byte window of each row. No rounding happens before the per-group
//     epilogue  y += scale * (V * 2^-f - zero * sum(X) * 2^-f).
//   * Every lane works on the same 16-byte column of every row ("window"
//     offsets are row-invariant), so the activation operand, its group masks
//     and the per-group constants are built once per workgroup into VGPRs.
//   * Workgroups take 16-row tiles round-robin; each tile is one contiguous
//     block of memory. The tile goes global -> LDS with 1 KB-per-instruction
//     DMA loads (buffer_load ... lds) into a ring of 3..8 tile buffers, the
//     first tiles being issued before the activation set-up so HBM is busy
//     from the start; the MFMA operands (codes and group headers) are read
//     back from LDS. The row windows are split over the waves and the
//     per-wave partial sums are added in a fixed order (deterministic).
//   * Rows longer than 48 windows use the register-only variant, which loads
//     the operands straight from HBM.
// Portable path (any even G): one wave per row, fp32 accumulation.

#include "i4_lane.h"

#include <algorithm>
#include <type_traits>

namespace tqhip {
namespace {

constexpr int kChunk = 64;     // bytes of one weight row covered by one MFMA pair ("window")
constexpr int kTile = 16;      // weight rows per MFMA tile
constexpr int kPiece = 1024;   // bytes one wave streams per 16-byte-per-lane load
constexpr int kCachePolicyStream = 2;     // buffer-load cache-policy bits: nt (non-temporal)
#ifndef TQ_DMA_INFLIGHT_KB
#define TQ_DMA_INFLIGHT_KB 96  // weight bytes in flight per CU the DMA ring aims for
#endif
constexpr size_t kInflightPerCu = static_cast<size_t>(TQ_DMA_INFLIGHT_KB) * 1024;
#ifndef TQ_DMA_WAVES_PER_CU
#define TQ_DMA_WAVES_PER_CU 32  // resident waves per CU the DMA-staged kernels aim for
#endif
constexpr int kDmaWavesPerCu = TQ_DMA_WAVES_PER_CU;
// Occupancy bound of a DMA-staged instance: three windows per wave need more
// than the 64 VGPRs that eight waves per SIMD leave.
constexpr int dma_waves_per_simd(int cpw) { return cpw >= 3 ? std::min(6, kDmaWavesPerCu / 4) : kDmaWavesPerCu / 4; }
constexpr int kPipeWavesPerSimd = 4;     // register-path kernel: launch bound (VGPR budget 128)
constexpr int kPipeSlots = 2;            // register-path kernel: tiles loaded ahead of the one computed
constexpr int kPipeWgsPerCu = 2;         // register-path kernel: workgroups per CU in the grid
constexpr size_t kLdsBytes = 160 * 1024;  // LDS per CU (gfx950)
constexpr int kMaxDepth = 8;              // DMA ring slots at most
constexpr int kMaxGroup = 3;              // matrices sharing x in one DMA-staged launch (qkv)

__device__ inline float wave_max(float v) { return xor_max_wave(v); }

__device__ inline float wave_sum(float v) { return xor_sum_wave(v); }

// Position of element i of a group inside its 8-element block, in the order
// the weight operand presents it: even elements (low nibbles) first, then odd.
__device__ inline int plane_pos(int i) {
    const int j = i & 7;
    return (i & ~7) + ((j & 1) ? 4 + (j >> 1) : (j >> 1));
}

// Three signed base-256 digits of X (|X| <= 2^22): X = d0 + 256*d1 + 65536*d2.
__device__ inline void planes_of(int X, int &d0, int &d1, int &d2) {
    d0 = ((X + 128) & 255) - 128;
    const int X1 = (X - d0) >> 8;
    d1 = ((X1 + 128) & 255) - 128;
    d2 = (X1 - d1) >> 8;
}

struct Geom {
    int M, K, G, gb, Gr, row_bytes, T, NW;
    int rbp;      // LDS row pitch of a staged tile (>= row_bytes, odd multiple of 16)
    int pieces;   // 1 KB pieces per staged tile
    int xoff;     // LDS byte offset of the activation set-up (staged kernel)
    int tbuf;     // bytes of one DMA tile buffer (DMA-staged kernel)
    int depth;    // DMA ring slots (DMA-staged kernel)
    // DMA-staged kernel: 1..3 matrices sharing x (pair / qkv), their tiles
    // numbered one after the other; tile_end[j] = tiles of matrices 0..j.
    int ksplit;  // split-K kernel: workgroups (row-window parts) per tile
    // register-path kernel with AMAX: each workgroup's largest output and its row (first row of
    // equal values) at amax_v / amax_i [blockIdx.x]
    float *amax_v;
    int *amax_i;
    int nmat;
    int tile_end[kMaxGroup];
    int mrows[kMaxGroup];
    const uint8_t *mw[kMaxGroup];
    float *my[kMaxGroup];
};

// Matrix of the group that holds global tile t, and t's index within it.
struct TileRef {
    const uint8_t *w;
    float *y;
    int M, tile;
};

// Tile -> matrix lookup for the 1..3 matrices of gm (tiles numbered one
// matrix after the other): the base values plus differences added under the
// two comparisons, copied out of the kernel argument once, so a lookup inside
// a loop is a few scalar selects and adds. (Selects among the fields
// themselves are turned by the compiler into an indexed load -- from the
// kernel argument, or from scratch memory for a local copy -- issued and
// waited for inside the loop.)
struct TileMap {
    unsigned long long w0, dw1, dw2, y0, dy1, dy2;
    int M0, dM1, dM2, end0, end1;
    __device__ explicit TileMap(const Geom &gm) {
        const unsigned long long w1 = reinterpret_cast<unsigned long long>(gm.mw[1]);
        const unsigned long long y1 = reinterpret_cast<unsigned long long>(gm.my[1]);
        w0 = reinterpret_cast<unsigned long long>(gm.mw[0]);
        dw1 = w1 - w0;
        dw2 = reinterpret_cast<unsigned long long>(gm.mw[2]) - w1;
        y0 = reinterpret_cast<unsigned long long>(gm.my[0]);
        dy1 = y1 - y0;
        dy2 = reinterpret_cast<unsigned long long>(gm.my[2]) - y1;
        M0 = gm.mrows[0];
        dM1 = gm.mrows[1] - gm.mrows[0];
        dM2 = gm.mrows[2] - gm.mrows[1];
        end0 = gm.tile_end[0];
        end1 = gm.tile_end[1];
    }
    __device__ TileRef at(int t) const {
        const bool a = t >= end0, b = t >= end1;
        TileRef r;
        r.w = reinterpret_cast<const uint8_t *>(w0 + (a ? dw1 : 0ull) + (b ? dw2 : 0ull));
        r.y = reinterpret_cast<float *>(y0 + (a ? dy1 : 0ull) + (b ? dy2 : 0ull));
        r.M = M0 + (a ? dM1 : 0) + (b ? dM2 : 0);
        r.tile = t - (a ? end0 : 0) - (b ? end1 - end0 : 0);
        return r;
    }
};

// LDS view of an activation set-up: groups gbase .. gbase+n-1 (the whole
// vector for a workgroup-wide set-up, or the few groups one wave's windows
// touch for a wave-local one).
struct XPlanes {
    int8_t *pl;    // 3 planes x stride bytes, 8-element blocks in operand order
    int *pre;      // per group: inclusive prefix over its 8-element blocks of sum(X)
    float *gexp;   // 2^-f per group
    int stride;    // bytes per plane
    int gbase;     // first group held
    int ngroups;   // groups held
};

// Wave-local set-up: 64 lanes x 8 elements cover the (at most 8) groups of G=64
// or (at most 4) groups of G=128 that one wave's <= 3 windows touch.
constexpr int kWaveXBytes = 3 * 64 * 8 + 64 * 4 + 8 * 4;  // planes + prefixes + exponents

// The first 8-element block of activations each thread converts (fast path):
// loaded at kernel entry, ahead of the weight stream, so its latency is not
// stretched by the tile loads queued behind it.
struct XFirst {
    float v[8];
};

template <int GT>
__device__ inline void load_x_first(XFirst &xf, const float *__restrict__ x, int K, int Kp) {
    if constexpr (GT == 64 || GT == 128) {
        // branch-free (clamped address, then masked) so the compiler can wait
        // for exactly these loads while weight DMAs issued after them are pending
        // clamped index, then masked: indices at or past K (threads past Kp
        // included, as Kp >= K) give 0. The loads stay scalar-element loads so
        // no wide load straddles the end of x.
        const int b = threadIdx.x;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int k = 8 * b + i;
            const float v = x[min(k, K - 1)];
            xf.v[i] = k < K ? v : 0.f;
        }
        (void)Kp;
    }
}

typedef unsigned v2u __attribute__((ext_vector_type(2)));

__device__ inline unsigned lds_addr(const void *p) {
    return static_cast<unsigned>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)p));
}

// LDS reads the compiler does not see as such: it would otherwise wait for
// every global->LDS transfer in flight before them (it cannot tell that these
// addresses are not among the transfers' targets). Complete on return.
__device__ inline float4 lds_read_f4(const float *p) {
    float4 v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return v;
}

__device__ inline void lds_read4_u2(const int8_t *const (&p)[4], v2u (&v)[4]) {
    asm volatile(
        "ds_read_b64 %0, %4\n\tds_read_b64 %1, %5\n\tds_read_b64 %2, %6\n\tds_read_b64 %3, %7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
        : "v"(lds_addr(p[0])), "v"(lds_addr(p[1])), "v"(lds_addr(p[2])), "v"(lds_addr(p[3]))
        : "memory");
}

__device__ inline void lds_read3_u32(const int *p1, const int *p0, const int *p2, int &v1, int &v0, float &v2) {
    int r2;
    asm volatile("ds_read_b32 %0, %3\n\tds_read_b32 %1, %4\n\tds_read_b32 %2, %5\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v1), "=&v"(v0), "=&v"(r2)
                 : "v"(lds_addr(p1)), "v"(lds_addr(p0)), "v"(lds_addr(p2))
                 : "memory");
    v2 = __builtin_bit_cast(float, r2);
}

// LDS stores the compiler does not see as such (same reason); they complete
// before the next s_waitcnt lgkmcnt(0), which every barrier here includes.
__device__ inline void lds_write3_u2(const void *p, int stride, v2u a, v2u b, v2u c) {
    const unsigned o = lds_addr(p);
    asm volatile("ds_write_b64 %0, %1\n\tds_write_b64 %2, %3\n\tds_write_b64 %4, %5"
                 :
                 : "v"(o), "v"(a), "v"(o + stride), "v"(b), "v"(o + 2 * stride), "v"(c)
                 : "memory");
}

__device__ inline void lds_write_u32(const void *p, unsigned v) {
    asm volatile("ds_write_b32 %0, %1" : : "v"(lds_addr(p)), "v"(v) : "memory");
}

// ---- 1. activations -> per-group exponent, integer planes, prefix block sums
// GT = 64 or 128: one lane per 8-element block, group max and prefix by DPP.
// ONE_ROUND: the caller guarantees Kp / 8 <= blockDim.x, so only the values
// already loaded by load_x_first are used (no further global loads here), and
// the LDS stores go through lds_write_* (global->LDS transfers may be in
// flight, and the compiler would wait for all of them before each store).
template <int GT, bool ONE_ROUND = false>
__device__ void prepare_x(const XPlanes &xp, const float *__restrict__ x, int K, int Gr, int Kp, const XFirst &xf) {
    if constexpr (GT == 64 || GT == 128) {
        constexpr int LPG = GT / 8;  // lanes (blocks) per group: 8 or 16
        const int nblk = Kp / 8;
        // every lane of a block-group takes part in the DPP steps, so the loop
        // runs whole waves and masks work past the last block instead
        const int stride = blockDim.x;
        const int nrounds = ONE_ROUND ? 1 : (nblk + stride - 1) / stride;
        const int lane = threadIdx.x & 63;
        for (int rd = 0; rd < nrounds; ++rd) {
            const int b = rd * stride + threadIdx.x;
            const bool live = b < nblk;
            float v[8];
            float m = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int k = 8 * b + i;
                if (ONE_ROUND || rd == 0)
                    v[i] = xf.v[i];
                else
                    v[i] = (live && k < K) ? x[k] : 0.f;
                m = fmaxf(m, abs_or_inf(v[i]));
            }
            m = fmaxf(m, dpp_f<kDppXor1>(m));
            m = fmaxf(m, dpp_f<kDppXor2>(m));
            m = fmaxf(m, dpp_f<kDppHalfMirror>(m));
            if constexpr (LPG == 16) m = fmaxf(m, dpp_f<kDppRor8>(m));
            const int f = group_exponent(m);
            unsigned w[3][2] = {{0u, 0u}, {0u, 0u}, {0u, 0u}};
            int sum = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int X = static_cast<int>(rintf(ldexpf(v[i], f)));
                sum += X;
                int d[3];
                planes_of(X, d[0], d[1], d[2]);
                const int word = i & 1, byte = i >> 1;  // even elements -> first dword
#pragma unroll
                for (int p = 0; p < 3; ++p) w[p][word] |= (static_cast<unsigned>(d[p]) & 0xFFu) << (8 * byte);
            }
            // inclusive prefix of the block sums within the group (Hillis-Steele over LPG lanes)
            const int j = lane & (LPG - 1);
            int s = sum, t;
            t = dpp_i<kDppShr1>(s);
            s += (j >= 1) ? t : 0;
            t = dpp_i<kDppShr2>(s);
            s += (j >= 2) ? t : 0;
            t = dpp_i<kDppShr4>(s);
            s += (j >= 4) ? t : 0;
            if constexpr (LPG == 16) {
                t = dpp_i<kDppShr8>(s);
                s += (j >= 8) ? t : 0;
            }
            if (live) {
                if constexpr (ONE_ROUND) {
                    lds_write3_u2(xp.pl + 8 * b, Kp, v2u{w[0][0], w[0][1]}, v2u{w[1][0], w[1][1]},
                                  v2u{w[2][0], w[2][1]});
                    lds_write_u32(xp.pre + b, static_cast<unsigned>(s));
                    if (j == 0) lds_write_u32(xp.gexp + b / LPG, __builtin_bit_cast(unsigned, group_unscale(m, f)));
                } else {
#pragma unroll
                    for (int p = 0; p < 3; ++p)
                        *reinterpret_cast<uint2 *>(xp.pl + p * Kp + 8 * b) = make_uint2(w[p][0], w[p][1]);
                    xp.pre[b] = s;
                    if (j == 0) xp.gexp[b / LPG] = group_unscale(m, f);
                }
            }
        }
    } else {
        const int G = Kp / Gr;
        const int lane = threadIdx.x & 63;
        const int wave = threadIdx.x >> 6;
        const int nw = blockDim.x >> 6;
        for (int g = wave; g < Gr; g += nw) {
            const int base = g * G;
            float m = 0.f;
            for (int i = lane; i < G; i += 64) {
                const int k = base + i;
                if (k < K) m = fmaxf(m, abs_or_inf(x[k]));
            }
            m = wave_max(m);
            const int f = group_exponent(m);
            for (int i = lane; i < G; i += 64) {
                const int k = base + i;
                const int X = (k < K) ? static_cast<int>(rintf(ldexpf(x[k], f))) : 0;
                int d0, d1, d2;
                planes_of(X, d0, d1, d2);
                const int pos = base + plane_pos(i);
                xp.pl[pos] = static_cast<int8_t>(d0);
                xp.pl[Kp + pos] = static_cast<int8_t>(d1);
                xp.pl[2 * Kp + pos] = static_cast<int8_t>(d2);
                int s = X;  // G % 8 == 0, so each 8-lane block is entirely active here
                s += __shfl_xor(s, 1);
                s += __shfl_xor(s, 2);
                s += __shfl_xor(s, 4);
                if ((i & 7) == 0) xp.pre[(base + i) >> 3] = s;  // block sum; prefixed below
            }
            if (lane == 0) xp.gexp[g] = group_unscale(m, f);
        }
        __syncthreads();
        // turn block sums into per-group inclusive prefixes (one thread per group)
        for (int g = threadIdx.x; g < Gr; g += blockDim.x) {
            int s = 0;
            for (int b = g * (G / 8); b < (g + 1) * (G / 8); ++b) {
                s += xp.pre[b];
                xp.pre[b] = s;
            }
        }
    }
}

// Wave-local variant of prepare_x (GT = 64 or 128): lane l converts block l of
// groups gfirst, gfirst+1, ... into this wave's own LDS slice. No barrier is
// needed before build_operands: the same wave reads what it wrote.
template <int GT>
__device__ void prepare_x_wave(const XPlanes &xp, const float *__restrict__ x, int K, int Gr, const XFirst &xf) {
    constexpr int LPG = GT / 8;
    const int lane = threadIdx.x & 63;
    const int j = lane & (LPG - 1);
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, abs_or_inf(xf.v[i]));
    m = fmaxf(m, dpp_f<kDppXor1>(m));
    m = fmaxf(m, dpp_f<kDppXor2>(m));
    m = fmaxf(m, dpp_f<kDppHalfMirror>(m));
    if constexpr (LPG == 16) m = fmaxf(m, dpp_f<kDppRor8>(m));
    const int f = group_exponent(m);
    unsigned w[3][2] = {{0u, 0u}, {0u, 0u}, {0u, 0u}};
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int X = static_cast<int>(rintf(ldexpf(xf.v[i], f)));
        sum += X;
        int d[3];
        planes_of(X, d[0], d[1], d[2]);
        const int word = i & 1, byte = i >> 1;  // even elements -> first dword
#pragma unroll
        for (int p = 0; p < 3; ++p) w[p][word] |= (static_cast<unsigned>(d[p]) & 0xFFu) << (8 * byte);
    }
    int s = sum, t;
    t = dpp_i<kDppShr1>(s);
    s += (j >= 1) ? t : 0;
    t = dpp_i<kDppShr2>(s);
    s += (j >= 2) ? t : 0;
    t = dpp_i<kDppShr4>(s);
    s += (j >= 4) ? t : 0;
    if constexpr (LPG == 16) {
        t = dpp_i<kDppShr8>(s);
        s += (j >= 8) ? t : 0;
    }
#pragma unroll
    for (int p = 0; p < 3; ++p) *reinterpret_cast<uint2 *>(xp.pl + p * xp.stride + 8 * lane) = make_uint2(w[p][0], w[p][1]);
    xp.pre[lane] = s;
    if (j == 0) xp.gexp[lane / LPG] = group_unscale(m, f);
}

// The 8 activations lane l of a wave-local set-up converts: block l of the
// groups starting at gfirst (zeros past the vector end).
template <int GT>
__device__ inline void load_x_wave(XFirst &xf, const float *__restrict__ x, int K, int Gr, int gfirst) {
    const int lane = threadIdx.x & 63;
    const int g = gfirst + lane / (GT / 8);
    const int k0 = g * GT + 8 * (lane & (GT / 8 - 1));
#pragma unroll
    for (int i = 0; i < 8; ++i) xf.v[i] = (g < Gr && k0 + i < K) ? x[k0 + i] : 0.f;
}

// ---- 2. per-lane, row-invariant activation operands and group constants for
// windows t0 .. t0+nch-1 (CPW slots; unused slots get a zero operand).
// HIDDEN: read LDS through lds_read_* (needed where global->LDS transfers are
// in flight, which the compiler would otherwise wait for before every read).
// Header offset (within its row) and mask of the group slot each lane reads
// for each of this wave's windows: the same values build_operands produces,
// from the geometry alone, so the header loads can go out before the
// activation set-up.
template <int GT, int CPW>
__device__ inline void header_slots(const Geom &gm, int t0, int nch, int (&HO)[CPW], unsigned (&HM)[CPW]) {
    const int gb = GT ? kI4Header + GT / 2 : gm.gb;
    const int kq = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int t = t0 + min(c, nch - 1);
        const int gq = (kChunk * t) / gb + kq;
        const int wend = min(kChunk * (t + 1), gm.row_bytes);
        const bool valid = c < nch && gq < gm.Gr && gq * gb < wend;
        HO[c] = valid ? gq * gb : 0;
        HM[c] = valid ? 0xFFFFFFFFu : 0u;
    }
}

template <int GT, int CPW, bool HIDDEN = false>
__device__ void build_operands(const XPlanes &xp, const Geom &gm, int t0, int nch, v4i (&A0)[CPW], v4i (&A1)[CPW],
                               float (&E)[CPW], float (&C)[CPW], int (&HO)[CPW], unsigned (&HM)[CPW]) {
    const int G = GT ? GT : gm.G;
    const int gb = GT ? kI4Header + GT / 2 : gm.gb;
    const int Gr = gm.Gr, rb = gm.row_bytes;
    const int lane = threadIdx.x & 63;
    const int am = lane & 15;  // activation-operand row = 4*slot + plane
    const int ah = am >> 2, ap = am & 3;
    const int kq = lane >> 4;  // k quad; also the epilogue's group slot
    const int apc = min(ap, 2);
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int t = t0 + min(c, nch - 1);
        const bool own = c < nch;
        const int gt = (kChunk * t) / gb;  // group holding the window's first byte
        // activation operand: all reads are issued unconditionally, then masked
        unsigned lo[4], hi[4];
        const int8_t *src[4];
        bool use[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // q = 2*u + dw
            const int o = kChunk * t + 4 * (4 * kq + q);
            const int g = o / gb;
            const int r = o - g * gb;
            use[q] = own && o < rb && ap < 3 && r >= kI4Header && g - gt == ah;
            const int blk = use[q] ? ((g - xp.gbase) * G + 2 * (r - kI4Header)) >> 3 : 0;  // local block
            src[q] = xp.pl + apc * xp.stride + 8 * blk;
        }
        v2u v[4];
        if constexpr (HIDDEN) {
            lds_read4_u2(src, v);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const v2u *>(src[q]);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            lo[q] = use[q] ? v[q].x : 0u;
            hi[q] = use[q] ? v[q].y : 0u;
        }
        A0[c] = v4i{static_cast<int>(lo[0]), static_cast<int>(hi[0]), static_cast<int>(lo[1]), static_cast<int>(hi[1])};
        A1[c] = v4i{static_cast<int>(lo[2]), static_cast<int>(hi[2]), static_cast<int>(lo[3]), static_cast<int>(hi[3])};
        // group slot kq of this window: its data bytes inside the window
        const int gq = gt + kq;
        const int wbeg = kChunk * t, wend = min(kChunk * (t + 1), rb);
        const int dbeg = max(gq * gb + kI4Header, wbeg), dend = min((gq + 1) * gb, wend);
        const bool valid = own && gq < Gr && gq * gb < wend;
        int sum = 0;
        const int gl = min(max(gq - xp.gbase, 0), xp.ngroups - 1);  // local group (clamped when invalid)
        const bool data = valid && dend > dbeg;
        const int b0 = gl * (G / 8) + (dbeg - gq * gb - kI4Header) / 4;  // first block in the window
        const int b1 = gl * (G / 8) + (dend - gq * gb - kI4Header) / 4;  // one past the last
        float ge;
        if constexpr (HIDDEN) {
            // unconditional reads at clamped in-range indices, then masked
            const int nb = xp.ngroups * (G / 8);
            int p1, p0;
            lds_read3_u32(xp.pre + min(max(b1 - 1, 0), nb - 1), xp.pre + min(max(b0 - 1, 0), nb - 1),
                          reinterpret_cast<const int *>(xp.gexp + gl), p1, p0, ge);
            if (data) sum = p1 - (b0 > gl * (G / 8) ? p0 : 0);
        } else {
            if (data) sum = xp.pre[b1 - 1] - (b0 > gl * (G / 8) ? xp.pre[b0 - 1] : 0);
            ge = xp.gexp[gl];
        }
        E[c] = valid ? ge : 0.f;
        C[c] = static_cast<float>(sum) * E[c];
        HO[c] = valid ? gq * gb : 0;
        HM[c] = valid ? 0xFFFFFFFFu : 0u;
    }
}

// Splits one 16-byte column of codes into the two int8 MFMA operands and
// accumulates this lane's share of scale * (sum(q*X) - zero * sum(X)) * 2^-f.
__device__ __forceinline__ float window_step(float a, const v4i &d, unsigned h, const v4i &A0, const v4i &A1, float E,
                                             float C) {
    const unsigned d0 = static_cast<unsigned>(d.x), d1 = static_cast<unsigned>(d.y);
    const unsigned d2 = static_cast<unsigned>(d.z), d3 = static_cast<unsigned>(d.w);
    const v4i b0 = {static_cast<int>(d0 & kNibbles), static_cast<int>((d0 >> 4) & kNibbles),
                    static_cast<int>(d1 & kNibbles), static_cast<int>((d1 >> 4) & kNibbles)};
    const v4i b1 = {static_cast<int>(d2 & kNibbles), static_cast<int>((d2 >> 4) & kNibbles),
                    static_cast<int>(d3 & kNibbles), static_cast<int>((d3 >> 4) & kNibbles)};
    v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, b0, v4i{0, 0, 0, 0}, 0, 0, 0);
    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, b1, D, 0, 0, 0);
    const float V =
        fmaf(static_cast<float>(D.z), 65536.f, fmaf(static_cast<float>(D.y), 256.f, static_cast<float>(D.x)));
    // A masked header gives scale = zero = 0, and V = E = C = 0 there, so an
    // empty group slot adds exactly 0.
    const float s = half_bits(h);
    const float z = half_bits(h >> 16);
    return fmaf(s, fmaf(V, E, -z * C), a);
}

// ============================================================================================
// DMA-staged kernel (rows of up to 48 windows): tiles go global -> LDS directly (buffer_load ... lds, 16 bytes per lane) into a
// ring of D tile buffers (D = gm.depth, 3..8, picked on the host from the LDS
// budget), so D tiles are in flight while the activation set-up runs and
// D - 1 while a tile is contracted, without spending VGPRs on the staging.
// Waits on the transfers are explicit (vmcnt counts of whole tiles).
__device__ __forceinline__ void wait_vmem(int n) {
    // s_waitcnt vmcnt(n) with expcnt/lgkmcnt left free (gfx9 encoding)
    switch (n) {
#define TQ_VMWAIT(N) case N: __builtin_amdgcn_s_waitcnt(((N) & 15) | (7 << 4) | (15 << 8) | (((N) >> 4) << 14)); break;
        TQ_VMWAIT(0) TQ_VMWAIT(1) TQ_VMWAIT(2) TQ_VMWAIT(3) TQ_VMWAIT(4) TQ_VMWAIT(5) TQ_VMWAIT(6) TQ_VMWAIT(7)
        TQ_VMWAIT(8) TQ_VMWAIT(9) TQ_VMWAIT(10) TQ_VMWAIT(11) TQ_VMWAIT(12) TQ_VMWAIT(13) TQ_VMWAIT(14)
        TQ_VMWAIT(15) TQ_VMWAIT(16) TQ_VMWAIT(17) TQ_VMWAIT(18) TQ_VMWAIT(19) TQ_VMWAIT(20) TQ_VMWAIT(21)
        TQ_VMWAIT(22) TQ_VMWAIT(23) TQ_VMWAIT(24) TQ_VMWAIT(25) TQ_VMWAIT(26) TQ_VMWAIT(27) TQ_VMWAIT(28)
#undef TQ_VMWAIT
        default: __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); break;
    }
}

// Global->LDS copy of one tile: each of this wave's PW DMAs moves 1 KB
// (16 bytes per lane, source byte poff[s], landing at dst + pdst[s] + 16*lane).
// (Not a template: clang's host pass rejected the template form in the kernel
// and silently dropped the kernel's host stub. pw is a constant at every call.)
// Every lane of every DMA is live (no branch), so the compiler can count the
// transfers issued after earlier loads and the per-wave count is exactly pw.
__device__ __forceinline__ void dma_tile(const uint8_t *w, int M, int rb, int tile, unsigned char *dst, const int *poff,
                                         const int *pdst, int pw) {
    const __amdgpu_buffer_rsrc_t rs = rows_rsrc(w, M, rb, tile * kTile);
#pragma unroll
    for (int s = 0; s < pw; ++s)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(dst + pdst[s]), 16,
                                                 poff[s], 0, 0, 0);
}

// dma_tile with the non-temporal hint: the DMA ring reads every tile once, in
// 1 KB pieces of one contiguous 16-row block, so no line is read twice and the
// caches need not keep any. Measured on the lm_head-sized stream: 8% faster
// than the default policy. The kernels whose waves read parts of lines that
// other waves also read (row segments, windows) lose with it.
__device__ __forceinline__ void dma_tile_stream(const uint8_t *w, int M, int rb, int tile, unsigned char *dst,
                                                const int *poff, const int *pdst, int pw) {
    const __amdgpu_buffer_rsrc_t rs = rows_rsrc(w, M, rb, tile * kTile);
#pragma unroll
    for (int s = 0; s < pw; ++s)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(dst + pdst[s]), 16,
                                                 poff[s], 0, 0, kCachePolicyStream);
}

// Workgroup barrier for LDS traffic that leaves weight DMAs in flight: waits
// for this wave's own LDS operations only (a __syncthreads() here would also
// wait for every pending global->LDS transfer). The empty asm statements keep
// the compiler from moving memory accesses across it.
__device__ inline void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0), vmcnt/expcnt untouched
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int GT, int CPW, int PW, int NWMAX>
__global__ __launch_bounds__(64 * NWMAX, dma_waves_per_simd(CPW)) void i4_matvec_dma(const uint8_t *__restrict__ w,
                                                                             const float *__restrict__ x,
                                                                             float *__restrict__ y, Geom gm) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int NW = gm.NW;
    const int rb = gm.row_bytes;  // (w, y, gm.M: see gm.mw / gm.my / gm.mrows)
    const int G = GT ? GT : gm.G;
    const int Kp = gm.Gr * G;
    const int NWP = (NW + 3) & ~3;
    const int tbuf = gm.tbuf;  // one tile as in memory + 64 bytes of slack, multiple of 16, >= 1 KB
    const int D = gm.depth;    // ring slots, 3..8

    unsigned char *stage = smem;                                 // [D][tbuf]
    float *part = reinterpret_cast<float *>(smem + D * tbuf);    // [2][16][NWP]
    XPlanes xp;
    xp.pl = reinterpret_cast<int8_t *>(part + 2 * kTile * NWP);
    xp.stride = Kp;
    xp.pre = reinterpret_cast<int *>(xp.pl + 3 * Kp);
    xp.gexp = reinterpret_cast<float *>(xp.pre + Kp / 8);
    xp.gbase = 0;
    xp.ngroups = gm.Gr;
    XFirst xf;
    load_x_first<GT>(xf, x, gm.K, Kp);

    const int tiles = gm.tile_end[gm.nmat - 1];
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int ntile = wg < tiles ? (tiles - 1 - wg) / nwg + 1 : 0;
    auto tile_of = [&](int i) { return wg + i * nwg; };
    const TileMap map(gm);
    const int last = max(ntile - 1, 0);

    // 1 KB pieces of a tile this wave moves (piece j -> wave j % NW). Every
    // wave issues exactly PW DMAs per tile (surplus slots repeat the last
    // piece), so the wait counts below are exact. The last piece is moved
    // back to end at the buffer's end; the bytes it shares with the piece
    // before it are written twice with the same values.
    int poff[PW], pdst[PW];
#pragma unroll
    for (int s = 0; s < PW; ++s) {
        const int j = min(wave + s * NW, gm.pieces - 1);
        pdst[s] = min(kPiece * j, tbuf - kPiece);
        poff[s] = pdst[s] + 16 * lane;
    }
    auto dma = [&](int i, unsigned char *dst) {
        const TileRef r = map.at(tile_of(i));
        dma_tile_stream(r.w, r.M, rb, r.tile, dst, poff, pdst, PW);
    };
    // the first three tiles go out before the activation set-up (repeats of
    // the last tile when the workgroup has fewer; they are never read) ...
    dma(0, stage);
    dma(min(1, last), stage + tbuf);
    dma(min(2, last), stage + 2 * tbuf);

    prepare_x<GT, true>(xp, x, gm.K, gm.Gr, Kp, xf);
    // ... and the rest of the ring once the activations have been read
    for (int t = 3; t < D; ++t) dma(min(t, last), stage + t * tbuf);
    lds_barrier();
    const int t0 = (gm.T * wave) / NW;
    const int nch = (gm.T * (wave + 1)) / NW - t0;  // 1..CPW by construction on the host
    v4i A0[CPW], A1[CPW];
    float E[CPW], C[CPW];
    int HO[CPW];
    unsigned HM[CPW];
    build_operands<GT, CPW, true>(xp, gm, t0, nch, A0, A1, E, C, HO, HM);
    const int bn = lane & 15, kq = lane >> 4;
    int RO[CPW], RH[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int t = t0 + min(c, nch - 1);
        RO[c] = bn * rb + kChunk * t + 16 * kq;
        RH[c] = bn * rb + HO[c];
    }
    for (int i = threadIdx.x; i < 2 * kTile * NWP; i += blockDim.x) lds_write_u32(part + i, 0u);

    auto reduce_prev = [&](int i) {  // partial sums of tile i (written before the last barrier)
        const float *pb = part + (i & 1) * (kTile * NWP);
        if (threadIdx.x < kTile) {
            const float *pr = pb + threadIdx.x * NWP;
            float s = 0.f;
            for (int q = 0; q < NWP / 4; ++q) {  // fixed order; padding slots hold 0
                const float4 v = lds_read_f4(pr + 4 * q);
                s += v.x;
                s += v.y;
                s += v.z;
                s += v.w;
            }
            const TileRef r = map.at(tile_of(i));
            const int row = r.tile * kTile + threadIdx.x;
            if (row < r.M) store_y(r.y + row, s);
        }
    };

    int b = 0;  // ring slot of tile i
    for (int i = 0; i < ntile; ++i) {
        // tiles issued so far: D at the start, then one per iteration from
        // i = 1 while tiles remain; tile i has landed once at most the later
        // ones are pending
        const int later = D + max(0, min(i - 1, ntile - D)) - i - 1;
        wait_vmem(later * PW);
        lds_barrier();  // every wave's pieces of tile i are in LDS; tile i-1's slot is free
        if (i >= 1 && i + D - 1 < ntile)
            dma(i + D - 1, stage + (b == 0 ? D - 1 : b - 1) * tbuf);
        const unsigned char *buf = stage + b * tbuf;
        float a = 0.f;
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            const v4i d = *reinterpret_cast<const v4i *>(buf + RO[c]);
            const unsigned h = *reinterpret_cast<const unsigned *>(buf + RH[c]) & HM[c];
            a = window_step(a, d, h, A0[c], A1[c], E[c], C[c]);
        }
        a = sum_rows4(a);  // the four group slots of each row
        if (lane < kTile) lds_write_u32(part + (i & 1) * (kTile * NWP) + lane * NWP + wave, __builtin_bit_cast(unsigned, a));
        if (i > 0) reduce_prev(i - 1);
        b = b == D - 1 ? 0 : b + 1;
    }
    wait_vmem(0);  // no DMA may still be writing this workgroup's LDS at exit
    __syncthreads();
    if (ntile > 0) reduce_prev(ntile - 1);
}

// Register-path kernel: every wave loads its own windows of each tile straight
// into VGPRs (16 rows x 16 bytes per window load, plus the group headers), P
// tiles ahead of the one it computes. No weight bytes pass through LDS; LDS
// holds the activation set-up and the per-wave partial sums, reduced in fixed
// order after one LDS-only barrier per tile. Tiles go round-robin over the
// workgroups (blockIdx.x + k * gridDim.x) across the 1..3 matrices of gm.
// Every wave issues the same loads for every tile slot (zero-length loads past
// its last tile), so the compiler's waits count exactly the loads in flight.
template <int GT, int CPW, int NWMAX, int P, bool GROUP, bool AMAX = false>
__global__ __launch_bounds__(64 * NWMAX, kPipeWavesPerSimd) void i4_matvec_pipe(const uint8_t *__restrict__ w,
                                                                         const float *__restrict__ x,
                                                                         float *__restrict__ y, Geom gm) {
    // GROUP: 1..3 matrices through gm.mw / gm.my / gm.mrows; else the one
    // matrix w -> y of gm.M rows (fewer scalar instructions per tile)
    // AMAX (one matrix): the workgroup's argmax as well (argmax_ref: the first row of the
    // largest value; a NaN is never taken), one partial per workgroup
    static_assert(!(AMAX && GROUP), "argmax of one matrix");
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int NW = gm.NW;
    const int rb = gm.row_bytes;
    const int G = GT ? GT : gm.G;
    const int Kp = gm.Gr * G;
    const int NWP = (NW + 3) & ~3;
    float *part = reinterpret_cast<float *>(smem);  // [2][16][NWP]
    const int t0 = (gm.T * wave) / NW;
    const int nch = (gm.T * (wave + 1)) / NW - t0;  // 1..CPW by construction on the host
    XPlanes xp;
    xp.pl = reinterpret_cast<int8_t *>(part + 2 * kTile * NWP);
    xp.stride = Kp;
    xp.pre = reinterpret_cast<int *>(xp.pl + 3 * Kp);
    xp.gexp = reinterpret_cast<float *>(xp.pre + Kp / 8);
    xp.gbase = 0;
    xp.ngroups = gm.Gr;
    XFirst xf;
    load_x_first<GT>(xf, x, gm.K, Kp);

    const int tiles = gm.tile_end[gm.nmat - 1];
    const int wg = blockIdx.x, nwg = gridDim.x;  // tile of round k: wg + k * nwg
    const int ntile = wg < tiles ? (tiles - 1 - wg) / nwg + 1 : 0;
    const int bn = lane & 15, kq = lane >> 4;
    int DO[CPW], HOr[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) DO[c] = bn * rb + kChunk * (t0 + min(c, nch - 1)) + 16 * kq;

    // rows of this workgroup's k-th tile; past its last tile: no rows (every load reads 0)
    const TileMap map(gm);
    auto tile_of = [&](int t) {
        if constexpr (GROUP) return map.at(t);
        TileRef r;
        r.w = w;
        r.y = y;
        r.M = gm.M;
        r.tile = t;
        return r;
    };
    auto tile_rsrc = [&](int k) {
        const bool live = k < ntile;
        const TileRef r = tile_of(live ? wg + k * nwg : 0);
        return rows_rsrc(r.w, live ? r.M : 0, rb, r.tile * kTile);
    };
    v4i d[P][CPW];
    unsigned h[P][CPW];
    auto load_d = [&](int k, v4i (&dd)[CPW]) {
        const __amdgpu_buffer_rsrc_t rs = tile_rsrc(k);
#pragma unroll
        for (int c = 0; c < CPW; ++c) dd[c] = __builtin_amdgcn_raw_buffer_load_b128(rs, DO[c], 0, 0);
    };
    auto load_h = [&](int k, unsigned (&hh)[CPW]) {
        const __amdgpu_buffer_rsrc_t rs = tile_rsrc(k);
#pragma unroll
        for (int c = 0; c < CPW; ++c) hh[c] = __builtin_amdgcn_raw_buffer_load_b32(rs, HOr[c], 0, 0);
    };
    // The first P tiles' codes go out before the activation set-up. With one
    // window per wave their headers go with them (their offsets depend on the
    // geometry only); with more, after the set-up (measured faster there).
    int HO[CPW];
    unsigned HM[CPW];
    header_slots<GT, CPW>(gm, t0, nch, HO, HM);
#pragma unroll
    for (int c = 0; c < CPW; ++c) HOr[c] = bn * rb + HO[c];
#pragma unroll
    for (int s = 0; s < P; ++s) {
        load_d(s, d[s]);
        if constexpr (CPW == 1) load_h(s, h[s]);
    }

    // (A wave-local set-up -- each wave converting only the groups its
    // windows touch, with no barrier -- measured slower here: eight waves
    // fetching x instead of one workgroup.)
    prepare_x<GT, true>(xp, x, gm.K, gm.Gr, Kp, xf);
    lds_barrier();
    v4i A0[CPW], A1[CPW];
    float E[CPW], C[CPW];
    int HO2[CPW];
    unsigned HM2[CPW];
    build_operands<GT, CPW, true>(xp, gm, t0, nch, A0, A1, E, C, HO2, HM2);  // (the same header slots)
    if constexpr (CPW > 1) {
#pragma unroll
        for (int s = 0; s < P; ++s) load_h(s, h[s]);
    }

    // Whole rounds of the P register slots: every slot is loaded and computed
    // the same way in every round (zero-length loads past the last tile),
    // which keeps the compiler's waits exact.
    const int nround = (ntile + P - 1) / P * P;
    for (int k0 = 0; k0 < nround; k0 += P) {
#pragma unroll
        for (int s = 0; s < P; ++s) {
            const int k = k0 + s;
            float a = 0.f;
#pragma unroll
            for (int c = 0; c < CPW; ++c) a = window_step(a, d[s][c], h[s][c] & HM[c], A0[c], A1[c], E[c], C[c]);
            if constexpr (P > 1) {  // (one tile per workgroup: nothing follows)
                load_d(k + P, d[s]);  // this slot's next tile
                load_h(k + P, h[s]);
            }
            a = sum_rows4(a);  // the four group slots of each row
            float *pb = part + (k & 1) * (kTile * NWP);
            if (lane < kTile) {
                lds_write_u32(pb + lane * NWP + wave, __builtin_bit_cast(unsigned, a));
                for (int q = NW + wave; q < NWP; q += NW) lds_write_u32(pb + lane * NWP + q, 0u);  // padding slots
            }
            // every wave's sums of tile k are in; the buffer written next (tile
            // k + 1) was read before this barrier
            lds_barrier();
            if (wave == 0 && lane < kTile && k < ntile) {
                float sum = 0.f;
                for (int q = 0; q < NWP / 4; ++q) {  // fixed order; padding slots hold 0
                    const float4 v = lds_read_f4(pb + lane * NWP + 4 * q);
                    sum += v.x;
                    sum += v.y;
                    sum += v.z;
                    sum += v.w;
                }
                const TileRef r = tile_of(wg + k * nwg);
                const int row = r.tile * kTile + lane;
                if (row < r.M) {
                    store_y(r.y + row, sum);
                    if constexpr (AMAX) {
                        if (sum > bv || (sum == bv && row < bi)) {
                            bv = sum;
                            bi = row;
                        }
                    }
                }
            }
        }
    }
    if constexpr (AMAX) {
        static_assert(kTile == 16, "candidates in lanes 0..15");
        if (wave == 0) {  // lanes 0..15 hold the candidates, the others (-inf, max)
            const auto step = [&](auto dl) {
                constexpr int DL = decltype(dl)::value;
                const float v = lane_xor<DL>(bv, lane);
                const int i = __float_as_int(lane_xor<DL>(__int_as_float(bi), lane));
                if (v > bv || (v == bv && i < bi)) {
                    bv = v;
                    bi = i;
                }
            };
            step(std::integral_constant<int, 8>{});
            step(std::integral_constant<int, 4>{});
            step(std::integral_constant<int, 2>{});
            step(std::integral_constant<int, 1>{});
            if (lane == 0) {
                gm.amax_v[blockIdx.x] = bv;
                gm.amax_i[blockIdx.x] = bi;
            }
        }
    }
    if constexpr (P > 1) wait_vmem(0);  // the loads issued past the last tile have returned before the wave ends
}

// Wave-private DMA ring: no workgroup barrier per tile. Each wave moves only
// the bytes its own windows read: of every row of a 16-row tile, the segment
// from the first group header its windows need to the end of its last window
// (nc 16-byte chunks per row, 16 * nc chunks = at most PD DMAs of 64 lanes;
// element e of the tile segment lands at 16 e of the wave's ring slot). The
// wave's ring holds D tiles; it waits only for its own transfers. Row sums
// of every tile go to LDS per (tile, row, wave) and are added in fixed wave
// order after the loop, so waves never wait for each other inside it.
template <int GT, int CPW, int PD, int NWMAX>
__global__ __launch_bounds__(64 * NWMAX, 2) void i4_matvec_seg(const uint8_t *__restrict__ w,
                                                             const float *__restrict__ x, float *__restrict__ y,
                                                             Geom gm) {
    (void)w;
    (void)y;  // (w, y, gm.M: see the tile map)
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int NW = gm.NW;
    const int rb = gm.row_bytes;
    const int G = GT ? GT : gm.G;
    const int Kp = gm.Gr * G;
    const int NWP = (NW + 3) & ~3;
    const int D = gm.depth;
    const int tiles = gm.tile_end[gm.nmat - 1];
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int ntile = wg < tiles ? (tiles - 1 - wg) / nwg + 1 : 0;

    // LDS: [NW waves][D slots][PD KB] rings, then the activation set-up, which
    // the per-tile sums [ntile][16][NWP] overlay once the operands are built
    unsigned char *ring = smem + static_cast<size_t>(wave) * D * (PD * kPiece);
    unsigned char *shared_area = smem + static_cast<size_t>(NW) * D * (PD * kPiece);
    float *part = reinterpret_cast<float *>(shared_area);
    XPlanes xp;
    xp.pl = reinterpret_cast<int8_t *>(shared_area);
    xp.stride = Kp;
    xp.pre = reinterpret_cast<int *>(xp.pl + 3 * Kp);
    xp.gexp = reinterpret_cast<float *>(xp.pre + Kp / 8);
    xp.gbase = 0;
    xp.ngroups = gm.Gr;
    XFirst xf;
    load_x_first<GT>(xf, x, gm.K, Kp);

    const int t0 = (gm.T * wave) / NW;
    const int nch = (gm.T * (wave + 1)) / NW - t0;  // 1..CPW by construction on the host
    int HO[CPW];
    unsigned HM[CPW];
    header_slots<GT, CPW>(gm, t0, nch, HO, HM);
    // this wave's segment of a row: [sb, sb + 16 nc), sb 16-aligned, covering
    // its windows and the headers they use (masked headers read offset 0 and
    // are never used)
    int lo = kChunk * t0;
#pragma unroll
    for (int c = 0; c < CPW; ++c)
        if (HM[c]) lo = min(lo, HO[c]);
    const int sb = __builtin_amdgcn_readfirstlane(lo & ~15);
    const int nc = __builtin_amdgcn_readfirstlane((kChunk * (t0 + nch) - sb + 15) / 16);  // <= 64 PD / 16 on the host
    const TileMap map(gm);

    // DMA sources of this lane: element e = 64 i + lane of the tile segment,
    // row e / nc, chunk e % nc (elements past 16 nc repeat the last one; they
    // land in the slot's unused tail)
    int poff[PD], pdst[PD];
#pragma unroll
    for (int i = 0; i < PD; ++i) {
        const int e = min(64 * i + lane, 16 * nc - 1);
        const int row = e / nc, ch = e - row * nc;
        poff[i] = row * rb + sb + 16 * ch;
        pdst[i] = kPiece * i;
    }
    auto dma = [&](int k, unsigned char *dst) {  // the wave's segment of its k-th tile (no rows past the last tile)
        const bool live = k < ntile;
        const TileRef r = map.at(live ? wg + k * nwg : 0);
        dma_tile(r.w, live ? r.M : 0, rb, r.tile, dst, poff, pdst, PD);
    };
    // the first two tiles go out before the activation set-up (a fixed count,
    // so the compiler's wait for the activation loads stays exact), the rest
    // of the ring after it
    dma(0, ring);
    dma(1, ring + PD * kPiece);
    prepare_x<GT, true>(xp, x, gm.K, gm.Gr, Kp, xf);
    for (int k = 2; k < D; ++k) dma(k, ring + k * (PD * kPiece));
    lds_barrier();
    v4i A0[CPW], A1[CPW];
    float E[CPW], C[CPW];
    int HO2[CPW];
    unsigned HM2[CPW];
    build_operands<GT, CPW, true>(xp, gm, t0, nch, A0, A1, E, C, HO2, HM2);
    lds_barrier();  // every wave is done with the set-up: the sums may overlay it
    for (int i = threadIdx.x; i < ntile * kTile * NWP; i += blockDim.x) lds_write_u32(part + i, 0u);  // padding stays 0
    lds_barrier();

    const int bn = lane & 15, kq = lane >> 4;
    int RO[CPW], RH[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int t = t0 + min(c, nch - 1);
        RO[c] = 16 * (bn * nc) + kChunk * t + 16 * kq - sb;
        RH[c] = 16 * (bn * nc) + (HM[c] ? HO[c] - sb : 0);
    }
    int issued = D;  // tiles whose DMAs are out (past ntile: zero-length)
    int b = 0;
    for (int k = 0; k < ntile; ++k) {
        wait_vmem((issued - k - 1) * PD);  // this wave's transfers of tile k have landed
        const unsigned char *buf = ring + b * (PD * kPiece);
        float a = 0.f;
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            const v4i d = *reinterpret_cast<const v4i *>(buf + RO[c]);
            const unsigned h = *reinterpret_cast<const unsigned *>(buf + RH[c]) & HM[c];
            a = window_step(a, d, h, A0[c], A1[c], E[c], C[c]);
        }
        // the slot's reads are complete (their values are used above): refill it
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (issued < ntile) {
            dma(issued, ring + b * (PD * kPiece));
            ++issued;
        }
        a = sum_rows4(a);  // the four group slots of each row
        if (lane < kTile) lds_write_u32(part + (k * kTile + lane) * NWP + wave, __builtin_bit_cast(unsigned, a));
        b = b == D - 1 ? 0 : b + 1;
    }
    wait_vmem(0);  // no transfer may still be writing this workgroup's LDS
    __syncthreads();
    for (int i = threadIdx.x; i < ntile * kTile; i += blockDim.x) {
        const int k = i / kTile, row_in = i - k * kTile;
        const float *pr = part + i * NWP;
        float sum = 0.f;
        for (int q = 0; q < NWP / 4; ++q) {  // fixed order; padding slots hold 0
            const float4 v = lds_read_f4(pr + 4 * q);
            sum += v.x;
            sum += v.y;
            sum += v.z;
            sum += v.w;
        }
        const TileRef r = map.at(wg + k * nwg);
        const int row = r.tile * kTile + row_in;
        if (row < r.M) store_y(r.y + row, sum);
    }
}

// One meeting of two partial sums of a row in a split-K tile: a 64-bit slot
// that is 0 when empty and (1 << 32 | float bits) when it holds the first
// arrival's value. Each side swaps its own value in; the side that gets a
// full slot back arrives second, adds the two in fixed order (first + second
// operand of the tree, whatever the arrival order) and empties the slot for
// the next launch. The value travels inside the atomic itself, so no other
// store has to be made visible first: one round trip to the device-coherent
// level per meeting.
__device__ inline bool meet_partial(unsigned long long *slot, bool second_operand, float &v) {
    const unsigned long long mine = (1ull << 32) | __builtin_bit_cast(unsigned, v);
    const unsigned long long old = __hip_atomic_exchange(slot, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((old >> 32) == 0) return false;  // first arrival: the other side carries on
    const float o = __builtin_bit_cast(float, static_cast<unsigned>(old));
    v = second_operand ? o + v : v + o;
    __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// Split-K variant for long rows and few tiles (down projections): the windows
// of every tile are split into S <= 4 parts, one workgroup per (tile, part). A
// workgroup converts only the activations of its part's groups, DMAs only the
// part's bytes of its 16 rows and reads the group headers straight from
// global memory. The S row sums meet in a binary tree of 64-bit exchange
// slots (meet_partial): parts 2j and 2j+1 meet first, then the winners of
// the two pairs (a part without a sibling goes straight up), so the sums are
// added as (p0 + p1) + (p2 + p3) whatever the arrival order (deterministic),
// and the last arrival stores the row. Slots: [tile][3][16], level-one pair
// slots 0 and 1, level-two slot 2; every launch leaves them empty.
template <int GT, int CPW, int PW, int NWMAX>
__global__ __launch_bounds__(64 * NWMAX, dma_waves_per_simd(CPW)) void i4_matvec_split(
    const uint8_t *__restrict__ w, const float *__restrict__ x, float *__restrict__ y, Geom gm,
    unsigned long long *__restrict__ slots) {
    static_assert(GT == 64 || GT == 128, "one activation block per thread needs a compile-time group size");
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int NW = gm.NW;
    const int M = gm.M, rb = gm.row_bytes, gb = gm.gb;
    const int NWP = (NW + 3) & ~3;
    const int S = gm.ksplit;
    const int tile = blockIdx.x / S, part = blockIdx.x - tile * S;
    const int tb = (gm.T * part) / S, te = (gm.T * (part + 1)) / S;  // windows [tb, te)
    const int Tp = te - tb;
    const int pitch = kChunk * Tp;  // LDS bytes per row
    const int byte_lo = kChunk * tb, byte_hi = min(kChunk * te, rb);
    const int g_lo = byte_lo / gb, g_hi = (byte_hi - 1) / gb + 1;  // groups the part touches
    const int ng = g_hi - g_lo;

    unsigned char *stage = smem;                                   // [16][pitch]
    float *part_sum = reinterpret_cast<float *>(smem + gm.tbuf);   // [16][NWP]
    XPlanes xp;
    xp.pl = reinterpret_cast<int8_t *>(part_sum + kTile * NWP);
    xp.stride = ng * GT;
    xp.pre = reinterpret_cast<int *>(xp.pl + 3 * xp.stride);
    xp.gexp = reinterpret_cast<float *>(xp.pre + xp.stride / 8);
    xp.gbase = g_lo;
    xp.ngroups = ng;

    // 1. the part's bytes of the 16 rows: Tp DMAs of 1 KB, chunk c = 64 j + lane
    //    -> row c / (4 Tp), 16-byte column c % (4 Tp); surplus slots repeat the last
    const __amdgpu_buffer_rsrc_t rs = rows_rsrc(w, M, rb, tile * kTile);
#pragma unroll
    for (int s = 0; s < PW; ++s) {
        const int j = min(wave + s * NW, Tp - 1);
        const int c = 64 * j + lane;
        const int r = c / (4 * Tp), col = c - r * (4 * Tp);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(stage + 1024 * j), 16,
                                                 r * rb + byte_lo + 16 * col, 0, 0, 0);
    }
    // 2. this lane's group headers (row bn, group slot kq of each of its windows)
    const int t0 = min(tb + (Tp * wave) / NW, te - 1);
    const int nch_raw = tb + (Tp * (wave + 1)) / NW - (tb + (Tp * wave) / NW);  // 0..CPW
    const int nch = max(nch_raw, 1);  // an idle wave still addresses one valid window
    const int bn = lane & 15, kq = lane >> 4;
    unsigned hraw[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int t = t0 + min(c, nch - 1);
        const int gq = min((kChunk * t) / gb + kq, gm.Gr - 1);
        hraw[c] = __builtin_amdgcn_raw_buffer_load_b32(rs, bn * rb + gq * gb, 0, 0);
    }
    // 3. the part's activations
    XFirst xf;
    load_x_first<GT>(xf, x + g_lo * GT, min(gm.K - g_lo * GT, ng * GT), ng * GT);
    prepare_x<GT, true>(xp, x + g_lo * GT, min(gm.K - g_lo * GT, ng * GT), ng, ng * GT, xf);
    wait_vmem(0);
    for (int i = threadIdx.x; i < kTile * NWP; i += blockDim.x)
        if (i % NWP >= NW) part_sum[i] = 0.f;  // padding slots of the fixed-order sums
    lds_barrier();
    v4i A0[CPW], A1[CPW];
    float E[CPW], C[CPW];
    int HO[CPW];
    unsigned HM[CPW];
    build_operands<GT, CPW, false>(xp, gm, t0, nch, A0, A1, E, C, HO, HM);
    float a = 0.f;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int t = t0 + min(c, nch - 1);
        const v4i d = *reinterpret_cast<const v4i *>(stage + bn * pitch + kChunk * (t - tb) + 16 * kq);
        a = window_step(a, d, hraw[c] & HM[c], A0[c], A1[c], E[c], C[c]);
    }
    if (nch_raw <= 0) a = 0.f;  // a part one window short of the widest leaves a wave idle
    a = sum_rows4(a);
    if (lane < kTile) part_sum[lane * NWP + wave] = a;
    __syncthreads();
    // 4. this part's 16 row sums climb the exchange tree; the last arrival stores
    if (threadIdx.x < kTile) {
        const float4 *pr = reinterpret_cast<const float4 *>(part_sum + threadIdx.x * NWP);
        float v = 0.f;
        for (int q = 0; q < NWP / 4; ++q) {
            const float4 u = pr[q];
            v += u.x;
            v += u.y;
            v += u.z;
            v += u.w;
        }
        unsigned long long *ts = slots + static_cast<size_t>(tile) * (3 * kTile) + threadIdx.x;
        bool alive = true;
        if ((part ^ 1) < S) alive = meet_partial(ts + (part >> 1) * kTile, part & 1, v);
        const int node = part >> 1, nodes = (S + 1) >> 1;
        if (alive && (node ^ 1) < nodes) alive = meet_partial(ts + 2 * kTile, node & 1, v);
        const int row = tile * kTile + threadIdx.x;
        if (alive && row < M) store_y(y + row, v);
    }
}


// ============================================================================================
// Register-only kernel (rows of 49..96 windows): operands straight from HBM.
template <int GT, int CPW>
__global__ __launch_bounds__(1024, 4) void i4_matvec_reg(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                         float *__restrict__ y, Geom gm) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int NW = gm.NW;
    const int M = gm.M, rb = gm.row_bytes;
    const int G = GT ? GT : gm.G;
    const int Kp = gm.Gr * G;
    const int NWP = (NW + 3) & ~3;
    float *part = reinterpret_cast<float *>(smem);  // [16][NWP]
    XPlanes xp;
    xp.pl = reinterpret_cast<int8_t *>(part + kTile * NWP);
    xp.stride = Kp;
    xp.pre = reinterpret_cast<int *>(xp.pl + 3 * Kp);
    xp.gexp = reinterpret_cast<float *>(xp.pre + Kp / 8);
    xp.gbase = 0;
    xp.ngroups = gm.Gr;

    const int tiles = (M + kTile - 1) / kTile;

    const int t0 = (gm.T * wave) / NW;
    const int nch = (gm.T * (wave + 1)) / NW - t0;
    const int bn = lane & 15, kq = lane >> 4;
    XFirst xf;
    load_x_first<GT>(xf, x, gm.K, Kp);
    prepare_x<GT>(xp, x, gm.K, gm.Gr, Kp, xf);
    for (int i = threadIdx.x; i < kTile * NWP; i += blockDim.x) part[i] = 0.f;
    __syncthreads();
    v4i A0[CPW], A1[CPW];
    float E[CPW], C[CPW];
    int HO[CPW];
    unsigned HM[CPW];
    build_operands<GT, CPW>(xp, gm, t0, nch, A0, A1, E, C, HO, HM);
    int DO[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) DO[c] = kChunk * (t0 + min(c, nch - 1)) + 16 * kq;

    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {  // round-robin, as in i4_matvec_dma
        const int row0 = tile * kTile;
        const __amdgpu_buffer_rsrc_t rs = rows_rsrc(w, M, rb, row0);
        const int lb = (min(row0 + bn, M - 1) - row0) * rb;
        v4i d[CPW];
        unsigned h[CPW];
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            d[c] = __builtin_amdgcn_raw_buffer_load_b128(rs, lb + DO[c], 0, 0);
            h[c] = __builtin_amdgcn_raw_buffer_load_b32(rs, lb + HO[c], 0, 0);
        }
        float a = 0.f;
#pragma unroll
        for (int c = 0; c < CPW; ++c) a = window_step(a, d[c], h[c] & HM[c], A0[c], A1[c], E[c], C[c]);
        a = sum_rows4(a);
        if (lane < kTile) part[lane * NWP + wave] = a;
        __syncthreads();
        if (threadIdx.x < kTile) {
            const float4 *pr = reinterpret_cast<const float4 *>(part + threadIdx.x * NWP);
            float s = 0.f;
            for (int q = 0; q < NWP / 4; ++q) {
                const float4 v = pr[q];
                s += v.x;
                s += v.y;
                s += v.z;
                s += v.w;
            }
            const int row = row0 + threadIdx.x;
            if (row < M) y[row] = s;
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void i4_matvec_rowwave(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                         float *__restrict__ y, int M, int K, int G, int gb, int Gr,
                                                         unsigned long long row_bytes) {
    const int lane = threadIdx.x & 63;
    const int wv = static_cast<int>((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nwv = static_cast<int>((gridDim.x * blockDim.x) >> 6);
    for (int row = wv; row < M; row += nwv) {
        const uint8_t *rp = w + static_cast<size_t>(row) * row_bytes;
        float acc = 0.f;
        for (int g = lane; g < Gr; g += 64) {
            const uint8_t *gp = rp + static_cast<size_t>(g) * gb;
            const float s = half_bits(gp[0] | (gp[1] << 8));
            const float z = half_bits(gp[2] | (gp[3] << 8));
            const int col = g * G;
            const int n = min(G, K - col);
            float part = 0.f;
            for (int i = 0; i < n; ++i) {
                const unsigned b = gp[kI4Header + (i >> 1)];
                const int q = (i & 1) ? static_cast<int>(b >> 4) : static_cast<int>(b & 15u);
                part = fmaf((static_cast<float>(q) - z) * s, x[col + i], part);
            }
            acc += part;
        }
        acc = wave_sum(acc);
        if (lane == 0) y[row] = acc;
    }
}

// Lets `fn` take `lds` bytes of dynamic LDS. Above the default 64 KB the
// limit is raised once per kernel, to what the CU's 160 KB leaves beside the
// kernel's static LDS; `limit` caches that figure (0: not raised yet).
int fit_dynamic_lds(const void *fn, size_t lds, size_t &limit) {
    if (lds <= 64 * 1024) return kOk;
    if (limit == 0) {
        hipFuncAttributes attr{};
        if (hipFuncGetAttributes(&attr, fn) != hipSuccess) return kLaunchFailed;
        if (attr.sharedSizeBytes >= static_cast<size_t>(kLdsBytes)) return kTooLarge;
        const size_t cap = kLdsBytes - attr.sharedSizeBytes;
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(cap)) != hipSuccess)
            return kLaunchFailed;
        limit = cap;
    }
    return lds <= limit ? kOk : kTooLarge;
}

size_t xplanes_bytes(const Geom &gm) {
    const size_t Kp = static_cast<size_t>(gm.Gr) * gm.G;
    return 3 * Kp + (Kp / 8) * 4 + static_cast<size_t>(gm.Gr) * 4;
}

template <typename KernelT>
int launch_with_lds(KernelT kernel, int grid, int threads, size_t lds, const uint8_t *w, const float *x, float *y,
                    const Geom &gm, hipStream_t stream, size_t &limit) {
    const int fit = fit_dynamic_lds(reinterpret_cast<const void *>(kernel), lds, limit);
    if (fit != kOk) return fit;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(threads), lds, stream, w, x, y, gm);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

int pipe_grid(int tiles) { return std::max(1, std::min(tiles, device_cu_count() * kPipeWgsPerCu)); }

template <int GT, int CPW, int NWMAX, bool AMAX = false>
int launch_pipe(const uint8_t *w, const float *x, float *y, const Geom &gm, hipStream_t stream) {
    const int tiles = gm.tile_end[gm.nmat - 1];
    const int NWP = (gm.NW + 3) & ~3;
    const size_t lds = static_cast<size_t>(2 * kTile * NWP) * 4 + xplanes_bytes(gm) + 16;
    const int grid = pipe_grid(tiles);
    // one tile per workgroup: nothing to load ahead (a second register slot
    // would only add a round of zero-length loads and an idle iteration)
    const bool one = tiles <= grid;
    if constexpr (AMAX) {
        static size_t limit_a1 = 0, limit_a = 0;
        if (gm.nmat != 1) return kBadShape;
        return one ? launch_with_lds(i4_matvec_pipe<GT, CPW, NWMAX, 1, false, true>, grid, 64 * gm.NW, lds, w, x, y,
                                     gm, stream, limit_a1)
                   : launch_with_lds(i4_matvec_pipe<GT, CPW, NWMAX, kPipeSlots, false, true>, grid, 64 * gm.NW, lds, w,
                                     x, y, gm, stream, limit_a);
    }
    if (gm.nmat > 1) {
        static size_t limit_g1 = 0, limit_g = 0;
        return one ? launch_with_lds(i4_matvec_pipe<GT, CPW, NWMAX, 1, true>, grid, 64 * gm.NW, lds, w, x, y, gm,
                                     stream, limit_g1)
                   : launch_with_lds(i4_matvec_pipe<GT, CPW, NWMAX, kPipeSlots, true>, grid, 64 * gm.NW, lds, w, x, y,
                                     gm, stream, limit_g);
    }
    static size_t limit_1 = 0, limit = 0;
    return one ? launch_with_lds(i4_matvec_pipe<GT, CPW, NWMAX, 1, false>, grid, 64 * gm.NW, lds, w, x, y, gm, stream,
                                 limit_1)
               : launch_with_lds(i4_matvec_pipe<GT, CPW, NWMAX, kPipeSlots, false>, grid, 64 * gm.NW, lds, w, x, y, gm,
                                 stream, limit);
}

// Wave-private ring for three windows per wave. Measured against the
// workgroup ring (i4_matvec_dma): faster for rows of more than 24 windows and
// for fewer than 32 tiles per CU (-7% to -17%); as fast or slower at 37 tiles
// per CU with 23 windows (the 151936x2560 lm_head), and slower for two windows
// per wave. One workgroup per CU with a three-tile ring up to 8 tiles per CU,
// else two with two-tile rings.
template <int GT, int CPW, int NWMAX>
int launch_seg(const uint8_t *w, const float *x, float *y, const Geom &gm, hipStream_t stream) {
    constexpr int PD = 4;  // DMAs per wave per tile: a row segment of at most 64 B of header lead-in + 3 windows
    static_assert(kChunk * CPW + 48 <= 16 * PD * 4, "segment fits the slot");
    const int tiles = gm.tile_end[gm.nmat - 1];
    const int NWP = (gm.NW + 3) & ~3;
    const int cus = device_cu_count();
    const int wgs = tiles <= 8 * cus ? 1 : 2, depth = wgs == 1 ? 3 : 2;
    const int grid = std::max(1, std::min(tiles, cus * wgs));
    const int per_wg = (tiles + grid - 1) / grid;
    const size_t rings = static_cast<size_t>(gm.NW) * depth * PD * kPiece;
    const size_t shared_area = std::max(xplanes_bytes(gm), static_cast<size_t>(per_wg) * kTile * NWP * 4);
    const size_t lds = rings + shared_area + 16;
    if (lds > kLdsBytes) return kTooLarge;
    Geom g2 = gm;
    g2.depth = depth;
    static size_t limit = 0;
    return launch_with_lds(i4_matvec_seg<GT, CPW, PD, NWMAX>, grid, 64 * gm.NW, lds, w, x, y, g2, stream, limit);
}

template <int GT, int CPW, int PW, int NWMAX>
int launch_dma(const uint8_t *w, const float *x, float *y, const Geom &gm, hipStream_t stream) {
    static size_t limit = 0;
    const int tiles = gm.tile_end[gm.nmat - 1];
    const int NWP = (gm.NW + 3) & ~3;
    Geom g2 = gm;
    const size_t tile = static_cast<size_t>(kTile) * gm.row_bytes;
    const size_t tbuf = std::max<size_t>((tile + kChunk + 15) / 16 * 16, kPiece);
    const size_t fixed = static_cast<size_t>(2 * kTile * NWP) * 4 + xplanes_bytes(gm) + 16;
    // Workgroups per CU: as many as the wave budget allows (at most 2) while a
    // three-slot ring still fits. Ring depth: enough tiles in flight per CU
    // for the HBM latency-bandwidth product, within the LDS left.
    if ((GT == 64 || GT == 128) && static_cast<size_t>(gm.Gr) * GT / 8 > static_cast<size_t>(64 * gm.NW))
        return kTooLarge;  // the activation set-up assumes one 8-element block per thread
    int wgs = std::max(1, std::min(4, 4 * dma_waves_per_simd(CPW) / gm.NW));
    {
        // The DMA ring pays off only for long rows over many tiles: one window
        // per wave, or at most two tiles per workgroup slot, run faster on the
        // register path -- except three windows per wave over more tiles than
        // the register path has workgroups (9728x2560: 7.6 us on the
        // wave-private ring below, 9.7 us on the register path).
        const size_t lds2 = 2 * tbuf + fixed;
        int wgs2 = wgs;
        while (wgs2 > 1 && static_cast<size_t>(wgs2) * lds2 > kLdsBytes) --wgs2;
        const int slots = device_cu_count() * wgs2;
        const bool pipe_one_round = CPW != 3 || tiles <= device_cu_count() * kPipeWgsPerCu;
        if (CPW == 1 || (tiles <= 2 * slots && pipe_one_round)) return launch_pipe<GT, CPW, NWMAX>(w, x, y, gm, stream);
    }
    if constexpr (CPW == 3) {
        if (gm.T > 24 || tiles < 32 * device_cu_count()) {
            const int st = launch_seg<GT, CPW, NWMAX>(w, x, y, gm, stream);
            if (st != kTooLarge) return st;
        }
    }
    while (wgs > 1 && static_cast<size_t>(wgs) * (3 * tbuf + fixed) > kLdsBytes) --wgs;
    if (3 * tbuf + fixed > kLdsBytes) return kTooLarge;
    const int grid = std::max(1, std::min(tiles, device_cu_count() * wgs));
    const int per_wg = (tiles + grid - 1) / grid;
    const size_t lds_cap = kLdsBytes / wgs;
    int depth = static_cast<int>(std::min<size_t>(kMaxDepth, (lds_cap - fixed) / tbuf));
    const size_t want = (kInflightPerCu + static_cast<size_t>(wgs) * tile - 1) / (static_cast<size_t>(wgs) * tile) + 1;
    depth = std::max(3, std::min({depth, static_cast<int>(want), std::max(3, per_wg)}));
    g2.tbuf = static_cast<int>(tbuf);
    g2.depth = depth;
    const size_t lds = depth * tbuf + fixed;
    return launch_with_lds(i4_matvec_dma<GT, CPW, PW, NWMAX>, grid, 64 * gm.NW, lds, w, x, y, g2, stream, limit);
}


template <int GT, int CPW, int PW, int NWMAX>
int launch_split(const uint8_t *w, const float *x, float *y, Geom gm, int S, int Tmax, hipStream_t stream) {
    static size_t limit = 0;
    const int tiles = (gm.M + kTile - 1) / kTile;
    const int NWP = (gm.NW + 3) & ~3;
    const int ng = (kChunk * Tmax + gm.gb - 1) / gm.gb + 1;  // groups one part can touch
    const size_t kp = static_cast<size_t>(ng) * GT;
    if (kp / 8 > static_cast<size_t>(64 * gm.NW)) return kTooLarge;  // one activation block per thread
    gm.tbuf = kTile * kChunk * Tmax;
    gm.ksplit = S;
    const size_t lds = gm.tbuf + static_cast<size_t>(kTile * NWP) * 4 + 3 * kp + kp / 8 * 4 + ng * 4 + 16;
    if (lds > kLdsBytes) return kTooLarge;
    if (S < 2 || S > 4) return kTooLarge;  // the exchange tree has two levels
    unsigned long long *slots = nullptr;
    const int st = scratch_split_slots(stream, static_cast<size_t>(tiles) * 3 * kTile, &slots);
    if (st != kOk) return st;
    const int fit = fit_dynamic_lds(reinterpret_cast<const void *>(i4_matvec_split<GT, CPW, PW, NWMAX>), lds, limit);
    if (fit != kOk) return fit;
    hipLaunchKernelGGL((i4_matvec_split<GT, CPW, PW, NWMAX>), dim3(tiles * S), dim3(64 * gm.NW), lds, stream, w, x, y,
                       gm, slots);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

// Split-K when the rows are long and the tiles few: S parts of at least 8
// windows, enough workgroups for about two per CU.
template <int GT>
int launch_split_for(const uint8_t *w, const float *x, float *y, Geom gm, hipStream_t stream) {
    const int tiles = (gm.M + kTile - 1) / kTile;
    const int slots = 2 * device_cu_count();
    if (gm.T < 24 || 2 * tiles > slots || gm.row_bytes % 16 != 0) return kTooLarge;
    const int S = std::min({4, slots / tiles, gm.T / 8});
    if (S < 2) return kTooLarge;
    const int Tmax = (gm.T + S - 1) / S;
    if (Tmax <= 8) {
        gm.NW = Tmax;
        return launch_split<GT, 1, 1, 8>(w, x, y, gm, S, Tmax, stream);
    }
    if (Tmax <= 16) {
        gm.NW = (Tmax + 1) / 2;
        return launch_split<GT, 2, 2, 8>(w, x, y, gm, S, Tmax, stream);
    }
    if (Tmax <= 24) {
        gm.NW = (Tmax + 2) / 3;
        return launch_split<GT, 3, 3, 8>(w, x, y, gm, S, Tmax, stream);
    }
    gm.NW = (Tmax + 2) / 3;
    return launch_split<GT, 3, 3, 16>(w, x, y, gm, S, Tmax, stream);
}

template <int GT, int CPW>
int launch_reg(const uint8_t *w, const float *x, float *y, const Geom &gm, hipStream_t stream) {
    static size_t limit = 0;
    const int tiles = (gm.M + kTile - 1) / kTile;
    const int NWP = (gm.NW + 3) & ~3;
    const size_t lds = static_cast<size_t>(kTile * NWP) * 4 + xplanes_bytes(gm) + 16;
    const int grid = std::max(1, std::min(tiles, device_cu_count()));
    return launch_with_lds(i4_matvec_reg<GT, CPW>, grid, 64 * gm.NW, lds, w, x, y, gm, stream, limit);
}

// Picks windows-per-wave, pieces-per-wave and waves for a row of T 64-byte windows.
template <int GT>
int launch_mfma_for(const uint8_t *w, const float *x, float *y, Geom gm, hipStream_t stream) {
    const int T = gm.T;
    auto pw_of = [&](int nw) { return (gm.pieces + nw - 1) / nw; };
    if (T <= 8) {
        gm.NW = T;
        switch (pw_of(gm.NW)) {
            case 1: return launch_dma<GT, 1, 1, 8>(w, x, y, gm, stream);
            case 2: return launch_dma<GT, 1, 2, 8>(w, x, y, gm, stream);
            case 3: return launch_dma<GT, 1, 3, 8>(w, x, y, gm, stream);
            default: return launch_dma<GT, 1, 4, 8>(w, x, y, gm, stream);
        }
    }
    if (T <= 16) {
        gm.NW = (T + 1) / 2;
        switch (pw_of(gm.NW)) {
            case 1: case 2: return launch_dma<GT, 2, 2, 8>(w, x, y, gm, stream);
            case 3: return launch_dma<GT, 2, 3, 8>(w, x, y, gm, stream);
            default: return launch_dma<GT, 2, 4, 8>(w, x, y, gm, stream);
        }
    }
    if (T <= 24) {
        gm.NW = (T + 2) / 3;
        return pw_of(gm.NW) <= 3 ? launch_dma<GT, 3, 3, 8>(w, x, y, gm, stream)
                                 : launch_dma<GT, 3, 4, 8>(w, x, y, gm, stream);
    }
    if (T <= 48) {
        gm.NW = (T + 2) / 3;
        return pw_of(gm.NW) <= 3 ? launch_dma<GT, 3, 3, 16>(w, x, y, gm, stream)
                                 : launch_dma<GT, 3, 4, 16>(w, x, y, gm, stream);
    }
    if (T <= 64) {
        gm.NW = (T + 3) / 4;
        return launch_reg<GT, 4>(w, x, y, gm, stream);
    }
    if (T <= 96) {
        gm.NW = (T + 5) / 6;
        return launch_reg<GT, 6>(w, x, y, gm, stream);
    }
    return kTooLarge;
}

}  // namespace

int launch_i4_matvec_generic(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                             hipStream_t stream) {
    if (out_dim < 1 || in_dim < 1) return kBadShape;
    if (group_size < 2 || (group_size & 1)) return kBadGroup;
    if (!w || !x || !y) return kBadShape;  // nothing is launched on a null operand
    const int gb = i4_group_bytes(group_size);
    const int Gr = i4_groups(in_dim, group_size);
    const unsigned long long rb = i4_row_bytes(in_dim, group_size);
    const int waves_per_block = 4;
    const int grid = std::max(1, std::min((out_dim + waves_per_block - 1) / waves_per_block, device_cu_count() * 8));
    hipLaunchKernelGGL(i4_matvec_rowwave, dim3(grid), dim3(64 * waves_per_block), 0, stream, w, x, y, out_dim,
                       in_dim, group_size, gb, Gr, rb);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

namespace {

// The geometry of one matrix for the MFMA kernels (launch_i4_matvec's fast groups).
Geom one_matrix_geom(const uint8_t *w, float *y, int out_dim, int in_dim, int group_size) {
    const size_t rb = i4_row_bytes(in_dim, group_size);
    Geom gm;
    gm.M = out_dim;
    gm.K = in_dim;
    gm.G = group_size;
    gm.gb = i4_group_bytes(group_size);
    gm.Gr = i4_groups(in_dim, group_size);
    gm.row_bytes = static_cast<int>(rb);
    gm.T = static_cast<int>((rb + kChunk - 1) / kChunk);
    gm.NW = 1;
    int rbp = static_cast<int>((rb + 15) & ~static_cast<size_t>(15));
    if (((rbp / 16) & 1) == 0) rbp += 16;  // odd multiple of 16: 16-row column reads avoid bank conflicts
    gm.rbp = rbp;
    gm.pieces = static_cast<int>((static_cast<size_t>(kTile) * rb + kPiece - 1) / kPiece);
    gm.xoff = 0;
    gm.tbuf = 0;
    gm.depth = 0;
    gm.nmat = 1;
    for (int j = 0; j < kMaxGroup; ++j) {
        gm.tile_end[j] = (out_dim + kTile - 1) / kTile;
        gm.mrows[j] = out_dim;
        gm.mw[j] = w;
        gm.my[j] = y;
    }
    gm.ksplit = 1;
    gm.amax_v = nullptr;
    gm.amax_i = nullptr;
    return gm;
}

}  // namespace

int launch_i4_matvec(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                     hipStream_t stream) {
    if (out_dim < 1 || in_dim < 1) return kBadShape;
    if (group_size < 2 || (group_size & 1)) return kBadGroup;
    if (!w || !x || !y) return kBadShape;  // nothing is launched on a null operand
    const size_t rb = i4_row_bytes(in_dim, group_size);
    const bool fast_group = (group_size % 8 == 0) && group_size >= 40;
    if (!fast_group || rb * kTile * 2 >= (1ull << 31))
        return launch_i4_matvec_generic(w, x, y, out_dim, in_dim, group_size, stream);
    Geom gm = one_matrix_geom(w, y, out_dim, in_dim, group_size);
    int st;
    {
        const I4Mat m{w, x, y, out_dim, in_dim};
        st = launch_i4_matvec_set_fit(1, &m, group_size, stream);
        if (st != kNotFused) return st;
    }
    if ((group_size == 64 || group_size == 128)) {
        st = group_size == 64 ? launch_split_for<64>(w, x, y, gm, stream) : launch_split_for<128>(w, x, y, gm, stream);
        if (st != kTooLarge) return st;
    }
    if (group_size == 64)
        st = launch_mfma_for<64>(w, x, y, gm, stream);
    else if (group_size == 128)
        st = launch_mfma_for<128>(w, x, y, gm, stream);
    else
        st = launch_mfma_for<0>(w, x, y, gm, stream);
    if (st == kTooLarge) return launch_i4_matvec_generic(w, x, y, out_dim, in_dim, group_size, stream);
    return st;
}

namespace {

// The register-path geometry launch_i4_matvec uses for this one matrix, and its workgroup count,
// when that is its choice at G = 64 with at most cap workgroups: not the set kernel, rows of at
// most 8 windows (the split-K and longer-row kernels start above), within the register path's
// activation set-up limit.
bool amax_plan(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size, int cap, Geom &gm,
               int &grid) {
    if (out_dim < 1 || in_dim < 1 || group_size != 64) return false;
    const size_t rb = i4_row_bytes(in_dim, group_size);
    if (rb * kTile * 2 >= (1ull << 31)) return false;
    const I4Mat m{w, x, y, out_dim, in_dim};
    if (i4_set_fit_takes(1, &m, group_size)) return false;
    gm = one_matrix_geom(w, y, out_dim, in_dim, group_size);
    if (gm.T > 8) return false;
    gm.NW = gm.T;
    if (static_cast<size_t>(gm.Gr) * 64 / 8 > static_cast<size_t>(64 * gm.NW)) return false;
    grid = pipe_grid(gm.tile_end[0]);
    return grid <= cap;
}

}  // namespace

bool i4_matvec_amax_takes(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                          int cap) {
    Geom gm;
    int grid = 0;
    return amax_plan(w, x, y, out_dim, in_dim, group_size, cap, gm, grid);
}

int launch_i4_matvec_amax(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                          float *pv, int *pi, int cap, int *parts, hipStream_t stream) {
    if (out_dim < 1 || in_dim < 1 || !w || !x || !y || !pv || !pi || !parts) return kBadShape;
    Geom gm;
    int grid = 0;
    if (!amax_plan(w, x, y, out_dim, in_dim, group_size, cap, gm, grid)) return kNotFused;
    gm.amax_v = pv;
    gm.amax_i = pi;
    *parts = grid;
    return launch_pipe<64, 1, 8, true>(w, x, y, gm, stream);
}

// Matvecs of n (<= 3) matrices that share x, in_dim and group_size (the
// reference's pair and qkv forms): one DMA-staged launch whose tiles run over
// the matrices one after the other, else one launch per matrix.
int launch_i4_matvec_group(int n, const uint8_t *const *w, float *const *y, const int *out_dim, const float *x,
                           int in_dim, int group_size, hipStream_t stream) {
    if (n < 1 || n > kMaxGroup || in_dim < 1) return kBadShape;
    if (group_size < 2 || (group_size & 1)) return kBadGroup;
    if (!x) return kBadShape;
    for (int j = 0; j < n; ++j)
        if (out_dim[j] < 1 || !w[j] || !y[j]) return kBadShape;
    const size_t rb = i4_row_bytes(in_dim, group_size);
    const int T = static_cast<int>((rb + kChunk - 1) / kChunk);
    {  // the set kernel takes all n in one launch where it applies (rows sharing x)
        I4Mat m[kMaxGroup];
        for (int j = 0; j < n; ++j) m[j] = I4Mat{w[j], x, y[j], out_dim[j], in_dim};
        const int st = launch_i4_matvec_set_fit(n, m, group_size, stream);
        if (st != kNotFused) return st;
    }
    const bool grouped = n > 1 && (group_size % 8 == 0) && group_size >= 40 && T <= 48 &&
                         rb * kTile * 2 < (1ull << 31);
    if (!grouped) {
        for (int j = 0; j < n; ++j) {
            const int st = launch_i4_matvec(w[j], x, y[j], out_dim[j], in_dim, group_size, stream);
            if (st != kOk) return st;
        }
        return kOk;
    }
    Geom gm;
    gm.M = out_dim[0];
    gm.K = in_dim;
    gm.G = group_size;
    gm.gb = i4_group_bytes(group_size);
    gm.Gr = i4_groups(in_dim, group_size);
    gm.row_bytes = static_cast<int>(rb);
    gm.T = T;
    gm.NW = 1;
    gm.rbp = 0;
    gm.pieces = static_cast<int>((static_cast<size_t>(kTile) * rb + kPiece - 1) / kPiece);
    gm.xoff = 0;
    gm.tbuf = 0;
    gm.depth = 0;
    gm.nmat = n;
    gm.ksplit = 1;
    int end = 0;
    for (int j = 0; j < kMaxGroup; ++j) {
        const int jj = std::min(j, n - 1);  // unused slots repeat the last matrix (never selected)
        if (j < n) end += (out_dim[j] + kTile - 1) / kTile;
        gm.tile_end[j] = end;
        gm.mrows[j] = out_dim[jj];
        gm.mw[j] = w[jj];
        gm.my[j] = y[jj];
    }
    const int st = group_size == 64    ? launch_mfma_for<64>(w[0], x, y[0], gm, stream)
                   : group_size == 128 ? launch_mfma_for<128>(w[0], x, y[0], gm, stream)
                                       : launch_mfma_for<0>(w[0], x, y[0], gm, stream);
    if (st != kTooLarge) return st;
    for (int j = 0; j < n; ++j) {  // the staged kernel does not fit: one launch per matrix
        const int sj = launch_i4_matvec(w[j], x, y[j], out_dim[j], in_dim, group_size, stream);
        if (sj != kOk) return sj;
    }
    return kOk;
}

}  // namespace tqhip
