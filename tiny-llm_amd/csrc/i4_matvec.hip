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
//   * A workgroup owns a contiguous range of 16-row tiles; each tile is one
//     contiguous block of memory. The tile is streamed into LDS with
//     coalesced 1 KB-per-instruction loads kept two tiles ahead in VGPRs,
//     double-buffered in LDS, and the MFMA operands (codes and group headers)
//     are read back from LDS. The row windows are split over the waves and the
//     per-wave partial sums are added in a fixed order (deterministic).
//   * Rows longer than 48 windows use the register-only variant, which loads
//     the operands straight from HBM.
// Portable path (any even G): one wave per row, fp32 accumulation.

#include "tq_common.h"

#include <algorithm>

namespace tqhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;     // bytes of one weight row covered by one MFMA pair ("window")
constexpr int kTile = 16;      // weight rows per MFMA tile
constexpr int kPiece = 1024;   // bytes one wave streams per 16-byte-per-lane load
constexpr unsigned kNibbles = 0x0F0F0F0Fu;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family word 3)

// DPP controls (gfx9): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_ror:8, row_shr:n.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppRor8 = 0x128;
constexpr int kDppShr1 = 0x111, kDppShr2 = 0x112, kDppShr4 = 0x114, kDppShr8 = 0x118;

__device__ inline float half_bits(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xFFFFu)));
}

__device__ inline float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ inline float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

template <int CTRL>
__device__ inline float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ inline int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Position of element i of a group inside its 8-element block, in the order
// the weight operand presents it: even elements (low nibbles) first, then odd.
__device__ inline int plane_pos(int i) {
    const int j = i & 7;
    return (i & ~7) + ((j & 1) ? 4 + (j >> 1) : (j >> 1));
}

__device__ inline int group_exponent(float m) {
    if (!(m > 0.f)) return 0;
    int e;
    frexpf(m, &e);  // m in [2^(e-1), 2^e)
    return min(22 - e, 149);
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
};

// LDS view of the activation set-up shared by both kernels.
struct XPlanes {
    int8_t *pl;    // 3 planes x Kp bytes, 8-element blocks in operand order
    int *pre;      // per group: inclusive prefix over its 8-element blocks of sum(X)
    float *gexp;   // 2^-f per group
};

// ---- 1. activations -> per-group exponent, integer planes, prefix block sums
// GT = 64 or 128: one lane per 8-element block, group max and prefix by DPP.
template <int GT>
__device__ void prepare_x(const XPlanes &xp, const float *__restrict__ x, int K, int Gr, int Kp) {
    if constexpr (GT == 64 || GT == 128) {
        constexpr int LPG = GT / 8;  // lanes (blocks) per group: 8 or 16
        const int nblk = Kp / 8;
        // every lane of a block-group takes part in the DPP steps, so the loop
        // runs whole waves and masks work past the last block instead
        const int stride = blockDim.x;
        const int nrounds = (nblk + stride - 1) / stride;
        const int lane = threadIdx.x & 63;
        for (int rd = 0; rd < nrounds; ++rd) {
            const int b = rd * stride + threadIdx.x;
            const bool live = b < nblk;
            float v[8];
            float m = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int k = 8 * b + i;
                v[i] = (live && k < K) ? x[k] : 0.f;
                m = fmaxf(m, fabsf(v[i]));
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
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    *reinterpret_cast<uint2 *>(xp.pl + p * Kp + 8 * b) = make_uint2(w[p][0], w[p][1]);
                xp.pre[b] = s;
                if (j == 0) xp.gexp[b / LPG] = ldexpf(1.f, -f);
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
                if (k < K) m = fmaxf(m, fabsf(x[k]));
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
            if (lane == 0) xp.gexp[g] = ldexpf(1.f, -f);
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

// ---- 2. per-lane, row-invariant activation operands and group constants for
// windows t0 .. t0+nch-1 (CPW slots; unused slots get a zero operand).
template <int GT, int CPW>
__device__ void build_operands(const XPlanes &xp, const Geom &gm, int t0, int nch, v4i (&A0)[CPW], v4i (&A1)[CPW],
                               float (&E)[CPW], float (&C)[CPW], int (&HO)[CPW], unsigned (&HM)[CPW]) {
    const int G = GT ? GT : gm.G;
    const int gb = GT ? kI4Header + GT / 2 : gm.gb;
    const int Gr = gm.Gr, rb = gm.row_bytes, Kp = Gr * G;
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
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // q = 2*u + dw
            const int o = kChunk * t + 4 * (4 * kq + q);
            const int g = o / gb;
            const int r = o - g * gb;
            const bool use = own && o < rb && ap < 3 && r >= kI4Header && g - gt == ah;
            const int blk = use ? (g * G + 2 * (r - kI4Header)) >> 3 : 0;
            const uint2 v = *reinterpret_cast<const uint2 *>(xp.pl + apc * Kp + 8 * blk);
            lo[q] = use ? v.x : 0u;
            hi[q] = use ? v.y : 0u;
        }
        A0[c] = v4i{static_cast<int>(lo[0]), static_cast<int>(hi[0]), static_cast<int>(lo[1]), static_cast<int>(hi[1])};
        A1[c] = v4i{static_cast<int>(lo[2]), static_cast<int>(hi[2]), static_cast<int>(lo[3]), static_cast<int>(hi[3])};
        // group slot kq of this window: its data bytes inside the window
        const int gq = gt + kq;
        const int wbeg = kChunk * t, wend = min(kChunk * (t + 1), rb);
        const int dbeg = max(gq * gb + kI4Header, wbeg), dend = min((gq + 1) * gb, wend);
        const bool valid = own && gq < Gr && gq * gb < wend;
        int sum = 0;
        if (valid && dend > dbeg) {
            const int b0 = gq * (G / 8) + (dbeg - gq * gb - kI4Header) / 4;  // first block in the window
            const int b1 = gq * (G / 8) + (dend - gq * gb - kI4Header) / 4;  // one past the last
            sum = xp.pre[b1 - 1] - (b0 > gq * (G / 8) ? xp.pre[b0 - 1] : 0);
        }
        E[c] = valid ? xp.gexp[min(gq, Gr - 1)] : 0.f;
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

__device__ inline __amdgpu_buffer_rsrc_t rows_rsrc(const uint8_t *w, int M, int row_bytes, int row0) {
    const size_t rem = static_cast<size_t>(M - row0) * row_bytes;
    const int nrec = rem > 0xFFFFFFFFull ? -1 : static_cast<int>(static_cast<unsigned>(rem));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w) + static_cast<size_t>(row0) * row_bytes,
                                             static_cast<short>(0), nrec, kBufferFlags);
}

// ============================================================================================
// LDS-staged kernel (rows of up to 48 windows).
//   GT: compile-time group size (0 = run time). CPW: windows per wave.
//   PW: 1 KB pieces per wave per tile. NWMAX: waves per workgroup bound.
template <int GT, int CPW, int PW, int NWMAX>
__global__ __launch_bounds__(64 * NWMAX, 4) void i4_matvec_lds(const uint8_t *__restrict__ w,
                                                               const float *__restrict__ x, float *__restrict__ y,
                                                               Geom gm) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int NW = gm.NW;
    const int M = gm.M, rb = gm.row_bytes, rbp = gm.rbp;
    const int G = GT ? GT : gm.G;
    const int Kp = gm.Gr * G;
    const int NWP = (NW + 3) & ~3;
    const int tbuf = kTile * rbp + kChunk;  // bytes of one staged tile (slack for the last window)

    unsigned char *stage = smem;                                         // [2][tbuf]
    float *part = reinterpret_cast<float *>(smem + 2 * tbuf);            // [2][16][NWP]
    XPlanes xp;
    xp.pl = reinterpret_cast<int8_t *>(part + 2 * kTile * NWP);
    xp.pre = reinterpret_cast<int *>(xp.pl + 3 * Kp);
    xp.gexp = reinterpret_cast<float *>(xp.pre + Kp / 8);

    const int tiles = (M + kTile - 1) / kTile;
    const int my0 = static_cast<int>(static_cast<long long>(tiles) * blockIdx.x / gridDim.x);
    const int my1 = static_cast<int>(static_cast<long long>(tiles) * (blockIdx.x + 1) / gridDim.x);
    const int ntile = my1 - my0;

    // Pieces of a tile this lane moves: tile-relative byte offset and its LDS
    // destination (row-padded). Identical for every tile.
    int poff[PW], pdst[PW];
    bool pown[PW];
#pragma unroll
    for (int s = 0; s < PW; ++s) {
        const int j = wave + s * NW;
        const int o = kPiece * j + 16 * lane;
        // o and the tile size 16*rb are multiples of 16: a 16-byte piece lies
        // entirely inside the tile or entirely past it (the last piece's tail).
        pown[s] = j < gm.pieces && o < kTile * rb;
        poff[s] = o;
        const int row = o / rb;
        pdst[s] = row * rbp + (o - row * rb);
    }
    const bool aligned16 = (rb & 15) == 0;  // a 16-byte piece never straddles two rows

    auto issue = [&](v4i (&v)[PW], int tile) {
        const __amdgpu_buffer_rsrc_t rs = rows_rsrc(w, M, rb, tile * kTile);
#pragma unroll
        for (int s = 0; s < PW; ++s)
            if (pown[s]) v[s] = __builtin_amdgcn_raw_buffer_load_b128(rs, poff[s], 0, 0);
    };
    auto stash = [&](const v4i (&v)[PW], unsigned char *buf) {
#pragma unroll
        for (int s = 0; s < PW; ++s) {
            if (!pown[s]) continue;
            if (aligned16) {
                *reinterpret_cast<v4i *>(buf + pdst[s]) = v[s];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int o = poff[s] + 4 * e;
                    const int row = o / rb;
                    *reinterpret_cast<int *>(buf + row * rbp + (o - row * rb)) = v[s][e];
                }
            }
        }
    };

    // Tiles my0 and my0+1 start streaming before the activation set-up.
    v4i V0[PW], V1[PW];
    if (ntile > 0) issue(V0, my0);
    if (ntile > 1) issue(V1, my0 + 1);

    prepare_x<GT>(xp, x, gm.K, gm.Gr, Kp);
    __syncthreads();

    const int t0 = (gm.T * wave) / NW;
    const int nch = (gm.T * (wave + 1)) / NW - t0;  // 1..CPW by construction on the host
    v4i A0[CPW], A1[CPW];
    float E[CPW], C[CPW];
    int HO[CPW];
    unsigned HM[CPW];
    build_operands<GT, CPW>(xp, gm, t0, nch, A0, A1, E, C, HO, HM);
    // LDS offsets of this lane's operand column and headers within a staged tile
    const int bn = lane & 15, kq = lane >> 4;
    int RO[CPW], RH[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int t = t0 + min(c, nch - 1);
        RO[c] = bn * rbp + kChunk * t + 16 * kq;
        RH[c] = bn * rbp + HO[c];
    }

    if (ntile > 0) stash(V0, stage);
    if (ntile > 2) issue(V0, my0 + 2);

    auto reduce_prev = [&](int i) {  // partial sums of tile i (written before the last barrier)
        const float *pb = part + (i & 1) * (kTile * NWP);
        if (threadIdx.x < kTile) {
            const float4 *pr = reinterpret_cast<const float4 *>(pb + threadIdx.x * NWP);
            float s = 0.f;
            for (int q = 0; q < NWP / 4; ++q) {  // fixed order; padding slots hold 0
                const float4 v = pr[q];
                s += v.x;
                s += v.y;
                s += v.z;
                s += v.w;
            }
            const int row = (my0 + i) * kTile + threadIdx.x;
            if (row < M) y[row] = s;
        }
    };
    auto compute = [&](int i) {
        const unsigned char *buf = stage + (i & 1) * tbuf;
        float a = 0.f;
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            const v4i d = *reinterpret_cast<const v4i *>(buf + RO[c]);
            const unsigned h = *reinterpret_cast<const unsigned *>(buf + RH[c]) & HM[c];
            a = window_step(a, d, h, A0[c], A1[c], E[c], C[c]);
        }
        a += __shfl_xor(a, 16);  // the four group slots of each row
        a += __shfl_xor(a, 32);
        float *pb = part + (i & 1) * (kTile * NWP);
        if (lane < kTile) pb[lane * NWP + wave] = a;
    };

    for (int i = threadIdx.x; i < 2 * kTile * NWP; i += blockDim.x) part[i] = 0.f;

    // Pipeline: tile i is in LDS buffer i&1, tile i+1 in VGPRs (V1/V0 by parity),
    // tile i+2 being fetched.
    for (int i = 0; i < ntile; i += 2) {
        __syncthreads();
        if (i + 1 < ntile) stash(V1, stage + tbuf);
        if (i + 3 < ntile) issue(V1, my0 + i + 3);
        compute(i);
        if (i > 0) reduce_prev(i - 1);
        if (i + 1 >= ntile) break;
        __syncthreads();
        if (i + 2 < ntile) stash(V0, stage);
        if (i + 4 < ntile) issue(V0, my0 + i + 4);
        compute(i + 1);
        reduce_prev(i);
    }
    __syncthreads();
    if (ntile > 0) reduce_prev(ntile - 1);
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
    xp.pre = reinterpret_cast<int *>(xp.pl + 3 * Kp);
    xp.gexp = reinterpret_cast<float *>(xp.pre + Kp / 8);

    const int tiles = (M + kTile - 1) / kTile;
    const int my0 = static_cast<int>(static_cast<long long>(tiles) * blockIdx.x / gridDim.x);
    const int my1 = static_cast<int>(static_cast<long long>(tiles) * (blockIdx.x + 1) / gridDim.x);

    const int t0 = (gm.T * wave) / NW;
    const int nch = (gm.T * (wave + 1)) / NW - t0;
    const int bn = lane & 15, kq = lane >> 4;
    prepare_x<GT>(xp, x, gm.K, gm.Gr, Kp);
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

    for (int tile = my0; tile < my1; ++tile) {
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
        a += __shfl_xor(a, 16);
        a += __shfl_xor(a, 32);
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

int device_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        TQ_HIP_CHECK(hipGetDevice(&dev));
        TQ_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        if (cus < 1) cus = 1;
    }
    return cus;
}

size_t xplanes_bytes(const Geom &gm) {
    const size_t Kp = static_cast<size_t>(gm.Gr) * gm.G;
    return 3 * Kp + (Kp / 8) * 4 + static_cast<size_t>(gm.Gr) * 4;
}

template <typename KernelT>
int launch_with_lds(KernelT kernel, int grid, int threads, size_t lds, const uint8_t *w, const float *x, float *y,
                    const Geom &gm, hipStream_t stream, bool &raised) {
    if (lds > 160 * 1024) return kTooLarge;
    if (lds > 64 * 1024 && !raised) {
        TQ_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        raised = true;
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(threads), lds, stream, w, x, y, gm);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

template <int GT, int CPW, int PW, int NWMAX>
int launch_lds(const uint8_t *w, const float *x, float *y, const Geom &gm, hipStream_t stream) {
    static bool raised = false;
    const int tiles = (gm.M + kTile - 1) / kTile;
    const int NWP = (gm.NW + 3) & ~3;
    const size_t tbuf = static_cast<size_t>(kTile) * gm.rbp + kChunk;
    const size_t lds = 2 * tbuf + static_cast<size_t>(2 * kTile * NWP) * 4 + xplanes_bytes(gm) + 16;
    // 16 resident waves per CU when LDS allows it.
    const int by_waves = std::max(1, 16 / NWMAX);
    const int by_lds = std::max(1, static_cast<int>((160 * 1024) / lds));
    const int grid = std::max(1, std::min(tiles, device_cus() * std::min(by_waves, by_lds)));
    return launch_with_lds(i4_matvec_lds<GT, CPW, PW, NWMAX>, grid, 64 * gm.NW, lds, w, x, y, gm, stream, raised);
}

template <int GT, int CPW>
int launch_reg(const uint8_t *w, const float *x, float *y, const Geom &gm, hipStream_t stream) {
    static bool raised = false;
    const int tiles = (gm.M + kTile - 1) / kTile;
    const int NWP = (gm.NW + 3) & ~3;
    const size_t lds = static_cast<size_t>(kTile * NWP) * 4 + xplanes_bytes(gm) + 16;
    const int grid = std::max(1, std::min(tiles, device_cus()));
    return launch_with_lds(i4_matvec_reg<GT, CPW>, grid, 64 * gm.NW, lds, w, x, y, gm, stream, raised);
}

// Picks windows-per-wave, pieces-per-wave and waves for a row of T 64-byte windows.
template <int GT>
int launch_mfma_for(const uint8_t *w, const float *x, float *y, Geom gm, hipStream_t stream) {
    const int T = gm.T;
    auto pw_of = [&](int nw) { return (gm.pieces + nw - 1) / nw; };
    if (T <= 8) {
        gm.NW = T;
        switch (pw_of(gm.NW)) {
            case 1: return launch_lds<GT, 1, 1, 8>(w, x, y, gm, stream);
            case 2: return launch_lds<GT, 1, 2, 8>(w, x, y, gm, stream);
            case 3: return launch_lds<GT, 1, 3, 8>(w, x, y, gm, stream);
            default: return launch_lds<GT, 1, 4, 8>(w, x, y, gm, stream);
        }
    }
    if (T <= 16) {
        gm.NW = (T + 1) / 2;
        switch (pw_of(gm.NW)) {
            case 1: case 2: return launch_lds<GT, 2, 2, 8>(w, x, y, gm, stream);
            case 3: return launch_lds<GT, 2, 3, 8>(w, x, y, gm, stream);
            default: return launch_lds<GT, 2, 4, 8>(w, x, y, gm, stream);
        }
    }
    if (T <= 24) {
        gm.NW = (T + 2) / 3;
        return pw_of(gm.NW) <= 3 ? launch_lds<GT, 3, 3, 8>(w, x, y, gm, stream)
                                 : launch_lds<GT, 3, 4, 8>(w, x, y, gm, stream);
    }
    if (T <= 48) {
        gm.NW = (T + 2) / 3;
        return pw_of(gm.NW) <= 3 ? launch_lds<GT, 3, 3, 16>(w, x, y, gm, stream)
                                 : launch_lds<GT, 3, 4, 16>(w, x, y, gm, stream);
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
    const int gb = i4_group_bytes(group_size);
    const int Gr = i4_groups(in_dim, group_size);
    const unsigned long long rb = i4_row_bytes(in_dim, group_size);
    const int waves_per_block = 4;
    const int grid = std::max(1, std::min((out_dim + waves_per_block - 1) / waves_per_block, device_cus() * 8));
    hipLaunchKernelGGL(i4_matvec_rowwave, dim3(grid), dim3(64 * waves_per_block), 0, stream, w, x, y, out_dim,
                       in_dim, group_size, gb, Gr, rb);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

int launch_i4_matvec(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                     hipStream_t stream) {
    if (out_dim < 1 || in_dim < 1) return kBadShape;
    if (group_size < 2 || (group_size & 1)) return kBadGroup;
    const size_t rb = i4_row_bytes(in_dim, group_size);
    const bool fast_group = (group_size % 8 == 0) && group_size >= 40;
    if (!fast_group || rb * kTile * 2 >= (1ull << 31))
        return launch_i4_matvec_generic(w, x, y, out_dim, in_dim, group_size, stream);
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
    int st;
    if (group_size == 64)
        st = launch_mfma_for<64>(w, x, y, gm, stream);
    else if (group_size == 128)
        st = launch_mfma_for<128>(w, x, y, gm, stream);
    else
        st = launch_mfma_for<0>(w, x, y, gm, stream);
    if (st == kTooLarge) return launch_i4_matvec_generic(w, x, y, out_dim, in_dim, group_size, stream);
    return st;
}

}  // namespace tqhip
