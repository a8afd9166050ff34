// i4_matvec.hip -- batch=1 i4 HQQ (asymmetric uint4, fp16 scale/zero per group) matvec for gfx950.
//
// Computes y[o] = sum_g sum_i (q[o,g,i] - zero[o,g]) * scale[o,g] * x[g*G + i], the
// contract of the reference's matvec_i4_ref (kernels/matvec/matvec_i4_ref.cpp:45-103),
// on the reference's interleaved layout: every row is ceil(K/G) groups of
// [scale fp16 | zero fp16 | G/2 bytes of codes], low nibble = even element.
//
// Fast path (G % 8 == 0, G >= 40): integer MFMA.
//   * Activations are turned, once per workgroup, into exact integers
//     X = rint(x * 2^f_g) with one power-of-two exponent per group (|X| < 2^22),
//     split into three signed base-256 digits ("planes") d0 + 256*d1 + 65536*d2.
//   * The weight codes are used as they are: the packed dword is split into its
//     even and odd nibbles with two AND masks, giving 8 int8 values 0..15.
//   * v_mfma_i32_16x16x64_i8 contracts 16 weight rows against a 16-row
//     activation operand whose rows are (group slot h, plane p), so one MFMA
//     pair yields the exact integer sums sum(q*X) per plane and per group for
//     a 64-byte window of each row. No float rounding happens before the
//     per-group epilogue  y += scale * (V * 2^-f - zero * sum(X) * 2^-f).
//   * The weight stream is read with 16-byte buffer loads at row-invariant
//     offsets: every lane touches the same 16-byte column of every row, so the
//     activation operand, its group masks and the per-group constants are
//     computed once per workgroup and kept in VGPRs for all rows.
//   * A workgroup splits each row's 64-byte windows over its waves and sums
//     the per-wave partials through LDS in a fixed order (deterministic).
// Generic path (any even G): one wave per row, fp32 accumulation.

#include "tq_common.h"

#include <algorithm>

namespace tqhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;     // bytes of one weight row covered by one MFMA pair
constexpr int kTile = 16;      // weight rows per MFMA tile
constexpr int kMaxWaves = 16;  // waves per workgroup (1024 threads)
constexpr unsigned kNibbles = 0x0F0F0F0Fu;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family word 3)

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

// Position of element i of a group inside its 8-element block, in the order
// the weight operand presents it: even elements (low nibbles) first, then odd.
__device__ inline int plane_pos(int i) {
    const int j = i & 7;
    return (i & ~7) + ((j & 1) ? 4 + (j >> 1) : (j >> 1));
}

struct Geom {
    int M, K, G, gb, Gr, row_bytes, T, NW;
};

// Rows of 16-row tiles handled per LDS reduction round, by windows per wave.
template <int CPW>
struct Rounds {
    static constexpr int R = CPW <= 2 ? 8 : CPW <= 3 ? 4 : CPW <= 4 ? 3 : 1;
};

template <int CPW>
__global__ __launch_bounds__(1024) void i4_matvec_mfma(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                        float *__restrict__ y, Geom gm) {
    constexpr int R = Rounds<CPW>::R;
    extern __shared__ __align__(16) unsigned char smem[];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int NW = gm.NW;
    const int G = gm.G, gb = gm.gb, Gr = gm.Gr, K = gm.K, M = gm.M;
    const int row_bytes = gm.row_bytes;
    const int Kp = Gr * G;  // padded element count (multiple of 8)

    int8_t *pl = reinterpret_cast<int8_t *>(smem);                 // 3 planes x Kp bytes
    int *dsum = reinterpret_cast<int *>(smem + 3 * Kp);            // sum of X per 8-element block
    float *gexp = reinterpret_cast<float *>(dsum + Kp / 8);        // 2^-f per group
    float *part = gexp + Gr;                                       // [2][R][NW][16] partial row sums

    // ---- 1. activations -> per-group exponent, integer planes, block sums (LDS)
    for (int g = wave; g < Gr; g += NW) {
        const int base = g * G;
        float m = 0.f;
        for (int i = lane; i < G; i += 64) {
            const int k = base + i;
            if (k < K) m = fmaxf(m, fabsf(x[k]));
        }
        m = wave_max(m);
        int f = 0;
        if (m > 0.f) {
            int e;
            frexpf(m, &e);  // m in [2^(e-1), 2^e)
            f = min(22 - e, 149);
        }
        for (int i = lane; i < G; i += 64) {
            const int k = base + i;
            const int X = (k < K) ? static_cast<int>(rintf(ldexpf(x[k], f))) : 0;
            const int d0 = ((X + 128) & 255) - 128;
            const int X1 = (X - d0) >> 8;
            const int d1 = ((X1 + 128) & 255) - 128;
            const int d2 = (X1 - d1) >> 8;
            const int pos = base + plane_pos(i);
            pl[pos] = static_cast<int8_t>(d0);
            pl[Kp + pos] = static_cast<int8_t>(d1);
            pl[2 * Kp + pos] = static_cast<int8_t>(d2);
            int s = X;  // G % 8 == 0, so each 8-lane block is entirely active here
            s += __shfl_xor(s, 1);
            s += __shfl_xor(s, 2);
            s += __shfl_xor(s, 4);
            if ((i & 7) == 0) dsum[(base + i) >> 3] = s;
        }
        if (lane == 0) gexp[g] = ldexpf(1.f, -f);
    }
    __syncthreads();

    // ---- 2. per-lane, row-invariant operands for this wave's windows
    const int t0 = (gm.T * wave) / NW;
    const int nch = (gm.T * (wave + 1)) / NW - t0;  // <= CPW by construction on the host
    const int am = lane & 15;                        // activation-operand row = 4*slot + plane
    const int ah = am >> 2, ap = am & 3;
    const int kq = lane >> 4;                        // k quad; also the epilogue's group slot
    const int bn = lane & 15;                        // weight row within the tile

    // Waves with fewer than CPW windows repeat their last window (a cache hit)
    // with a zero activation operand and a zero header mask, so the streaming
    // loop below has no per-window branches and can issue all loads up front.
    v4i A0[CPW], A1[CPW];
    float E[CPW], C[CPW];
    int DO[CPW], HO[CPW];
    unsigned HM[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        A0[c] = v4i{0, 0, 0, 0};
        A1[c] = v4i{0, 0, 0, 0};
        E[c] = 0.f;
        C[c] = 0.f;
        HM[c] = 0u;
        const int t = t0 + min(c, nch - 1);
        DO[c] = kChunk * t + 16 * kq;
        HO[c] = 0;
        if (c >= nch) continue;
        const int gt = (kChunk * t) / gb;  // group holding the window's first byte
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int dw = 0; dw < 2; ++dw) {
                const int o = kChunk * t + 4 * (4 * kq + 2 * u + dw);
                unsigned lo = 0, hi = 0;
                if (o < row_bytes && ap < 3) {
                    const int g = o / gb;
                    const int r = o - g * gb;
                    if (r >= kI4Header && g - gt == ah) {
                        const int blk = (g * G + 2 * (r - kI4Header)) >> 3;
                        const uint2 v = *reinterpret_cast<const uint2 *>(pl + ap * Kp + 8 * blk);
                        lo = v.x;
                        hi = v.y;
                    }
                }
                if (u == 0) {
                    A0[c][2 * dw] = static_cast<int>(lo);
                    A0[c][2 * dw + 1] = static_cast<int>(hi);
                } else {
                    A1[c][2 * dw] = static_cast<int>(lo);
                    A1[c][2 * dw + 1] = static_cast<int>(hi);
                }
            }
        }
        const int gq = gt + kq;
        const int wend = min(kChunk * (t + 1), row_bytes);
        if (gq < Gr && gq * gb < wend) {
            int sum = 0;
            for (int cd = 0; cd < kChunk / 4; ++cd) {
                const int o = kChunk * t + 4 * cd;
                if (o >= row_bytes) break;
                const int g = o / gb;
                const int r = o - g * gb;
                if (g == gq && r >= kI4Header) sum += dsum[(g * G + 2 * (r - kI4Header)) >> 3];
            }
            E[c] = gexp[gq];
            C[c] = static_cast<float>(sum) * E[c];
            HO[c] = gq * gb;
            HM[c] = 0xFFFFFFFFu;
        }
    }

    // ---- 3. stream the rows: R tiles of 16 rows per round, windows split over the waves
    const int tiles = (M + kTile - 1) / kTile;
    const int my0 = static_cast<int>(static_cast<long long>(tiles) * blockIdx.x / gridDim.x);
    const int my1 = static_cast<int>(static_cast<long long>(tiles) * (blockIdx.x + 1) / gridDim.x);
    int buf = 0;
    for (int b0 = my0; b0 < my1; b0 += R) {
        const int nb = min(R, my1 - b0);
        const int row0 = b0 * kTile;
        const size_t rem = static_cast<size_t>(M - row0) * row_bytes;
        const int nrec = rem > 0xFFFFFFFFull ? -1 : static_cast<int>(static_cast<unsigned>(rem));
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(w) + static_cast<size_t>(row0) * row_bytes, static_cast<short>(0), nrec,
            kBufferFlags);
        // (a) issue every load of the round; tiles past the WG's range repeat the last one
        v4i dat[R][CPW];
        unsigned hdr[R][CPW];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int rr = min(r, nb - 1);
            const int row = min(row0 + rr * kTile + bn, M - 1);
            const int lb = (row - row0) * row_bytes;
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                dat[r][c] = __builtin_amdgcn_raw_buffer_load_b128(rs, lb + DO[c], 0, 0);
                hdr[r][c] = __builtin_amdgcn_raw_buffer_load_b32(rs, lb + HO[c], 0, 0);
            }
        }
        // (b) contract and apply the group scales
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float a = 0.f;
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                const v4i d = dat[r][c];
                const unsigned d0 = static_cast<unsigned>(d.x), d1 = static_cast<unsigned>(d.y);
                const unsigned d2 = static_cast<unsigned>(d.z), d3 = static_cast<unsigned>(d.w);
                const v4i b0 = {static_cast<int>(d0 & kNibbles), static_cast<int>((d0 >> 4) & kNibbles),
                                static_cast<int>(d1 & kNibbles), static_cast<int>((d1 >> 4) & kNibbles)};
                const v4i b1 = {static_cast<int>(d2 & kNibbles), static_cast<int>((d2 >> 4) & kNibbles),
                                static_cast<int>(d3 & kNibbles), static_cast<int>((d3 >> 4) & kNibbles)};
                v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0[c], b0, v4i{0, 0, 0, 0}, 0, 0, 0);
                D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1[c], b1, D, 0, 0, 0);
                const float V = fmaf(static_cast<float>(D.z), 65536.f,
                                     fmaf(static_cast<float>(D.y), 256.f, static_cast<float>(D.x)));
                // A masked header gives scale = zero = 0, and V = E = C = 0 there,
                // so an empty group slot adds exactly 0.
                const unsigned h = hdr[r][c] & HM[c];
                const float s = half_bits(h);
                const float z = half_bits(h >> 16);
                a = fmaf(s, fmaf(V, E[c], -z * C[c]), a);
            }
            acc[r] = a;
        }
        // (c) sum the four group slots of each row, then the waves, in a fixed order
        float *pb = part + buf * (R * NW * kTile);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = acc[r];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (lane < kTile) pb[(r * NW + wave) * kTile + lane] = v;
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < nb * kTile; idx += blockDim.x) {
            const int r = idx / kTile, n = idx % kTile;
            float s = 0.f;
            for (int wv = 0; wv < NW; ++wv) s += pb[(r * NW + wv) * kTile + n];
            const int row = (b0 + r) * kTile + n;
            if (row < M) y[row] = s;
        }
        buf ^= 1;
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

template <int CPW>
int launch_mfma_cpw(const uint8_t *w, const float *x, float *y, const Geom &gm, hipStream_t stream) {
    constexpr int R = Rounds<CPW>::R;
    const int tiles = (gm.M + kTile - 1) / kTile;
    const int Kp = gm.Gr * gm.G;
    const size_t lds = static_cast<size_t>(3 * Kp) + static_cast<size_t>(Kp / 8) * 4 + static_cast<size_t>(gm.Gr) * 4 +
                       static_cast<size_t>(2 * R * gm.NW * kTile) * 4;
    if (lds > 160 * 1024) return kTooLarge;
    // Aim for about 16 resident waves per CU.
    const int wg_per_cu = std::max(1, 16 / gm.NW);
    const int grid = std::max(1, std::min(tiles, device_cus() * wg_per_cu));
    if (lds > 64 * 1024) {
        static bool raised = false;
        if (!raised) {
            TQ_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(i4_matvec_mfma<CPW>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
            raised = true;
        }
    }
    hipLaunchKernelGGL(i4_matvec_mfma<CPW>, dim3(grid), dim3(64 * gm.NW), lds, stream, w, x, y, gm);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
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
    if (!fast_group || rb * kTile * 8 >= (1ull << 31))
        return launch_i4_matvec_generic(w, x, y, out_dim, in_dim, group_size, stream);
    Geom gm;
    gm.M = out_dim;
    gm.K = in_dim;
    gm.G = group_size;
    gm.gb = i4_group_bytes(group_size);
    gm.Gr = i4_groups(in_dim, group_size);
    gm.row_bytes = static_cast<int>(rb);
    gm.T = static_cast<int>((rb + kChunk - 1) / kChunk);
    int cpw = (gm.T + kMaxWaves - 1) / kMaxWaves;
    if (cpw == 5) cpw = 6;
    if (cpw > 6) return launch_i4_matvec_generic(w, x, y, out_dim, in_dim, group_size, stream);
    gm.NW = (gm.T + cpw - 1) / cpw;
    int st = kTooLarge;
    switch (cpw) {
        case 1: st = launch_mfma_cpw<1>(w, x, y, gm, stream); break;
        case 2: st = launch_mfma_cpw<2>(w, x, y, gm, stream); break;
        case 3: st = launch_mfma_cpw<3>(w, x, y, gm, stream); break;
        case 4: st = launch_mfma_cpw<4>(w, x, y, gm, stream); break;
        case 6: st = launch_mfma_cpw<6>(w, x, y, gm, stream); break;
        default: break;
    }
    if (st == kTooLarge) return launch_i4_matvec_generic(w, x, y, out_dim, in_dim, group_size, stream);
    return st;
}

}  // namespace tqhip
