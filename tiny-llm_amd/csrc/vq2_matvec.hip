// vq2_matvec.hip -- batch=1 VQ2 (d=4, 256-entry fp16 codebook) matvec for gfx950.
//
// Computes y[o] = sum_b codebook[idx[o][b]] . x[4b : 4b+4], the contract of the
// reference's matvec_vq2_ref (kernels/matvec/matvec_vq2_ref.cpp:52-81), on the
// layout [codebook 256 x 4 fp16 = 2048 B][out_dim x in_dim/4 uint8 indices].
//
// Four kernels:
// - vq2_matvec_table (index rows 16-byte aligned, in_dim <= 1024, at least 256 rows per CU):
//   per workgroup a table of every codebook entry's dot product with every 4-element block of
//   x, built with fp32 MFMAs in LDS; a lookup is then one 4-byte LDS read and one add (see its
//   comment).
// - vq2_matvec_copies (index rows dword-aligned, in_dim % 16 == 0): 16 bank-
//   interleaved fp32 copies of the codebook in LDS make every lookup
//   conflict-free; tiles of 4 rows per wave, the next tile's index dwords in
//   flight during the current tile's lookups, and a short halving reduction
//   over the wave (see its comment).
// - vq2_matvec_kernel (any other in_dim): one fp32 codebook copy in LDS, one
//   byte load per index. A wave owns a tile of kRows rows and sweeps the row in
//   steps of 64 lanes x 4 indices; each lane keeps the 16 activations of its 4
//   indices in VGPRs and reuses them for all kRows rows.
// - vq2_matvec_rows (index rows dword-aligned, at most kDirectLookups lookups): one wave per
//   row and no LDS at all. A grid this small cannot amortise building a 64 KB codebook
//   replica per workgroup, so every lookup is an 8-byte load of the fp16 entry from the
//   2 KB codebook in global memory (it stays in each CU's L1 after the first touch). One
//   launch serves up to kSetMaxMats matrices with their own activations
//   (launch_vq2_matvec_set: a decoder layer's q/k/v or gate/up).
// All accumulate in fp32.

#include "lane_sum.h"
#include "tq_common.h"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace tqhip {
namespace {

constexpr int kRows = 8;  // rows per wave tile
constexpr int kWavesPerBlock = 4;
constexpr int kBufferFlags = 0x00020000;

__device__ inline float half_bits(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xFFFFu)));
}

// Index rows at any byte alignment: one byte load per index.
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
                unsigned q = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (b + j < nb) q |= static_cast<unsigned>(__builtin_amdgcn_raw_buffer_load_b8(rs, r * nb + b + j, 0, 0)) << (8 * j);
                float a = acc[r];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (b + j < nb) {  // past the row end: nothing (entry 0 may be non-finite)
                        const float4 c = cb[(q >> (8 * j)) & 0xFFu];
                        a = fmaf(c.x, xv[j].x, a);
                        a = fmaf(c.y, xv[j].y, a);
                        a = fmaf(c.z, xv[j].z, a);
                        a = fmaf(c.w, xv[j].w, a);
                    }
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

// ---- Bank-conflict-free variant (index rows dword-aligned).
// A lookup reads a random codebook entry per lane, so with one codebook copy
// the lanes of an LDS pass collide on banks. Here LDS holds 16 interleaved
// fp32 copies: copy c of entry e is float4 number 16 e + c, and lane l reads
// copy l % 16. Entry rows are 256 bytes apart (a whole number of bank sweeps),
// so a lane's banks are 4 (l % 16) .. +3 whatever entry it reads: the 16 lanes
// served together never share a bank. 16 copies x 256 entries x 16 B = 64 KB.
//
// A wave owns tiles of R rows and covers a row chunk of 256 index bytes with
// 64 lanes x 4 indices (one dword per lane per row). The next tile's index
// dwords are loaded while the current tile is computed. The R per-lane sums
// are reduced over the wave by halving exchanges (R - 1 + log2(64 / R)
// shuffles instead of 6 R).
constexpr int kCopies = 16;
constexpr int kVq2Waves = 16;  // waves per workgroup (the 64 KB codebook is shared by all of them)
constexpr int kVq2Rows = 4;    // rows per wave tile

template <int R>
__device__ inline void vq2_load_rows(const __amdgpu_buffer_rsrc_t &rs, int nb, int off, unsigned (&q)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) q[r] = __builtin_amdgcn_raw_buffer_load_b32(rs, r * nb + off, 0, 0);
}

template <int R, bool ONE_CHUNK>
__global__ __launch_bounds__(64 * kVq2Waves) void vq2_matvec_copies(const uint8_t *__restrict__ w,
                                                                    const float *__restrict__ x,
                                                                    float *__restrict__ y, int M, int K) {
    __shared__ float4 cb[kVq2Entries * kCopies];
    for (int i = threadIdx.x; i < kVq2Entries * kCopies; i += blockDim.x) {
        const uint16_t *h = reinterpret_cast<const uint16_t *>(w) + kVq2Dim * (i / kCopies);
        cb[i] = make_float4(half_bits(h[0]), half_bits(h[1]), half_bits(h[2]), half_bits(h[3]));
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int nb = K / kVq2Dim;           // index bytes per row (a multiple of 4)
    const int nchunk = ONE_CHUNK ? 1 : (nb + 255) / 256;  // 256-byte chunks of a row (ONE_CHUNK: nb <= 256)
    const uint8_t *idx = w + kVq2CodebookBytes;
    const int tiles = (M + R - 1) / R;
    const int gw = blockIdx.x * kVq2Waves + wave;
    const int nw = gridDim.x * kVq2Waves;
    const int ntile = gw < tiles ? (tiles - 1 - gw) / nw + 1 : 0;  // this wave's tiles
    const int nstep = ntile * nchunk;                                // (tile, chunk) steps
    const float4 *cbl = cb + (lane & (kCopies - 1));  // this lane's copy: entry e at cbl[16 e]

    // indices of step s: tile gw + (s / nchunk) nw, chunk s % nchunk; this
    // lane's dword is bytes 256 chunk + 4 lane .. +3 of each of the R rows.
    // Steps past the last and bytes past the row end read 0.
    auto load_step = [&](int s, unsigned (&q)[R]) {
        const int t = s / nchunk, ch = s - t * nchunk;
        const int tile = gw + t * nw;
        const int row0 = tile * R;
        const size_t rem = s < nstep ? static_cast<size_t>(M - row0) * nb : 0;
        const int nrec = rem > 0xFFFFFFFFull ? -1 : static_cast<int>(static_cast<unsigned>(rem));
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(idx) + static_cast<size_t>(s < nstep ? row0 : 0) * nb, static_cast<short>(0), nrec,
            kBufferFlags);
        const int b = 256 * ch + 4 * lane;
        const int off = b < nb ? b : 0x40000000;
#pragma unroll
        for (int r = 0; r < R; ++r) q[r] = __builtin_amdgcn_raw_buffer_load_b32(rs, r * nb + off, 0, 0);
    };
    // activations of this lane's 4 indices of a chunk (0 past the row end)
    auto xvals = [&](int ch, float4 (&xv)[4]) {
        const int b = 256 * ch + 4 * lane;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float *xp = x + 4 * (b + j);
            xv[j] = (b + j < nb) ? make_float4(xp[0], xp[1], xp[2], xp[3]) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };

    float4 xv[4];
    xvals(0, xv);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    // one step: lookups of q, and at a tile's last chunk the reduction and store
    auto step = [&](int s, const unsigned (&q)[R]) {
        const int t = s / nchunk, ch = s - t * nchunk;
        if constexpr (!ONE_CHUNK) xvals(ch, xv);  // (with one chunk, loaded once before the loop)
        // a lane past the row end adds nothing: its index 0 and zero activations would still
        // give NaN for a non-finite entry 0, which the row never uses
        if (256 * ch + 4 * lane < nb) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float a = acc[r];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 c = cbl[kCopies * ((q[r] >> (8 * j)) & 0xFFu)];
                    a = fmaf(c.x, xv[j].x, a);
                    a = fmaf(c.y, xv[j].y, a);
                    a = fmaf(c.z, xv[j].z, a);
                    a = fmaf(c.w, xv[j].w, a);
                }
                acc[r] = a;
            }
        }
        if (ch + 1 < nchunk) return;
        // halving exchanges: after the exchange over lane bit `bit`, half the
        // rows remain, each summed over both lanes of the pair
        float v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = acc[r];
        constexpr int kSteps = R == 8 ? 3 : R == 4 ? 2 : R == 2 ? 1 : 0;  // log2 R
        int row = 0;
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {  // (unrolled: every index below is a constant)
            const int h = (R >> st) / 2, bit = 32 >> st;
            const bool upper = (lane & bit) != 0;
#pragma unroll
            for (int r = 0; r < h; ++r) {
                // both halves summed over the pair, then the lane keeps its
                // half (a select of two sums: a select of two array elements
                // is compiled as a run-time index into the array)
                const float lo = v[r] + __shfl_xor(v[r], bit);
                const float hi = v[r + h] + __shfl_xor(v[r + h], bit);
                v[r] = upper ? hi : lo;
            }
            row += upper ? h : 0;
        }
        float sum = v[0];
#pragma unroll
        for (int bit = 32 / R; bit > 0; bit /= 2) sum += __shfl_xor(sum, bit);
        const int r0 = (gw + t * nw) * R;
        if ((lane & (64 / R - 1)) == 0 && r0 + row < M) y[r0 + row] = sum;
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;
    };

    // two register sets, alternating: the next step's indices are in flight
    // during every step's lookups
    unsigned qa[R], qb[R];
    load_step(0, qa);
    for (int s = 0; s < nstep; s += 2) {
        load_step(s + 1, qb);
        step(s, qa);
        if (s + 1 >= nstep) break;
        load_step(s + 2, qa);
        step(s + 1, qb);
    }
}

// ---- One wave per row, codebook entries gathered from global memory (small launches).
// Lane l takes index dwords l, l + 64, ... of the row (indices 4 b .. 4 b + 3) and their
// activations; the 64 lane sums are added by a butterfly over the wave. Measured on MI355X
// against vq2_matvec_copies: 896x896 2.5 vs 5.2 us, 3072x1024 3.3-3.6 vs 5.1-5.3 us (the
// one-launch floor for its 0.8 MB is 3.3 us), 4864x896 4.1 vs 5.3, 2001x3056 4.7 vs 7.9; from
// about 8M lookups (16384x2048, 32768x896) the replica kernel is faster.
constexpr long long kDirectLookups = 4ll << 20;
// A launch of this kernel serves up to kSetMaxMats matrices, each with its own activations
// (a layer's q/k/v, gate/up, or rotated copies of x): workgroups are numbered matrix after
// matrix and a workgroup finds its matrix with scalar compares against the kernel argument.
// A row's bits do not depend on the other matrices of the launch.
// Staged activations (XM != 0 or ROT; 8-wave workgroups): every workgroup first builds its
// matrix's activations in LDS, and the rows read them from there.
// - XM, the prologue shared by the launch's matrices (one x): 1 x = silu(x) * x2 (swiglu's
//   operations); 2 x = rmsnorm((x + d1) + d2) * nw (add_rmsnorm's: a double sum of squares,
//   a float mean, 1 / sqrt(mean + eps), (h * scale) * w), workgroup 0 storing the sum to hout.
// - ROT: then each matrix's own BiIP rotation, with biip_rotate_kernel's operations in its
//   order (division by the scale, sign product, butterfly stages, the 1 / sqrt(block)
//   product).
// The rows see exactly the values the separate launches would have written.
struct Vq2Mat {
    const uint8_t *w;
    const float *x;
    float *y;
    int M, K;
    int blk0;                  // first workgroup of this matrix
    const float *scale, *sign;  // ROT: the matrix's rotation (scale may be null)
};
struct Vq2SetArgs {
    Vq2Mat m[kSetMaxMats];
    int n;
};
// The staged launches carry at most three records (a layer's q/k/v at most): five fewer
// records in the kernel argument measured 0.17 us less per launch in the decode engine.
constexpr int kStagedMaxMats = 3;
struct Vq2StagedArgs {
    Vq2Mat m[kStagedMaxMats];
    int n;
    int lg_bs;        // ROT: log2 of the rotation block
    float inv_sqrt;   // ROT: 1 / sqrt(block), as the host computes it for biip_rotate
    SetPrologue pro;  // XM != 0
};
template <int WAVES>
__device__ inline double vq2_block_sum(double v) {
    v = xor_sum_wave(v);
    __shared__ double red[WAVES];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = red[0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += red[w];
    return t;
}
// One step of a row's dot product: the four entries of index dword q against 16 activations.
__device__ inline float vq2_accum(float acc, const uint2 *c, const float4 *xv) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        acc = fmaf(half_bits(c[jj].x), xv[jj].x, acc);
        acc = fmaf(half_bits(c[jj].x >> 16), xv[jj].y, acc);
        acc = fmaf(half_bits(c[jj].y), xv[jj].z, acc);
        acc = fmaf(half_bits(c[jj].y >> 16), xv[jj].w, acc);
    }
    return acc;
}

// The workgroup's matrix: scalar compares against the kernel argument, every field selected
// in registers. (A helper that returned the record, or a reference into the argument, made the
// compiler copy the argument to scratch memory.)
#define TQ_VQ2_SELECT(a, m, cap)                                                          \
    Vq2Mat m = (a).m[0];                                                                  \
    {                                                                                     \
        int j_ = 0;                                                                       \
        _Pragma("unroll") for (int i_ = 1; i_ < (cap); ++i_) j_ =                         \
            (i_ < (a).n && static_cast<int>(blockIdx.x) >= (a).m[i_].blk0) ? i_ : j_;      \
        _Pragma("unroll") for (int i_ = 1; i_ < (cap); ++i_) if (i_ == j_) m = (a).m[i_]; \
    }

// Row `row` of one matrix, x from global memory, its 64 lane sums added over the wave.
template <bool XALIGN>
__device__ inline float vq2_row(const uint8_t *w, const float *x, int K, int row, int lane) {
    const int nb = K / kVq2Dim;  // index bytes per row (a multiple of 4)
    const unsigned *qrow = reinterpret_cast<const unsigned *>(w + kVq2CodebookBytes + static_cast<size_t>(row) * nb);
    const uint2 *cbg = reinterpret_cast<const uint2 *>(w);  // entry e: 4 fp16 in 8 bytes
    float acc = 0.f;
    for (int d = lane; 4 * d < nb; d += 64) {
        const unsigned q = qrow[d];
        float4 xv[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const float *xp = x + 16 * d + 4 * jj;
            xv[jj] = XALIGN ? *reinterpret_cast<const float4 *>(xp) : make_float4(xp[0], xp[1], xp[2], xp[3]);
        }
        uint2 c[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) c[jj] = cbg[(q >> (8 * jj)) & 0xFFu];
        acc = vq2_accum(acc, c, xv);
    }
    return sum_wave(acc);  // DPP and row swaps in registers, a fixed order
}

// One matrix per launch (32 bytes of kernel arguments: the set form's 8 records and their
// selection took 4.0 against 3.5 us at 3072x1024).
template <bool XALIGN>
__global__ __launch_bounds__(256) void vq2_matvec_row1(const uint8_t *__restrict__ w, const float *__restrict__ x,
                                                       float *__restrict__ y, int M, int K) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const float acc = vq2_row<XALIGN>(w, x, K, row, threadIdx.x & 63);
    if ((threadIdx.x & 63) == 0) y[row] = acc;
}

template <bool XALIGN>
__global__ __launch_bounds__(256) void vq2_matvec_rows(Vq2SetArgs a) {
    TQ_VQ2_SELECT(a, m, kSetMaxMats);
    const int row = (static_cast<int>(blockIdx.x) - m.blk0) * 4 + (threadIdx.x >> 6);
    if (row >= m.M) return;
    const float acc = vq2_row<XALIGN>(m.w, m.x, m.K, row, threadIdx.x & 63);
    if ((threadIdx.x & 63) == 0) m.y[row] = acc;
}

// The staged form: 8 waves, each taking RPW rows, so that a workgroup's activation build serves
// 8 RPW rows. Lane l of wave w holds activations 256 (8 p + w) + 4 l + 0..3 in pass p (NP
// passes of 2048 cover K): 16-byte loads of every prologue operand, and a BiIP block (at most
// 256 activations, a power of two dividing K) lies within one wave, so the rotation's radix-2
// stages run in registers -- stage h < 4 inside the lane, stage h >= 4 against lane l ^ (h / 4)
// -- with no barrier. Each stage makes the same adds and subtracts, in the same order, as
// biip_rotate_kernel (whose radix-4 form is two radix-2 stages), so the values match its bits.
// The 2 KB codebook goes to LDS once per workgroup and the lookups read it there. Every load
// that does not wait for the prologue goes out first (the codebook, the rows' index dwords, the
// prologue operands); the prologue runs in registers (one barrier for the RMSNorm's sum) while
// they arrive. Measured on MI355X at the Qwen2.5-0.5B rotated-VQ2 shapes against the previous
// form (one activation per thread and pass, LDS butterfly with a barrier per two stages,
// codebook entries gathered from global memory, one row per wave): see the launcher.
constexpr int kRotWaves = 8;
constexpr int kStagedPass = 64 * kRotWaves * 4;  // activations per pass
template <int NP, int XM, bool ROT, int RPW>
__global__ __launch_bounds__(64 * kRotWaves) void vq2_matvec_staged(Vq2StagedArgs a) {
    extern __shared__ __align__(16) float xs[];  // the matrix's activations
    __shared__ uint2 cbl[256];                   // its codebook's fp16 entries
    constexpr int NIT = 2 * NP;                  // index dwords per lane and row (K / 16 <= 128 NP)
    TQ_VQ2_SELECT(a, m, kStagedMaxMats);
    const float *const d1 = a.pro.d1, *const d2 = a.pro.d2, *const nw = a.pro.nw, *const x2 = a.pro.x2;
    float *const hout = a.pro.hout;
    const float eps = a.pro.eps;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int blk = static_cast<int>(blockIdx.x) - m.blk0;
    const int K = m.K, M = m.M, nb = K / kVq2Dim;
    if (t < 256) cbl[t] = reinterpret_cast<const uint2 *>(m.w)[t];
    unsigned qv[RPW][NIT];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = (blk * RPW + r) * kRotWaves + wave;
        const unsigned *qrow =
            reinterpret_cast<const unsigned *>(m.w + kVq2CodebookBytes + static_cast<size_t>(row < M ? row : 0) * nb);
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int d = lane + 64 * it;
            qv[r][it] = row < M && 4 * d < nb ? qrow[d] : 0u;
        }
    }
    // activations 4 e .. 4 e + 3 of pass p, e = 64 (8 p + w) + l (whole float4s: K % 16 == 0)
    typedef float f4e __attribute__((ext_vector_type(4)));
    f4e v[NP], p1[NP], p2[NP], p3[NP], sc[NP], sg[NP];
    const f4e zero = {0.f, 0.f, 0.f, 0.f}, one = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int e = 64 * (kRotWaves * p + wave) + lane;
        const bool ok = 4 * e < K;
        v[p] = ok ? reinterpret_cast<const f4e *>(m.x)[e] : zero;
        if constexpr (XM == 2) {
            p1[p] = ok && d1 ? reinterpret_cast<const f4e *>(d1)[e] : zero;
            p2[p] = ok && d2 ? reinterpret_cast<const f4e *>(d2)[e] : zero;
            p3[p] = ok ? reinterpret_cast<const f4e *>(nw)[e] : zero;
        } else if constexpr (XM == 1) {
            p1[p] = ok ? reinterpret_cast<const f4e *>(x2)[e] : zero;
        }
        if constexpr (ROT) {
            sc[p] = ok && m.scale ? reinterpret_cast<const f4e *>(m.scale)[e] : one;
            sg[p] = ok ? reinterpret_cast<const f4e *>(m.sign)[e] : zero;
        }
    }
    if constexpr (XM == 2) {  // add_rmsnorm's operations
        double ss = 0.0;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if (d1) v[p][c] = v[p][c] + p1[p][c];
                if (d2) v[p][c] = v[p][c] + p2[p][c];
                ss += static_cast<double>(v[p][c]) * static_cast<double>(v[p][c]);
            }
            const int e = 64 * (kRotWaves * p + wave) + lane;
            if (hout && blockIdx.x == 0 && 4 * e < K) reinterpret_cast<f4e *>(hout)[e] = v[p];
        }
        ss = vq2_block_sum<kRotWaves>(ss);
        const float mean_sq = static_cast<float>(ss / K);
        const float scale = 1.0f / sqrtf(mean_sq + eps);
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int c = 0; c < 4; ++c) v[p][c] = (v[p][c] * scale) * p3[p][c];
    } else if constexpr (XM == 1) {  // swiglu's operations
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int c = 0; c < 4; ++c) v[p][c] = (v[p][c] / (1.0f + expf(-v[p][c]))) * p1[p][c];
    }
    {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            f4e f = v[p];
            if constexpr (ROT) {  // biip_rotate_kernel's operations
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    f[c] = m.scale ? (f[c] / sc[p][c]) * sg[p][c] : f[c] * sg[p][c];
                // stage h: (u, c) at (j, j + h) of a block -> (u + c, u - c)
                if (a.lg_bs > 0) {
                    const float u0 = f[0], u1 = f[1], u2 = f[2], u3 = f[3];
                    f[0] = u0 + u1;
                    f[1] = u0 - u1;
                    f[2] = u2 + u3;
                    f[3] = u2 - u3;
                }
                if (a.lg_bs > 1) {
                    const float u0 = f[0], u1 = f[1], u2 = f[2], u3 = f[3];
                    f[0] = u0 + u2;
                    f[1] = u1 + u3;
                    f[2] = u0 - u2;
                    f[3] = u1 - u3;
                }
                // stages h = 4 .. 128: the pair's other elements are in lane l ^ (h / 4); the lane
                // with that bit set holds the second ones (u - c, c its own)
                auto stage = [&](auto dlc) {
                    constexpr int DL = decltype(dlc)::value;
                    const bool hi = lane & DL;
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const float o = lane_xor<DL>(f[c], lane);
                        f[c] = hi ? o - f[c] : f[c] + o;
                    }
                };
                if (a.lg_bs > 2) stage(std::integral_constant<int, 1>{});
                if (a.lg_bs > 3) stage(std::integral_constant<int, 2>{});
                if (a.lg_bs > 4) stage(std::integral_constant<int, 4>{});
                if (a.lg_bs > 5) stage(std::integral_constant<int, 8>{});
                if (a.lg_bs > 6) stage(std::integral_constant<int, 16>{});
                if (a.lg_bs > 7) stage(std::integral_constant<int, 32>{});
#pragma unroll
                for (int c = 0; c < 4; ++c) f[c] = f[c] * a.inv_sqrt;
            }
            const int e = 64 * (kRotWaves * p + wave) + lane;
            if (4 * e < K) reinterpret_cast<f4e *>(xs)[e] = f;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = (blk * RPW + r) * kRotWaves + wave;
        if (row >= M) break;
        float acc = 0.f;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int d = lane + 64 * it;
            if (4 * d >= nb) break;
            uint2 cv[4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) cv[jj] = cbl[(qv[r][it] >> (8 * jj)) & 0xFFu];
            float4 xv[4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) xv[jj] = *reinterpret_cast<const float4 *>(xs + 16 * d + 4 * jj);
            acc = vq2_accum(acc, cv, xv);
        }
        acc = sum_wave(acc);  // vq2_row's order
        if (lane == 0) m.y[row] = acc;
    }
}

// The matrix the one-wave-per-row kernel takes: index rows dword-aligned, at most
// kDirectLookups lookups.
bool rows_kernel_takes(const uint8_t *w, int out_dim, int in_dim) {
    return (in_dim % 16) == 0 && (reinterpret_cast<uintptr_t>(w) % 4) == 0 &&
           static_cast<long long>(out_dim) * (in_dim / kVq2Dim) <= kDirectLookups;
}

int launch_rows(Vq2SetArgs &a, int n, int blocks, bool xalign, hipStream_t stream) {
    if (n == 1) {
        const Vq2Mat &m = a.m[0];
        if (xalign)
            hipLaunchKernelGGL(vq2_matvec_row1<true>, dim3(blocks), dim3(256), 0, stream, m.w, m.x, m.y, m.M, m.K);
        else
            hipLaunchKernelGGL(vq2_matvec_row1<false>, dim3(blocks), dim3(256), 0, stream, m.w, m.x, m.y, m.M, m.K);
        return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
    }
    for (int k = n; k < kSetMaxMats; ++k) a.m[k] = a.m[n - 1];  // never selected (k >= n)
    a.n = n;
    if (xalign)
        hipLaunchKernelGGL(vq2_matvec_rows<true>, dim3(blocks), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(vq2_matvec_rows<false>, dim3(blocks), dim3(256), 0, stream, a);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}


// ---- Dot-product table (large launches, index rows 16-byte aligned, in_dim <= 1024).
// A lookup of the replica kernel costs four fp32 FMAs and a 16-byte LDS read per index, which
// bounds it by VALU and LDS issue (151936x896: 16 us). Here the products are formed once per
// workgroup: T[c][b] = codebook[c] . x[4 b .. 4 b + 3] for every entry c and index position b of
// the row, and a lookup is one 4-byte LDS read and one add. The whole table (256 x in_dim / 4
// fp32) does not fit in LDS at in_dim 896, so the row's index dwords d are taken in two passes,
// d mod 4 in {0, 1}, then {2, 3}, each with a 128 KB table of two 64 KB sub-tables:
//   pass p, sub-table s (d mod 4 = 2 p + s): entry (c, byte j, q = d / 4) at byte
//   s * 65536 + 256 c + 64 j + 4 q holds T[c][4 d + j], and 0 past the row end.
// Lane (rho = lane / 16, q = lane % 16) loads 16 bytes, dwords 4 q .. 4 q + 3, of rows
// 16 (wave + 16 i) + 4 r + rho (r = 0..3): a load instruction moves 4 x 256 contiguous bytes.
// In pass p the lane looks up bytes of dwords 4 q + 2 p and 4 q + 2 p + 1; at step k it takes
// byte jl = (k + rho) & 3, so the 32 lanes of an LDS pass read banks (16 jl + q) mod 32, all
// different. One v_perm forms the address from the index byte, the lane's 64 jl + 4 q and
// the sub-table number.
// The table is built with v_mfma_f32_32x32x2_f32 (codebook entries x positions, the four
// components as two k-steps); a 32-position tile is two bytes j x 16 q, so its LDS stores
// are conflict-free as well. The first batch's index loads go out right after the codebook and
// x loads and before anything waits for them (a conversion there would make the index stream
// wait for a round trip); the other batches follow once the first table is built (see step 3
// in the kernel). Measured on MI355X (cold weights, 256 workgroups): 151936x896 11.6-11.8 us
// (replica kernel 15.6), 131072x1024 11.3 (13.5), 65536x896 8.5 (8.8). Per workgroup, each
// lookup pass takes ~1.3 us (LDS issue) and the second table ~0.9 us.
constexpr int kTabWaves = 16;           // waves per workgroup
constexpr int kTabBatchRows = 16;       // rows of a wave's batch (4 per load instruction x 4)
constexpr int kTabMaxBatches = 4;       // batches per wave held in VGPRs: <= 1024 rows per workgroup
constexpr int kTabMinRowsPerCu = 256;   // fewer rows: the replica kernel (65536 rows at 256 CUs)
constexpr int kTabMaxDim = 1024;        // 64 index dwords per row: 16 lanes x 16 bytes

template <int CTRL>
__device__ inline float tab_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int BMAX>
__global__ __launch_bounds__(64 * kTabWaves) void vq2_matvec_table(const uint8_t *__restrict__ w,
                                                                   const float *__restrict__ x,
                                                                   float *__restrict__ y, int M, int K,
                                                                   int rows_per_wg) {
    __shared__ __align__(16) unsigned char tab[2 * 65536];
    typedef float f16v __attribute__((ext_vector_type(16)));
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = K / kVq2Dim, nd = nb / 4;  // index bytes and dwords per row
    const int r0 = blockIdx.x * rows_per_wg;
    const int nrows = min(rows_per_wg, M - r0);
    if (nrows <= 0) return;
    const uint16_t *cbh = reinterpret_cast<const uint16_t *>(w);
    const int rho = lane >> 4, q = lane & 15;
    const int nbatch = (nrows + kTabBatchRows - 1) / kTabBatchRows;
    const int mynb = wave < nbatch ? (nbatch - 1 - wave) / kTabWaves + 1 : 0;  // this wave's batches (<= BMAX)

    // 1. table operands, raw: tile t = 2 wave + tt covers entries 32 (t & 7) + 0..31 and
    //    positions of sub-table (t >> 4), bytes 2 ((t >> 3) & 1) + 0..1; MFMA column n = lane % 32
    //    is byte 2 ((t >> 3) & 1) + n / 16 of dword 4 (n % 16) + 2 p + sub-table
    uint16_t cbr[2][2];
    float xr[2][2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int t = 2 * wave + tt, c0 = 32 * (t & 7), ts = t >> 3;
        const int j = 2 * (ts & 1) + ((lane >> 4) & 1), qn = lane & 15;
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            const int e = 2 * k2 + (lane >> 5);
            cbr[tt][k2] = cbh[kVq2Dim * (c0 + (lane & 31)) + e];
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int b = 4 * (4 * qn + 2 * p + (ts >> 1)) + j;
                xr[p][tt][k2] = x[b < nb ? kVq2Dim * b + e : 0];
            }
        }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // 2. the index loads of this wave's first batch (out-of-range offsets read 0 and fetch
    //    nothing); the other batches follow once the first table is built (step 3)
    const uint8_t *idx = w + kVq2CodebookBytes + static_cast<size_t>(r0) * nb;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(idx), static_cast<short>(0),
                                                                        nrows * nb, kBufferFlags);
    uint4 q4[BMAX][4];
    const bool qok = 4 * q < nd;
    auto issue = [&](int i) {
        const int row0 = kTabBatchRows * (wave + kTabWaves * i) + rho;
        const bool ok = i < mynb && qok;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            q4[i][r] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? (row0 + 4 * r) * nb + 16 * q : 0xFFFFFFF0u, 0, 0));
    };
    issue(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    float av[2][2], bv[2][2][2];
    bool pad[2][2];  // the tile column lies past the row end: its entries are stored as 0
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int ts = (2 * wave + tt) >> 3;
        const int j = 2 * (ts & 1) + ((lane >> 4) & 1), qn = lane & 15;
#pragma unroll
        for (int p = 0; p < 2; ++p) pad[p][tt] = 4 * (4 * qn + 2 * p + (ts >> 1)) + j >= nb;
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            av[tt][k2] = half_bits(cbr[tt][k2]);
#pragma unroll
            for (int p = 0; p < 2; ++p) bv[p][tt][k2] = pad[p][tt] ? 0.f : xr[p][tt][k2];
        }
    }
    unsigned loff[2][4], sel[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const unsigned jl = (k + rho) & 3;
        loff[0][k] = 64u * jl + 4u * q;
        loff[1][k] = loff[0][k] | 0x10000u;
        sel[k] = 0x0C020000u | ((4u + jl) << 8);  // bytes: loff.0, index byte jl, loff.2, zero
    }
    auto build = [&](int p) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = 2 * wave + tt, c0 = 32 * (t & 7), ts = t >> 3;
            f16v d = {};
            d = __builtin_amdgcn_mfma_f32_32x32x2f32(av[tt][0], bv[p][tt][0], d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_32x32x2f32(av[tt][1], bv[p][tt][1], d, 0, 0, 0);
            const unsigned base = ((ts >> 1) << 16) + 64 * (2 * (ts & 1) + ((lane >> 4) & 1)) + 4 * (lane & 15);
#pragma unroll
            for (int r = 0; r < 16; ++r) {  // D row 8 (r / 4) + 4 (lane / 32) + r % 4 = entry offset
                const int c = c0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                *reinterpret_cast<float *>(tab + base + 256 * c) = pad[p][tt] ? 0.f : d[r];
            }
        }
    };

    float acc[BMAX][4];
#pragma unroll
    for (int i = 0; i < BMAX; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][r] = 0.f;
    // 3. the first table, then the rest of the index stream. Issued whole before the first table,
    //    the stream queued the cold codebook's read behind all 34 MB of index reads (the table
    //    was ready ~4 us after the start at 151936x896); with the first batch alone in flight
    //    the codebook arrives early and the first pass's lookups overlap the stream (12.5 ->
    //    11.7 us, 131072x1024 12.4 -> 11.3). The first batch keeps HBM busy meanwhile.
    build(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 1; i < BMAX; ++i) issue(i);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        if (p) {
            __syncthreads();  // every lookup of the first pass is done
            build(1);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < BMAX; ++i) {
            if (i < mynb) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float s = acc[i][r];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const unsigned dw = p == 0 ? (h ? q4[i][r].y : q4[i][r].x) : (h ? q4[i][r].w : q4[i][r].z);
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            s += *reinterpret_cast<const float *>(tab + __builtin_amdgcn_perm(dw, loff[h][k], sel[k]));
                    }
                    acc[i][r] = s;
                }
            }
        }
    }

    // 4. per batch: the 4 row sums of each lane added over its 16 lanes by halving exchanges
    //    (row_mirror, row_half_mirror, then quad swaps); lanes 4 m + 0 of each 16 keep row
    //    4 m + rho's total
#pragma unroll
    for (int i = 0; i < BMAX; ++i) {
        if (i < mynb) {
            float v0 = acc[i][0], v1 = acc[i][1], v2 = acc[i][2], v3 = acc[i][3];
            const bool u8 = lane & 8, u4 = lane & 4;
            {
                const float lo0 = v0 + tab_dpp<0x140>(v0), hi0 = v2 + tab_dpp<0x140>(v2);
                const float lo1 = v1 + tab_dpp<0x140>(v1), hi1 = v3 + tab_dpp<0x140>(v3);
                v0 = u8 ? hi0 : lo0;
                v1 = u8 ? hi1 : lo1;
            }
            {
                const float lo = v0 + tab_dpp<0x141>(v0), hi = v1 + tab_dpp<0x141>(v1);
                v0 = u4 ? hi : lo;
            }
            v0 += tab_dpp<0x4E>(v0);
            v0 += tab_dpp<0xB1>(v0);
            const int row = kTabBatchRows * (wave + kTabWaves * i) + 4 * ((lane >> 2) & 3) + rho;
            if ((lane & 3) == 0 && row < nrows) y[r0 + row] = v0;
        }
    }
}

}  // namespace

int launch_vq2_matvec(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, hipStream_t stream) {
    if (out_dim < 1 || in_dim < kVq2Dim || in_dim % kVq2Dim) return kBadShape;
    if (!w || !x || !y) return kBadShape;  // nothing is launched on a null operand
    const int cus = device_cu_count();
    const bool aligned = (in_dim % 16) == 0 && (reinterpret_cast<uintptr_t>(w) % 4) == 0;
    if (rows_kernel_takes(w, out_dim, in_dim)) {
        Vq2SetArgs a{};
        a.m[0] = Vq2Mat{w, x, y, out_dim, in_dim, 0, nullptr, nullptr};
        return launch_rows(a, 1, (out_dim + 3) / 4, (reinterpret_cast<uintptr_t>(x) & 15) == 0, stream);
    }
    if (in_dim % 64 == 0 && in_dim <= kTabMaxDim && (reinterpret_cast<uintptr_t>(w) % 16) == 0 &&
        static_cast<long long>(out_dim) >= static_cast<long long>(kTabMinRowsPerCu) * cus) {
        // index rows 16-byte aligned and large: the dot-product table, one workgroup per CU (at
        // most 1024 rows each, more workgroups beyond 1024 rows per CU)
        constexpr int kMaxRows = kTabWaves * kTabBatchRows * kTabMaxBatches;
        const int grid = std::max(cus, (out_dim + kMaxRows - 1) / kMaxRows);
        const int rpw = (out_dim + grid - 1) / grid;
        const int batches = ((rpw + kTabBatchRows - 1) / kTabBatchRows + kTabWaves - 1) / kTabWaves;
        switch (batches) {
            case 1: hipLaunchKernelGGL(vq2_matvec_table<1>, dim3(grid), dim3(64 * kTabWaves), 0, stream, w, x, y, out_dim, in_dim, rpw); break;
            case 2: hipLaunchKernelGGL(vq2_matvec_table<2>, dim3(grid), dim3(64 * kTabWaves), 0, stream, w, x, y, out_dim, in_dim, rpw); break;
            case 3: hipLaunchKernelGGL(vq2_matvec_table<3>, dim3(grid), dim3(64 * kTabWaves), 0, stream, w, x, y, out_dim, in_dim, rpw); break;
            case 4: hipLaunchKernelGGL(vq2_matvec_table<4>, dim3(grid), dim3(64 * kTabWaves), 0, stream, w, x, y, out_dim, in_dim, rpw); break;
            default: return kBadShape;  // unreachable: rpw <= kMaxRows
        }
        return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
    }
    if (aligned) {
        // index rows dword-aligned: the conflict-free kernel (16 waves x 4-row
        // tiles measured fastest at 3072..16384 rows, within 4% of the best at
        // 151936 rows)
        const bool one = in_dim <= 1024;  // one 256-byte chunk of indices per row
        const int tiles = (out_dim + kVq2Rows - 1) / kVq2Rows;
        const int g = std::max(1, std::min((tiles + kVq2Waves - 1) / kVq2Waves, 2 * cus));
        auto kernel = one ? vq2_matvec_copies<kVq2Rows, true> : vq2_matvec_copies<kVq2Rows, false>;
        hipLaunchKernelGGL(kernel, dim3(g), dim3(64 * kVq2Waves), 0, stream, w, x, y, out_dim, in_dim);
        return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
    }
    const int tiles = (out_dim + kRows - 1) / kRows;
    const int grid = std::max(1, std::min((tiles + kWavesPerBlock - 1) / kWavesPerBlock, cus * 8));
    hipLaunchKernelGGL(vq2_matvec_kernel, dim3(grid), dim3(64 * kWavesPerBlock), 0, stream, w, x, y, out_dim,
                       in_dim);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

// The matrices the one-wave-per-row kernel takes go into one launch per kSetMaxMats of them
// (a launch is closed early once it holds more than 2 kDirectLookups lookups, where the replica
// kernel would be faster); any other matrix is launched alone by launch_vq2_matvec. Every row
// gets the same bits as from launch_vq2_matvec.
int launch_vq2_matvec_set(int n, const I4Mat *mats, hipStream_t stream) {
    if (n < 0 || (n > 0 && !mats)) return kBadShape;
    for (int i = 0; i < n; ++i)
        if (mats[i].M < 1 || mats[i].K < kVq2Dim || mats[i].K % kVq2Dim || !mats[i].w || !mats[i].x || !mats[i].y)
            return kBadShape;
    Vq2SetArgs a{};
    int nb = 0, blocks = 0;
    long long lookups = 0;
    bool xalign = true;
    for (int i = 0; i < n; ++i) {
        const I4Mat &mt = mats[i];
        if (!rows_kernel_takes(mt.w, mt.M, mt.K)) {
            const int st = launch_vq2_matvec(mt.w, mt.x, mt.y, mt.M, mt.K, stream);
            if (st != kOk) return st;
            continue;
        }
        const long long lk = static_cast<long long>(mt.M) * (mt.K / kVq2Dim);
        if (nb == kSetMaxMats || (nb > 0 && lookups + lk > 2 * kDirectLookups)) {
            const int st = launch_rows(a, nb, blocks, xalign, stream);
            if (st != kOk) return st;
            nb = blocks = 0;
            lookups = 0;
            xalign = true;
        }
        a.m[nb++] = Vq2Mat{mt.w, mt.x, mt.y, mt.M, mt.K, blocks, nullptr, nullptr};
        blocks += (mt.M + 3) / 4;
        lookups += lk;
        xalign = xalign && (reinterpret_cast<uintptr_t>(mt.x) & 15) == 0;
    }
    return nb > 0 ? launch_rows(a, nb, blocks, xalign, stream) : kOk;
}

// n VQ2 matvecs in ONE launch of the one-wave-per-row kernel with staged activations: the
// prologue pro (kind 1 or 2, shared by the matrices, which then share x and K; null for none),
// then, where sign is given, each matrix's own BiIP rotation (rotate as launch_biip_rotate, the
// block size shared by the launch). Each output has the bits of the separate swiglu /
// add_rmsnorm, biip_rotate and launch_vq2_matvec launches. kNotFused (nothing launched) when a
// matrix is not one the kernel takes, the set needs more than one launch, the block does not
// divide a row length, or there is nothing to stage.
int launch_vq2_matvec_set_pro(int n, const I4Mat *mats, const float *const *scale, const float *const *sign,
                              int block_size, const SetPrologue *pro, hipStream_t stream) {
    const int xm = pro ? pro->kind : 0;
    if (n < 1 || n > kStagedMaxMats || xm < 0 || xm > 2 || (!sign && !xm)) return kNotFused;
    if (xm == 1 && !pro->x2) return kNotFused;
    if (xm == 2 && !pro->nw) return kNotFused;
    // a rotation block lies within one wave's 256 activations
    if (sign && (block_size < 1 || block_size > 256 || (block_size & (block_size - 1)))) return kNotFused;
    auto a16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };  // null passes
    if (pro && !(a16(pro->x2) && a16(pro->d1) && a16(pro->d2) && a16(pro->nw) && a16(pro->hout))) return kNotFused;
    Vq2StagedArgs a{};
    int rows = 0, kmax = 0;
    long long lookups = 0;
    for (int i = 0; i < n; ++i) {
        const I4Mat &mt = mats[i];
        if (mt.M < 1 || mt.K < kVq2Dim || mt.K % kVq2Dim || !rows_kernel_takes(mt.w, mt.M, mt.K) || !a16(mt.x))
            return kNotFused;
        if (sign && (!sign[i] || mt.K % block_size || !a16(sign[i]) || !a16(scale[i]))) return kNotFused;
        if (xm && (mt.x != mats[0].x || mt.K != mats[0].K)) return kNotFused;
        rows += mt.M;
        lookups += static_cast<long long>(mt.M) * (mt.K / kVq2Dim);
        kmax = std::max(kmax, mt.K);
    }
    // up to 5 passes of 2048 activations (the RMSNorm's operands: 3)
    if (lookups > 2 * kDirectLookups || kmax > (xm == 2 ? 6144 : 10240)) return kNotFused;
    // Rows per wave: 4 when the set has enough rows to keep 300 workgroups (the build is then
    // shared by 32 rows) and K <= 6144 (with 5 passes the index dwords of 4 rows went to
    // scratch memory), else 1.
    const int passes = (kmax + kStagedPass - 1) / kStagedPass;
    const int rpw = passes <= 3 && rows >= 4 * kRotWaves * 300 ? 4 : 1;
    int blocks = 0;
    for (int i = 0; i < n; ++i) {
        const I4Mat &mt = mats[i];
        a.m[i] = Vq2Mat{mt.w, mt.x, mt.y, mt.M, mt.K, blocks, sign ? scale[i] : nullptr, sign ? sign[i] : nullptr};
        blocks += (mt.M + kRotWaves * rpw - 1) / (kRotWaves * rpw);
    }
    for (int k = n; k < kStagedMaxMats; ++k) a.m[k] = a.m[n - 1];  // never selected (k >= n)
    a.n = n;
    if (pro) a.pro = *pro;
    if (sign) {
        int lg = 0;
        while ((1 << lg) < block_size) ++lg;
        a.lg_bs = lg;
        a.inv_sqrt = 1.0f / std::sqrt(static_cast<float>(block_size));  // as launch_biip_rotate computes it
    }
    const dim3 grid(blocks), block(64 * kRotWaves);
    const size_t lds = static_cast<size_t>(kmax) * 4;
    auto go = [&](auto npc, auto rc) {  // the instance of (xm, rotation); xm was checked above
        constexpr int NP = decltype(npc)::value, R = decltype(rc)::value;
        if (xm == 0)
            hipLaunchKernelGGL((vq2_matvec_staged<NP, 0, true, R>), grid, block, lds, stream, a);
        else if (xm == 1 && sign)
            hipLaunchKernelGGL((vq2_matvec_staged<NP, 1, true, R>), grid, block, lds, stream, a);
        else if (xm == 1)
            hipLaunchKernelGGL((vq2_matvec_staged<NP, 1, false, R>), grid, block, lds, stream, a);
        else if (sign)
            hipLaunchKernelGGL((vq2_matvec_staged<NP, 2, true, R>), grid, block, lds, stream, a);
        else
            hipLaunchKernelGGL((vq2_matvec_staged<NP, 2, false, R>), grid, block, lds, stream, a);
    };
    auto go_np = [&](auto rc) {
        if (passes <= 1)
            go(std::integral_constant<int, 1>{}, rc);
        else if (passes == 2)
            go(std::integral_constant<int, 2>{}, rc);
        else if (passes == 3)
            go(std::integral_constant<int, 3>{}, rc);
        else if constexpr (decltype(rc)::value == 1)
            go(std::integral_constant<int, 5>{}, rc);
    };
    if (rpw == 4)
        go_np(std::integral_constant<int, 4>{});
    else
        go_np(std::integral_constant<int, 1>{});
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

int launch_vq2_matvec_set_rot(int n, const I4Mat *mats, const float *const *scale, const float *const *sign,
                              int block_size, hipStream_t stream) {
    if (!sign) return kNotFused;
    return launch_vq2_matvec_set_pro(n, mats, scale, sign, block_size, nullptr, stream);
}

// The staged launch would take these shapes: a set of matrices of row length K with the given
// rows, with prologue kind xm (the engine decides its fused layers with it).
bool vq2_set_takes(int n, const int *M, int K, int xm) {
    long long lookups = 0;
    for (int i = 0; i < n; ++i) {
        if (M[i] < 1 || K % 16 || static_cast<long long>(M[i]) * (K / kVq2Dim) > kDirectLookups) return false;
        lookups += static_cast<long long>(M[i]) * (K / kVq2Dim);
    }
    return n >= 1 && n <= kStagedMaxMats && lookups <= 2 * kDirectLookups && K <= (xm == 2 ? 6144 : 10240);
}

}  // namespace tqhip
