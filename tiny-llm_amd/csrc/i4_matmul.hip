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
//      elements per step. Each step the workgroup loads its W slice
//      (group header + 16 code bytes per thread-unit) and the fp16 X slice
//      into registers one step ahead, dequantizes W as q * scale - zero * scale
//      with one rounding to fp16 (v_fma_mix) into LDS, and contracts with
//      v_mfma_f32_32x32x16_f16 (fp32 accumulation).
//      fp16 and bf16 MFMA run at the same rate on gfx950; fp16 keeps 8x
//      finer rounding of both operands.
// Other group sizes: one i4 matvec per token column.

#include "tq_common.h"

#include <algorithm>
#include <mutex>

namespace tqhip {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));

constexpr int kStepK = 64;             // K elements per main-loop step
constexpr int kRowHalves = kStepK + 8;  // LDS row stride in halves (144 B: conflict-free 16-byte reads)
constexpr int kThreads = 256;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void *base, size_t bytes) {
    const int nrec = bytes > 0xFFFFFFFFull ? -1 : static_cast<int>(static_cast<unsigned>(bytes));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), nrec, kBufferFlags);
}

// ---- 1. X (fp32, column n = token) -> fp16 * 2^e_n, rows padded to Kp
__global__ __launch_bounds__(256) void x_to_f16(const float *__restrict__ x, int K, int Kp, _Float16 *__restrict__ xh,
                                                  float *__restrict__ xinv) {
    const int n = blockIdx.x;
    const float *xc = x + static_cast<size_t>(n) * K;
    float m = 0.f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) m = fmaxf(m, fabsf(xc[k]));
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
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
    for (int k = threadIdx.x; k < Kp; k += blockDim.x)
        hc[k] = static_cast<_Float16>(k < K ? ldexpf(xc[k], e) : 0.f);
    if (threadIdx.x == 0) xinv[n] = ldexpf(1.f, -e);
}

__device__ inline float half_bits_f(unsigned h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h & 0xFFFFu)));
}

// fp16 pair {q0 * s + c, q1 * s + c}: each computed exactly and rounded once
// to fp16 (v_fma_mix with fp32 operands).
__device__ inline unsigned fma_pair_f16(float q0, float q1, float s, float c) {
    unsigned r;
    asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,0,0]" : "=v"(r) : "v"(q0), "v"(s), "v"(c));
    asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel_hi:[0,0,0]" : "+v"(r) : "v"(q1), "v"(s), "v"(c));
    return r;
}

// Dequantizes 32 consecutive elements (16 code bytes, low nibble first) of one
// group to fp16: q * scale - zero * scale with one rounding to fp16 (within
// one fp16 rounding of the reference's fp32 (q - zero) * scale).
__device__ inline void dequant32(const unsigned (&c)[4], unsigned hdr, bool valid, u4v (&out)[2][2]) {
    const float s = valid ? half_bits_f(hdr) : 0.f;
    const float nzs = valid ? -(half_bits_f(hdr >> 16) * s) : 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const unsigned lo = c[d] & 0x0F0F0F0Fu;         // elements 8d + 0, 2, 4, 6
        const unsigned hi = (c[d] >> 4) & 0x0F0F0F0Fu;  // elements 8d + 1, 3, 5, 7
        unsigned pk[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float q0 = static_cast<float>((lo >> (8 * b)) & 0xFFu);
            const float q1 = static_cast<float>((hi >> (8 * b)) & 0xFFu);
            pk[b] = fma_pair_f16(q0, q1, s, nzs);
        }
        out[d >> 1][d & 1] = u4v{pk[0], pk[1], pk[2], pk[3]};
    }
}

// ---- 2. MFMA tile kernel
//   WM x WN blocks of 32x32 per wave, WAVES_M x WAVES_N waves (= 4).
template <int WM, int WN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(kThreads) void i4_matmul_mfma(const uint8_t *__restrict__ w,
                                                           const _Float16 *__restrict__ xh,
                                                           const float *__restrict__ xinv, float *__restrict__ y,
                                                           int M, int N, int K, int Kp, int G, int row_bytes) {
    static_assert(WAVES_M * WAVES_N == 4, "four waves");
    constexpr int BM = 32 * WM * WAVES_M;
    constexpr int BN = 32 * WN * WAVES_N;
    constexpr int UNITS = 2 * BM / kThreads;  // 32-element W units per thread per step
    constexpr int XCH = BN * 8 / kThreads;    // 16-byte X chunks per thread per step
    static_assert(UNITS >= 1 && XCH >= 1, "tile too small for the thread count");
    __shared__ __align__(16) _Float16 sw[2][BM * kRowHalves];
    __shared__ __align__(16) _Float16 sx[2][BN * kRowHalves];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    const int gb = 4 + G / 2;
    const int groups = (K + G - 1) / G;
    const int steps = Kp / kStepK;

    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + static_cast<size_t>(m0) * row_bytes,
                                                static_cast<size_t>(M - m0) * row_bytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(xh + static_cast<size_t>(n0) * Kp,
                                                static_cast<size_t>(N - n0) * Kp * 2);

    // per-thread load slots
    int urow[UNITS], uhalf[UNITS];
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
        const int id = tid + u * kThreads;
        urow[u] = id >> 1;
        uhalf[u] = id & 1;
    }
    int xrow[XCH], xcol[XCH];
#pragma unroll
    for (int c = 0; c < XCH; ++c) {
        const int id = tid + c * kThreads;
        xrow[c] = id >> 3;  // token within the tile
        xcol[c] = id & 7;   // 16-byte chunk within the 128-byte step slice
    }

    unsigned wc[UNITS][4], wh[UNITS];
    bool wv[UNITS];
    u4v xv[XCH];
    auto load_step = [&](int s) {
#pragma unroll
        for (int u = 0; u < UNITS; ++u) {
            const int k0 = s * kStepK + 32 * uhalf[u];
            const int g = k0 / G;
            wv[u] = g < groups;
            const int gg = min(g, groups - 1);
            const int base = urow[u] * row_bytes + gg * gb;
            const int cb = base + 4 + (k0 - gg * G) / 2;
            wh[u] = __builtin_amdgcn_raw_buffer_load_b32(wr, base, 0, 0);
#pragma unroll
            for (int d = 0; d < 4; ++d) wc[u][d] = __builtin_amdgcn_raw_buffer_load_b32(wr, cb + 4 * d, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < XCH; ++c)
            xv[c] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                xr, (xrow[c] * Kp + s * kStepK) * 2 + 16 * xcol[c], 0, 0));
    };
    auto store_step = [&](int b) {
#pragma unroll
        for (int u = 0; u < UNITS; ++u) {
            u4v o[2][2];
            dequant32(wc[u], wh[u], wv[u], o);
            _Float16 *dst = &sw[b][urow[u] * kRowHalves + 32 * uhalf[u]];
            *reinterpret_cast<u4v *>(dst) = o[0][0];
            *reinterpret_cast<u4v *>(dst + 8) = o[0][1];
            *reinterpret_cast<u4v *>(dst + 16) = o[1][0];
            *reinterpret_cast<u4v *>(dst + 24) = o[1][1];
        }
#pragma unroll
        for (int c = 0; c < XCH; ++c) *reinterpret_cast<u4v *>(&sx[b][xrow[c] * kRowHalves + 8 * xcol[c]]) = xv[c];
    };

    f16x acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = f16x{};

    const int li = lane & 31, lk = 8 * (lane >> 5);
    load_step(0);
    store_step(0);
    __syncthreads();
    for (int s = 0; s < steps; ++s) {
        const int b = s & 1;
        if (s + 1 < steps) load_step(s + 1);
#pragma unroll
        for (int kk = 0; kk < kStepK; kk += 16) {
            h8 a[WM], bb[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i)
                a[i] = *reinterpret_cast<const h8 *>(&sw[b][(32 * (wm * WM + i) + li) * kRowHalves + kk + lk]);
#pragma unroll
            for (int j = 0; j < WN; ++j)
                bb[j] = *reinterpret_cast<const h8 *>(&sx[b][(32 * (wn * WN + j) + li) * kRowHalves + kk + lk]);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bb[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < steps) store_step(b ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds rows (r/4)*8 + (lane/32)*4 + r%4 of column lane%32
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        const int n = n0 + 32 * (wn * WN + j) + li;
        if (n >= N) continue;
        const float sc = xinv[n];
        float *yc = y + static_cast<size_t>(n) * M;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int m = m0 + 32 * (wm * WM + i) + 8 * r4 + 4 * (lane >> 5);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (m + q < M) yc[m + q] = acc[i][j][4 * r4 + q] * sc;
            }
        }
    }
}

// Grow-only device workspace for the fp16 copy of X (one per process; the
// launches that use it are ordered on their streams by the caller).
struct Workspace {
    std::mutex mu;
    void *ptr = nullptr;
    size_t bytes = 0;
};
Workspace &workspace() {
    static Workspace ws;
    return ws;
}

void *workspace_at_least(size_t bytes) {
    Workspace &ws = workspace();
    std::lock_guard<std::mutex> lock(ws.mu);
    if (ws.bytes < bytes) {
        if (ws.ptr) {
            TQ_HIP_CHECK(hipDeviceSynchronize());  // earlier launches may still read it
            TQ_HIP_CHECK(hipFree(ws.ptr));
        }
        const size_t want = std::max(bytes, ws.bytes * 2);
        TQ_HIP_CHECK(hipMalloc(&ws.ptr, want));
        ws.bytes = want;
    }
    return ws.ptr;
}

template <int WM, int WN, int WAVES_M, int WAVES_N>
int launch_tiles(const uint8_t *w, const _Float16 *xh, const float *xinv, float *y, int M, int N, int K, int Kp, int G,
                 int rb, hipStream_t stream) {
    constexpr int BM = 32 * WM * WAVES_M, BN = 32 * WN * WAVES_N;
    const dim3 grid((M + BM - 1) / BM, (N + BN - 1) / BN);
    hipLaunchKernelGGL((i4_matmul_mfma<WM, WN, WAVES_M, WAVES_N>), grid, dim3(kThreads), 0, stream, w, xh, xinv, y, M,
                       N, K, Kp, G, rb);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

}  // namespace

int launch_i4_matmul(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                     hipStream_t stream) {
    if (M < 1 || K < 1 || N < 1 || group_size < 2 || (group_size & 1)) return kBadShape;
    const size_t rb = i4_row_bytes(K, group_size);
    const size_t Kp = (static_cast<size_t>(K) + kStepK - 1) / kStepK * kStepK;
    const bool mfma = group_size % 32 == 0 && rb * static_cast<size_t>(M) < (1ull << 31) &&
                      Kp * 2 * static_cast<size_t>(N) < (1ull << 31);
    if (!mfma) {
        for (int n = 0; n < N; ++n) {
            const int st = launch_i4_matvec(w, x + static_cast<size_t>(n) * K, y + static_cast<size_t>(n) * M, M, K,
                                            group_size, stream);
            if (st != kOk) return st;
        }
        return kOk;
    }
    const size_t xh_bytes = (Kp * 2 * N + 255) / 256 * 256;
    unsigned char *ws = static_cast<unsigned char *>(workspace_at_least(xh_bytes + 4 * static_cast<size_t>(N)));
    _Float16 *xh = reinterpret_cast<_Float16 *>(ws);
    float *xinv = reinterpret_cast<float *>(ws + xh_bytes);
    hipLaunchKernelGGL(x_to_f16, dim3(N), dim3(256), 0, stream, x, K, static_cast<int>(Kp), xh, xinv);
    if (hipGetLastError() != hipSuccess) return kLaunchFailed;
    const int ikp = static_cast<int>(Kp), irb = static_cast<int>(rb);
    if (N <= 32) return launch_tiles<2, 1, 4, 1>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
    if (N <= 64) return launch_tiles<2, 1, 2, 2>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
    return launch_tiles<2, 2, 2, 2>(w, xh, xinv, y, M, N, K, ikp, group_size, irb, stream);
}

}  // namespace tqhip
