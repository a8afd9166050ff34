// i4_set.hip -- one launch over a set of i4 HQQ@64 matvecs, each with its own
// activation vector, output, row count and row length.
//
// A decoder layer's matvec set (q, k, v, o, gate, up, down: four distinct
// activation vectors) is about 8 MB at Qwen2.5-0.5B scale, a microsecond or two
// of HBM time, while every separate launch costs a few microseconds of dispatch
// and load latency. This kernel covers the whole set with one grid:
//   * Every workgroup belongs to one matrix (the matrices' workgroups are
//     numbered one after the other, the longest rows first so they start
//     first); the matrix is found with a few scalar compares against the
//     kernel argument.
//   * The workgroup's activation loads are issued first, then half of the weight
//     loads of its rows; the activations are turned into exact integer operands
//     in LDS (one power-of-two exponent per group of 64), the other half of the
//     weight loads goes out, and one barrier later every wave reads its slices
//     from LDS.
//   * Rows of up to 32 half-groups (K <= 1024) take one half-wave each (two rows
//     per half-wave on larger sets), longer rows (K <= 10240) one wave each over
//     1..5 slots of 64 half-groups (two rows per wave when every long-row matrix
//     of the launch has >= 2048 rows); lane u computes half-group u (32 weights: 16
//     code bytes and the group header) with v_dot4 on the code nibbles and the
//     activation digits, exact before a per-half-group fp32 epilogue.
// The same kernel serves single-matrix and pair / qkv launches of decode size
// (launch_i4_matvec_set_fit), so a matrix gives the same bits alone or in a set.
// Numerics: the only rounding before the epilogue is x -> X (relative 2^-23 of the
// group's largest |x|); measured rel L2 ~4e-7 against the double-accumulating reference
// (kernels/matvec/matvec_i4_ref.cpp:45-103).
#include "i4_set_core.h"

#include <algorithm>

namespace tqhip {
namespace {

struct SetMat {
    const uint8_t *w;
    const float *x;
    float *y;
    int M, K;
    int blk0;   // first workgroup of this matrix
    int shape;  // 0: one row per half-wave (K <= 1024); s = 1..5: one row per wave over s slots
};
// C: the records the kernel argument holds. Launches of up to kSetSmallMats matrices (a decode
// engine's launches, single and fused matvecs) carry that many; five fewer records in the
// argument measured 0.17 us less per launch (VQ2 staged launches, decode engine).
constexpr int kSetSmallMats = 3;
template <int C>
struct SetArgs {
    SetMat m[C];
    int n;
    SetPrologue pro;  // XM != 0 instances only
};

// XM: the activation prologue (0 none; 1 x = silu(x) * x2; 2 x = rmsnorm((x + d1) + d2) * nw,
// workgroup 0 storing the sum to hout), with its operands in pro. GLU: every row of m is computed
// together with the same row of w2 (a matrix of m's shape reading the same x), and the row's
// output is swiglu(m row, w2 row), as the separate outputs would give it in a SwiGLU prologue.
template <int S, int R, int XM, bool GLU = false>
__device__ __forceinline__ void set_rows(const SetMat &m, int blk, unsigned char *lds, const SetPrologue &pro,
                                         const uint8_t *w2 = nullptr) {
    // 16-byte activation loads per thread: the chunks of the widest row of this shape
    constexpr int NX = ((S == 0 ? 256 : 512 * S) + kSetThreads - 1) / kSetThreads;
    constexpr int NR = GLU ? 2 * R : R;     // rows per lane (GLU: R of m, then the same R of w2)
    constexpr int NS = S == 0 ? 1 : S;      // half-group slots per lane
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int U = 2 * ((m.K + 63) / 64), rb = 18 * U;  // half-groups and bytes per row
    const int C = 8 * U;                                 // 16-byte activation chunks the rows read
    unsigned char *xp = lds;                                              // C / 2 blocks of operands
    float2 *hs = reinterpret_cast<float2 *>(lds + (C / 2) * kBlockBytes);  // U (sum(X), 2^-f)

    // 1. the activations first: chunk t + kSetThreads i, clamped to the last one (zeroed past K
    // in stage_x). (Plain 16-byte loads: with a 16-byte buffer load whose elements are used
    // as floats, this compiler shrinks the load to its first dword and reuses that dword.)
    const float4 *x4 = reinterpret_cast<const float4 *>(m.x);
    const int Kc = m.K / 4;
    float4 xq[NX];
#pragma unroll
    for (int i = 0; i < NX; ++i) xq[i] = x4[min(t + kSetThreads * i, Kc - 1)];
    // the prologue's operands, loaded with x: up (XM 1); the deltas and the norm weight (XM 2)
    constexpr int NP = XM ? NX : 1, NQ = XM == 2 ? NX : 1;
    float4 pa[NP], pb[NQ], pw[NQ];
    if constexpr (XM == 1) {
        const float4 *u4 = reinterpret_cast<const float4 *>(pro.x2);
#pragma unroll
        for (int i = 0; i < NX; ++i) pa[i] = u4[min(t + kSetThreads * i, Kc - 1)];
    } else if constexpr (XM == 2) {
        const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 *d1 = reinterpret_cast<const float4 *>(pro.d1), *d2 = reinterpret_cast<const float4 *>(pro.d2);
        const float4 *w4 = reinterpret_cast<const float4 *>(pro.nw);
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int c = min(t + kSetThreads * i, Kc - 1);
            pa[i] = d1 ? d1[c] : zero;
            pb[i] = d2 ? d2[c] : zero;
            pw[i] = w4[c];
        }
    }

    // 2. the weights: lane u of a row takes half-group u (+ 64 per slot)
    const int half = S == 0 ? lane >> 5 : 0, u = S == 0 ? lane & 31 : lane;
    // the wave's first row (uniform, so the buffer resource stays in scalar registers); the
    // half-wave's row goes into the per-lane offset
    const int base = S == 0 ? (blk * kSetWaves + wave) * 2 * R : (blk * kSetWaves + wave) * R;
    const __amdgpu_buffer_rsrc_t wr = rows_rsrc(m.w, m.M, rb, base);  // rows past the matrix read 0
    const __amdgpu_buffer_rsrc_t wr2 = rows_rsrc(GLU ? w2 : m.w, m.M, rb, base);
    // Half of the lane's (row, slot) loads go out now, the other half once the activations
    // are converted. The activations are cold (a step's weights stream through every cache),
    // so their read waits in the memory queues behind whatever weight reads went out before
    // it; with half of the weight reads in flight it returns sooner, and the first half keeps
    // HBM busy meanwhile. Measured on MI355X (cold, one box): layer set 4.91 -> 4.78 us,
    // 2560x9728 7.82 -> 7.17, 9728x2560 7.30 -> 7.19, 2560x4096 4.34 -> 4.24.
    unsigned hd[NR * NS];
    v4i cd[NR * NS];
    constexpr int NU = NR * NS, NFIRST = NU > 1 ? NU / 2 : 1;
    auto issue = [&](int q) {  // row q / NS, slot q % NS
        const int r = q / NS, sl = q % NS;
        const int rr = GLU ? r % R : r;  // GLU: rows R.. are the same rows of w2
        const int unit = u + 64 * sl;
        const int off = (S == 0 ? 2 * rr + half : rr) * rb + (kI4Header + 32) * (unit >> 1);
        const __amdgpu_buffer_rsrc_t rs = GLU && r >= R ? wr2 : wr;
        hd[q] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
        cd[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + kI4Header + 16 * (unit & 1), 0, 0);
    };
#pragma unroll
    for (int q = 0; q < NFIRST; ++q) issue(q);
    // the first half is issued before the wait for the activations below (without the barrier
    // the compiler moved the weight loads behind it, serialising two HBM round trips)
    __builtin_amdgcn_sched_barrier(0);

    // 3. activations to integer operands in LDS, while the weights arrive. Every iteration
    // runs (stage_x writes only chunks below C): a loop that stopped early would let the
    // compiler sink the later activation loads behind the weight loads.
    if constexpr (XM == 1) {  // swiglu_ref (kernels/silu/swiglu_ref.cpp): silu(g) * u
#pragma unroll
        for (int i = 0; i < NX; ++i) xq[i] = swiglu4(xq[i], pa[i]);
    } else if constexpr (XM == 2) {
        // hidden + delta(s) in the runtime's order, then rmsnorm_ref (kernels/rmsnorm/rmsnorm_ref.cpp):
        // a double sum of squares, a float mean, 1 / sqrt(mean + eps), (h * scale) * w
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            if (pro.d1) xq[i] = add4(xq[i], pa[i]);
            if (pro.d2) xq[i] = add4(xq[i], pb[i]);
            if (t + kSetThreads * i < Kc) ss += sq4(xq[i]);
        }
        if (pro.hout && blockIdx.x == 0) {
            float4 *h4 = reinterpret_cast<float4 *>(pro.hout);
#pragma unroll
            for (int i = 0; i < NX; ++i)
                if (t + kSetThreads * i < Kc) h4[t + kSetThreads * i] = xq[i];
        }
        ss = set_block_sum(ss);
        const float scale = rms_scale(ss, m.K, pro.eps);
#pragma unroll
        for (int i = 0; i < NX; ++i) xq[i] = rms_apply(xq[i], scale, pw[i]);
    }
#pragma unroll
    for (int i = 0; i < NX; ++i) stage_x(xq[i], t + kSetThreads * i, Kc, C, xp, hs);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = NFIRST; q < NU; ++q) issue(q);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    // 4. the row sums; lanes past the row's half-groups read the last one (ignored)
    float p[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) p[r] = 0.f;
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
        const int unit = u + 64 * sl;
        const int ru = min(unit, U - 1);
        unsigned xv[24];
        const v4i *src = reinterpret_cast<const v4i *>(xp + ru * 4 * kBlockBytes);
#pragma unroll
        for (int k = 0; k < 6; ++k) {
            const v4i v = src[k];
            xv[4 * k] = v[0];
            xv[4 * k + 1] = v[1];
            xv[4 * k + 2] = v[2];
            xv[4 * k + 3] = v[3];
        }
        const float2 h = hs[ru];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const float v = half_group_int(cd[r * NS + sl], hd[r * NS + sl], xv, h);
            if (unit < U) p[r] += v;
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = base + (S == 0 ? 2 * r + half : r);
        const float sum = S == 0 ? sum_half_wave(p[r]) : sum_wave(p[r]);
        if constexpr (GLU) {
            const float sum2 = S == 0 ? sum_half_wave(p[R + r]) : sum_wave(p[R + r]);
            if (u == 0 && row < m.M) store_y(m.y + row, swiglu1(sum, sum2));
        } else {
            if (u == 0 && row < m.M) store_y(m.y + row, sum);
        }
    }
}

// SMAX: the largest shape in the launch (the register budget follows it); R: rows per
// half-wave for the short rows; RL: rows per wave for the long rows (two rows share the
// activation operands each wave reads from LDS and halve the workgroups that convert x).
template <int SMAX, int R, int RL, int XM, int C>
__global__ __launch_bounds__(kSetThreads) void i4_matvec_set(SetArgs<C> a) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int b = blockIdx.x;
    int j = 0;
#pragma unroll
    for (int i = 1; i < C; ++i) j = (i < a.n && b >= a.m[i].blk0) ? i : j;
    SetMat m = a.m[0];
#pragma unroll
    for (int i = 1; i < C; ++i)
        if (i == j) m = a.m[i];
    const int blk = b - m.blk0;
    if (m.shape == 0) {
        set_rows<0, R, XM>(m, blk, lds, a.pro);
    } else if (SMAX <= 1 || m.shape == 1) {
        set_rows<1, RL, XM>(m, blk, lds, a.pro);
    } else if (SMAX <= 2 || m.shape == 2) {
        set_rows<2, RL, XM>(m, blk, lds, a.pro);
    } else if (SMAX <= 3 || m.shape == 3) {
        set_rows<3, RL, XM>(m, blk, lds, a.pro);
    } else if (SMAX <= 4 || m.shape == 4) {
        set_rows<4, RL, XM>(m, blk, lds, a.pro);
    } else {
        set_rows<5, RL, XM>(m, blk, lds, a.pro);
    }
}

// A fused decode layer's gate / up pair as one launch with SwiGLU applied to its outputs: each
// workgroup computes rows of gate (m[0]) and the same rows of up (m[1]) from the shared x with the
// prologue pro, and stores act = silu(gate) * up to m[0].y, which the down projection then reads
// with no prologue. Every row has the bits its set launch gives it, and act the bits the SwiGLU
// prologue forms from the two outputs (the same swiglu1).
template <int S, int XM>
__global__ __launch_bounds__(kSetThreads) void i4_matvec_glu(SetArgs<2> a) {
    extern __shared__ __align__(16) unsigned char lds[];
    set_rows<S, 1, XM, true>(a.m[0], blockIdx.x, lds, a.pro, a.m[1].w);
}

// Shape of a matrix in the set kernel, or -1 when the kernel does not take it:
// G = 64, K % 4 == 0 and x 16-byte aligned (whole 16-byte activation loads), K <= 10240.
int set_shape(const I4Mat &mt, int group_size) {
    if (group_size != 64 || mt.K % 4 != 0 || mt.K > kSetMaxSlots * 64 * 32 ||
        (reinterpret_cast<uintptr_t>(mt.x) & 15) != 0)
        return -1;
    return mt.K <= 1024 ? 0 : (mt.K + 64 * 32 - 1) / (64 * 32);
}

template <int R, int RL, int XM, int C>
void launch_r(int smax, const dim3 &grid, const dim3 &block, size_t lds, hipStream_t stream, const SetArgs<C> &a) {
    switch (smax) {
        case 0: hipLaunchKernelGGL((i4_matvec_set<0, R, 1, XM, C>), grid, block, lds, stream, a); break;
        case 1: hipLaunchKernelGGL((i4_matvec_set<1, R, RL, XM, C>), grid, block, lds, stream, a); break;
        case 2: hipLaunchKernelGGL((i4_matvec_set<2, R, RL, XM, C>), grid, block, lds, stream, a); break;
        case 3: hipLaunchKernelGGL((i4_matvec_set<3, R, RL, XM, C>), grid, block, lds, stream, a); break;
        case 4: hipLaunchKernelGGL((i4_matvec_set<4, R, RL, XM, C>), grid, block, lds, stream, a); break;
        default: hipLaunchKernelGGL((i4_matvec_set<5, R, RL, XM, C>), grid, block, lds, stream, a); break;
    }
}

template <int XM, int C>
void launch_rr(int R, int RL, int smax, const dim3 &grid, const dim3 &block, size_t lds, hipStream_t stream,
               const SetArgs<C> &a) {
    if (R == 2)
        RL == 2 ? launch_r<2, 2, XM, C>(smax, grid, block, lds, stream, a)
                : launch_r<2, 1, XM, C>(smax, grid, block, lds, stream, a);
    else
        RL == 2 ? launch_r<1, 2, XM, C>(smax, grid, block, lds, stream, a)
                : launch_r<1, 1, XM, C>(smax, grid, block, lds, stream, a);
}

// Two long rows per wave when every long-row matrix of the launch has at least this many rows.
// Measured on MI355X (cold, one launch): 9728x2560 7.66 -> 7.38 us, 2560x9728 8.60 -> 7.82,
// 4096x2560 4.72 -> 4.40, 2560x4096 4.81 -> 4.36; the decode layer set, whose only long-row
// matrix (down, 896x4864) then has half the workgroups, 4.90 -> 5.83 (so it keeps one).
constexpr int kLongRowPairMinRows = 2048;
int long_rows_per_wave(const I4Mat *mats, const int *shape, int n) {
    bool any = false;
    for (int i = 0; i < n; ++i) {
        if (shape[i] == 0) continue;
        if (mats[i].M < kLongRowPairMinRows) return 1;
        any = true;
    }
    return any ? 2 : 1;
}

int launch_set(const I4Mat *mats, const int *shape, int n, hipStream_t stream, const SetPrologue *pro = nullptr) {
    SetArgs<kSetMaxMats> a{};
    if (pro) a.pro = *pro;
    int order[kSetMaxMats];
    for (int i = 0; i < n; ++i) order[i] = i;
    // longest rows first: their workgroups are dispatched first
    std::stable_sort(order, order + n, [&](int p, int q) { return shape[p] > shape[q]; });
    // Two short rows per half-wave once they fill more than one 16-row tile per CU: the
    // activations read from LDS and summed once serve both rows.
    long short_rows = 0;
    for (int k = 0; k < n; ++k)
        if (shape[k] == 0) short_rows += mats[k].M;
    const int R = short_rows > 16L * device_cu_count() ? 2 : 1;
    const int RL = long_rows_per_wave(mats, shape, n);
    int blocks = 0, smax = 0, umax = 0;
    for (int k = 0; k < n; ++k) {
        const I4Mat &mt = mats[order[k]];
        const int s = shape[order[k]];
        a.m[k] = SetMat{mt.w, mt.x, mt.y, mt.M, mt.K, blocks, s};
        const int per = s == 0 ? 2 * R * kSetWaves : RL * kSetWaves;  // rows per workgroup
        blocks += (mt.M + per - 1) / per;
        smax = std::max(smax, s);
        umax = std::max(umax, 2 * ((mt.K + 63) / 64));
    }
    for (int k = n; k < kSetMaxMats; ++k) a.m[k] = a.m[n - 1];  // never selected (k >= n)
    a.n = n;
    const size_t lds = static_cast<size_t>(umax) * (4 * kBlockBytes + 8);  // the widest row's operands
    const dim3 grid(blocks), block(kSetThreads);
    const int xm = pro ? pro->kind : 0;
    if (n <= kSetSmallMats) {  // the prologue launches always (launch_i4_matvec_set_pro)
        SetArgs<kSetSmallMats> s3{};
        for (int k = 0; k < kSetSmallMats; ++k) s3.m[k] = a.m[k];
        s3.n = a.n;
        s3.pro = a.pro;
        if (xm == 1)
            launch_rr<1, kSetSmallMats>(R, RL, smax, grid, block, lds, stream, s3);
        else if (xm == 2)
            launch_rr<2, kSetSmallMats>(R, RL, smax, grid, block, lds, stream, s3);
        else
            launch_rr<0, kSetSmallMats>(R, RL, smax, grid, block, lds, stream, s3);
    } else {
        if (xm) return kNotFused;  // prologue launches hold at most kSetSmallMats matrices
        launch_rr<0, kSetMaxMats>(R, RL, smax, grid, block, lds, stream, a);
    }
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

// Single-matrix and fused (pair / qkv) launches go through the set kernel while its grid
// stays within this many workgroups per CU: measured on MI355X against the MFMA kernels,
// 9728x2560 7.6 vs 8.5 us, 2560x9728 8.5 vs 13.0 us, 896x4864 4.0 vs 5.5 us; at
// 151936x896 (4748 workgroups) both take 19 us and at 151936x2560 the DMA ring wins
// (39 vs 69 us).
constexpr int kSetMaxBlocksPerCu = 8;

}  // namespace

namespace {

// Whether launch_i4_matvec_set_fit launches the set kernel for these matrices; their shapes at shape.
bool set_fit_shapes(int n, const I4Mat *mats, int group_size, int *shape) {
    if (n < 1 || n > kSetMaxMats) return false;
    for (int i = 0; i < n; ++i) {
        shape[i] = set_shape(mats[i], group_size);
        if (shape[i] < 0 || mats[i].M < 1) return false;
    }
    const int RL = long_rows_per_wave(mats, shape, n);
    long blocks = 0;
    for (int i = 0; i < n; ++i)
        blocks += shape[i] == 0 ? (mats[i].M + 4 * kSetWaves - 1) / (4 * kSetWaves)
                                : (mats[i].M + RL * kSetWaves - 1) / (RL * kSetWaves);
    return blocks <= static_cast<long>(kSetMaxBlocksPerCu) * device_cu_count();
}

}  // namespace

int launch_i4_matvec_set_fit(int n, const I4Mat *mats, int group_size, hipStream_t stream) {
    int shape[kSetMaxMats];
    if (!set_fit_shapes(n, mats, group_size, shape)) return kNotFused;
    return launch_set(mats, shape, n, stream);
}

bool i4_set_fit_takes(int n, const I4Mat *mats, int group_size) {
    int shape[kSetMaxMats];
    return set_fit_shapes(n, mats, group_size, shape);
}

bool set_kernel_takes(int K, int group_size) {
    const I4Mat probe{nullptr, nullptr, nullptr, 1, K};  // (a null x is 16-byte aligned)
    return K >= 1 && set_shape(probe, group_size) >= 0;
}

int launch_i4_matvec_set_pro(int n, const I4Mat *mats, int group_size, const SetPrologue &pro, hipStream_t stream) {
    if (n < 1 || n > kSetSmallMats || pro.kind < 1 || pro.kind > 2) return kNotFused;
    const auto al = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (!al(pro.x2) || !al(pro.d1) || !al(pro.d2) || !al(pro.nw) || !al(pro.hout) ||
        (pro.kind == 1 && !pro.x2) || (pro.kind == 2 && !pro.nw))
        return kNotFused;
    int shape[kSetMaxMats];
    for (int i = 0; i < n; ++i) {
        shape[i] = set_shape(mats[i], group_size);
        if (shape[i] < 0 || mats[i].M < 1 || mats[i].x != mats[0].x || mats[i].K != mats[0].K) return kNotFused;
    }
    return launch_set(mats, shape, n, stream, &pro);
}

int launch_i4_matvec_glu(const I4Mat &gate, const I4Mat &up, int group_size, const SetPrologue &pro,
                         hipStream_t stream) {
    const auto al = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const int shape = set_shape(gate, group_size);
    if (shape < 0 || set_shape(up, group_size) != shape || gate.M < 1 || up.M != gate.M || up.K != gate.K ||
        up.x != gate.x || !gate.w || !up.w || !gate.x || !gate.y || pro.kind != 2 || !pro.nw || !al(pro.d1) ||
        !al(pro.d2) || !al(pro.nw) || !al(pro.hout))
        return kNotFused;
    SetArgs<2> a{};
    a.m[0] = SetMat{gate.w, gate.x, gate.y, gate.M, gate.K, 0, shape};
    a.m[1] = SetMat{up.w, up.x, nullptr, up.M, up.K, 0, shape};
    a.n = 2;
    a.pro = pro;
    const int per = shape == 0 ? 2 * kSetWaves : kSetWaves;  // rows (pairs) per workgroup
    const dim3 grid((gate.M + per - 1) / per), block(kSetThreads);
    const size_t lds = static_cast<size_t>(2 * ((gate.K + 63) / 64)) * (4 * kBlockBytes + 8);
    switch (shape) {
        case 0: hipLaunchKernelGGL((i4_matvec_glu<0, 2>), grid, block, lds, stream, a); break;
        case 1: hipLaunchKernelGGL((i4_matvec_glu<1, 2>), grid, block, lds, stream, a); break;
        case 2: hipLaunchKernelGGL((i4_matvec_glu<2, 2>), grid, block, lds, stream, a); break;
        case 3: hipLaunchKernelGGL((i4_matvec_glu<3, 2>), grid, block, lds, stream, a); break;
        case 4: hipLaunchKernelGGL((i4_matvec_glu<4, 2>), grid, block, lds, stream, a); break;
        default: hipLaunchKernelGGL((i4_matvec_glu<5, 2>), grid, block, lds, stream, a); break;
    }
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

int launch_i4_matvec_set(int n, const I4Mat *mats, int group_size, hipStream_t stream) {
    if (n < 0 || (n > 0 && !mats)) return kBadShape;
    if (group_size < 2 || (group_size & 1)) return kBadGroup;
    for (int i = 0; i < n; ++i)
        if (mats[i].M < 1 || mats[i].K < 1 || !mats[i].w || !mats[i].x || !mats[i].y) return kBadShape;
    // the matrices the set kernel takes, in launches of up to kSetMaxMats; the others alone
    I4Mat batch[kSetMaxMats];
    int shape[kSetMaxMats], nb = 0;
    for (int i = 0; i < n; ++i) {
        const int s = set_shape(mats[i], group_size);
        if (s < 0) {
            const int st = launch_i4_matvec(mats[i].w, mats[i].x, mats[i].y, mats[i].M, mats[i].K, group_size, stream);
            if (st != kOk) return st;
            continue;
        }
        batch[nb] = mats[i];
        shape[nb++] = s;
        if (nb == kSetMaxMats) {
            const int st = launch_set(batch, shape, nb, stream);
            if (st != kOk) return st;
            nb = 0;
        }
    }
    return nb > 0 ? launch_set(batch, shape, nb, stream) : kOk;
}

}  // namespace tqhip
