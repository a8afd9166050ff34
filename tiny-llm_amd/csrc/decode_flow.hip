// decode_flow.hip -- one decode token's layers as one cooperative launch, phases linked by
// data flow (decode_flow.h has the plan, the tags and why no vector is overwritten early).
//
// The engine's graph runs a token of a fused i4 file as five launches per layer (q/k/v,
// attention, o, gate/up, down): each launch spends a few microseconds in dispatch and in the
// round trip of activations written by the launch before it, whatever its bytes. Here the
// whole layer stack is one launch of one 512-thread workgroup per CU, all resident at once
// (cooperative launch), and each phase waits only for the vectors it reads:
//   * a task (a block of rows, or two attention heads) first issues the weight loads of its
//     rows, then polls the tagged input pairs at device scope (sc1: served where all XCDs
//     meet) until every tag matches, so the weights travel while it waits;
//   * rows are computed with the set kernel's own code (i4_set_core.h) and the attention with
//     the engine's (decode_attn.h), so every value has the bits the graph's launches give it;
//   * gate/up computes the same row of both matrices in one half-wave and stores
//     silu(gate) * up, the down projection's input, directly.
// Every wait is bounded by wall-clock time: a workgroup whose inputs do not arrive in time
// stores an error code and leaves, the others see it and leave too, and the engine runs the
// token again through its graph.

#include "decode_attn.h"
#include "decode_flow.h"
#include "i4_set_core.h"

#include <algorithm>

namespace tqhip {

namespace {

typedef unsigned u4v __attribute__((ext_vector_type(4)));
constexpr int kScopeDevice = 16;  // buffer cache policy sc1: coherent where all XCDs meet

__device__ inline __amdgpu_buffer_rsrc_t pairs_rsrc(const uint2 *v, int n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint2 *>(v), static_cast<short>(0), 8 * n, kBufferFlags);
}

// Elements 4c .. 4c + 3 of a tagged vector (two 16-byte loads at device scope); bad |= 1 unless
// all four carry `tag`. (The empty asm keeps every loaded dword: this compiler has been seen to
// shrink a 16-byte buffer load whose elements were used as floats to its first dword.)
__device__ inline float4 tagged_chunk(__amdgpu_buffer_rsrc_t r, int c, unsigned tag, int &bad) {
    const u4v a = __builtin_amdgcn_raw_buffer_load_b128(r, 32 * c, 0, kScopeDevice);
    const u4v b = __builtin_amdgcn_raw_buffer_load_b128(r, 32 * c + 16, 0, kScopeDevice);
    unsigned a0 = a[0], a1 = a[1], a2 = a[2], a3 = a[3], b0 = b[0], b1 = b[1], b2 = b[2], b3 = b[3];
    asm volatile("" : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(b0), "+v"(b1), "+v"(b2), "+v"(b3));
    bad |= (a1 != tag) | (a3 != tag) | (b1 != tag) | (b3 != tag);
    return make_float4(__uint_as_float(a0), __uint_as_float(a2), __uint_as_float(b0), __uint_as_float(b2));
}

typedef unsigned u2v __attribute__((ext_vector_type(2)));

// One element of a tagged vector (an 8-byte load at device scope).
__device__ inline float tagged_one(__amdgpu_buffer_rsrc_t r, int i, unsigned tag, int &bad) {
    const u2v p = __builtin_amdgcn_raw_buffer_load_b64(r, 8 * i, 0, kScopeDevice);
    unsigned v0 = p[0], v1 = p[1];
    asm volatile("" : "+v"(v0), "+v"(v1));
    bad |= v1 != tag;
    return __uint_as_float(v0);
}

// Element i of a tagged vector: value and tag in one 8-byte store at device scope (written
// through this XCD's L2 to where every XCD reads it).
__device__ inline void put_tagged(__amdgpu_buffer_rsrc_t r, int i, float x, unsigned tag) {
    __builtin_amdgcn_raw_buffer_store_b64(u2v{__float_as_uint(x), tag}, r, 8 * i, 0, kScopeDevice);
}

// A global-address-space view of a pointer (plain loads through it stay global loads).
template <typename T>
__device__ inline const __attribute__((address_space(1))) T *gbl(const T *p) {
    return (const __attribute__((address_space(1))) T *)p;
}

typedef float f4v __attribute__((ext_vector_type(4)));

// 16 bytes at p + 16 c (global load).
__device__ inline float4 ld_f4(const float *p, int c) {
    const f4v v = gbl(reinterpret_cast<const f4v *>(p))[c];
    return make_float4(v[0], v[1], v[2], v[3]);
}

// The poll of one wait: whether the workgroup must look again (some input not there yet).
// Leaves with false and sets `failed` once the wait's time is up or another workgroup has
// reported an error (checked every 16th look).
struct Waiter {
    long long deadline;
    int looks = 0;
    bool failed = false;
    __device__ bool again(int bad, int *err, long long timeout) {
        if (!__syncthreads_or(bad)) return false;
        ++looks;
        if (looks == 1) deadline = static_cast<long long>(wall_clock64()) + timeout;
        const bool late = static_cast<long long>(wall_clock64()) > deadline;
        const bool other = (looks & 15) == 0 &&
                           __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
        if (__syncthreads_or(late || other)) {  // every thread decides alike
            if (late && threadIdx.x == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            failed = true;
            return false;
        }
        return true;
    }
};

// Waits until a sample of the newest input (64 elements spread over its n, polled by wave 0)
// carries `tag`: a workgroup that waits reads 512 bytes per look instead of its whole inputs.
// Workgroups with no task in a phase go on to poll their next one, so at any time most of the
// grid is waiting; reading whole vectors per look (up to 39 KB for the down projection's
// input) made those polls crowd out the producers' traffic. The whole inputs are read and
// checked once the sample is complete. Returns false when the wait failed.
__device__ bool sample_wait(const uint2 *v, int n, unsigned tag, Waiter &wt, int *err, long long timeout) {
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t r = pairs_rsrc(v, n);
    do {
        int bad = 0;
        if (threadIdx.x < 64) tagged_one(r, static_cast<int>((static_cast<long>(lane) * n) >> 6) + (n >> 7), tag, bad);
        if (!wt.again(bad, err, timeout)) break;
    } while (true);
    return !wt.failed;
}

// Inputs of more elements than this are sampled first (sample_wait); shorter ones are polled
// whole, one round trip less once they are there.
constexpr int kFlowSampleAbove = 2048;

// ---- one block of rows ----------------------------------------------------------------------
// The rows of set_rows (i4_set.hip) with their inputs and outputs in tagged vectors. XM: the
// activation prologue (0 none, 2 x = rmsnorm((x + d1) + d2) * nw; the qkv task 0 stores the
// pre-norm x to hout). PAIR: unit r < R is a row of w, unit R + r the same row of w2, and the
// row's output is swiglu(w row, w2 row). x == nullptr: the prologue's x is the embedding row.
struct RowsJob {
    const uint8_t *w, *w2;
    int M, K, blk;
    uint2 *y;
    const uint2 *x, *d1, *d2;
    const float *nw;
    uint2 *hout;
    unsigned tin, tout;  // the tag the inputs must carry, the tag of the outputs
    const uint2 *newest;  // the input written last (sampled before the whole inputs are read), or null
};

template <int S, int R, int XM, bool PAIR>
__device__ __attribute__((always_inline)) bool flow_rows(const RowsJob &j, const FlowArgs &a, unsigned char *lds) {
    constexpr int NX = ((S == 0 ? 256 : 512 * S) + kSetThreads - 1) / kSetThreads;
    constexpr int NR = PAIR ? 2 * R : R;  // weight units per lane and slot
    constexpr int NS = S == 0 ? 1 : S;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int U = 2 * ((j.K + 63) / 64), rb = 18 * U;
    const int C = 8 * U;
    const int Kc = j.K / 4;
    unsigned char *xp = lds;
    float2 *hs = reinterpret_cast<float2 *>(lds + (C / 2) * kBlockBytes);

    // 1. the rows' weights, all of them, before anything waits
    const int half = S == 0 ? lane >> 5 : 0, u = S == 0 ? lane & 31 : lane;
    const int base = S == 0 ? (j.blk * kSetWaves + wave) * 2 * R : (j.blk * kSetWaves + wave) * R;
    const __amdgpu_buffer_rsrc_t wr = rows_rsrc(j.w, j.M, rb, base);
    const __amdgpu_buffer_rsrc_t wr2 = rows_rsrc(PAIR ? j.w2 : j.w, j.M, rb, base);
    unsigned hd[NR * NS];
    v4i cd[NR * NS];
#pragma unroll
    for (int q = 0; q < NR * NS; ++q) {
        const int r = q / NS, sl = q % NS;
        const int rr = PAIR ? r % R : r;
        const int unit = u + 64 * sl;
        const int off = (S == 0 ? 2 * rr + half : rr) * rb + (kI4Header + 32) * (unit >> 1);
        const __amdgpu_buffer_rsrc_t rs = PAIR && r >= R ? wr2 : wr;
        hd[q] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
        cd[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + kI4Header + 16 * (unit & 1), 0, 0);
    }
    float4 pw[XM == 2 ? NX : 1];
    if constexpr (XM == 2) {
#pragma unroll
        for (int i = 0; i < NX; ++i) pw[i] = ld_f4(j.nw, min(t + kSetThreads * i, Kc - 1));
    }
    // the loads above stay ahead of the wait (the scheduler would otherwise move them to their
    // first use, after the inputs have arrived, and add their HBM round trip to the phase)
    __builtin_amdgcn_sched_barrier(0);

    // 2. the inputs: chunk t + kSetThreads i (clamped), polled until every tag is there
    float4 xq[NX], pa[XM == 2 ? NX : 1], pb[XM == 2 ? NX : 1];
    const __amdgpu_buffer_rsrc_t rx = pairs_rsrc(j.x, j.K), r1 = pairs_rsrc(j.d1, j.K), r2 = pairs_rsrc(j.d2, j.K);
    const int token = a.io[1];
    Waiter wt{};
    if (j.newest && j.K > kFlowSampleAbove && !sample_wait(j.newest, j.K, j.tin, wt, a.io + 4, a.timeout))
        return false;
    do {
        int bad = 0;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int c = min(t + kSetThreads * i, Kc - 1);
            if (j.x) {
                xq[i] = tagged_chunk(rx, c, j.tin, bad);
            } else if (a.embed_i4) {  // i4_embed_rows_kernel's decode: (q - zero) * scale
                const int gb = kI4Header + a.embed_gs / 2, groups = (j.K + a.embed_gs - 1) / a.embed_gs;
                const auto row = gbl(a.embed_i4 + static_cast<size_t>(token) * groups * gb);
                float e[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int k = 4 * c + q, g = k / a.embed_gs, ii = k - g * a.embed_gs;
                    const auto gp = row + static_cast<size_t>(g) * gb;
                    const float scale = half_bits(gp[0] | (gp[1] << 8));
                    const float zero = half_bits(gp[2] | (gp[3] << 8));
                    const uint8_t byte = gp[kI4Header + (ii >> 1)];
                    const int qv = (ii & 1) ? (byte >> 4) : (byte & 0x0F);
                    e[q] = (static_cast<float>(qv) - zero) * scale;
                }
                xq[i] = make_float4(e[0], e[1], e[2], e[3]);
            } else {
                xq[i] = ld_f4(a.embed_f32 + static_cast<size_t>(token) * j.K, c);
            }
            if constexpr (XM == 2) {
                pa[i] = j.d1 ? tagged_chunk(r1, c, j.tin, bad) : make_float4(0.f, 0.f, 0.f, 0.f);
                pb[i] = j.d2 ? tagged_chunk(r2, c, j.tin, bad) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        if (!wt.again(bad, a.io + 4, a.timeout)) break;
    } while (true);
    if (wt.failed) return false;

    // 3. the prologue (the set kernel's arithmetic) and the activations to integer operands
    if constexpr (XM == 2) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            if (j.d1) xq[i] = add4(xq[i], pa[i]);
            if (j.d2) xq[i] = add4(xq[i], pb[i]);
            if (t + kSetThreads * i < Kc) ss += sq4(xq[i]);
        }
        if (j.hout) {
            const __amdgpu_buffer_rsrc_t rh = pairs_rsrc(j.hout, j.K);
#pragma unroll
            for (int i = 0; i < NX; ++i) {
                const int c = t + kSetThreads * i;
                if (c < Kc) {
                    put_tagged(rh, 4 * c, xq[i].x, j.tout);
                    put_tagged(rh, 4 * c + 1, xq[i].y, j.tout);
                    put_tagged(rh, 4 * c + 2, xq[i].z, j.tout);
                    put_tagged(rh, 4 * c + 3, xq[i].w, j.tout);
                }
            }
        }
        ss = set_block_sum(ss);
        const float scale = rms_scale(ss, j.K, a.eps);
#pragma unroll
        for (int i = 0; i < NX; ++i) xq[i] = rms_apply(xq[i], scale, pw[i]);
    }
#pragma unroll
    for (int i = 0; i < NX; ++i) stage_x(xq[i], t + kSetThreads * i, Kc, C, xp, hs);
    __syncthreads();

    // 4. the row sums (set_rows' order), then the tagged outputs
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
    const __amdgpu_buffer_rsrc_t ry = pairs_rsrc(j.y, j.M);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = base + (S == 0 ? 2 * r + half : r);
        const float sum = S == 0 ? sum_half_wave(p[r]) : sum_wave(p[r]);
        if constexpr (PAIR) {
            const float sum2 = S == 0 ? sum_half_wave(p[R + r]) : sum_wave(p[R + r]);
            if (u == 0 && row < j.M) put_tagged(ry, row, swiglu1(sum, sum2), j.tout);
        } else {
            if (u == 0 && row < j.M) put_tagged(ry, row, sum, j.tout);
        }
    }
    __syncthreads();  // the LDS operands are rewritten by the workgroup's next task
    return true;
}

// Shapes the flow step serves (the engine checks them): rows of H and q_dim elements up to
// kFlowMaxShapeHq, rows of I elements up to the set kernel's 5 slots.
constexpr int kFlowMaxShapeHq = 2;  // H, q_dim <= 4096

template <int SMAX, int R, int XM, bool PAIR>
__device__ __attribute__((always_inline)) bool flow_rows_s(int shape, const RowsJob &j, const FlowArgs &a,
                                                           unsigned char *lds) {
    switch (shape) {
        case 0: return flow_rows<0, R, XM, PAIR>(j, a, lds);
        case 1: return flow_rows<1, R, XM, PAIR>(j, a, lds);
        case 2: return flow_rows<2, R, XM, PAIR>(j, a, lds);
        case 3: if constexpr (SMAX >= 3) return flow_rows<3, R, XM, PAIR>(j, a, lds);
                return false;
        case 4: if constexpr (SMAX >= 4) return flow_rows<4, R, XM, PAIR>(j, a, lds);
                return false;
        default: if constexpr (SMAX >= 5) return flow_rows<5, R, XM, PAIR>(j, a, lds);
                 return false;
    }
}

// Rows of one workgroup task for a shape: 16 R per task (S = 0) or 8 R (S > 0).
__host__ __device__ inline int flow_rows_per_task(int shape, int r) { return shape == 0 ? 16 * r : 8 * r; }

// ---- attention: two heads per workgroup ------------------------------------------------------
template <int HD>
__device__ __attribute__((always_inline)) bool flow_attention(int task, int layer, const FlowLayerPtrs &L,
                                                              const FlowArgs &a, unsigned char *lds) {
    const int sub = threadIdx.x >> 8, t = threadIdx.x & 255;
    AttnShared &S = reinterpret_cast<AttnShared *>(lds)[sub];
    int head = 2 * task + sub;
    const bool real = head < a.n_heads;
    if (!real) head = a.n_heads - 1;  // a duplicate run that keeps the workgroup's barriers in step
    const int kvh = head / a.heads_per_kv;
    const unsigned tag = flow_tag(static_cast<unsigned>(a.io[3]), a.n_layers, layer);
    const __amdgpu_buffer_rsrc_t rq = pairs_rsrc(a.vec[kVecQ], a.q_dim), rk = pairs_rsrc(a.vec[kVecK], a.kv_dim),
                                 rv = pairs_rsrc(a.vec[kVecV], a.kv_dim);
    const float *qb = L.qb, *kb = L.kb, *vb = L.vb;
    int *err = a.io + 4;
    const long long timeout = a.timeout;
    // q / k / v polled once the cache loads and the RoPE angles are under way; then the biases,
    // as attention_step adds them
    const auto fetch = [&](float &qv, float &kv, float &vv) {
        Waiter wt{};
        do {
            int bad = 0;
            if (t < HD) {
                qv = tagged_one(rq, head * HD + t, tag, bad);
                kv = tagged_one(rk, kvh * HD + t, tag, bad);
                vv = tagged_one(rv, kvh * HD + t, tag, bad);
            }
            if (!wt.again(bad, err, timeout)) break;
        } while (true);
        if (wt.failed) return false;
        if (t < HD) {
            const int qi = head * HD + t, ki = kvh * HD + t;
            qv = qb ? qv + attn_ld(qb + qi) : qv;
            kv = kb ? kv + attn_ld(kb + ki) : kv;
            vv = vb ? vv + attn_ld(vb + ki) : vv;
        }
        return true;
    };
    const __amdgpu_buffer_rsrc_t ro = pairs_rsrc(a.vec[kVecAttn], a.q_dim);
    // (the key row is prefetched into registers only at head_dim 64: at 128 and 256 its 32 or 64
    // float4 registers made this kernel spill)
    if (!attention_head<HD, HD <= 64>(S, t, head, a.heads_per_kv, fetch, L.qn, L.kn, L.kc, L.vc, a.io[0], a.max_seq,
                                      a.theta, a.eps, a.attn_scale, real,
                                      [&](int i, float o) { put_tagged(ro, i, o, tag); }))
        return false;
    __syncthreads();  // the LDS is the next task's
    return true;
}

// ---- the final norm ---------------------------------------------------------------------------
// add_rmsnorm<1024, PER> (decode_engine.hip) with 512 threads: thread r plays its threads r and
// r + 512, whose waves are this thread's wave w and w + 8, so the 64-lane butterflies and the
// 16 wave sums in wave order are the same additions.
template <int PER>
__device__ __attribute__((always_inline)) bool flow_final_norm(const FlowArgs &a, unsigned char *lds) {
#pragma clang fp contract(off)
    const int layer = a.n_layers - 1, n = a.H;
    const unsigned tag = flow_tag(static_cast<unsigned>(a.io[3]), a.n_layers, layer);
    const __amdgpu_buffer_rsrc_t hv = pairs_rsrc(a.vec[flow_buffer(kVecH0, layer)], n),
                                 ov = pairs_rsrc(a.vec[kVecO], n), fv = pairs_rsrc(a.vec[kVecFfn], n);
    float h[2][PER];
    Waiter wt{};
    if (!sample_wait(a.vec[kVecFfn], n, tag, wt, a.io + 4, a.timeout)) return false;
    do {
        int bad = 0;
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                const int i = threadIdx.x + 512 * s + 1024 * q;
                if (i < n) {
                    const float f = tagged_one(fv, i, tag, bad), o = tagged_one(ov, i, tag, bad);
                    h[s][q] = (tagged_one(hv, i, tag, bad) + o) + f;
                } else {
                    h[s][q] = 0.0f;
                }
            }
        if (!wt.again(bad, a.io + 4, a.timeout)) break;
    } while (true);
    if (wt.failed) return false;
    double *red = reinterpret_cast<double *>(lds);
    double ss[2] = {0.0, 0.0};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int q = 0; q < PER; ++q) ss[s] += static_cast<double>(h[s][q]) * static_cast<double>(h[s][q]);
        ss[s] = xor_sum_wave(ss[s]);
        if ((threadIdx.x & 63) == 0) red[(threadIdx.x >> 6) + 8 * s] = ss[s];
    }
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < 16; ++w) tot += red[w];
    const float mean_sq = static_cast<float>(tot / n);
    const float scale = 1.0f / sqrtf(mean_sq + a.eps);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = threadIdx.x + 512 * s + 1024 * q;
            if (i < n) a.normed[i] = (h[s][q] * scale) * a.final_norm[i];
        }
    return true;
}

// ---- the kernel -------------------------------------------------------------------------------
// The description lives in HBM (the engine uploads it once), not in the kernel argument: held
// in the argument, its fields stayed live in registers across the whole layer loop and the
// kernel spilled about a hundred VGPRs; read through a pointer, with a compiler barrier before
// each phase, each phase reloads the fields it uses (scalar loads, cache hits).
template <int HD>
__global__ __launch_bounds__(kSetThreads) void decode_flow(const FlowArgs *args) {
    extern __shared__ __align__(16) unsigned char lds[];
    const FlowArgs &a = *args;
    const int L = a.n_layers, wg = blockIdx.x;
    // The layer records, copied once into LDS (after the phases' scratch): a phase then starts
    // from an LDS read instead of a dependent HBM load of its weight pointers.
    FlowLayerPtrs *layers = reinterpret_cast<FlowLayerPtrs *>(lds + a.lds_table);
    {
        const unsigned *src = reinterpret_cast<const unsigned *>(a.layers);
        unsigned *dst = reinterpret_cast<unsigned *>(layers);
        const int words = L * static_cast<int>(sizeof(FlowLayerPtrs) / 4);
        for (int i = threadIdx.x; i < words; i += kSetThreads) dst[i] = src[i];
        __syncthreads();
    }
    const unsigned run = static_cast<unsigned>(a.io[3]);
    const int rq = flow_rows_per_task(a.shape_h, 1);
    const int tq = (a.q_dim + rq - 1) / rq, tk = (a.kv_dim + rq - 1) / rq;
    for (int l = 0; l < L; ++l) {
        asm volatile("" ::: "memory");
        const FlowLayerPtrs &Ly = layers[l];
        const unsigned tin = flow_tag(run, L, l - 1), tout = flow_tag(run, L, l);
        // q / k / v: the three matrices' blocks one after the other
        for (int i = 0;; ++i) {
            const int t = flow_task(a.plan, kFlowQkv, wg, i);
            if (t < 0) break;
            const int m = t < tq ? 0 : t < tq + tk ? 1 : 2;
            const int blk = m == 0 ? t : m == 1 ? t - tq : t - tq - tk;
            RowsJob j{};
            j.w = m == 0 ? Ly.q : m == 1 ? Ly.k : Ly.v;
            j.M = m == 0 ? a.q_dim : a.kv_dim;
            j.K = a.H;
            j.blk = blk;
            j.y = a.vec[m == 0 ? kVecQ : m == 1 ? kVecK : kVecV];
            if (l > 0) {
                j.x = a.vec[flow_buffer(kVecH0, l - 1)];
                j.d1 = a.vec[kVecO];
                j.d2 = a.vec[kVecFfn];
                j.newest = j.d2;
            }
            j.nw = Ly.in_ln;
            j.hout = t == 0 ? a.vec[flow_buffer(kVecH0, l)] : nullptr;
            j.tin = tin;
            j.tout = tout;
            if (!flow_rows_s<kFlowMaxShapeHq, 1, 2, false>(a.shape_h, j, a, lds)) return;
        }
        asm volatile("" ::: "memory");
        for (int i = 0;; ++i) {
            const int t = flow_task(a.plan, kFlowAttn, wg, i);
            if (t < 0) break;
            if (!flow_attention<HD>(t, l, Ly, a, lds)) return;
        }
        asm volatile("" ::: "memory");
        for (int i = 0;; ++i) {
            const int t = flow_task(a.plan, kFlowO, wg, i);
            if (t < 0) break;
            RowsJob j{};
            j.w = Ly.o;
            j.M = a.H;
            j.K = a.q_dim;
            j.blk = t;
            j.y = a.vec[kVecO];
            j.x = a.vec[kVecAttn];
            j.newest = j.x;
            j.tin = tout;
            j.tout = tout;
            if (!flow_rows_s<kFlowMaxShapeHq, 2, 0, false>(a.shape_q, j, a, lds)) return;
        }
        asm volatile("" ::: "memory");
        for (int i = 0;; ++i) {
            const int t = flow_task(a.plan, kFlowGateUp, wg, i);
            if (t < 0) break;
            RowsJob j{};
            j.w = Ly.gate;
            j.w2 = Ly.up;
            j.M = a.I;
            j.K = a.H;
            j.blk = t;
            j.y = a.vec[kVecAct];
            j.x = a.vec[flow_buffer(kVecH0, l)];
            j.d1 = a.vec[kVecO];
            j.newest = j.d1;
            j.nw = Ly.post_ln;
            j.tin = tout;
            j.tout = tout;
            // two row pairs per half-wave for rows of up to 1024 elements, one per wave above
            const bool ok = a.shape_h == 0 ? flow_rows<0, 2, 2, true>(j, a, lds)
                                           : flow_rows_s<kFlowMaxShapeHq, 1, 2, true>(a.shape_h, j, a, lds);
            if (!ok) return;
        }
        asm volatile("" ::: "memory");
        for (int i = 0;; ++i) {
            const int t = flow_task(a.plan, kFlowDown, wg, i);
            if (t < 0) break;
            RowsJob j{};
            j.w = Ly.down;
            j.M = a.H;
            j.K = a.I;
            j.blk = t;
            j.y = a.vec[kVecFfn];
            j.x = a.vec[kVecAct];
            j.newest = j.x;
            j.tin = tout;
            j.tout = tout;
            if (!flow_rows_s<5, 2, 0, false>(a.shape_i, j, a, lds)) return;
        }
    }
    asm volatile("" ::: "memory");
    if (flow_task(a.plan, kFlowNorm, wg, 0) == 0) {
        if (a.H <= 1024)
            flow_final_norm<1>(a, lds);
        else if (a.H <= 4096)
            flow_final_norm<4>(a, lds);
        else
            flow_final_norm<16>(a, lds);
    }
}

}  // namespace

// Whether the flow step serves rows of these widths (H and q_dim up to 4096).
bool flow_shapes_ok(int H, int q_dim) {
    const auto shape = [](int K) { return K <= 1024 ? 0 : (K + 2047) / 2048; };
    return shape(H) <= kFlowMaxShapeHq && shape(q_dim) <= kFlowMaxShapeHq;
}

// The LDS of the phases' scratch: the widest row's operands, two attention heads, the final
// norm's sums. The layer records follow at that offset (flow_lds_table + layers * 128 bytes).
size_t flow_lds_table(int H, int q_dim, int I) {
    const int kmax = H > q_dim ? (H > I ? H : I) : (q_dim > I ? q_dim : I);
    const size_t rows = static_cast<size_t>(2 * ((kmax + 63) / 64)) * (4 * kBlockBytes + 8);
    const size_t attn = 2 * sizeof(AttnShared);
    return (std::max(rows, attn) + 255) / 256 * 256;
}

int flow_tasks(int kind, int H, int q_dim, int kv_dim, int I, int n_heads, int shape_h, int shape_q, int shape_i,
               int rd) {
    switch (kind) {
        case kFlowQkv: {
            const int r = flow_rows_per_task(shape_h, 1);
            return (q_dim + r - 1) / r + 2 * ((kv_dim + r - 1) / r);
        }
        case kFlowAttn:
            return (n_heads + 1) / 2;
        case kFlowO:
            return (H + flow_rows_per_task(shape_q, 2) - 1) / flow_rows_per_task(shape_q, 2);
        case kFlowGateUp:
            return (I + flow_rows_per_task(shape_h, rd) - 1) / flow_rows_per_task(shape_h, rd);
        case kFlowDown:
            return (H + flow_rows_per_task(shape_i, 2) - 1) / flow_rows_per_task(shape_i, 2);
        default:
            return 1;
    }
}

const void *flow_kernel(int head_dim) {
    switch (head_dim) {
        case 64: return reinterpret_cast<const void *>(decode_flow<64>);
        case 128: return reinterpret_cast<const void *>(decode_flow<128>);
        case 256: return reinterpret_cast<const void *>(decode_flow<256>);
        default: return nullptr;
    }
}

}  // namespace tqhip
