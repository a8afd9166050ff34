// decode_attn.h -- one query head of a decode step's attention, shared by the engine's
// attention launch (decode_engine.hip, one head per 256-thread workgroup) and the data-flow
// decode kernel (decode_flow.hip, two heads per 512-thread workgroup), so both give the
// same bits.
//
// A head finishes its q head and the k / v head of its group from the raw projections
// (biases, optional per-head RMSNorm for q and k, RoPE as rope_ref, kernels/rope/rope_ref.cpp:
// pairs (i, i + half), inv_freq = theta^(-2i/d), angle = pos * inv_freq), writes k and v at
// `pos` into the cache (the group's first head only), then attends over positions 0..pos
// (attention_decode_ref, kernels/attention/attention_decode_ref.cpp: scores q.k * scale,
// softmax, sum of p * v). Every head of a group computes the new k / v itself and uses its
// own copy at position pos, so no head reads a cache row another workgroup is writing.
//
// Latency is the cost here (14 heads at Qwen2.5-0.5B), so the memory round trips are
// overlapped: thread t's key row for position t (head_dim <= 128) and the first eight value
// rows of its slice are issued at entry, and the RoPE angles are computed while they are in
// flight. Thread j scores position j of a chunk of up to 4096 positions; the softmax over a
// chunk is max / exp / sum, and across chunks the running max rescales the partial sums.
// Thread t accumulates dimension t % hd over every (256 / hd)-th position, in position order.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

#include "lane_sum.h"

namespace tqhip {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnChunk = 4096;  // scores of one chunk of positions in LDS
constexpr int kAttnMaxHd = 256;

// One head's LDS.
struct AttnShared {
    __attribute__((aligned(16))) float qs[kAttnMaxHd];
    __attribute__((aligned(16))) float ks[kAttnMaxHd];
    float vs[kAttnMaxHd];
    float sc[kAttnChunk];
    float part[kAttnThreads];
    float norm_scale[2];
    double dred[kAttnThreads / 64];
    float fred[kAttnThreads / 64];
};

// Sum / max over the head's 256 threads (t = the thread's index within them) in a fixed
// order: a 64-lane butterfly, then the four wave results in wave order. Every thread of the
// workgroup must call them (they hold a workgroup barrier). red is written before the barrier
// and read after it; the caller passes an array no thread writes again before a later barrier.
__device__ inline double attn_sum(double v, double *red, int t) {
    v = xor_sum_wave(v);
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    double r = 0.0;
    for (int w = 0; w < kAttnThreads / 64; ++w) r += red[w];
    return r;
}

__device__ inline float attn_max(float v, float *red, int t) {
    v = xor_max_wave(v);
    if ((t & 63) == 0) red[t >> 6] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < kAttnThreads / 64; ++w) r = fmaxf(r, red[w]);
    return r;
}

// Global-address-space loads and stores of the KV cache (plain pointers would be flat
// accesses, which also count against the LDS wait counter).
typedef float attn_f4v __attribute__((ext_vector_type(4)));
__device__ inline float4 attn_ld4(const float *p) {
    const attn_f4v v = *(const __attribute__((address_space(1))) attn_f4v *)p;
    return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ inline float attn_ld(const float *p) { return *(const __attribute__((address_space(1))) float *)p; }
__device__ inline void attn_st(float *p, float v) { *(__attribute__((address_space(1))) float *)p = v; }

// 1 / rms of one head in LDS (rmsnorm_ref on a head slice), summed by one wave.
__device__ inline float head_rms_scale(const float *x, int hd, float eps) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    double ss = 0.0;
    for (int i = lane; i < hd; i += 64) ss += static_cast<double>(x[i]) * static_cast<double>(x[i]);
    ss = xor_sum_wave(ss);
    return 1.0f / sqrtf(static_cast<float>(ss / hd) + eps);
}

// One head, run by 256 threads (t = 0..255 among them; every thread of the workgroup enters,
// with the same pos, so the barriers match). fetch(qv, kv, vv) gives thread t < HD its element
// of the head's q and of its group's k and v, biases added; it is called by every thread after
// the cache loads and the RoPE angles, which do not depend on them, are under way, and returns
// false to abandon the head (then so does attention_head). `writes`: the head stores its k / v
// (when it is its group's first head) and its output; false for a duplicate run that only
// keeps a workgroup's barriers in step. out(i, value) stores output element i of the
// attention vector (head * HD + d). PREFETCH_KEY: thread t loads its key row at entry into
// registers (HD / 4 of them); the dot products are the same either way.
template <int HD, bool PREFETCH_KEY = (HD <= 128), int NV = 8, typename Fetch, typename Out>
__device__ inline bool attention_head(AttnShared &S, int t, int head, int heads_per_kv, Fetch fetch, const float *qn,
                                      const float *kn, float *kcache, float *vcache, int pos, int max_seq, float theta,
                                      float eps, float scale, bool writes, Out out) {
#pragma clang fp contract(off)
    constexpr int hd = HD, half = HD / 2, slices = kAttnThreads / HD;
    constexpr bool kPrefetchKey = PREFETCH_KEY;
    const int kvh = head / heads_per_kv;
    const int seq = pos + 1;
    const int d = t % hd, slice = t / hd;
    const float *kh = kcache + static_cast<size_t>(kvh) * max_seq * hd;
    const float *vh = vcache + static_cast<size_t>(kvh) * max_seq * hd;

    // The prefetch loads are unconditional (a thread without a row to prefetch reads row 0, which
    // every step before this one has written, and never uses it): loads under branches leave the
    // compiler unable to count them, and its waits for q / k / v then wait for every load.
    // The first wave's key rows (positions 0..63) and the first eight value rows of each slice are
    // requested without waiting for the position, whose load is a round trip of its own: rows past
    // it (but below max_seq) are read and never used. The other waves' key rows go out after q / k /
    // v, once the position is known, so that a long cache is not read beyond the sequence.
    float4 kreg[kPrefetchKey ? HD / 4 : 1];
    const bool key_pre = kPrefetchKey && t < seq && t != pos && t < kAttnChunk;
    if constexpr (kPrefetchKey) {
        if (t < 64) {  // (wave-uniform) the other waves' rows go out once q / k / v are in, below
            const float *kr = kh + static_cast<size_t>(t < max_seq ? t : 0) * hd;
#pragma unroll
            for (int i = 0; i < HD / 4; ++i) kreg[i] = attn_ld4(kr + 4 * i);
        }
    }
    static_assert(NV == 8 || NV == 16, "value rows loaded ahead: 8 at entry, 8 more after q / k / v");
    float vreg[NV];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int p = slice + u * slices;
        vreg[u] = attn_ld(vh + static_cast<size_t>(p < max_seq ? p : 0) * hd + d);
    }
    // the q / k norm weights of element t (files without them: the key cache instead, unused)
    const float qnw = attn_ld((qn ? qn : kh) + (t < hd ? t : 0)), knw = attn_ld((kn ? kn : kh) + (t < hd ? t : 0));
    float c = 0.0f, s = 0.0f;
    // (HD 64: lanes half..63 take the angle of element t - half too, for the rotation in registers)
    if (t < half || (HD == 64 && t < 64)) {
        const int i = t < half ? t : t - half;
        const float inv_freq = powf(theta, -static_cast<float>(2 * i) / static_cast<float>(hd));
        const float angle = static_cast<float>(pos) * inv_freq;
        c = cosf(angle);
        s = sinf(angle);
    }
    float qv = 0.0f, kv = 0.0f, vv = 0.0f;
    __builtin_amdgcn_sched_barrier(0);  // the cache loads above stay ahead of fetch's waits
    if (!fetch(qv, kv, vv)) return false;
    if constexpr (kPrefetchKey) {
        if (t >= 64) {  // (wave-uniform) rows 64.. of the sequence, now that the position is known
            const float *kr = kh + static_cast<size_t>(key_pre ? t : 0) * hd;
#pragma unroll
            for (int i = 0; i < HD / 4; ++i) kreg[i] = attn_ld4(kr + 4 * i);
        }
    }
#pragma unroll
    for (int u = 8; u < NV; ++u) {  // the next value rows, in flight through the scores and the softmax
        const int p = slice + u * slices;
        vreg[u] = attn_ld(vh + static_cast<size_t>(p < max_seq ? p : 0) * hd + d);
    }
    if constexpr (HD == 64) {
        // The head is wave 0's, element t in lane t: the q / k norms (rmsnorm_ref on the head,
        // the sum of squares as head_rms_scale forms it) and the rotation (element t with
        // element t ^ 32, through a row swap) in registers, then one barrier. The same
        // operations on the same values as the LDS form below.
        if (t < 64) {
            if (qn) {
                const double sq = xor_sum_wave(0.0 + static_cast<double>(qv) * static_cast<double>(qv));
                const double sk = xor_sum_wave(0.0 + static_cast<double>(kv) * static_cast<double>(kv));
                const float rq = 1.0f / sqrtf(static_cast<float>(sq / hd) + eps);
                const float rk = 1.0f / sqrtf(static_cast<float>(sk / hd) + eps);
                qv = (qv * rq) * qnw;
                kv = (kv * rk) * knw;
            }
            const float qp = lane_xor<32>(qv, t), kp = lane_xor<32>(kv, t);
            if (t < half) {
                qv = qv * c - qp * s;
                kv = kv * c - kp * s;
            } else {
                qv = qv * c + qp * s;
                kv = kv * c + kp * s;
            }
            S.qs[t] = qv;
            S.ks[t] = kv;
            S.vs[t] = vv;
        }
        __syncthreads();
    } else {
    if (t < hd) {
        S.qs[t] = qv;
        S.ks[t] = kv;
        S.vs[t] = vv;
    }
    __syncthreads();
    if (qn) {
        const int wave = t >> 6;
        if (wave < 2) {
            const float s0 = head_rms_scale(wave == 0 ? S.qs : S.ks, hd, eps);
            if ((t & 63) == 0) S.norm_scale[wave] = s0;
        }
        __syncthreads();
        if (t < hd) {
            S.qs[t] = (S.qs[t] * S.norm_scale[0]) * qnw;
            S.ks[t] = (S.ks[t] * S.norm_scale[1]) * knw;
        }
        __syncthreads();
    }
    if (t < half) {
        float *xs[2] = {S.qs, S.ks};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float *x = xs[h];
            const float x0 = x[t], x1 = x[t + half];
            const float r0 = x0 * c - x1 * s;
            const float r1 = x1 * c + x0 * s;
            x[t] = r0;
            x[t + half] = r1;
        }
    }
    __syncthreads();
    }
    if (writes && head % heads_per_kv == 0 && t < hd) {
        attn_st(kcache + (static_cast<size_t>(kvh) * max_seq + pos) * hd + t, S.ks[t]);
        attn_st(vcache + (static_cast<size_t>(kvh) * max_seq + pos) * hd + t, S.vs[t]);
    }

    float m = -INFINITY, l = 0.0f, acc = 0.0f;
    const float4 *q4 = reinterpret_cast<const float4 *>(S.qs);
    for (int c0 = 0; c0 < seq; c0 += kAttnChunk) {
        const int len = min(kAttnChunk, seq - c0);
        for (int j = t; j < len; j += kAttnThreads) {
            const int p = c0 + j;
            float dot = 0.0f;
            if (kPrefetchKey && p == t && key_pre) {
#pragma unroll
                for (int i = 0; i < HD / 4; ++i) {
                    const float4 a = q4[i], b = kreg[kPrefetchKey ? i : 0];
                    dot += a.x * b.x;
                    dot += a.y * b.y;
                    dot += a.z * b.z;
                    dot += a.w * b.w;
                }
            } else if (p == pos) {  // this step's own key, in LDS
                const float4 *kr = reinterpret_cast<const float4 *>(S.ks);
#pragma unroll
                for (int i = 0; i < HD / 4; ++i) {
                    const float4 a = q4[i], b = kr[i];
                    dot += a.x * b.x;
                    dot += a.y * b.y;
                    dot += a.z * b.z;
                    dot += a.w * b.w;
                }
            } else {
                const float *kr = kh + static_cast<size_t>(p) * hd;
#pragma unroll
                for (int i = 0; i < HD / 4; ++i) {
                    const float4 a = q4[i], b = attn_ld4(kr + 4 * i);
                    dot += a.x * b.x;
                    dot += a.y * b.y;
                    dot += a.z * b.z;
                    dot += a.w * b.w;
                }
            }
            S.sc[j] = dot * scale;
        }
        // Each thread reduces only the scores it wrote; the value sums read the others' after
        // attn_sum's barrier. fred and dred are each written once per chunk, and the chunk ends
        // with a barrier.
        float cmax = -INFINITY;
        for (int j = t; j < len; j += kAttnThreads) cmax = fmaxf(cmax, S.sc[j]);
        cmax = attn_max(cmax, S.fred, t);
        const float m_new = fmaxf(m, cmax);
        double csum = 0.0;
        for (int j = t; j < len; j += kAttnThreads) {
            const float p = expf(S.sc[j] - m_new);
            S.sc[j] = p;
            csum += p;
        }
        csum = attn_sum(csum, S.dred, t);
        const float rescale = expf(m - m_new);
        l = l * rescale + static_cast<float>(csum);
        acc = acc * rescale;
        // The slice's positions j = slice, slice + slices, ... < len, added to acc in position
        // order (acc + p * v each). Branch-free, eight positions at a time: their LDS reads and
        // cache loads all go out before the first add (with a branch per position each LDS read
        // was waited for before the next was issued), reads past the chunk are clamped to its
        // last score, and the terms of positions past it are dropped by a select.
        const float vpos = S.vs[d];  // position pos: this step's own value row, from LDS
        int j = slice;
        if (c0 == 0) {  // the first NV positions of the slice, loaded ahead
            float scv[NV];
#pragma unroll
            for (int u = 0; u < NV; ++u) scv[u] = S.sc[min(slice + u * slices, len - 1)];
#pragma unroll
            for (int u = 0; u < NV; ++u) {
                const int jj = slice + u * slices;
                const float term = scv[u] * (jj == pos ? vpos : vreg[u]);
                acc = jj < len ? acc + term : acc;
            }
            j = slice + NV * slices;
        }
        for (; j < len; j += 8 * slices) {
            float vb8[8], sc8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int jj = j + u * slices, p = c0 + jj;
                // rows past the chunk and row pos (being written by this step) are not read: row 0
                // instead, whose term is dropped (pos > 0 whenever a position past the first
                // NV exists)
                const bool use = jj < len && p != pos;
                vb8[u] = attn_ld(vh + static_cast<size_t>(use ? p : 0) * hd + d);
                sc8[u] = S.sc[min(jj, len - 1)];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int jj = j + u * slices;
                const float term = sc8[u] * (c0 + jj == pos ? vpos : vb8[u]);
                acc = jj < len ? acc + term : acc;
            }
        }
        m = m_new;
        __syncthreads();
    }
    S.part[t] = acc;
    __syncthreads();
    if (slice == 0) {
        float o = S.part[d];
        for (int s2 = 1; s2 < slices; ++s2) o += S.part[s2 * hd + d];
        if (writes) out(head * hd + d, o * (1.0f / l));
    }
    return true;
}

}  // namespace
}  // namespace tqhip
