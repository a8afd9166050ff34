// decode_engine.hip -- device-resident decode engine for dense i4 / VQ2 Qwen2 / Qwen3 models.
//
// The "gpu_decode" boundary of the reference (kernels/dispatch.h:337-378: create /
// step / reset / destroy / logits on an opaque engine). The reference's CUDA engine
// (kernels/cuda/gpu_engine.cu) serves f32 / f16 files; this one serves the i4
// HQQ and VQ2 files whose projections the library's matvec kernels run. Weights stay
// where tqhip_model_upload put them (one HBM allocation per model), activations,
// the fp32 KV cache and the argmax live in one more allocation, and a step is
// one HIP-graph replay on the engine's stream: only the token id and the next
// token cross PCIe.
//
// One step follows QwenModel::forward_token (runtime/qwen_forward_token.cpp:83-700)
// for a Qwen2.x layer: embedding row, RMSNorm, fused q/k/v matvec, biases,
// optional per-head q/k RMSNorm (Qwen3 dense), RoPE, KV write, attention over
// positions 0..pos, o matvec, residual, RMSNorm, fused gate/up matvec, SwiGLU,
// down matvec, residual, final RMSNorm, lm_head matvec, argmax. The small
// kernels below fuse the elementwise work between the matvecs: residual add
// with the following RMSNorm, and biases, q/k norm, RoPE, the KV write and the
// attention in one launch.

#include "../../include/tqhip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

#include "decode_attn.h"
#include "decode_flow.h"
#include "lane_sum.h"
#include "tq_common.h"

// The elementwise steps below round every product and sum separately, as the
// reference's scalar C++ does; contraction into FMAs would change low bits.
#pragma clang fp contract(off)

namespace tqhip {

namespace {

constexpr int kNormThreads = 1024;
constexpr int kMaxHidden = 16 * kNormThreads;  // values per thread kept in registers
constexpr int kArgmaxThreads = 256, kArgmaxPerThread = 8;
constexpr int kArgmaxPerBlock = kArgmaxThreads * kArgmaxPerThread;
constexpr int kArgmaxParts = 4096;  // argmax partial slots: blocks of argmax_partial or lm_head workgroups

// Fixed-order block sum: a 64-lane butterfly, then every thread adds the wave
// totals in wave order, so all threads hold the same value.
template <int NT>
__device__ double block_sum(double v, double *red) {
    v = xor_sum_wave(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < NT / 64; ++w) t += red[w];
    __syncthreads();
    return t;
}

// hidden += delta, then += delta2 (each when given); out = rmsnorm(hidden) * w. rmsnorm_ref
// (kernels/rmsnorm/rmsnorm_ref.cpp): double sum of squares, float mean,
// 1 / sqrt(mean + eps), then (x * scale) * w. NT threads hold PER values each.
// The launch is latency-bound: many waves issuing one load each finish sooner
// than one wave issuing many (6.5 vs 3.4 us at hidden 896).
template <int NT, int PER>
__global__ __launch_bounds__(NT) void add_rmsnorm(float *__restrict__ hidden, const float *__restrict__ delta,
                                                  const float *__restrict__ delta2, const float *__restrict__ w,
                                                  float *__restrict__ out, int n, float eps) {
    __shared__ double red[NT / 64];
    float h[PER], dl[PER], dl2[PER], wv[PER];
    // Every load is issued before the first store, so they share one round trip.
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int i = threadIdx.x + j * NT;
        h[j] = i < n ? hidden[i] : 0.0f;
        dl[j] = delta && i < n ? delta[i] : 0.0f;
        dl2[j] = delta2 && i < n ? delta2[i] : 0.0f;
        wv[j] = i < n ? w[i] : 0.0f;
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int i = threadIdx.x + j * NT;
        if (delta) h[j] = h[j] + dl[j];
        if (delta2) h[j] = h[j] + dl2[j];
        if (delta || delta2) {
            if (i < n) hidden[i] = h[j];
        }
        ss += static_cast<double>(h[j]) * static_cast<double>(h[j]);
    }
    ss = block_sum<NT>(ss, red);
    const float mean_sq = static_cast<float>(ss / n);
    const float scale = 1.0f / sqrtf(mean_sq + eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int i = threadIdx.x + j * NT;
        if (i < n) out[i] = (h[j] * scale) * wv[j];
    }
}

void launch_add_rmsnorm(float *hidden, const float *delta, const float *delta2, const float *w, float *out, int n,
                        float eps, hipStream_t s) {
    if (n <= kNormThreads)
        add_rmsnorm<kNormThreads, 1><<<1, kNormThreads, 0, s>>>(hidden, delta, delta2, w, out, n, eps);
    else if (n <= 4 * kNormThreads)
        add_rmsnorm<kNormThreads, 4><<<1, kNormThreads, 0, s>>>(hidden, delta, delta2, w, out, n, eps);
    else
        add_rmsnorm<kNormThreads, kMaxHidden / kNormThreads><<<1, kNormThreads, 0, s>>>(hidden, delta, delta2, w, out, n,
                                                                                          eps);
}

// Row `*token` of an fp32 embedding table.
// A step's first launch: the position and the token the host wrote to pinned memory (host_io[0],
// host_io[1]; read at system scope) go to device memory (io[0], io[1]), where the step's later
// launches read them, and the token's embedding row is decoded into out. i4 rows decode as
// i4_embed_rows_kernel decodes them: (q - zero) * scale, one subtraction and one product
// (dequant_i4_row, kernels/ref_ops.h:183-205); fp32 rows are copied.
__device__ __forceinline__ int pinned_load(const int *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ __launch_bounds__(256) void step_begin_i4(const uint8_t *__restrict__ embed, const int *host_io, int *io,
                                                     int dim, int group_size, float *__restrict__ out) {
    const int pos = pinned_load(host_io), tok = pinned_load(host_io + 1);
    if (threadIdx.x == 0) {
        io[0] = pos;
        io[1] = tok;
    }
    const int groups = (dim + group_size - 1) / group_size;
    const int gbytes = kI4Header + group_size / 2;
    const uint8_t *r = embed + static_cast<size_t>(tok) * groups * gbytes;
    for (int k = threadIdx.x; k < dim; k += blockDim.x) {
        const int g = k / group_size, i = k - g * group_size;
        const uint8_t *gp = r + static_cast<size_t>(g) * gbytes;
        const float scale = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(gp[0] | (gp[1] << 8))));
        const float zero = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(gp[2] | (gp[3] << 8))));
        const uint8_t b = gp[kI4Header + (i >> 1)];
        const int q = (i & 1) ? (b >> 4) : (b & 0x0F);
        out[k] = (static_cast<float>(q) - zero) * scale;
    }
}

__global__ void step_begin_f32(const float *table, const int *host_io, int *io, float *out, int n) {
    const int pos = pinned_load(host_io), tok = pinned_load(host_io + 1);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        io[0] = pos;
        io[1] = tok;
    }
    const size_t base = static_cast<size_t>(tok) * n;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = table[base + i];
}

// One workgroup per query head: attention_head (decode_attn.h) on the raw q / k / v
// projections, biases added at entry.
template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attention_step(
    int heads_per_kv, int max_seq, float theta, float eps, float scale, const int *pos_ptr, const float *q,
    const float *k, const float *v, const float *qb, const float *kb, const float *vb, const float *qn,
    const float *kn, float *kcache, float *vcache, float *out) {
    __shared__ AttnShared sh;
    const int t = threadIdx.x;
    const int head = blockIdx.x, kvh = head / heads_per_kv;
    // q / k / v and their biases do not depend on the position: their loads go out before the
    // position's, and the fetch below only adds the biases (the KV-cache prefetch, which needs
    // the position, then does not delay them)
    // (unconditional loads, so that the compiler can count them: threads past the head and absent
    // biases read element 0 of the projection instead, which they never use)
    const int qi = t < HD ? head * HD + t : 0, ki = t < HD ? kvh * HD + t : 0;
    const float rq = q[qi], rk = k[ki], rv = v[ki];
    const float bq = (qb ? qb : q)[qi], bk = (kb ? kb : k)[ki], bv = (vb ? vb : v)[ki];
    __builtin_amdgcn_sched_barrier(0);
    const auto fetch = [&](float &qv, float &kv, float &vv) {
        if (t < HD) {
            qv = qb ? rq + bq : rq;
            kv = kb ? rk + bk : rk;
            vv = vb ? rv + bv : rv;
        }
        return true;
    };
    attention_head<HD, (HD <= 128), 16>(sh, t, head, heads_per_kv, fetch, qn, kn, kcache, vcache, *pos_ptr, max_seq,
                                        theta, eps, scale, true, [&](int i, float o) { out[i] = o; });
}

// gate = silu(gate) * up (swiglu_ref, kernels/silu/swiglu_ref.cpp).
__global__ void swiglu(float *gate, const float *up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float g = gate[i];
        const float s = g / (1.0f + expf(-g));
        gate[i] = s * up[i];
    }
}

// First index of the largest value (argmax_ref, kernels/argmax/argmax_ref.cpp):
// each block scans its slice, the final block reduces the block winners; ties
// go to the lower index.
__device__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__device__ void block_argmax(float &bv, int &bi) {
    __shared__ float rv[kArgmaxThreads / 64];
    __shared__ int ri[kArgmaxThreads / 64];
    const int lane = threadIdx.x & 63;
    const auto step = [&](auto dl) {  // lane l ^ dl's candidate, exchanged in registers
        constexpr int DL = decltype(dl)::value;
        better(bv, bi, lane_xor<DL>(bv, lane), __float_as_int(lane_xor<DL>(__int_as_float(bi), lane)));
    };
    step(std::integral_constant<int, 32>{});
    step(std::integral_constant<int, 16>{});
    step(std::integral_constant<int, 8>{});
    step(std::integral_constant<int, 4>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 1>{});
    if ((threadIdx.x & 63) == 0) {
        rv[threadIdx.x >> 6] = bv;
        ri[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    bv = rv[0];
    bi = ri[0];
    for (int w = 1; w < kArgmaxThreads / 64; ++w) better(bv, bi, rv[w], ri[w]);
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial(const float *x, int n, float *pv, int *pi) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    const int base = blockIdx.x * kArgmaxPerBlock;
    for (int j = 0; j < kArgmaxPerThread; ++j) {
        const int i = base + j * kArgmaxThreads + threadIdx.x;
        if (i < n) better(bv, bi, x[i], i);
    }
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

// The token goes to out and, when host_out is given (pinned memory), to host_out at system scope.
__global__ __launch_bounds__(kArgmaxThreads) void argmax_final(const float *pv, const int *pi, int nb, int *out,
                                                               int *host_out) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int b = threadIdx.x; b < nb; b += kArgmaxThreads) better(bv, bi, pv[b], pi[b]);
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
        const int tok = bi == 0x7fffffff ? 0 : bi;
        *out = tok;
        if (host_out) __hip_atomic_store(host_out, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// fp16 -> fp32 of the fp16 vectors a VQ2 file may carry (norms, biases); the
// reference converts them once at load with half_to_float (runtime/qwen_model.cpp:182-190).
__global__ void f16_to_f32(const _Float16 *src, float *dst, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = static_cast<float>(src[i]);
}

// BiIP rotation ahead of one projection (RotParams, runtime/qwen_model.h:316-320).
struct Rot {
    const float *sign = nullptr, *scale = nullptr;
    int bs = 0;
};

struct Layer {
    Rot rq, rk, rv, ro, rg, ru, rd;
    bool rotated = false;
    const float *in_ln = nullptr, *post_ln = nullptr;
    const float *qb = nullptr, *kb = nullptr, *vb = nullptr, *qn = nullptr, *kn = nullptr;
    const uint8_t *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    const uint8_t *gate = nullptr, *up = nullptr, *down = nullptr;
};

struct Engine {
    tqhip_model_config c{};
    int pd = 3, lm_dtype = 3;  // projection dtype and lm_head dtype: 3 i4, 4 VQ2
    int q_dim = 0, kv_dim = 0, gs = 0, max_seq = 0, amax_blocks = 0;
    float attn_scale = 0.0f;
    const void *embed = nullptr;
    bool embed_i4 = false;
    const uint8_t *lm_head = nullptr;
    const float *final_norm = nullptr;
    std::vector<Layer> layers;
    float *hidden = nullptr, *normed = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr,
          *o = nullptr, *gate = nullptr, *up = nullptr, *ffn = nullptr, *logits = nullptr, *kv = nullptr,
          *amax_v = nullptr, *rotbuf = nullptr;
    // Fused layers (i4 files without rotations whose projections the set kernel takes): the
    // residual adds, the RMSNorms and SwiGLU run inside the next projection's launch (its
    // activation prologue), and the layers' hidden states alternate between hidden and hidden2.
    bool fused = false;
    bool fused_rot = false;  // VQ2 rotations inside the matvec launches (unless TQHIP_DECODE_UNFUSED)
    // Fused i4 layers: gate/up as one launch storing silu(gate) * up, down without a prologue
    // (TQHIP_DECODE_NO_GLU=1: gate and up stored, SwiGLU in down's prologue; the same bits)
    bool glu = false;
    // An i4 lm_head on the register-path kernel forms each workgroup's argmax as it stores the
    // logits, and one launch reduces the partials (TQHIP_DECODE_NO_AMAX=1: the two-launch argmax
    // over the logits; the same token)
    bool amax_fused = false;
    float *hidden2 = nullptr;
    size_t rotbuf_floats = 0;
    int *amax_i = nullptr, *dev_io = nullptr;  // dev_io: pos, token, next, run, flow error
    int *host_io = nullptr;  // pinned: a step's position and token in (0, 1), its next token out (2)
    // The data-flow step (decode_flow.hip): one cooperative launch for the layers, then the
    // lm_head and the argmax; the graph above stays as the fallback.
    bool flow = false;
    FlowArgs fa{};
    void *flow_mem = nullptr;  // HBM: the launch's FlowArgs, then the per-layer pointers
    size_t flow_lds = 0;
    unsigned run = 0;
    size_t layer_stride = 0;                    // floats per layer and plane: n_kv_heads * max_seq * head_dim
    void *arena = nullptr;
    hipStream_t stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool eager = false;  // TQHIP_DECODE_EAGER=1: launch the step kernel by kernel (for profilers)
    ScratchSet *scratch = nullptr;  // the matvec launches' split-K slots: owned by the engine's graph
    int seq_len = 0;
};

int mv(const Engine &e, const uint8_t *w, int dtype, const float *x, float *y, int M, int K, hipStream_t s) {
    return dtype == 4 ? launch_vq2_matvec(w, x, y, M, K, s) : launch_i4_matvec(w, x, y, M, K, e.gs, s);
}

// mv_rot (runtime/qwen_model.cpp:229-238): the activation rotated into rotbuf
// first when the projection carries a rotation (for VQ2, inside the matvec launch where
// that takes it: the same bits, one launch fewer).
int mvr(const Engine &e, const uint8_t *w, int dtype, const float *x, float *y, int M, int K, const Rot &r,
        hipStream_t s) {
    if (r.sign && dtype == 4 && e.fused_rot) {
        const I4Mat m1{w, x, y, M, K};
        const int st = launch_vq2_matvec_set_rot(1, &m1, &r.scale, &r.sign, r.bs, s);
        if (st != kNotFused) return st;
    }
    if (r.sign) {
        const int st = launch_biip_rotate(x, e.rotbuf, K, r.scale, r.sign, r.bs, s);
        if (st != kOk) return st;
        x = e.rotbuf;
    }
    return mv(e, w, dtype, x, y, M, K, s);
}

// Projections of one x that all carry a rotation with the same block: the n
// rotations in one launch (into rotbuf, K floats apart), then the n matvecs, each
// on its own rotated copy, as one set launch. kNotFused when the rotations differ
// in presence or block, or rotbuf cannot hold n copies.
int mv_rotated_set(const Engine &e, int n, const uint8_t *const *w, float *const *y, const int *m, int K,
                   const Rot *const *r, hipStream_t s) {
    if (static_cast<size_t>(n) * K > e.rotbuf_floats) return kNotFused;
    for (int j = 0; j < n; ++j)
        if (!r[j]->sign || r[j]->bs != r[0]->bs) return kNotFused;
    if (e.pd == 4 && e.fused_rot) {  // VQ2: the rotations inside the set launch where it takes them
        I4Mat mats[3];
        const float *sc[3], *sg[3];
        for (int j = 0; j < n; ++j) {
            mats[j] = I4Mat{w[j], e.normed, y[j], m[j], K};
            sc[j] = r[j]->scale;
            sg[j] = r[j]->sign;
        }
        const int st = launch_vq2_matvec_set_rot(n, mats, sc, sg, r[0]->bs, s);
        if (st != kNotFused) return st;
    }
    float *xr[3];
    const float *sc[3], *sg[3];
    for (int j = 0; j < n; ++j) {
        xr[j] = e.rotbuf + static_cast<size_t>(j) * K;
        sc[j] = r[j]->scale;
        sg[j] = r[j]->sign;
    }
    int st = launch_biip_rotate_n(n, e.normed, xr, K, sc, sg, r[0]->bs, s);
    if (st != kOk) return st;
    I4Mat mats[3];
    for (int j = 0; j < n; ++j) mats[j] = I4Mat{w[j], xr[j], y[j], m[j], K};
    return e.pd == 4 ? launch_vq2_matvec_set(n, mats, s) : launch_i4_matvec_set(n, mats, e.gs, s);
}

int forward(Engine &e) {
    hipStream_t s = e.stream;
    const int H = e.c.hidden_size, I = e.c.intermediate_size;
    const float eps = e.c.rms_norm_eps;
    int st = kOk;
    // the position and token from the host's pinned words, and the token's embedding row
    if (e.embed_i4) {
        step_begin_i4<<<1, 256, 0, s>>>(static_cast<const uint8_t *>(e.embed), e.host_io, e.dev_io, H, e.gs, e.hidden);
    } else {
        step_begin_f32<<<(H + 255) / 256, 256, 0, s>>>(static_cast<const float *>(e.embed), e.host_io, e.dev_io,
                                                        e.hidden, H);
    }
    if (!e.fused) launch_add_rmsnorm(e.hidden, nullptr, nullptr, e.layers[0].in_ln, e.normed, H, eps, s);
    // A fused launch that does not apply returns kNotFused; the engine chose fused layers
    // only where every one applies, so that is a launch failure here. i4: the set kernel's
    // prologue; VQ2: the staged launch, which also applies the projections' rotations.
    auto fused_set = [&](int n, const I4Mat *m, const Rot *const *rot, const SetPrologue &p) {
        int r;
        if (e.pd == 3) {
            r = launch_i4_matvec_set_pro(n, m, e.gs, p, s);
        } else {
            const float *sc[3], *sg[3];
            for (int j = 0; j < n; ++j) {
                sc[j] = rot[j]->scale;
                sg[j] = rot[j]->sign;
            }
            r = launch_vq2_matvec_set_pro(n, m, sc, rot[0]->sign ? sg : nullptr, rot[0]->bs, &p, s);
        }
        return r == kNotFused ? static_cast<int>(kLaunchFailed) : r;
    };
    for (size_t li = 0; li < e.layers.size(); ++li) {
        const Layer &L = e.layers[li];
        float *kc = e.kv + (2 * li) * e.layer_stride, *vc = e.kv + (2 * li + 1) * e.layer_stride;
        // fused: this layer's hidden state, cur = (prev + o) + ffn of the layer before, stored by
        // the q/k/v launch (layer 0: the embedding, in hidden)
        float *cur = (li & 1) ? e.hidden2 : e.hidden, *prev = (li & 1) ? e.hidden : e.hidden2;
        const uint8_t *w3[3] = {L.q, L.k, L.v};
        float *y3[3] = {e.q, e.k, e.v};
        const int d3[3] = {e.q_dim, e.kv_dim, e.kv_dim};
        const Rot *r3[3] = {&L.rq, &L.rk, &L.rv};
        if (e.fused) {
            const float *xb = li == 0 ? e.hidden : prev;
            const I4Mat m3[3] = {{L.q, xb, e.q, e.q_dim, H}, {L.k, xb, e.k, e.kv_dim, H}, {L.v, xb, e.v, e.kv_dim, H}};
            const SetPrologue p{2, nullptr, li == 0 ? nullptr : e.o, li == 0 ? nullptr : e.ffn, L.in_ln,
                                li == 0 ? nullptr : cur, eps};
            if ((st = fused_set(3, m3, r3, p)) != kOk) return st;
        } else if (e.pd == 3 && !L.rotated) {
            if ((st = launch_i4_matvec_group(3, w3, y3, d3, e.normed, H, e.gs, s)) != kOk) return st;
        } else if (e.pd == 4 && !L.rotated) {
            const I4Mat m3[3] = {{L.q, e.normed, e.q, e.q_dim, H}, {L.k, e.normed, e.k, e.kv_dim, H},
                                 {L.v, e.normed, e.v, e.kv_dim, H}};
            if ((st = launch_vq2_matvec_set(3, m3, s)) != kOk) return st;
        } else if ((st = mv_rotated_set(e, 3, w3, y3, d3, H, r3, s)) != kNotFused) {
            if (st != kOk) return st;
        } else {
            for (int j = 0; j < 3; ++j)
                if ((st = mvr(e, w3[j], e.pd, e.normed, y3[j], d3[j], H, *r3[j], s)) != kOk) return st;
        }
        auto attn = e.c.head_dim == 64 ? attention_step<64> : e.c.head_dim == 128 ? attention_step<128>
                                                                                  : attention_step<256>;
        attn<<<e.c.n_heads, kAttnThreads, 0, s>>>(e.c.n_heads / e.c.n_kv_heads, e.max_seq, e.c.rope_theta,
                                                  e.c.rms_norm_eps, e.attn_scale, e.dev_io, e.q, e.k, e.v, L.qb,
                                                  L.kb, L.vb, L.qn, L.kn, kc, vc, e.attn);
        if ((st = mvr(e, L.o, e.pd, e.attn, e.o, H, e.q_dim, L.ro, s)) != kOk) return st;
        if (e.fused) {
            // gate/up read rmsnorm(cur + o) * post_ln; down reads silu(gate) * up
            const I4Mat m2[2] = {{L.gate, cur, e.gate, I, H}, {L.up, cur, e.up, I, H}};
            const Rot *r2[2] = {&L.rg, &L.ru}, *r1[1] = {&L.rd};
            const SetPrologue post{2, nullptr, e.o, nullptr, L.post_ln, nullptr, eps};
            if (e.glu) {  // i4: silu(gate) * up formed by the gate/up launch, down without a prologue
                st = launch_i4_matvec_glu(m2[0], m2[1], e.gs, post, s);
                if (st != kOk) return st == kNotFused ? static_cast<int>(kLaunchFailed) : st;
                const I4Mat m1{L.down, e.gate, e.ffn, H, I};
                st = launch_i4_matvec_set_fit(1, &m1, e.gs, s);
                if (st != kOk) return st == kNotFused ? static_cast<int>(kLaunchFailed) : st;
                continue;
            }
            if ((st = fused_set(2, m2, r2, post)) != kOk) return st;
            const I4Mat m1[1] = {{L.down, e.gate, e.ffn, H, I}};
            if ((st = fused_set(1, m1, r1, SetPrologue{1, e.up, nullptr, nullptr, nullptr, nullptr, eps})) != kOk)
                return st;
            continue;
        }
        launch_add_rmsnorm(e.hidden, e.o, nullptr, L.post_ln, e.normed, H, eps, s);
        const uint8_t *w2[2] = {L.gate, L.up};
        float *y2[2] = {e.gate, e.up};
        const int d2[2] = {I, I};
        const Rot *r2[2] = {&L.rg, &L.ru};
        if (e.pd == 3 && !L.rotated) {
            if ((st = launch_i4_matvec_group(2, w2, y2, d2, e.normed, H, e.gs, s)) != kOk) return st;
        } else if (e.pd == 4 && !L.rotated) {
            const I4Mat m2[2] = {{L.gate, e.normed, e.gate, I, H}, {L.up, e.normed, e.up, I, H}};
            if ((st = launch_vq2_matvec_set(2, m2, s)) != kOk) return st;
        } else if ((st = mv_rotated_set(e, 2, w2, y2, d2, H, r2, s)) != kNotFused) {
            if (st != kOk) return st;
        } else {
            for (int j = 0; j < 2; ++j)
                if ((st = mvr(e, w2[j], e.pd, e.normed, y2[j], d2[j], H, *r2[j], s)) != kOk) return st;
        }
        swiglu<<<(I + 255) / 256, 256, 0, s>>>(e.gate, e.up, I);
        if ((st = mvr(e, L.down, e.pd, e.gate, e.ffn, H, I, L.rd, s)) != kOk) return st;
        const float *next_ln = li + 1 < e.layers.size() ? e.layers[li + 1].in_ln : e.final_norm;
        launch_add_rmsnorm(e.hidden, e.ffn, nullptr, next_ln, e.normed, H, eps, s);
    }
    if (e.fused) {  // the last layer's (cur + o) + ffn, normed with the final norm
        float *last = ((e.layers.size() - 1) & 1) ? e.hidden2 : e.hidden;
        launch_add_rmsnorm(last, e.o, e.ffn, e.final_norm, e.normed, H, eps, s);
    }
    if (e.amax_fused) {
        int parts = 0;
        st = launch_i4_matvec_amax(e.lm_head, e.normed, e.logits, e.c.vocab_size, H, e.gs, e.amax_v, e.amax_i,
                                   kArgmaxParts, &parts, s);
        if (st != kOk) return st == kNotFused ? kLaunchFailed : st;  // (chosen at create where it applies)
        argmax_final<<<1, kArgmaxThreads, 0, s>>>(e.amax_v, e.amax_i, parts, e.dev_io + 2, e.host_io + 2);
        return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
    }
    if ((st = mv(e, e.lm_head, e.lm_dtype, e.normed, e.logits, e.c.vocab_size, H, s)) != kOk) return st;
    argmax_partial<<<e.amax_blocks, kArgmaxThreads, 0, s>>>(e.logits, e.c.vocab_size, e.amax_v, e.amax_i);
    argmax_final<<<1, kArgmaxThreads, 0, s>>>(e.amax_v, e.amax_i, e.amax_blocks, e.dev_io + 2, e.host_io + 2);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

int eager_forward(Engine &e) {
    ScratchScope scope(e.scratch);
    return forward(e);
}

// The data-flow step: the layers and the final norm as one cooperative launch, then the lm_head
// and the argmax as in the graph.
int flow_forward(Engine &e) {
    hipStream_t s = e.stream;
    const FlowArgs *dev_args = static_cast<const FlowArgs *>(e.flow_mem);
    void *args[] = {&dev_args};
    if (hipLaunchCooperativeKernel(flow_kernel(e.c.head_dim), dim3(e.fa.plan.wgs), dim3(512), args,
                                   static_cast<unsigned>(e.flow_lds), s) != hipSuccess)
        return kLaunchFailed;
    ScratchScope scope(e.scratch);
    const int st = mv(e, e.lm_head, e.lm_dtype, e.normed, e.logits, e.c.vocab_size, e.c.hidden_size, s);
    if (st != kOk) return st;
    argmax_partial<<<e.amax_blocks, kArgmaxThreads, 0, s>>>(e.logits, e.c.vocab_size, e.amax_v, e.amax_i);
    argmax_final<<<1, kArgmaxThreads, 0, s>>>(e.amax_v, e.amax_i, e.amax_blocks, e.dev_io + 2, nullptr);
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

// Sets up the data-flow step for an engine of fused i4 layers when TQHIP_DECODE_FLOW=1 (the
// graph stays the default: measured on MI355X, the flow step takes 0.65-0.71 ms per token of
// the Qwen2.5-0.5B-shaped file against 0.63-0.66 ms for the graph, the same logits): the
// per-layer pointer table in HBM, one 512-thread workgroup per CU (all resident at once;
// TQHIP_FLOW_WGS overrides the count, up to what fits), the task plan, the wait limit. Leaves
// e->flow false, with nothing to undo, wherever it does not apply.
int flow_setup(Engine *e) {
    const char *env = std::getenv("TQHIP_DECODE_FLOW");
    if (!env || env[0] != '1' || !e->fused || e->pd != 3 || e->eager) return kOk;
    const void *fn = flow_kernel(e->c.head_dim);
    const int H = e->c.hidden_size, I = e->c.intermediate_size, qd = e->q_dim;
    if (!fn || !set_kernel_takes(qd, e->gs) || !flow_shapes_ok(H, qd) || (!e->embed_i4 && H % 4 != 0)) return kOk;
    int dev = 0, coop = 0, cus = 0, rate_khz = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || rate_khz <= 0)
        return kOk;
    const size_t lds = flow_lds_table(H, qd, I) + e->layers.size() * sizeof(FlowLayerPtrs);
    if (lds > 64 * 1024 || hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, 512, lds) != hipSuccess || occ < 1)
        return kOk;
    int wgs = cus;
    if (const char *w = std::getenv("TQHIP_FLOW_WGS")) wgs = std::max(1, std::atoi(w));
    wgs = std::min(wgs, occ * cus);
    std::vector<FlowLayerPtrs> lp(e->layers.size());
    for (size_t i = 0; i < e->layers.size(); ++i) {
        const Layer &L = e->layers[i];
        lp[i] = FlowLayerPtrs{L.q, L.k, L.v, L.o, L.gate, L.up, L.down, L.in_ln, L.post_ln, L.qb, L.kb, L.vb, L.qn,
                              L.kn, e->kv + (2 * i) * e->layer_stride, e->kv + (2 * i + 1) * e->layer_stride};
    }
    const size_t head = (sizeof(FlowArgs) + 255) / 256 * 256, bytes = lp.size() * sizeof(FlowLayerPtrs);
    if (hipMalloc(&e->flow_mem, head + bytes) != hipSuccess) return kHipFailed;
    FlowLayerPtrs *dev_layers = reinterpret_cast<FlowLayerPtrs *>(static_cast<uint8_t *>(e->flow_mem) + head);
    if (hipMemcpy(dev_layers, lp.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) return kHipFailed;
    const auto shape = [](int K) { return K <= 1024 ? 0 : (K + 2047) / 2048; };
    FlowArgs &a = e->fa;  // (a.vec was set with the arena)
    a.layers = dev_layers;
    a.n_layers = e->c.n_layers;
    a.H = H;
    a.I = I;
    a.q_dim = qd;
    a.kv_dim = e->kv_dim;
    a.n_heads = e->c.n_heads;
    a.heads_per_kv = e->c.n_heads / e->c.n_kv_heads;
    a.max_seq = e->max_seq;
    a.eps = e->c.rms_norm_eps;
    a.theta = e->c.rope_theta;
    a.attn_scale = e->attn_scale;
    a.embed_i4 = e->embed_i4 ? static_cast<const uint8_t *>(e->embed) : nullptr;
    a.embed_f32 = e->embed_i4 ? nullptr : static_cast<const float *>(e->embed);
    a.embed_gs = e->gs;
    a.final_norm = e->final_norm;
    a.normed = e->normed;
    a.io = e->dev_io;
    a.shape_h = shape(H);
    a.shape_q = shape(qd);
    a.shape_i = shape(I);
    a.rd = a.shape_h == 0 ? 2 : 1;  // gate/up row pairs per half-wave, or per wave for longer rows
    // 100 ms per wait; TQHIP_FLOW_TIMEOUT_US sets another limit (tests force the fallback with 0)
    long long us = 100000;
    if (const char *t = std::getenv("TQHIP_FLOW_TIMEOUT_US")) us = std::max(0LL, std::atoll(t));
    a.timeout = static_cast<long long>(rate_khz) * us / 1000;
    int tasks[kFlowPhases];
    for (int k = 0; k < kFlowPhases; ++k)
        tasks[k] = flow_tasks(k, H, qd, e->kv_dim, I, e->c.n_heads, a.shape_h, a.shape_q, a.shape_i, a.rd);
    a.plan = flow_plan(wgs, tasks);
    a.lds_table = static_cast<int>(flow_lds_table(H, qd, I));
    if (hipMemcpy(e->flow_mem, &a, sizeof(FlowArgs), hipMemcpyHostToDevice) != hipSuccess) return kHipFailed;
    e->flow_lds = lds;
    e->flow = true;
    return kOk;
}

void release(Engine *e) {
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    if (e->exec) (void)hipGraphExecDestroy(e->exec);
    if (e->graph) (void)hipGraphDestroy(e->graph);
    scratch_set_free(e->scratch);
    if (e->arena) (void)hipFree(e->arena);
    if (e->host_io) (void)hipHostFree(e->host_io);
    if (e->flow_mem) (void)hipFree(e->flow_mem);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

// Resolves a tensor of the model with the expected dtype and shape.
struct Binder {
    void *model;
    std::string *err;
    const void *get(const std::string &name, int dtype, uint64_t d0, uint64_t d1, bool optional = false) {
        tqhip_tensor_info info;
        if (tqhip_model_find(model, name.c_str(), &info) != kOk) {
            if (!optional) *err = "gpu engine: missing tensor " + name;
            return nullptr;
        }
        const bool shape_ok = d1 == 0 ? (info.ndim == 1 && info.shape[0] == d0)
                                      : (info.ndim == 2 && info.shape[0] == d0 && info.shape[1] == d1);
        if (info.dtype != dtype || !shape_ok) {
            *err = "gpu engine: tensor " + name + " has an unexpected dtype or shape";
            return nullptr;
        }
        return info.device;
    }
};

int create(void *model, int max_seq_len, std::string *err, Engine **out) {
    tqhip_model_config c;
    if (tqhip_model_config_get(model, &c) != kOk) {
        *err = "gpu engine: no model";
        return kBadFile;
    }
    if ((c.file_dtype != 3 && c.file_dtype != 4) || c.model_type != 0) {
        *err = "gpu engine: serves dense (Qwen2 / Qwen3) i4 and VQ2 files only";
        return kBadFile;
    }
    if (max_seq_len <= 0) max_seq_len = c.max_seq_len;
    if (max_seq_len > c.max_seq_len) {
        *err = "gpu engine: max_seq_len " + std::to_string(max_seq_len) + " exceeds the model limit " +
               std::to_string(c.max_seq_len);
        return kBadShape;
    }
    if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256) {
        *err = "gpu engine: head_dim must be 64, 128 or 256";
        return kBadShape;
    }
    if (c.hidden_size > kMaxHidden) {
        *err = "gpu engine: hidden_size above " + std::to_string(kMaxHidden);
        return kBadShape;
    }
    const int st = tqhip_model_upload(model);
    if (st != kOk) {
        *err = "gpu engine: weight upload failed";
        return st;
    }
    Engine *e = new Engine;
    e->c = c;
    e->q_dim = c.n_heads * c.head_dim;
    e->kv_dim = c.n_kv_heads * c.head_dim;
    e->gs = c.quant_group_size;
    e->pd = c.file_dtype;
    e->max_seq = max_seq_len;
    e->attn_scale = 1.0f / std::sqrt(static_cast<float>(c.head_dim));
    const uint64_t H = c.hidden_size, I = c.intermediate_size, V = c.vocab_size;
    Binder b{model, err};
    bool ok = true;
    // fp16 vectors (VQ2 files) are converted into the arena after it exists:
    // (source, length, the pointer to patch).
    struct F16Vec {
        const void *src;
        int n;
        const float **slot;
    };
    std::vector<F16Vec> f16s;
    size_t f16_floats = 0;
    auto vec_into = [&](const std::string &n, uint64_t d, const float **slot, bool opt = false) {
        tqhip_tensor_info info;
        const bool half = e->pd == 4 && tqhip_model_find(model, n.c_str(), &info) == kOk && info.dtype == 1;
        const void *p = b.get(n, half ? 1 : 0, d, 0, opt);
        if (!p && (!opt || !err->empty())) ok = false;
        if (p && half) {
            f16s.push_back({p, static_cast<int>(d), slot});
            f16_floats += (d + 63) / 64 * 64;
            p = nullptr;  // patched after the arena is allocated
        }
        *slot = static_cast<const float *>(p);
    };
    auto vec = [&](const std::string &n, uint64_t d, bool opt = false) {
        const float *p = nullptr;
        vec_into(n, d, &p, opt);
        return p;
    };
    auto mat = [&](const std::string &n, uint64_t d0, uint64_t d1) {
        const uint8_t *p = static_cast<const uint8_t *>(b.get(n, e->pd, d0, d1));
        if (!p) ok = false;
        return p;
    };
    tqhip_tensor_info emb;
    if (tqhip_model_find(model, "model.embed_tokens.weight", &emb) != kOk) {
        *err = "gpu engine: missing tensor model.embed_tokens.weight";
        ok = false;
    } else {
        e->embed_i4 = emb.dtype == 3;
        e->embed = b.get("model.embed_tokens.weight", e->embed_i4 ? 3 : 0, V, H);  // i4 or fp32 [vocab, hidden]
        ok = e->embed != nullptr;
    }
    if (ok) vec_into("model.norm.weight", H, &e->final_norm);
    if (ok) {
        tqhip_tensor_info lm;
        if (tqhip_model_find(model, "lm_head.weight", &lm) == kOk) {
            e->lm_dtype = lm.dtype == 3 ? 3 : e->pd;  // an i4 lm_head in a VQ2 file, or the file's own
            e->lm_head = static_cast<const uint8_t *>(b.get("lm_head.weight", e->lm_dtype, V, H));
            ok = e->lm_head != nullptr;
        } else if (c.tied_embeddings && e->embed_i4) {
            e->lm_dtype = 3;
            e->lm_head = static_cast<const uint8_t *>(e->embed);
        } else {
            *err = c.tied_embeddings ? "gpu engine: a tied fp32 embedding needs an fp32 lm_head, which is not served"
                                     : "gpu engine: missing tensor lm_head.weight";
            ok = false;
        }
    }
    e->layers.resize(c.n_layers);
    for (int i = 0; ok && i < c.n_layers; ++i) {
        const std::string p = "model.layers." + std::to_string(i) + ".";
        Layer &L = e->layers[i];
        vec_into(p + "input_layernorm.weight", H, &L.in_ln);
        vec_into(p + "post_attention_layernorm.weight", H, &L.post_ln);
        L.q = mat(p + "self_attn.q_proj.weight", e->q_dim, H);
        L.k = mat(p + "self_attn.k_proj.weight", e->kv_dim, H);
        L.v = mat(p + "self_attn.v_proj.weight", e->kv_dim, H);
        L.o = mat(p + "self_attn.o_proj.weight", H, e->q_dim);
        L.gate = mat(p + "mlp.gate_proj.weight", I, H);
        L.up = mat(p + "mlp.up_proj.weight", I, H);
        L.down = mat(p + "mlp.down_proj.weight", H, I);
        if (!ok) break;
        vec_into(p + "self_attn.q_proj.bias", e->q_dim, &L.qb, true);
        vec_into(p + "self_attn.k_proj.bias", e->kv_dim, &L.kb, true);
        vec_into(p + "self_attn.v_proj.bias", e->kv_dim, &L.vb, true);
        vec_into(p + "self_attn.q_norm.weight", c.head_dim, &L.qn, true);
        vec_into(p + "self_attn.k_norm.weight", c.head_dim, &L.kn, true);
        // bind_rot (runtime/qwen_model.cpp:427-435): sign present = rotated; the
        // block is the largest of 256, 128, ..., 2 dividing in_features, else 1.
        auto rot = [&](const std::string &prefix, int in_f, Rot &r) {
            vec_into(prefix + ".rot_sign", in_f, &r.sign, true);
            vec_into(prefix + ".rot_scale", in_f, &r.scale, true);
            tqhip_tensor_info si;
            if (tqhip_model_find(model, (prefix + ".rot_sign").c_str(), &si) != kOk) return;
            r.bs = 1;
            for (int bs : {256, 128, 64, 32, 16, 8, 4, 2})
                if (in_f % bs == 0) {
                    r.bs = bs;
                    break;
                }
            L.rotated = true;
        };
        rot(p + "self_attn.q_proj", c.hidden_size, L.rq);
        rot(p + "self_attn.k_proj", c.hidden_size, L.rk);
        rot(p + "self_attn.v_proj", c.hidden_size, L.rv);
        rot(p + "self_attn.o_proj", e->q_dim, L.ro);
        rot(p + "mlp.gate_proj", c.hidden_size, L.rg);
        rot(p + "mlp.up_proj", c.hidden_size, L.ru);
        rot(p + "mlp.down_proj", c.intermediate_size, L.rd);
        if (ok && (L.qn == nullptr) != (L.kn == nullptr)) {
            *err = "gpu engine: layer " + std::to_string(i) + ": q_norm/k_norm must both be present or both absent";
            ok = false;
        }
    }
    if (!ok) {
        release(e);
        return kBadFile;
    }

    // One allocation: activations (each 256-byte aligned), the fp32 KV cache
    // [layer][k|v][kv_head][max_seq][head_dim], the argmax partials.
    e->layer_stride = static_cast<size_t>(c.n_kv_heads) * max_seq_len * c.head_dim;
    e->amax_blocks = (c.vocab_size + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
    const size_t counts[] = {H, H, static_cast<size_t>(e->q_dim), static_cast<size_t>(e->kv_dim),
                             static_cast<size_t>(e->kv_dim), static_cast<size_t>(e->q_dim), H, I, I, H, V,
                             2 * static_cast<size_t>(c.n_layers) * e->layer_stride,
                             static_cast<size_t>(kArgmaxParts), static_cast<size_t>(kArgmaxParts), 8,
                             f16_floats, std::max<size_t>(std::max<size_t>(3 * H, I), e->q_dim), H,
                             // the data-flow step's tagged vectors (8 bytes per element): h0, h1, q, k, v,
                             // attn, o, act, ffn
                             2 * H, 2 * H, 2 * static_cast<size_t>(e->q_dim), 2 * static_cast<size_t>(e->kv_dim),
                             2 * static_cast<size_t>(e->kv_dim), 2 * static_cast<size_t>(e->q_dim), 2 * H, 2 * I,
                             2 * H};
    float **slots[] = {&e->hidden, &e->normed, &e->q, &e->k, &e->v, &e->attn, &e->o, &e->gate, &e->up, &e->ffn,
                       &e->logits, &e->kv, &e->amax_v};
    constexpr int kSlots = 18 + kFlowVecs;
    size_t offs[kSlots], total = 0;
    for (int i = 0; i < kSlots; ++i) {
        offs[i] = total;
        total += (counts[i] * 4 + 255) / 256 * 256;
    }
    if (hipMalloc(&e->arena, total) != hipSuccess || hipStreamCreate(&e->stream) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void **>(&e->host_io), 8 * sizeof(int)) != hipSuccess) {
        *err = "gpu engine: HIP allocation failed";
        release(e);
        return kHipFailed;
    }
    for (int i = 0; i < 8; ++i) e->host_io[i] = 0;  // the set-up pass below runs position 0, token 0
    uint8_t *base = static_cast<uint8_t *>(e->arena);
    for (int i = 0; i < 13; ++i) *slots[i] = reinterpret_cast<float *>(base + offs[i]);
    e->amax_i = reinterpret_cast<int *>(base + offs[13]);
    e->dev_io = reinterpret_cast<int *>(base + offs[14]);
    if (hipMemsetAsync(e->arena, 0, total, e->stream) != hipSuccess) {
        *err = "gpu engine: HIP memset failed";
        release(e);
        return kHipFailed;
    }
    e->rotbuf = reinterpret_cast<float *>(base + offs[16]);
    e->rotbuf_floats = counts[16];
    e->hidden2 = reinterpret_cast<float *>(base + offs[17]);
    for (int i = 0; i < kFlowVecs; ++i) e->fa.vec[i] = reinterpret_cast<uint2 *>(base + offs[18 + i]);
    // fused layers where the set kernel takes every projection around a residual add, an
    // RMSNorm or SwiGLU: q/k/v and gate/up (rows of hidden_size) and down (intermediate_size)
    bool any_rot = false, aligned = true, rot_sets = true;
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    // a fused VQ2 launch rotates all of its matrices or none, with one block size
    const auto same = [](const Rot &a, const Rot &b) { return !a.sign == !b.sign && (!a.sign || a.bs == b.bs); };
    for (const Layer &L : e->layers) {
        any_rot = any_rot || L.rotated;
        aligned = aligned && al16(L.in_ln) && al16(L.post_ln);
        rot_sets = rot_sets && same(L.rq, L.rk) && same(L.rq, L.rv) && same(L.rg, L.ru);
    }
    const bool unfused = std::getenv("TQHIP_DECODE_UNFUSED") != nullptr;
    const int hs = static_cast<int>(c.hidden_size), is = static_cast<int>(c.intermediate_size);
    const int m3[3] = {e->q_dim, e->kv_dim, e->kv_dim}, m2[2] = {is, is}, m1[1] = {hs};
    const bool vq2_sets = vq2_set_takes(3, m3, hs, 2) && vq2_set_takes(2, m2, hs, 2) && vq2_set_takes(1, m1, is, 1);
    e->fused = !unfused && ((e->pd == 3 && !any_rot && aligned && set_kernel_takes(hs, e->gs) &&
                             set_kernel_takes(is, e->gs)) ||
                            (e->pd == 4 && rot_sets && vq2_sets));
    e->fused_rot = e->pd == 4 && !unfused;
    const char *no_glu = std::getenv("TQHIP_DECODE_NO_GLU");
    e->glu = e->fused && e->pd == 3 && !(no_glu && no_glu[0] == '1');
    const char *no_amax = std::getenv("TQHIP_DECODE_NO_AMAX");
    e->amax_fused = e->lm_dtype == 3 && !(no_amax && no_amax[0] == '1') &&
                    i4_matvec_amax_takes(e->lm_head, e->normed, e->logits, c.vocab_size, H, e->gs, kArgmaxParts);
    float *conv = reinterpret_cast<float *>(base + offs[15]);
    for (const F16Vec &f : f16s) {
        f16_to_f32<<<(f.n + 255) / 256, 256, 0, e->stream>>>(static_cast<const _Float16 *>(f.src), conv, f.n);
        *f.slot = conv;
        conv += (f.n + 63) / 64 * 64;
    }
    // One eager pass at position 0 with token 0 sizes the engine's scratch
    // outside the capture; its KV rows are rewritten by the first real step.
    e->scratch = scratch_set_new();
    ScratchScope scope(e->scratch);
    int rc = forward(*e);
    if (rc == kOk && hipStreamSynchronize(e->stream) != hipSuccess) rc = kLaunchFailed;
    const char *eager = std::getenv("TQHIP_DECODE_EAGER");
    e->eager = eager && eager[0] == '1';
    if (rc == kOk && !e->eager && hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
        rc = kLaunchFailed;
    if (rc == kOk && !e->eager) {
        const int fst = forward(*e);
        const hipError_t end = hipStreamEndCapture(e->stream, &e->graph);
        if (fst != kOk || end != hipSuccess) rc = fst != kOk ? fst : kLaunchFailed;
    }
    if (rc == kOk && !e->eager && hipGraphInstantiate(&e->exec, e->graph, nullptr, nullptr, 0) != hipSuccess)
        rc = kLaunchFailed;
    if (rc != kOk) {
        *err = "gpu engine: setting up the step graph failed";
        release(e);
        return rc;
    }
    if ((rc = flow_setup(e)) != kOk) {
        *err = "gpu engine: setting up the data-flow step failed";
        release(e);
        return rc;
    }
    *out = e;
    return kOk;
}

}  // namespace
}  // namespace tqhip

using namespace tqhip;

extern "C" {

int tqhip_decode_create(void *model, int max_seq_len, char *err, int err_len, void **engine) {
    if (!engine) return kBadShape;
    *engine = nullptr;
    std::string msg;
    Engine *e = nullptr;
    const int rc = model ? create(model, max_seq_len, &msg, &e) : kBadFile;
    if (rc != kOk) {
        if (msg.empty()) msg = "gpu engine: no model";
        if (err && err_len > 0) {
            std::strncpy(err, msg.c_str(), err_len - 1);
            err[err_len - 1] = 0;
        }
        return rc;
    }
    *engine = e;
    return kOk;
}

int tqhip_decode_step(void *engine, int token_id) {
    Engine *e = static_cast<Engine *>(engine);
    if (!e || token_id < 0 || token_id >= e->c.vocab_size || e->seq_len >= e->max_seq) return kBadShape;
    e->host_io[0] = e->seq_len;
    e->host_io[1] = token_id;
    if (e->flow) {
        e->host_io[3] = static_cast<int>(++e->run);
        e->host_io[4] = 0;
        if (hipMemcpyAsync(e->dev_io, e->host_io, 5 * sizeof(int), hipMemcpyHostToDevice, e->stream) != hipSuccess ||
            flow_forward(*e) != kOk ||
            hipMemcpyAsync(e->host_io + 2, e->dev_io + 2, 3 * sizeof(int), hipMemcpyDeviceToHost, e->stream) !=
                hipSuccess ||
            hipStreamSynchronize(e->stream) != hipSuccess)
            return kLaunchFailed;
        if (e->host_io[4] == 0) {
            e->seq_len += 1;
            return e->host_io[2];
        }
        // A wait of the data-flow step ran out: this engine keeps to its graph from now on, and
        // the token runs again through it (it rewrites every KV row at this position).
        std::fprintf(stderr, "tqhip: decode engine: the data-flow step timed out; using the step graph\n");
        e->flow = false;
    }
    // The step's first launch reads the position and token from host_io (pinned) and its last
    // launch writes the next token there: no copies around the graph. The host waits for that
    // word (the logits were stored by the launch before it); past a bound, or if the word never
    // comes, the stream is synchronised, which reports a failed launch.
    __atomic_store_n(&e->host_io[2], -1, __ATOMIC_SEQ_CST);
    if (e->eager ? eager_forward(*e) != kOk : hipGraphLaunch(e->exec, e->stream) != hipSuccess) return kLaunchFailed;
    const auto t0 = std::chrono::steady_clock::now();
    int next = -1;
    for (unsigned n = 0;; ++n) {
        next = __atomic_load_n(&e->host_io[2], __ATOMIC_ACQUIRE);
        if (next >= 0) break;
        if ((n & 1023) == 1023 && std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(200)) break;
    }
    if (next < 0) {
        if (hipStreamSynchronize(e->stream) != hipSuccess) return kLaunchFailed;
        next = __atomic_load_n(&e->host_io[2], __ATOMIC_ACQUIRE);
        if (next < 0) return kLaunchFailed;
    }
    e->seq_len += 1;
    return next;
}

void tqhip_decode_reset(void *engine) {
    if (engine) static_cast<Engine *>(engine)->seq_len = 0;
}

void tqhip_decode_destroy(void *engine) {
    Engine *e = static_cast<Engine *>(engine);
    if (!e) return;
    (void)hipStreamSynchronize(e->stream);
    release(e);
}

const float *tqhip_decode_logits(const void *engine) {
    return engine ? static_cast<const Engine *>(engine)->logits : nullptr;
}

int tqhip_decode_seq_len(const void *engine) { return engine ? static_cast<const Engine *>(engine)->seq_len : -1; }

int tqhip_decode_mode(const void *engine) {
    if (!engine) return -1;
    const Engine *e = static_cast<const Engine *>(engine);
    return (e->fused ? TQHIP_DECODE_FUSED : 0) | (e->flow ? TQHIP_DECODE_FLOW : 0) |
           (e->eager ? TQHIP_DECODE_EAGER : 0);
}

}  // extern "C"
