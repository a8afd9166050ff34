// decode_flow.h -- the plan of the data-flow decode step: its phases, the vectors each phase
// reads and writes, and which workgroup runs which task. Shared by the kernel
// (decode_flow.hip), the engine that launches it (decode_engine.hip) and the CPU model of its
// protocol (tests/flow_model.cpp), so all three follow one table.
//
// A token of a dense Qwen2 layer stack is, per layer l, five phases that each need the whole
// output of an earlier one:
//
//   qkv    h_l = (h_{l-1} + o_{l-1}) + ffn_{l-1} (layer 0: the embedding row), rmsnorm, q/k/v
//   attn   biases, q/k norm, RoPE, KV write at pos, attention over 0..pos
//   o      the o projection of the attention output
//   gateup rmsnorm(h_l + o_l), gate and up, act = silu(gate) * up
//   down   the down projection of act (ffn_l)
//
// and after the last layer one final norm. Every vector a phase writes goes to HBM as (value,
// tag) pairs, 8 bytes per element, stored at device scope; a phase's consumers poll the pairs
// they read until every tag is the one of the write they need, so no phase waits for more
// than its own inputs and no grid-wide barrier is used. The tag of a write of layer l in run r
// (one run per token) is r * (layers + 1) + l + 1 (mod 2^32): distinct from every tag of the
// previous run, and no vector keeps a value older than that.
//
// Why no vector is overwritten while a consumer may still read it: each phase reads whole
// vectors of earlier phases, and every workgroup that reads a phase's inputs also writes part
// of its output after the reads. A vector is next written two or more phases after its last
// read (h alternates between two buffers, see flow_buffer), and the writer of that later phase
// has, through the chain of whole-vector waits, seen the complete output of every phase in
// between, whose writers had all finished their reads.
#pragma once

#include <cstddef>
#include <cstdint>

#ifndef __HIPCC__  // the CPU model includes this without HIP
#ifndef __host__
#define __host__
#endif
#ifndef __device__
#define __device__
#endif
#endif

namespace tqhip {

enum FlowPhaseKind : int { kFlowQkv = 0, kFlowAttn, kFlowO, kFlowGateUp, kFlowDown, kFlowNorm, kFlowPhases };

// Tagged vectors. kVecH0 / kVecH1: the hidden state of even / odd layers.
enum FlowVecId : int { kVecH0 = 0, kVecH1, kVecQ, kVecK, kVecV, kVecAttn, kVecO, kVecAct, kVecFfn, kFlowVecs };

// One vector a phase of layer l reads: vector `vec` (for kVecH0, the buffer of layer l + dl)
// as written by layer l + dl. vec < 0: unused slot.
struct FlowRead {
    int vec, dl;
};

constexpr int kFlowMaxReads = 3;

// The reads of each phase kind, newest write first (the consumers poll that one first).
// qkv of layer 0 reads nothing (the embedding row is computed in place).
__host__ __device__ constexpr FlowRead flow_read(int kind, int j) {
    constexpr FlowRead none{-1, 0};
    switch (kind) {
        case kFlowQkv:  // ffn_{l-1}, o_{l-1}, h_{l-1}
            return j == 0 ? FlowRead{kVecFfn, -1} : j == 1 ? FlowRead{kVecO, -1} : FlowRead{kVecH0, -1};
        case kFlowAttn:  // q, k, v
            return j == 0 ? FlowRead{kVecQ, 0} : j == 1 ? FlowRead{kVecK, 0} : FlowRead{kVecV, 0};
        case kFlowO:
            return j == 0 ? FlowRead{kVecAttn, 0} : none;
        case kFlowGateUp:  // o_l, h_l
            return j == 0 ? FlowRead{kVecO, 0} : j == 1 ? FlowRead{kVecH0, 0} : none;
        case kFlowDown:
            return j == 0 ? FlowRead{kVecAct, 0} : none;
        case kFlowNorm:  // after the last layer L - 1: ffn, o, h of that layer
            return j == 0 ? FlowRead{kVecFfn, 0} : j == 1 ? FlowRead{kVecO, 0} : FlowRead{kVecH0, 0};
        default:
            return none;
    }
}

// The vectors a phase kind writes (up to 3; -1 unused), for layer l. qkv also stores h_l
// (workgroup of task 0).
__host__ __device__ constexpr int flow_write(int kind, int j) {
    switch (kind) {
        case kFlowQkv:
            return j == 0 ? kVecQ : j == 1 ? kVecK : j == 2 ? kVecV : -1;
        case kFlowAttn:
            return j == 0 ? kVecAttn : -1;
        case kFlowO:
            return j == 0 ? kVecO : -1;
        case kFlowGateUp:
            return j == 0 ? kVecAct : -1;
        case kFlowDown:
            return j == 0 ? kVecFfn : -1;
        default:
            return -1;  // the final norm writes the plain normed vector for the lm_head launch
    }
}

// The buffer of a read by layer l: h alternates between kVecH0 (even layers) and kVecH1.
__host__ __device__ constexpr int flow_buffer(int vec, int layer) {
    return vec == kVecH0 ? kVecH0 + (layer & 1) : vec;
}

__host__ __device__ constexpr uint32_t flow_tag(uint32_t run, int layers, int layer) {
    return run * static_cast<uint32_t>(layers + 1) + static_cast<uint32_t>(layer + 1);
}

// Task t of phase kind k runs on workgroup (first[k] + t) % wgs. The phases are laid out one
// after the other around the grid in the order q/k/v, attention, o, down, gate/up, so the
// largest, gate/up, wraps around onto the workgroups of q/k/v and attention, neither of which
// is next to it in the chain: as long as the tasks fit that way, no workgroup runs tasks of two
// consecutive phases (its second task would start only when its first is done, after the
// phase's inputs are there, and add its weight loads and first look to the chain).
struct FlowPlan {
    int wgs;
    int tasks[kFlowPhases];
    int first[kFlowPhases];
};

inline FlowPlan flow_plan(int wgs, const int (&tasks)[kFlowPhases]) {
    constexpr int order[kFlowPhases] = {kFlowQkv, kFlowAttn, kFlowO, kFlowDown, kFlowGateUp, kFlowNorm};
    FlowPlan p{};
    p.wgs = wgs;
    int at = 0;
    for (int k : order) {
        p.tasks[k] = tasks[k];
        p.first[k] = at % wgs;
        at += tasks[k];
    }
    return p;
}

// The task of phase kind k that workgroup wg runs as its i-th (i = 0, 1, ...), or -1.
__host__ __device__ inline int flow_task(const FlowPlan &p, int k, int wg, int i) {
    const int t = (wg - p.first[k] + p.wgs) % p.wgs + i * p.wgs;
    return t < p.tasks[k] ? t : -1;
}


#ifdef __HIPCC__
// The device-side description of one launch (the engine fills it and copies it to HBM).
struct FlowLayerPtrs {
    const uint8_t *q, *k, *v, *o, *gate, *up, *down;
    const float *in_ln, *post_ln, *qb, *kb, *vb, *qn, *kn;
    float *kc, *vc;  // this layer's KV cache planes [kv_head][max_seq][head_dim]
};

struct FlowArgs {
    const FlowLayerPtrs *layers;
    int n_layers, H, I, q_dim, kv_dim, n_heads, heads_per_kv, max_seq;
    float eps, theta, attn_scale;
    const uint8_t *embed_i4;  // the i4 embedding table (group size embed_gs), or
    const float *embed_f32;   // the fp32 one
    int embed_gs;
    const float *final_norm;
    float *normed;          // the final RMSNorm's output (plain floats, for the lm_head launch)
    uint2 *vec[kFlowVecs];  // the tagged vectors
    int *io;                // [0] position, [1] token, [3] run, [4] error (0: none)
    FlowPlan plan;
    int shape_h, shape_q, shape_i;  // set-kernel shapes of rows of H, q_dim and I elements
    int rd;                         // gate/up row pairs per half-wave (rows of H <= 1024) or wave
    long long timeout;              // wall-clock ticks one wait may take
    int lds_table;                  // LDS offset of the layer records (after the phases' scratch)
};

// decode_flow.hip
bool flow_shapes_ok(int H, int q_dim);
size_t flow_lds_table(int H, int q_dim, int I);  // LDS bytes before the layer records
int flow_tasks(int kind, int H, int q_dim, int kv_dim, int I, int n_heads, int shape_h, int shape_q, int shape_i,
               int rd);
const void *flow_kernel(int head_dim);  // decode_flow<head_dim>(const FlowArgs *), or null
#endif

}  // namespace tqhip
