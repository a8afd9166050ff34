// flow_model.cpp -- CPU model of the data-flow decode step's protocol (decode_flow.hip), on
// threads: the kernel's workgroups are threads, its tagged vectors are arrays of 64-bit
// atomics (value, tag), and each task reads, waits and writes exactly the vectors the kernel's
// task does, from the shared plan (tiny-llm_amd/csrc/decode_flow.h: flow_read, flow_write,
// flow_buffer, flow_tag, flow_plan, flow_task). The arithmetic is replaced by a mixing
// function of every value a task reads, so a stale or torn read changes the result. Random
// delays before tasks and between looks shuffle the interleavings.
//
// Checks (each prints "ok <name>" or "FAIL <name>: ..." and exits 1):
//   tokens    every token's result equals a sequential run of the same tasks, over several
//             tokens (the KV rows of earlier tokens are read), for several workgroup counts
//   timeout   a task that stalls past the wait limit: the others see the error and leave
//   planted   with the hidden state written into one buffer instead of alternating, a wait
//             never completes (the error is a timeout), never a wrong result
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>

#include "decode_flow.h"

using namespace tqhip;

namespace {

struct Shape {
    int L, H, QD, KD, I, HD, heads, kv_heads;
};

uint32_t mix(uint32_t a, uint32_t b) {
    uint32_t h = a * 0x9E3779B1u ^ (b + 0x7F4A7C15u + (a << 6) + (a >> 2));
    h ^= h >> 15;
    h *= 0x85EBCA77u;
    return h ^ (h >> 13);
}

struct Model {
    Shape s;
    int wgs;
    bool single_h = false;        // the planted mistake
    int stall_wg = -1, stall_layer = -1;  // a workgroup that stalls (timeout check)
    std::chrono::milliseconds limit{2000};
    std::vector<std::atomic<uint64_t>> vec[kFlowVecs];
    std::vector<uint32_t> kv;  // [layer][kv_head][pos] (one value per row, plain: written before any reader waits)
    std::vector<uint32_t> normed;
    std::atomic<int> err{0};
    FlowPlan plan;
    int rpt = 16, max_seq = 64;

    int len(int v) const {
        switch (v) {
            case kVecH0: case kVecH1: case kVecO: case kVecFfn: return s.H;
            case kVecQ: case kVecAttn: return s.QD;
            case kVecK: case kVecV: return s.KD;
            default: return s.I;
        }
    }
    int buffer(int v, int layer) const { return single_h && v == kVecH0 ? kVecH0 : flow_buffer(v, layer); }

    Model(Shape sh, int w) : s(sh), wgs(w) {
        for (int v = 0; v < kFlowVecs; ++v) {
            vec[v] = std::vector<std::atomic<uint64_t>>(len(v));
            for (auto &x : vec[v]) x = 0;
        }
        kv.assign(static_cast<size_t>(s.L) * s.kv_heads * max_seq, 0);
        normed.assign(s.H, 0);
        const int tasks[kFlowPhases] = {(s.QD + rpt - 1) / rpt + 2 * ((s.KD + rpt - 1) / rpt), (s.heads + 1) / 2,
                                        (s.H + rpt - 1) / rpt, (s.I + rpt - 1) / rpt, (s.H + rpt - 1) / rpt, 1};
        plan = flow_plan(wgs, tasks);
    }

    // Reads n elements of vector v (its buffer for layer `layer`) once each carries `tag`;
    // false when the wait ran out or another task reported an error.
    bool wait_read(int v, int layer, int lo, int n, uint32_t tag, uint32_t &acc, std::mt19937 &rng) {
        const auto t0 = std::chrono::steady_clock::now();
        std::vector<std::atomic<uint64_t>> &a = vec[buffer(v, layer)];
        for (;;) {
            bool ok = true;
            uint32_t sum = 0;
            for (int i = lo; i < lo + n; ++i) {
                const uint64_t p = a[i].load(std::memory_order_acquire);
                if (static_cast<uint32_t>(p >> 32) != tag) {
                    ok = false;
                    break;
                }
                sum = mix(sum, static_cast<uint32_t>(p));
            }
            if (ok) {
                acc = mix(acc, sum);
                return true;
            }
            if (err.load()) return false;
            if (std::chrono::steady_clock::now() - t0 > limit) {
                err = 1;
                return false;
            }
            if (rng() % 4 == 0) std::this_thread::sleep_for(std::chrono::microseconds(rng() % 50));
        }
    }
    void write(int v, int layer, int i, uint32_t x, uint32_t tag) {
        vec[buffer(v, layer)][i].store(static_cast<uint64_t>(x) | (static_cast<uint64_t>(tag) << 32),
                                       std::memory_order_release);
    }

    // One task of phase kind k of layer l (run r, position pos): the kernel's reads and writes.
    bool task(int k, int l, int t, uint32_t run, int pos, int token, std::mt19937 &rng) {
        const uint32_t tag = flow_tag(run, s.L, l);
        uint32_t acc = mix(static_cast<uint32_t>(k), static_cast<uint32_t>(l * 131 + t));
        if (stall_wg >= 0 && l == stall_layer && k == kFlowO && t == 0)
            std::this_thread::sleep_for(limit + limit);  // the stalled task (its outputs come too late)
        if (single_h && k == kFlowQkv && l > 0 && t != 0)  // task 0 (which stores h_l) runs first
            std::this_thread::sleep_for(std::chrono::milliseconds(5));
        if (k == kFlowAttn) {
            for (int sub = 0; sub < 2; ++sub) {
                const int head = std::min(2 * t + sub, s.heads - 1), kvh = head / (s.heads / s.kv_heads);
                uint32_t hacc = acc;
                if (!wait_read(kVecQ, l, head * s.HD, s.HD, tag, hacc, rng) ||
                    !wait_read(kVecK, l, kvh * s.HD, s.HD, tag, hacc, rng) ||
                    !wait_read(kVecV, l, kvh * s.HD, s.HD, tag, hacc, rng))
                    return false;
                const size_t base = (static_cast<size_t>(l) * s.kv_heads + kvh) * max_seq;
                const uint32_t kpos = mix(hacc, 7u);  // k / v of this position: every head of the group computes it
                for (int p = 0; p < pos; ++p) hacc = mix(hacc, kv[base + p]);
                hacc = mix(hacc, kpos);
                if (2 * t + sub < s.heads) {
                    if (head % (s.heads / s.kv_heads) == 0) kv[base + pos] = kpos;
                    for (int d = 0; d < s.HD; ++d) write(kVecAttn, l, head * s.HD + d, mix(hacc, d), tag);
                }
            }
            return true;
        }
        if (k == kFlowNorm) {
            for (int j = 0; j < kFlowMaxReads; ++j) {
                const FlowRead rd = flow_read(k, j);
                if (rd.vec >= 0 && !wait_read(rd.vec, l + rd.dl, 0, len(rd.vec), tag, acc, rng)) return false;
            }
            for (int i = 0; i < s.H; ++i) normed[i] = mix(acc, i);
            return true;
        }
        // a block of rows: wait for and read every input vector whole, then write the block
        if (!(k == kFlowQkv && l == 0)) {
            for (int j = 0; j < kFlowMaxReads; ++j) {
                const FlowRead rd = flow_read(k, j);
                if (rd.vec >= 0 && !wait_read(rd.vec, l + rd.dl, 0, len(rd.vec), flow_tag(run, s.L, l + rd.dl), acc, rng))
                    return false;
            }
        } else {
            acc = mix(acc, static_cast<uint32_t>(token));  // the embedding row
        }
        int out = flow_write(k, 0), blk = t;
        if (k == kFlowQkv) {
            const int tq = (s.QD + rpt - 1) / rpt, tk = (s.KD + rpt - 1) / rpt;
            out = t < tq ? kVecQ : t < tq + tk ? kVecK : kVecV;
            blk = t < tq ? t : t < tq + tk ? t - tq : t - tq - tk;
            if (t == 0)  // the hidden state h_l
                for (int i = 0; i < s.H; ++i) write(kVecH0, l, i, mix(acc, 1000000 + i), tag);
        }
        for (int r = blk * rpt; r < std::min(len(out), (blk + 1) * rpt); ++r) write(out, l, r, mix(acc, r), tag);
        return true;
    }

    // The kernel's loop on one workgroup.
    void workgroup(int wg, uint32_t run, int pos, int token, unsigned seed) {
        std::mt19937 rng(seed);
        for (int l = 0; l < s.L; ++l)
            for (int k : {kFlowQkv, kFlowAttn, kFlowO, kFlowGateUp, kFlowDown})
                for (int i = 0;; ++i) {
                    const int t = flow_task(plan, k, wg, i);
                    if (t < 0) break;
                    if (rng() % 3 == 0) std::this_thread::sleep_for(std::chrono::microseconds(rng() % 100));
                    if (!task(k, l, t, run, pos, token, rng)) return;
                }
        if (flow_task(plan, kFlowNorm, wg, 0) == 0) task(kFlowNorm, s.L - 1, 0, run, pos, token, rng);
    }

    bool step(uint32_t run, int pos, int token, unsigned seed) {
        err = 0;
        std::vector<std::thread> th;
        for (int wg = 0; wg < wgs; ++wg) th.emplace_back([=] { workgroup(wg, run, pos, token, seed * 977 + wg); });
        for (auto &x : th) x.join();
        return err.load() == 0;
    }
};

void check(bool ok, const char *name, const char *what) {
    if (!ok) {
        std::printf("FAIL %s: %s\n", name, what);
        std::exit(1);
    }
}

}  // namespace

int main() {
    const Shape sh{3, 64, 64, 32, 96, 16, 4, 2};
    // the sequential run: one workgroup (every task in plan order, no waiting ever fails)
    Model ref(sh, 1);
    std::vector<std::vector<uint32_t>> want;
    for (int r = 0; r < 5; ++r) {
        check(ref.step(r + 1, r, 3 * r + 1, 1), "tokens", "the sequential run failed");
        want.push_back(ref.normed);
    }
    for (int wgs : {2, 3, 7, 16, 40}) {
        Model m(sh, wgs);
        for (int r = 0; r < 5; ++r) {
            check(m.step(r + 1, r, 3 * r + 1, 100 * wgs + r), "tokens", "a wait ran out");
            check(m.normed == want[r], "tokens", "a token's result differs from the sequential run");
        }
    }
    std::printf("ok tokens\n");

    Model t(sh, 8);
    t.limit = std::chrono::milliseconds(50);
    t.stall_wg = 0;
    t.stall_layer = 1;
    const auto t0 = std::chrono::steady_clock::now();
    check(!t.step(1, 0, 1, 5), "timeout", "the stalled step reported success");
    check(std::chrono::steady_clock::now() - t0 < std::chrono::seconds(5), "timeout", "the workgroups did not leave");
    std::printf("ok timeout\n");

    Model p(sh, 16);
    p.single_h = true;
    p.limit = std::chrono::milliseconds(300);
    bool failed = false;
    for (int r = 0; r < 5 && !failed; ++r) {
        failed = !p.step(r + 1, r, 3 * r + 1, 7 + r);
        check(failed || p.normed == want[r], "planted", "a wrong result instead of a wait that runs out");
    }
    check(failed, "planted", "the shared hidden-state buffer was not caught");
    std::printf("ok planted\n");
    std::printf("all ok\n");
    return 0;
}
