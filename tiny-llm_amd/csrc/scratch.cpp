// scratch.cpp -- device scratch of the launches: the split-K exchange slots of
// the matvec and the tile arrival counters of the few-token prefill kernel (all
// zero between launches), and the prefill workspace (the fp16 copy of X of the
// prefill GEMM, or the few-token kernel's partial products).
//
// Who owns which buffer:
//   * Eager calls use the set of their (device, stream): launches on one stream
//     are ordered, launches on different streams never share a buffer.
//   * A graph (tqhip_ops_graph_create) or a decode engine owns a set of its
//     own. Its eager sizing pass and its capture run inside a ScratchScope, so
//     every launch captured into the graph names the owner's buffers, which
//     live exactly as long as the owner. Nothing an eager call does later
//     (growth, another stream) can touch them.
//   * Growth never happens under stream capture: a capture that would need a
//     larger buffer gets kHipFailed. A per-stream buffer that a foreign capture
//     (the caller's own hipStreamBeginCapture around a _dev call) has recorded
//     is marked and, when the stream later needs a larger one, retired instead
//     of freed: that graph may still be replayed.
//   * A fixed set (the allocation-free entry point) has preset buffers and can
//     not grow: a request beyond them is kTooLarge, which the launchers treat as
//     "this kernel does not fit" (split-K falls back to a non-split kernel).
#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "tq_common.h"

namespace tqhip {

struct ScratchBuf {
    void *p = nullptr;
    size_t cap = 0;
    bool captured = false;  // recorded into a graph: retire on growth, never free
};

namespace {
std::atomic<long> g_live_sets{0};
}  // namespace

struct ScratchSet {
    ScratchSet() { ++g_live_sets; }
    ~ScratchSet() { --g_live_sets; }
    ScratchSet(const ScratchSet &) = delete;
    ScratchSet &operator=(const ScratchSet &) = delete;
    std::mutex mu;
    ScratchBuf split;  // split-K exchange slots / arrival counters: zero between launches
    ScratchBuf xws;    // prefill workspace
    std::vector<void *> retired;
    bool fixed = false;  // preset buffers, no growth (allocation-free entry point)
};

namespace {

thread_local ScratchSet *t_scope = nullptr;

std::mutex g_streams_mu;
std::map<std::pair<int, hipStream_t>, ScratchSet *> g_streams;

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

ScratchSet *set_for(hipStream_t s) {
    if (t_scope) return t_scope;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_streams_mu);
    ScratchSet *&set = g_streams[{dev, s}];
    if (!set) set = new ScratchSet;
    return set;
}

void release_buf(ScratchSet &set, ScratchBuf &b) {
    if (b.p) {
        if (b.captured)
            set.retired.push_back(b.p);
        else
            (void)hipFree(b.p);
    }
    b = ScratchBuf{};
}

// b grown to at least `need` bytes (zero-filled when `zero`), for launches on s.
int grow(ScratchSet &set, ScratchBuf &b, size_t need, size_t floor_bytes, bool zero, hipStream_t s, void **out) {
    const bool cap = capturing(s);
    if (b.cap >= need) {
        if (cap) b.captured = true;
        *out = b.p;
        return kOk;
    }
    if (set.fixed) return kTooLarge;
    if (cap) return kHipFailed;  // no allocation inside a capture
    if (b.p && hipStreamSynchronize(s) != hipSuccess) return kHipFailed;  // earlier launches may still use it
    const size_t n = std::max({need, floor_bytes, (b.cap * 3) / 2});
    release_buf(set, b);
    void *p = nullptr;
    if (hipMalloc(&p, n) != hipSuccess) return kHipFailed;
    if (zero && hipMemsetAsync(p, 0, n, s) != hipSuccess) {
        (void)hipFree(p);
        return kHipFailed;
    }
    b.p = p;
    b.cap = n;
    *out = p;
    return kOk;
}

}  // namespace

int scratch_split_slots(hipStream_t s, size_t nslots, unsigned long long **slots) {
    ScratchSet *set = set_for(s);
    if (!set) return kHipFailed;
    std::lock_guard<std::mutex> lock(set->mu);
    void *p = nullptr;
    const int st = grow(*set, set->split, nslots * sizeof(unsigned long long), (size_t{1} << 14) * 8, true, s, &p);
    *slots = static_cast<unsigned long long *>(p);
    return st;
}

int scratch_prefill(hipStream_t s, size_t bytes, void **ws) {
    ScratchSet *set = set_for(s);
    if (!set) return kHipFailed;
    std::lock_guard<std::mutex> lock(set->mu);
    return grow(*set, set->xws, bytes, size_t{1} << 20, false, s, ws);
}

ScratchSet *scratch_set_new() { return new ScratchSet; }

ScratchSet *scratch_set_fixed(void *xws, size_t xws_bytes) {
    ScratchSet *set = new ScratchSet;
    set->fixed = true;
    set->xws.p = xws;
    set->xws.cap = xws_bytes;
    return set;
}

void scratch_set_free(ScratchSet *set) {
    if (!set) return;
    if (!set->fixed) {
        if (set->split.p) (void)hipFree(set->split.p);
        if (set->xws.p) (void)hipFree(set->xws.p);
        for (void *p : set->retired) (void)hipFree(p);
    }
    delete set;
}

ScratchScope::ScratchScope(ScratchSet *set) : prev_(t_scope) { t_scope = set; }
ScratchScope::~ScratchScope() { t_scope = prev_; }

void scratch_forget_stream(hipStream_t s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return;
    ScratchSet *set = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_streams_mu);
        auto it = g_streams.find({dev, s});
        if (it == g_streams.end()) return;
        set = it->second;
        g_streams.erase(it);
    }
    // Buffers a foreign graph recorded stay allocated (that graph may outlive the stream), and
    // so does their set. Otherwise the buffers and the set go: the stream is being destroyed,
    // so no other thread may still launch on it (the caller's contract, as for the stream).
    {
        std::lock_guard<std::mutex> lock(set->mu);
        if (set->split.captured || set->xws.captured || !set->retired.empty()) return;  // leaked on purpose
        if (set->split.p) (void)hipFree(set->split.p);
        if (set->xws.p) (void)hipFree(set->xws.p);
        set->split = ScratchBuf{};
        set->xws = ScratchBuf{};
    }
    delete set;
}

long scratch_live_sets() { return g_live_sets.load(); }

ScratchStats scratch_stats(hipStream_t s) {
    ScratchStats st{};
    ScratchSet *set = nullptr;
    if (t_scope) {
        set = t_scope;
    } else {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return st;
        std::lock_guard<std::mutex> lock(g_streams_mu);
        auto it = g_streams.find({dev, s});
        if (it == g_streams.end()) return st;
        set = it->second;
    }
    std::lock_guard<std::mutex> lock(set->mu);
    st.split_bytes = set->split.cap;
    st.prefill_bytes = set->xws.cap;
    st.split_captured = set->split.captured ? 1 : 0;
    st.prefill_captured = set->xws.captured ? 1 : 0;
    st.retired = static_cast<int>(set->retired.size());
    return st;
}

}  // namespace tqhip
