// scratch_harness.cpp -- host-side bookkeeping test of tiny-llm_amd/csrc/scratch.cpp.
//
// scratch.cpp is compiled with g++ and linked against this file, which defines
// the six HIP runtime calls it makes (hipGetDevice, hipStreamIsCapturing,
// hipStreamSynchronize, hipMalloc, hipMemsetAsync, hipFree) as recording mocks.
// No GPU and no HIP runtime are involved. Each check prints "ok <name>"; the
// first failure prints "FAIL <name>: <detail>" and exits 1.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>
#include <vector>

#include "tq_common.h"

namespace {

int g_dev = 0;
std::set<hipStream_t> g_capturing;
std::set<void *> g_live;
std::vector<void *> g_freed;
int g_mallocs = 0, g_syncs = 0, g_memsets = 0;
bool g_fail_malloc = false;
char g_arena[1 << 12];  // stands in for a fixed set's preset buffer

void check(bool ok, const char *name, const char *detail) {
    if (!ok) {
        std::printf("FAIL %s: %s\n", name, detail);
        std::exit(1);
    }
}

hipStream_t stream(int i) { return reinterpret_cast<hipStream_t>(static_cast<uintptr_t>(0x1000 * i)); }

}  // namespace

extern "C" {
hipError_t hipGetDevice(int *d) {
    *d = g_dev;
    return hipSuccess;
}
hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus *st) {
    *st = g_capturing.count(s) ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) {
    ++g_syncs;
    return hipSuccess;
}
hipError_t hipMalloc(void **p, size_t n) {
    if (g_fail_malloc) return hipErrorOutOfMemory;
    ++g_mallocs;
    *p = std::malloc(n);
    g_live.insert(*p);
    return hipSuccess;
}
hipError_t hipMemsetAsync(void *p, int v, size_t n, hipStream_t) {
    ++g_memsets;
    std::memset(p, v, n);
    return hipSuccess;
}
hipError_t hipFree(void *p) {
    if (!g_live.erase(p)) {
        std::printf("FAIL hipFree: pointer %p not live (double free or foreign)\n", p);
        std::exit(1);
    }
    g_freed.push_back(p);
    std::free(p);
    return hipSuccess;
}
}

using namespace tqhip;

int main() {
    unsigned long long *a = nullptr, *b = nullptr;
    void *x = nullptr, *x2 = nullptr;

    // 1. first request on stream 1 allocates and zero-fills the split slots
    check(scratch_split_slots(stream(1), 100, &a) == kOk && a, "eager_alloc", "request failed");
    check(g_mallocs == 1 && g_memsets == 1, "eager_alloc", "expected one hipMalloc and one zero fill");
    for (int i = 0; i < 100; ++i) check(a[i] == 0, "eager_alloc", "slots not zero");
    std::printf("ok eager_alloc\n");

    // 2. a request within capacity reuses the buffer
    check(scratch_split_slots(stream(1), 50, &b) == kOk && b == a && g_mallocs == 1, "reuse", "reallocated");
    std::printf("ok reuse\n");

    // 3. another stream never shares the buffer
    check(scratch_split_slots(stream(2), 50, &b) == kOk && b != a && g_mallocs == 2, "per_stream", "shared");
    std::printf("ok per_stream\n");

    // 4. under capture: a fitting request is served and marks the buffer captured ...
    g_capturing.insert(stream(1));
    check(scratch_split_slots(stream(1), 100, &b) == kOk && b == a, "capture_fit", "not served");
    check(scratch_stats(stream(1)).split_captured == 1, "capture_fit", "not marked captured");
    std::printf("ok capture_fit\n");
    // ... and a growing one fails without allocating or synchronising
    const int m0 = g_mallocs, s0 = g_syncs;
    check(scratch_split_slots(stream(1), 1 << 20, &b) == kHipFailed, "capture_grow", "growth under capture served");
    check(g_mallocs == m0 && g_syncs == s0, "capture_grow", "allocated or synchronised under capture");
    check(scratch_prefill(stream(1), 1 << 22, &x) == kHipFailed, "capture_grow", "prefill growth under capture");
    std::printf("ok capture_grow\n");
    g_capturing.erase(stream(1));

    // 5. growth after the capture: the stream is synchronised and the captured
    //    buffer retired, not freed (the graph may still replay it)
    check(scratch_split_slots(stream(1), 1 << 20, &b) == kOk && b != a, "retire", "no new buffer");
    check(g_syncs == s0 + 1, "retire", "stream not synchronised before the swap");
    check(g_live.count(a) == 1, "retire", "captured buffer was freed");
    check(scratch_stats(stream(1)).retired == 1 && scratch_stats(stream(1)).split_captured == 0, "retire",
          "bookkeeping");
    std::printf("ok retire\n");

    // 6. growth of a never-captured buffer frees the old one after synchronising
    check(scratch_prefill(stream(3), 1000, &x) == kOk, "free_on_grow", "first");
    check(scratch_prefill(stream(3), 8 << 20, &x2) == kOk && x2 != x, "free_on_grow", "second");
    check(g_live.count(x) == 0 && !g_freed.empty() && g_freed.back() == x, "free_on_grow", "old buffer not freed");
    std::printf("ok free_on_grow\n");

    // 7. inside a scope every request goes to the scope's set, whatever the stream
    ScratchSet *own = scratch_set_new();
    {
        ScratchScope scope(own);
        check(scratch_prefill(stream(3), 1000, &x) == kOk && x != x2, "scope", "served from the stream's set");
        void *x3 = nullptr;
        check(scratch_prefill(stream(4), 1000, &x3) == kOk && x3 == x, "scope", "another stream left the scope");
        check(scratch_stats(stream(9)).prefill_bytes >= 1000, "scope", "stats do not show the scope's set");
        {  // nested scopes restore the outer one
            ScratchSet *inner = scratch_set_new();
            ScratchScope s2(inner);
            check(scratch_stats(stream(3)).prefill_bytes == 0, "scope", "inner scope not selected");
            scratch_set_free(inner);
        }
        check(scratch_stats(stream(3)).prefill_bytes >= 1000, "scope", "outer scope not restored");
    }
    check(scratch_stats(stream(3)).prefill_bytes >= (8u << 20), "scope", "stream set changed by the scope");
    const size_t live_before = g_live.size();
    scratch_set_free(own);
    check(g_live.size() == live_before - 1, "scope", "owned set not freed");
    std::printf("ok scope\n");

    // 8. a fixed set never allocates: beyond its preset buffer the answer is kTooLarge
    ScratchSet *fixed = scratch_set_fixed(g_arena, sizeof g_arena);
    {
        ScratchScope scope(fixed);
        const int m1 = g_mallocs;
        check(scratch_prefill(stream(1), 100, &x) == kOk && x == g_arena, "fixed", "preset buffer not used");
        check(scratch_prefill(stream(1), sizeof g_arena + 1, &x) == kTooLarge, "fixed", "grew");
        check(scratch_split_slots(stream(1), 1, &b) == kTooLarge, "fixed", "split slots served");
        check(g_mallocs == m1, "fixed", "allocated");
    }
    scratch_set_free(fixed);  // must not free the preset buffer (a hipFree of it would fail above)
    std::printf("ok fixed\n");

    // 9. a failed allocation is an error code, not an abort, and leaves no buffer behind
    g_fail_malloc = true;
    check(scratch_prefill(stream(5), 1000, &x) == kHipFailed, "alloc_failure", "not reported");
    g_fail_malloc = false;
    check(scratch_prefill(stream(5), 1000, &x) == kOk, "alloc_failure", "no recovery");
    std::printf("ok alloc_failure\n");

    // 10. forgetting a stream frees its buffers and its set, unless a graph recorded a buffer
    const size_t l0 = g_live.size();
    const long n0 = scratch_live_sets();
    scratch_forget_stream(stream(5));
    check(g_live.size() == l0 - 1, "forget", "buffer of a destroyed stream kept");
    check(scratch_live_sets() == n0 - 1, "forget", "set of a destroyed stream kept");
    scratch_forget_stream(stream(1));  // holds a retired, captured buffer: everything stays
    check(g_live.size() == l0 - 1 && g_live.count(a) == 1, "forget", "a captured buffer was freed");
    check(scratch_live_sets() == n0 - 1, "forget", "the set of a captured buffer was deleted");
    scratch_forget_stream(stream(5));  // forgotten twice: nothing left to do
    check(scratch_live_sets() == n0 - 1, "forget", "second forget changed the sets");
    {  // a stream used, forgotten, and used again gets a fresh set
        void *y = nullptr;
        check(scratch_prefill(stream(6), 10, &y) == kOk, "forget", "alloc");
        check(scratch_live_sets() == n0, "forget", "no set for a new stream");
        scratch_forget_stream(stream(6));
        check(scratch_live_sets() == n0 - 1 && g_live.count(y) == 0, "forget", "set or buffer kept");
        check(scratch_prefill(stream(6), 10, &y) == kOk && scratch_live_sets() == n0, "forget", "reuse after forget");
        scratch_forget_stream(stream(6));
    }
    std::printf("ok forget\n");

    // 11. devices are separate: the same stream handle on device 1 gets its own set
    g_dev = 1;
    check(scratch_stats(stream(3)).prefill_bytes == 0, "per_device", "device 1 sees device 0's set");
    g_dev = 0;
    std::printf("ok per_device\n");
    std::printf("all ok\n");
    return 0;
}
