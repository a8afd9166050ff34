// host_copy.hip -- device results into pinned host memory, with completion words the host polls.
//
// A host-pointer call (capi.cpp) used to end with a device-to-host copy and a stream
// synchronisation; the host learnt of the result only after the copy's launch had ended and the
// runtime had seen it end. Here the copy is a kernel: workgroup b stores its slice of the floats
// into the pinned buffer, waits until its stores have completed, and then stores `seq` to its
// completion word at system scope. The host reads the words until every one holds this call's
// `seq` and then reads the buffer. (Every store of a workgroup precedes its completion word on the
// same path to host memory, and the host reads the buffer only after the last word.)

#include "tq_common.h"

namespace tqhip {
namespace {

constexpr int kCopyThreads = 256;

__global__ __launch_bounds__(kCopyThreads) void copy_to_host(const float *__restrict__ d, float *h, int n, int per_wg,
                                                             int *done, int seq) {
    const int b0 = blockIdx.x * per_wg, b1 = min(n, b0 + per_wg);
    for (int i = b0 + static_cast<int>(threadIdx.x); i < b1; i += kCopyThreads)
        __hip_atomic_store(h + i, d[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
    __syncthreads();                // and every other thread's
    if (threadIdx.x == 0) __hip_atomic_store(done + blockIdx.x, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace

int launch_copy_to_host(const float *d, float *h, size_t n, int *done, int max_wgs, int seq, hipStream_t stream,
                        int *wgs) {
    if (!d || !h || !done || n < 1 || n > (1u << 30) || max_wgs < 1) return kBadShape;
    constexpr int kPerWg = 8192;  // floats per workgroup
    const int nw = static_cast<int>((n + kPerWg - 1) / kPerWg);
    if (nw > max_wgs) return kTooLarge;
    hipLaunchKernelGGL(copy_to_host, dim3(nw), dim3(kCopyThreads), 0, stream, d, h, static_cast<int>(n), kPerWg, done,
                       seq);
    *wgs = nw;
    return hipGetLastError() == hipSuccess ? kOk : kLaunchFailed;
}

}  // namespace tqhip
