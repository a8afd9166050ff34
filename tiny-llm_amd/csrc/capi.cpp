// capi.cpp -- the C ABI declared in include/tqhip.h, and the "hip" registry variants.
//
// Host-pointer calls follow the reference's GPU-variant boundary
// (kernels/matvec/matvec_f16_cuda_resident_coal_ws.cu:88-159): weights are
// copied to HBM once and cached by host pointer + byte size, x/y go through a
// grow-only device workspace, and the call returns after y is back on the
// host. x and y are bounced through grow-only pinned host buffers: a copy from
// pageable memory is staged and synchronised inside the runtime, one from
// pinned memory is one DMA. One mutex guards the cache and workspaces, so
// concurrent callers (the reference's MoE expert pool calls mv from several
// threads) are serialised.

#include "../../include/tqhip.h"

#include <chrono>
#include <cstring>
#include <mutex>
#include <vector>
#include <unordered_map>

#include "dispatch.h"
#include "tq_common.h"

namespace tqhip {
namespace {

struct DeviceCopy {
    void *d = nullptr;
    size_t bytes = 0;
    uint64_t print = 0;
};

// Sampled content fingerprint (FNV-1a over up to 4 x 64 bytes). The cache is
// keyed by host pointer, as in the reference's CUDA variants; the fingerprint
// catches the common way that contract gets broken by accident: a freed
// weight buffer whose address is reused for a different tensor of the same
// size. It is not a full content check.
uint64_t fingerprint(const void *host, size_t bytes) {
    const unsigned char *p = static_cast<const unsigned char *>(host);
    uint64_t h = 0xCBF29CE484222325ull ^ bytes;
    const size_t n = bytes < 64 ? bytes : 64;
    const size_t offs[4] = {0, bytes / 3, (2 * bytes) / 3, bytes - n};
    for (size_t o : offs)
        for (size_t i = 0; i < n && o + i < bytes; ++i) {
            h ^= p[o + i];
            h *= 0x100000001B3ull;
        }
    return h;
}

struct HostBoundary {
    std::mutex mu;
    std::unordered_map<const void *, DeviceCopy> weights;
    float *dx = nullptr;
    size_t x_cap = 0;
    float *dy = nullptr;
    size_t y_cap = 0;
    float *hx = nullptr;  // pinned bounce buffers
    size_t hx_cap = 0;
    float *hy = nullptr;
    size_t hy_cap = 0;
    hipStream_t stream = nullptr;
    // Optional split of the last call (tqhip_host_timing): events around the copies and launches.
    bool timing = false;
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    float split_ms[3] = {0.f, 0.f, 0.f};

    hipStream_t get_stream() {
        if (!stream) TQ_HIP_CHECK(hipStreamCreate(&stream));  // default priority
        return stream;
    }
    const uint8_t *resident(const void *host, size_t bytes) {
        const uint64_t fp = fingerprint(host, bytes);
        auto it = weights.find(host);
        if (it != weights.end() && it->second.bytes == bytes && it->second.print == fp)
            return static_cast<const uint8_t *>(it->second.d);
        DeviceCopy &dc = weights[host];
        if (dc.d && dc.bytes != bytes) {
            TQ_HIP_CHECK(hipStreamSynchronize(get_stream()));
            TQ_HIP_CHECK(hipFree(dc.d));
            dc.d = nullptr;
        }
        if (!dc.d) TQ_HIP_CHECK(hipMalloc(&dc.d, bytes));
        TQ_HIP_CHECK(hipMemcpy(dc.d, host, bytes, hipMemcpyHostToDevice));
        dc.bytes = bytes;
        dc.print = fp;
        return static_cast<const uint8_t *>(dc.d);
    }
    float *ensure(float *&p, size_t &cap, size_t n) {
        if (n > cap) {
            if (p) {
                TQ_HIP_CHECK(hipStreamSynchronize(get_stream()));
                TQ_HIP_CHECK(hipFree(p));
            }
            p = nullptr;
            TQ_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&p), n * sizeof(float)));
            cap = n;
        }
        return p;
    }
    float *pinned(float *&p, size_t &cap, size_t n) {
        if (n > cap) {
            if (p) {
                TQ_HIP_CHECK(hipStreamSynchronize(get_stream()));
                TQ_HIP_CHECK(hipHostFree(p));
            }
            p = nullptr;
            TQ_HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&p), n * sizeof(float), hipHostMallocDefault));
            cap = n;
        }
        return p;
    }
    // Event i (0: before the upload, 1: after it, 2: after the launches, 3: after the download)
    // when timing is on.
    void mark(int i) {
        if (!timing) return;
        if (!ev[i]) TQ_HIP_CHECK(hipEventCreate(&ev[i]));
        TQ_HIP_CHECK(hipEventRecord(ev[i], get_stream()));
    }
    // After the call's synchronisation: the upload, kernel and download times of the call.
    void read_split() {
        if (!timing) return;
        for (int i = 0; i < 3; ++i) TQ_HIP_CHECK(hipEventElapsedTime(&split_ms[i], ev[i], ev[i + 1]));
    }
    // Completion words of the copy-out kernel (pinned, one per workgroup) and the call's number.
    int *done = nullptr;
    int seq = 0;
    static constexpr int kDoneWords = 4096;
    int *done_words() {
        if (!done) {
            TQ_HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&done), kDoneWords * sizeof(int), hipHostMallocDefault));
            for (int i = 0; i < kDoneWords; ++i) done[i] = 0;
        }
        return done;
    }
    void release() {
        for (auto &kv : weights)
            if (kv.second.d) TQ_HIP_CHECK(hipFree(kv.second.d));
        weights.clear();
    }
};

HostBoundary &boundary() {
    static HostBoundary b;
    return b;
}

void check_status(int st, const char *what) {
    if (st == kOk) return;
    const char *msg = st == kBadShape    ? "bad shape"
                      : st == kBadGroup  ? "bad group_size"
                      : st == kTooLarge  ? "shape too large"
                                         : "kernel launch failed";
    die(what, msg);
}

// x (n floats) into the device workspace through the pinned bounce buffer.
void upload(HostBoundary &hb, float *d, const float *h, size_t n, hipStream_t s) {
    float *p = hb.pinned(hb.hx, hb.hx_cap, n);
    std::memcpy(p, h, n * sizeof(float));
    hb.mark(0);
    TQ_HIP_CHECK(hipMemcpyAsync(d, p, n * sizeof(float), hipMemcpyHostToDevice, s));
    hb.mark(1);
}

// The outputs (pieces of the device workspace) back to the caller's arrays: the n floats at d
// into the pinned bounce buffer by the copy-out kernel, whose completion words the host reads
// (a device-to-host copy and a stream synchronisation took some 10 us more per call on MI355X),
// then one host copy per piece. A word that has not come within 200 ms hands over to a stream
// synchronisation, which reports a failed launch.
struct Piece {
    float *host;
    size_t off, n;
};
void download(HostBoundary &hb, const float *d, size_t n, const Piece *pieces, int np, hipStream_t s) {
    float *p = hb.pinned(hb.hy, hb.hy_cap, n);
    int *done = hb.done_words();
    const int seq = hb.seq = hb.seq == 0x7fffffff ? 1 : hb.seq + 1;
    int wgs = 0;
    hb.mark(2);
    const int st = launch_copy_to_host(d, p, n, done, HostBoundary::kDoneWords, seq, s, &wgs);
    if (st == kOk) {
        hb.mark(3);
        const auto t0 = std::chrono::steady_clock::now();
        bool all = false;
        for (unsigned k = 0; !all; ++k) {
            all = true;
            for (int b = 0; b < wgs && all; ++b) all = __atomic_load_n(done + b, __ATOMIC_ACQUIRE) == seq;
            if (!all && (k & 255) == 255 && std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(200))
                break;
        }
        if (!all || hb.timing) TQ_HIP_CHECK(hipStreamSynchronize(s));  // (the split's events have ended)
        if (!all)
            for (int b = 0; b < wgs; ++b)
                if (__atomic_load_n(done + b, __ATOMIC_ACQUIRE) != seq) die("tqhip: copy-out", "a completion word never came");
    } else {  // (more floats than the completion words cover) a copy and a synchronisation
        TQ_HIP_CHECK(hipMemcpyAsync(p, d, n * sizeof(float), hipMemcpyDeviceToHost, s));
        hb.mark(3);
        TQ_HIP_CHECK(hipStreamSynchronize(s));
    }
    hb.read_split();
    for (int i = 0; i < np; ++i) std::memcpy(pieces[i].host, p + pieces[i].off, pieces[i].n * sizeof(float));
}

}  // namespace
}  // namespace tqhip

using namespace tqhip;

extern "C" {

void tqhip_matvec_i4(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size) {
    if (out_dim < 1 || in_dim < 1 || group_size < 2 || (group_size & 1)) check_status(kBadShape, "tqhip_matvec_i4");
    HostBoundary &hb = boundary();
    std::lock_guard<std::mutex> lock(hb.mu);
    hipStream_t s = hb.get_stream();
    const uint8_t *dw = hb.resident(w, static_cast<size_t>(out_dim) * i4_row_bytes(in_dim, group_size));
    float *dx = hb.ensure(hb.dx, hb.x_cap, in_dim);
    float *dy = hb.ensure(hb.dy, hb.y_cap, out_dim);
    upload(hb, dx, x, in_dim, s);
    check_status(launch_i4_matvec(dw, dx, dy, out_dim, in_dim, group_size, s), "tqhip_matvec_i4");
    const Piece out[1] = {{y, 0, static_cast<size_t>(out_dim)}};
    download(hb, dy, out_dim, out, 1, s);
}

void tqhip_matvec_pair_i4(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2, int out_dim,
                          int in_dim, int group_size) {
    if (out_dim < 1 || in_dim < 1 || group_size < 2 || (group_size & 1))
        check_status(kBadShape, "tqhip_matvec_pair_i4");
    HostBoundary &hb = boundary();
    std::lock_guard<std::mutex> lock(hb.mu);
    hipStream_t s = hb.get_stream();
    const size_t wb = static_cast<size_t>(out_dim) * i4_row_bytes(in_dim, group_size);
    const uint8_t *d1 = hb.resident(w1, wb);
    const uint8_t *d2 = hb.resident(w2, wb);
    float *dx = hb.ensure(hb.dx, hb.x_cap, in_dim);
    float *dy = hb.ensure(hb.dy, hb.y_cap, 2 * static_cast<size_t>(out_dim));
    upload(hb, dx, x, in_dim, s);
    const uint8_t *ws[2] = {d1, d2};
    float *ys[2] = {dy, dy + out_dim};
    const int ms[2] = {out_dim, out_dim};
    check_status(launch_i4_matvec_group(2, ws, ys, ms, dx, in_dim, group_size, s), "tqhip_matvec_pair_i4");
    const size_t n = static_cast<size_t>(out_dim);
    const Piece out[2] = {{y1, 0, n}, {y2, n, n}};
    download(hb, dy, 2 * n, out, 2, s);
}

void tqhip_matvec_qkv_i4(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq,
                         float *yk, float *yv, int q_dim, int kv_dim, int in_dim, int group_size) {
    if (q_dim < 1 || kv_dim < 1 || in_dim < 1 || group_size < 2 || (group_size & 1))
        check_status(kBadShape, "tqhip_matvec_qkv_i4");
    HostBoundary &hb = boundary();
    std::lock_guard<std::mutex> lock(hb.mu);
    hipStream_t s = hb.get_stream();
    const size_t rb = i4_row_bytes(in_dim, group_size);
    const uint8_t *dq = hb.resident(wq, static_cast<size_t>(q_dim) * rb);
    const uint8_t *dk = hb.resident(wk, static_cast<size_t>(kv_dim) * rb);
    const uint8_t *dv = hb.resident(wv, static_cast<size_t>(kv_dim) * rb);
    float *dx = hb.ensure(hb.dx, hb.x_cap, in_dim);
    float *dy = hb.ensure(hb.dy, hb.y_cap, static_cast<size_t>(q_dim) + 2 * static_cast<size_t>(kv_dim));
    upload(hb, dx, x, in_dim, s);
    const uint8_t *ws[3] = {dq, dk, dv};
    float *ys[3] = {dy, dy + q_dim, dy + q_dim + kv_dim};
    const int ms[3] = {q_dim, kv_dim, kv_dim};
    check_status(launch_i4_matvec_group(3, ws, ys, ms, dx, in_dim, group_size, s), "tqhip_matvec_qkv_i4");
    const size_t nq = static_cast<size_t>(q_dim), nk = static_cast<size_t>(kv_dim);
    const Piece out[3] = {{yq, 0, nq}, {yk, nq, nk}, {yv, nq + nk, nk}};
    download(hb, dy, nq + 2 * nk, out, 3, s);
}

void tqhip_matvec_vq2(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim) {
    if (out_dim < 1 || in_dim < 4 || in_dim % 4) check_status(kBadShape, "tqhip_matvec_vq2");
    HostBoundary &hb = boundary();
    std::lock_guard<std::mutex> lock(hb.mu);
    hipStream_t s = hb.get_stream();
    const uint8_t *dw = hb.resident(w, vq2_bytes(out_dim, in_dim));
    float *dx = hb.ensure(hb.dx, hb.x_cap, in_dim);
    float *dy = hb.ensure(hb.dy, hb.y_cap, out_dim);
    upload(hb, dx, x, in_dim, s);
    check_status(launch_vq2_matvec(dw, dx, dy, out_dim, in_dim, s), "tqhip_matvec_vq2");
    const Piece out[1] = {{y, 0, static_cast<size_t>(out_dim)}};
    download(hb, dy, out_dim, out, 1, s);
}

void tqhip_matmul_i4(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size) {
    if (M < 1 || K < 1 || N < 1 || group_size < 2 || (group_size & 1)) check_status(kBadShape, "tqhip_matmul_i4");
    HostBoundary &hb = boundary();
    std::lock_guard<std::mutex> lock(hb.mu);
    hipStream_t s = hb.get_stream();
    const uint8_t *dw = hb.resident(w, static_cast<size_t>(M) * i4_row_bytes(K, group_size));
    float *dx = hb.ensure(hb.dx, hb.x_cap, static_cast<size_t>(K) * N);
    float *dy = hb.ensure(hb.dy, hb.y_cap, static_cast<size_t>(M) * N);
    upload(hb, dx, x, static_cast<size_t>(K) * N, s);
    check_status(launch_i4_matmul(dw, dx, dy, M, K, N, group_size, s), "tqhip_matmul_i4");
    const Piece out[1] = {{y, 0, static_cast<size_t>(M) * N}};
    download(hb, dy, static_cast<size_t>(M) * N, out, 1, s);
}

void tqhip_biip_rotate(const float *x, float *y, int dim, const float *scale, const float *sign, int block_size) {
    if (dim < 1 || block_size < 1 || (block_size & (block_size - 1)) || dim % block_size)
        check_status(kBadShape, "tqhip_biip_rotate");
    HostBoundary &hb = boundary();
    std::lock_guard<std::mutex> lock(hb.mu);
    hipStream_t s = hb.get_stream();
    // scale and sign are per-layer model constants: cached in HBM like weights
    const float *dscale =
        scale ? reinterpret_cast<const float *>(hb.resident(scale, static_cast<size_t>(dim) * sizeof(float))) : nullptr;
    const float *dsign = reinterpret_cast<const float *>(hb.resident(sign, static_cast<size_t>(dim) * sizeof(float)));
    float *dx = hb.ensure(hb.dx, hb.x_cap, dim);
    upload(hb, dx, x, dim, s);
    check_status(launch_biip_rotate(dx, dx, dim, dscale, dsign, block_size, s), "tqhip_biip_rotate");
    const Piece out[1] = {{y, 0, static_cast<size_t>(dim)}};
    download(hb, dx, dim, out, 1, s);
}

void tqhip_host_timing(int on) {
    HostBoundary &hb = boundary();
    std::lock_guard<std::mutex> lock(hb.mu);
    hb.timing = on != 0;
}

void tqhip_host_timing_last(float *upload_ms, float *kernel_ms, float *download_ms) {
    HostBoundary &hb = boundary();
    std::lock_guard<std::mutex> lock(hb.mu);
    if (upload_ms) *upload_ms = hb.split_ms[0];
    if (kernel_ms) *kernel_ms = hb.split_ms[1];
    if (download_ms) *download_ms = hb.split_ms[2];
}

void tqhip_release_weights(void) {
    HostBoundary &hb = boundary();
    std::lock_guard<std::mutex> lock(hb.mu);
    if (hb.stream) TQ_HIP_CHECK(hipStreamSynchronize(hb.stream));
    hb.release();
}

int tqhip_matvec_i4_dev(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                        void *stream) {
    return launch_i4_matvec(w, x, y, out_dim, in_dim, group_size, static_cast<hipStream_t>(stream));
}
int tqhip_matvec_pair_i4_dev(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2, int out_dim,
                             int in_dim, int group_size, void *stream) {
    const uint8_t *ws[2] = {w1, w2};
    float *ys[2] = {y1, y2};
    const int ms[2] = {out_dim, out_dim};
    return launch_i4_matvec_group(2, ws, ys, ms, x, in_dim, group_size, static_cast<hipStream_t>(stream));
}
int tqhip_matvec_qkv_i4_dev(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq,
                            float *yk, float *yv, int q_dim, int kv_dim, int in_dim, int group_size, void *stream) {
    const uint8_t *ws[3] = {wq, wk, wv};
    float *ys[3] = {yq, yk, yv};
    const int ms[3] = {q_dim, kv_dim, kv_dim};
    return launch_i4_matvec_group(3, ws, ys, ms, x, in_dim, group_size, static_cast<hipStream_t>(stream));
}
int tqhip_matvec_i4_generic_dev(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                                void *stream) {
    return launch_i4_matvec_generic(w, x, y, out_dim, in_dim, group_size, static_cast<hipStream_t>(stream));
}
int tqhip_dequant_i4_rows_dev(const uint8_t *embed, const int *rows, int n, int dim, int group_size, float *out,
                              void *stream) {
    return launch_i4_embed_rows(embed, rows, n, dim, group_size, out, static_cast<hipStream_t>(stream));
}
int tqhip_biip_rotate_dev(const float *x, float *y, int dim, const float *scale, const float *sign, int block_size,
                          void *stream) {
    return launch_biip_rotate(x, y, dim, scale, sign, block_size, static_cast<hipStream_t>(stream));
}
int tqhip_matvec_vq2_dev(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, void *stream) {
    return launch_vq2_matvec(w, x, y, out_dim, in_dim, static_cast<hipStream_t>(stream));
}
int tqhip_matmul_i4_dev(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                        void *stream) {
    return launch_i4_matmul(w, x, y, M, K, N, group_size, static_cast<hipStream_t>(stream));
}
int tqhip_matvec_i4_set_dev(const tqhip_i4_mat *mats, int n, int group_size, void *stream) {
    return launch_i4_matvec_set(n, reinterpret_cast<const I4Mat *>(mats), group_size, static_cast<hipStream_t>(stream));
}
int tqhip_matvec_vq2_set_dev(const tqhip_i4_mat *mats, int n, void *stream) {
    return launch_vq2_matvec_set(n, reinterpret_cast<const I4Mat *>(mats), static_cast<hipStream_t>(stream));
}
int tqhip_matmul_i4_noalloc_dev(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                                void *stream) {
    static_assert(TQHIP_NOALLOC_SCRATCH_BYTES == kNoAllocScratchBytes, "header and library agree on the size");
    return launch_i4_matmul_noalloc(w, x, y, M, K, N, group_size, static_cast<hipStream_t>(stream));
}

int tqhip_set_matvec_i4_impl_by_name(const char *name) { return tinyqwen::set_matvec_i4_impl_by_name(name) ? 1 : 0; }
const char *tqhip_matvec_i4_impl_name(void) { return tinyqwen::matvec_i4_impl_name(); }
const char *tqhip_available_matvec_i4_impls(void) { return tinyqwen::available_matvec_i4_impls(); }
int tqhip_set_matvec_vq2_impl_by_name(const char *name) {
    return tinyqwen::set_matvec_vq2_impl_by_name(name) ? 1 : 0;
}
const char *tqhip_matvec_vq2_impl_name(void) { return tinyqwen::matvec_vq2_impl_name(); }
const char *tqhip_available_matvec_vq2_impls(void) { return tinyqwen::available_matvec_vq2_impls(); }
int tqhip_set_matmul_i4_impl_by_name(const char *name) { return tinyqwen::set_matmul_i4_impl_by_name(name) ? 1 : 0; }
int tqhip_set_ops_impl_by_name(const char *name) { return tinyqwen::set_ops_impl_by_name(name) ? 1 : 0; }
const char *tqhip_ops_impl_name(void) { return tinyqwen::ops_impl_name(); }
void tqhip_biip_rotate_activation(const float *x, float *y, int dim, const float *scale, const float *sign,
                                  int block_size) {
    tinyqwen::biip_rotate_activation(x, y, dim, scale, sign, block_size);
}
void tqhip_dispatch_matvec_i4(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size) {
    tinyqwen::matvec_i4(w, x, y, out_dim, in_dim, group_size);
}
void tqhip_dispatch_matvec_pair_i4(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2,
                                   int out_dim, int in_dim, int group_size) {
    tinyqwen::matvec_pair_i4(w1, w2, x, y1, y2, out_dim, in_dim, group_size);
}
void tqhip_dispatch_matvec_qkv_i4(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq,
                                  float *yk, float *yv, int q_dim, int kv_dim, int in_dim, int group_size) {
    tinyqwen::matvec_qkv_i4(wq, wk, wv, x, yq, yk, yv, q_dim, kv_dim, in_dim, group_size);
}
void tqhip_dispatch_matvec_vq2(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim) {
    tinyqwen::matvec_vq2(w, x, y, out_dim, in_dim);
}
void tqhip_dispatch_matmul_i4(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size) {
    tinyqwen::matmul_i4(w, x, y, M, K, N, group_size);
}
void tqhip_dispatch_matmul_vq2(const uint8_t *w, const float *x, float *y, int M, int K, int N) {
    tinyqwen::matmul_vq2(w, x, y, M, K, N);
}

size_t tqhip_i4_row_bytes(int in_dim, int group_size) { return i4_row_bytes(in_dim, group_size); }
size_t tqhip_vq2_tensor_bytes(int rows, int cols) { return vq2_bytes(rows, cols); }

int tqhip_device_count(void) {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess ? n : 0;
}
int tqhip_device_name(char *buf, int len) {
    hipDeviceProp_t p;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) return -1;
    std::snprintf(buf, static_cast<size_t>(len), "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return 0;
}
void *tqhip_malloc(size_t bytes) {
    void *p = nullptr;
    return hipMalloc(&p, bytes) == hipSuccess ? p : nullptr;
}
int tqhip_free(void *p) { return hipFree(p) == hipSuccess ? 0 : -1; }
int tqhip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    return hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) == hipSuccess ? 0 : -1;
}
int tqhip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    return hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
int tqhip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    return hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice) == hipSuccess ? 0 : -1;
}
int tqhip_memset(void *dst, int value, size_t bytes) { return hipMemset(dst, value, bytes) == hipSuccess ? 0 : -1; }
int tqhip_synchronize(void) { return hipDeviceSynchronize() == hipSuccess ? 0 : -1; }
void *tqhip_stream_create(void) {
    hipStream_t s = nullptr;
    return hipStreamCreate(&s) == hipSuccess ? static_cast<void *>(s) : nullptr;
}
int tqhip_stream_destroy(void *stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (hipStreamSynchronize(s) != hipSuccess) return -1;
    scratch_forget_stream(s);  // its scratch, unless a graph recorded it
    return hipStreamDestroy(s) == hipSuccess ? 0 : -1;
}
int tqhip_stream_synchronize(void *stream) {
    return hipStreamSynchronize(static_cast<hipStream_t>(stream)) == hipSuccess ? 0 : -1;
}
void *tqhip_event_create(void) {
    hipEvent_t e = nullptr;
    return hipEventCreate(&e) == hipSuccess ? static_cast<void *>(e) : nullptr;
}
int tqhip_event_destroy(void *event) { return hipEventDestroy(static_cast<hipEvent_t>(event)) == hipSuccess ? 0 : -1; }
int tqhip_event_record(void *event, void *stream) {
    return hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)) == hipSuccess ? 0 : -1;
}
int tqhip_event_elapsed_ms(void *start, void *stop, float *ms) {
    if (hipEventSynchronize(static_cast<hipEvent_t>(stop)) != hipSuccess) return -1;
    return hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)) == hipSuccess ? 0
                                                                                                                 : -1;
}

static int launch_op(const tqhip_op &op, hipStream_t s) {
    const uint8_t *w = static_cast<const uint8_t *>(op.w);
    switch (op.kind) {
        case TQHIP_OP_I4_MATVEC: return launch_i4_matvec(w, op.x, op.y, op.out_dim, op.in_dim, op.group_size, s);
        case TQHIP_OP_I4_PAIR:
        case TQHIP_OP_I4_QKV: {
            const int n = op.kind == TQHIP_OP_I4_PAIR ? 2 : 3;
            const uint8_t *ws[3] = {w, static_cast<const uint8_t *>(op.w2), static_cast<const uint8_t *>(op.w3)};
            float *ys[3] = {op.y, op.y2, op.y3};
            const int ms[3] = {op.out_dim, op.kind == TQHIP_OP_I4_PAIR ? op.out_dim : op.out_dim2, op.out_dim2};
            return launch_i4_matvec_group(n, ws, ys, ms, op.x, op.in_dim, op.group_size, s);
        }
        case TQHIP_OP_VQ2_MATVEC: return launch_vq2_matvec(w, op.x, op.y, op.out_dim, op.in_dim, s);
        case TQHIP_OP_I4_MATMUL: return launch_i4_matmul(w, op.x, op.y, op.out_dim, op.in_dim, op.n, op.group_size, s);
        case TQHIP_OP_I4_SET:
            return launch_i4_matvec_set(op.n, static_cast<const I4Mat *>(op.w), op.group_size, s);
        case TQHIP_OP_VQ2_SET: return launch_vq2_matvec_set(op.n, static_cast<const I4Mat *>(op.w), s);
        case TQHIP_OP_BIIP_ROTATE:
            return launch_biip_rotate(op.x, op.y, op.in_dim, static_cast<const float *>(op.w2),
                                      static_cast<const float *>(op.w3), op.group_size, s);
        default: return kBadShape;
    }
}

int tqhip_run_ops(const tqhip_op *ops, int n_ops, int repeats, void *stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int r = 0; r < repeats; ++r) {
        for (int i = 0; i < n_ops; ++i) {
            const int st = launch_op(ops[i], s);
            if (st != kOk) return st;
        }
    }
    return kOk;
}

int tqhip_run_ops_timed(const tqhip_op *ops, int n_ops, int repeats, void *stream, float *op_ms) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n_ops < 1 || repeats < 1) return kBadShape;
    std::vector<hipEvent_t> ev(2 * static_cast<size_t>(n_ops));
    for (auto &e : ev)
        if (hipEventCreate(&e) != hipSuccess) return kLaunchFailed;
    for (int i = 0; i < n_ops; ++i) op_ms[i] = 0.f;
    int st = kOk;
    for (int r = 0; r < repeats && st == kOk; ++r) {
        for (int i = 0; i < n_ops && st == kOk; ++i) {
            if (hipEventRecord(ev[2 * i], s) != hipSuccess) st = kLaunchFailed;
            if (st == kOk) st = launch_op(ops[i], s);
            if (st == kOk && hipEventRecord(ev[2 * i + 1], s) != hipSuccess) st = kLaunchFailed;
        }
        if (st == kOk && hipEventSynchronize(ev.back()) != hipSuccess) st = kLaunchFailed;
        for (int i = 0; i < n_ops && st == kOk; ++i) {
            float ms = 0.f;
            if (hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]) != hipSuccess) st = kLaunchFailed;
            op_ms[i] += ms / repeats;
        }
    }
    for (auto &e : ev) (void)hipEventDestroy(e);
    return st;
}

// An op list captured once into a HIP graph and replayed: a device-resident
// decode loop issues the same calls every token with the same buffers, and a
// replay costs the GPU about 1.6 us per kernel instead of about 2.8 us for
// separate launches (measured on MI355X).
// The graph owns its scratch (split-K slots, prefill X copy): the eager sizing
// pass and the capture run inside a ScratchScope of that set, so no later call
// on any stream can grow, free or share what the replays use.
struct tqhip_ops_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    ScratchSet *scratch = nullptr;
};

int tqhip_ops_graph_create(const tqhip_op *ops, int n_ops, void *stream, void **graph_out) {
    if (!graph_out || n_ops < 1 || !stream) return kBadShape;  // (the null stream cannot be captured)
    *graph_out = nullptr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    ScratchSet *scratch = scratch_set_new();
    hipGraph_t g = nullptr;
    int st = kOk;
    {
        ScratchScope scope(scratch);
        // One eager pass first: it sizes the graph's scratch and sets kernel
        // attributes, neither of which may happen inside a capture.
        st = tqhip_run_ops(ops, n_ops, 1, stream);
        if (st == kOk && hipStreamSynchronize(s) != hipSuccess) st = kLaunchFailed;
        if (st == kOk && hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) st = kLaunchFailed;
        if (st == kOk) {
            for (int i = 0; i < n_ops && st == kOk; ++i) st = launch_op(ops[i], s);
            const hipError_t end = hipStreamEndCapture(s, &g);
            if (st == kOk && end != hipSuccess) st = kLaunchFailed;
        }
    }
    hipGraphExec_t exec = nullptr;
    if (st == kOk && hipGraphInstantiate(&exec, g, nullptr, nullptr, 0) != hipSuccess) st = kLaunchFailed;
    if (st != kOk) {
        if (g) (void)hipGraphDestroy(g);
        (void)hipStreamSynchronize(s);
        scratch_set_free(scratch);
        return st;
    }
    auto *h = new tqhip_ops_graph;
    h->graph = g;
    h->exec = exec;
    h->scratch = scratch;
    *graph_out = h;
    return kOk;
}

int tqhip_ops_graph_launch(void *graph, void *stream) {
    if (!graph || !stream) return kBadShape;
    auto *h = static_cast<tqhip_ops_graph *>(graph);
    return hipGraphLaunch(h->exec, static_cast<hipStream_t>(stream)) == hipSuccess ? kOk : kLaunchFailed;
}

int tqhip_ops_graph_destroy(void *graph) {
    if (!graph) return kOk;
    auto *h = static_cast<tqhip_ops_graph *>(graph);
    int st = kOk;
    if (h->exec && hipGraphExecDestroy(h->exec) != hipSuccess) st = kLaunchFailed;
    if (h->graph && hipGraphDestroy(h->graph) != hipSuccess) st = kLaunchFailed;
    // replays may still be running on any stream: wait for the device before
    // the scratch they use goes back
    if (hipDeviceSynchronize() != hipSuccess) st = kLaunchFailed;
    scratch_set_free(h->scratch);
    delete h;
    return st;
}

}  // extern "C"

static_assert(sizeof(tqhip_i4_mat) == sizeof(I4Mat) && offsetof(tqhip_i4_mat, w) == offsetof(I4Mat, w) &&
                  offsetof(tqhip_i4_mat, x) == offsetof(I4Mat, x) && offsetof(tqhip_i4_mat, y) == offsetof(I4Mat, y) &&
                  offsetof(tqhip_i4_mat, out_dim) == offsetof(I4Mat, M) &&
                  offsetof(tqhip_i4_mat, in_dim) == offsetof(I4Mat, K),
              "tqhip_i4_mat is the library's I4Mat");

// Self-registration as the "hip" variants (kernels/dispatch.h:459-474 idiom).
TINYQWEN_MATVEC_I4_VARIANT(tqhip_matvec_i4, "hip");
TINYQWEN_MATVEC_I4_PAIR_VARIANT(tqhip_matvec_pair_i4, "hip");
TINYQWEN_MATVEC_QKV_I4_VARIANT(tqhip_matvec_qkv_i4, "hip");
TINYQWEN_MATVEC_VQ2_VARIANT(tqhip_matvec_vq2, "hip");
TINYQWEN_MATMUL_I4_VARIANT(tqhip_matmul_i4, "hip");
TINYQWEN_BIIP_ROTATE_VARIANT(tqhip_biip_rotate, "hip");
