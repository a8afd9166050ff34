// tq_common.h -- shared definitions for the MI355X quantized-projection library.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include <hip/hip_runtime.h>

namespace tqhip {

// i4 group layout (runtime/tiny_format.h:58-78 of the reference):
//   [scale fp16 | zero fp16 | group_size/2 bytes of codes], low nibble = even element.
constexpr int kI4Header = 4;

// VQ2 layout (runtime/tiny_format.h:80-103): [codebook 256 x 4 fp16][rows x cols/4 u8].
constexpr int kVq2Dim = 4;
constexpr int kVq2Entries = 256;
constexpr int kVq2CodebookBytes = kVq2Entries * kVq2Dim * 2;

inline int i4_group_bytes(int group_size) { return kI4Header + group_size / 2; }
inline int i4_groups(int in_dim, int group_size) { return (in_dim + group_size - 1) / group_size; }
inline size_t i4_row_bytes(int in_dim, int group_size) {
    return static_cast<size_t>(i4_groups(in_dim, group_size)) * i4_group_bytes(group_size);
}
inline size_t vq2_bytes(int rows, int cols) {
    return kVq2CodebookBytes + static_cast<size_t>(rows) * (static_cast<size_t>(cols) / kVq2Dim);
}

// Fail fast, as the reference's GPU variants do (TINYQWEN_CUDA_CHECK +
// abort): the dispatch signatures have no error return.
[[noreturn]] inline void die(const char *what, const char *detail) {
    std::fprintf(stderr, "tqhip: %s: %s\n", what, detail);
    std::fflush(stderr);
    std::abort();
}

inline void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) die(what, hipGetErrorString(e));
}

#define TQ_HIP_CHECK(expr) ::tqhip::check_hip((expr), #expr)

// Error codes returned by the device-pointer entry points.
enum Status : int {
    kOk = 0,
    kBadShape = -1,      // a dimension is < 1, in_dim % 4 != 0 for VQ2, or an operand pointer is null
    kBadGroup = -2,      // group_size is odd or < 2
    kTooLarge = -3,      // a byte offset does not fit the 32-bit buffer range
    kLaunchFailed = -4,  // hipGetLastError after the launch was not hipSuccess
    kBadFile = -5,       // a .tqwen file was unreadable, invalid or of an unsupported kind
    kHipFailed = -6,     // a HIP allocation or copy failed
    kNoScratch = -7,     // the allocation-free entry point's static scratch is too small for the call
    kNotFused = 1,       // a fused path does not apply to these operands; nothing was launched
};

// Device-pointer launchers (defined in the .hip files). All return a Status.
int launch_i4_matvec(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                     hipStream_t stream);
int launch_i4_matvec_generic(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim,
                             int group_size, hipStream_t stream);
// n (1..3) matrices sharing x, in_dim and group_size (pair / qkv), one launch where possible.
int launch_i4_matvec_group(int n, const uint8_t *const *w, float *const *y, const int *out_dim, const float *x,
                           int in_dim, int group_size, hipStream_t stream);
// One matrix of a matvec set (tqhip_i4_mat): its own activations, output and shape.
struct I4Mat {
    const uint8_t *w;
    const float *x;
    float *y;
    int M, K;
};
constexpr int kSetMaxMats = 8;  // matrices per set launch
// n independent matvecs sharing a group size: one launch per kSetMaxMats matrices the set
// kernel takes (G = 64, K % 4 == 0, K <= 10240, x 16-byte aligned), the others one by one.
int launch_i4_matvec_set(int n, const I4Mat *mats, int group_size, hipStream_t stream);
// The set kernel for a single or fused launch when every matrix takes it and its grid is small
// enough to beat the MFMA kernels; kNotFused (nothing launched) otherwise.
int launch_i4_matvec_set_fit(int n, const I4Mat *mats, int group_size, hipStream_t stream);
bool i4_set_fit_takes(int n, const I4Mat *mats, int group_size);  // whether the call above would launch
// Activation prologue of a set launch whose matrices all read the same x (the decode engine's
// fused launches), applied as the activations are loaded:
//   kind 1: x = silu(x) * x2 (swiglu_ref);
//   kind 2: h = (x + d1) + d2 (d1, d2 optional), x = rmsnorm(h) * nw (rmsnorm_ref, eps), and
//           workgroup 0 also stores h to hout when hout is given.
struct SetPrologue {
    int kind;
    const float *x2, *d1, *d2, *nw;
    float *hout;
    float eps;
};
// The set kernel with a prologue for up to 3 matrices sharing x (mats[i].x equal, 16-byte aligned
// like x2, d1, d2, nw and hout); kNotFused (nothing launched) when the set kernel does not take them.
int launch_i4_matvec_set_pro(int n, const I4Mat *mats, int group_size, const SetPrologue &pro, hipStream_t stream);
// Whether the set kernel takes rows of K elements at this group size (with x 16-byte aligned).
bool set_kernel_takes(int K, int group_size);
// A decode layer's gate / up pair (same shape, same x) with the kind-2 prologue pro, as one launch
// storing act = silu(gate) * up to gate.y (up.y is not written): each value has the bits of the
// set launch of the pair followed by a kind-1 (SwiGLU) prologue. kNotFused when the set kernel
// does not take the shape or an operand is misaligned.
int launch_i4_matvec_glu(const I4Mat &gate, const I4Mat &up, int group_size, const SetPrologue &pro,
                         hipStream_t stream);
// launch_i4_matvec (same kernel, same bits) with each workgroup's argmax of y (argmax_ref: first
// row of the largest value; NaN never taken) at pv / pi [0 .. *parts): applies where
// launch_i4_matvec takes the register-path kernel for one matrix at G = 64 with at most cap
// workgroups; kNotFused (nothing launched) otherwise.
int launch_i4_matvec_amax(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                          float *pv, int *pi, int cap, int *parts, hipStream_t stream);
bool i4_matvec_amax_takes(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size,
                          int cap);  // whether the call above would launch
int launch_vq2_matvec(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, hipStream_t stream);
// n independent VQ2 matvecs (I4Mat: weights, activations, output, shape) in as few launches as
// the one-wave-per-row kernel allows; each output has the bits launch_vq2_matvec gives it.
int launch_vq2_matvec_set(int n, const I4Mat *mats, hipStream_t stream);
// The same with each matrix's activations BiIP-rotated first (scale may be null, sign not), in
// one launch; kNotFused when that launch does not take the set.
int launch_vq2_matvec_set_rot(int n, const I4Mat *mats, const float *const *scale, const float *const *sign,
                              int block_size, hipStream_t stream);
// One launch with the activations staged per workgroup, for up to 3 matrices: the prologue pro
// (SetPrologue kind 1 or 2, the matrices sharing x; null for none), then, with sign given, each
// matrix's BiIP rotation; kNotFused when that launch does not take the set. vq2_set_takes: whether it would take n
// matrices of these rows and row length K (4-byte aligned weights).
int launch_vq2_matvec_set_pro(int n, const I4Mat *mats, const float *const *scale, const float *const *sign,
                              int block_size, const SetPrologue *pro, hipStream_t stream);
bool vq2_set_takes(int n, const int *M, int K, int xm);
int launch_i4_embed_rows(const uint8_t *embed, const int *rows, int n, int dim, int group_size, float *out,
                         hipStream_t stream);
int launch_biip_rotate(const float *x, float *y, int dim, const float *scale, const float *sign, int block_size,
                       hipStream_t stream);
// n (1..3) rotations of one x with their own scale (may be null) / sign / output, one launch.
int launch_biip_rotate_n(int n, const float *x, float *const *y, int dim, const float *const *scale,
                         const float *const *sign, int block_size, hipStream_t stream);
int launch_i4_matmul(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                     hipStream_t stream);
// The same without any allocation: X's fp16 copy goes to the library's static
// device array (kNoAllocScratchBytes per device); kNoScratch when it does not fit.
int launch_i4_matmul_noalloc(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                             hipStream_t stream);
constexpr size_t kNoAllocScratchBytes = size_t{16} << 20;
// Bytes of prefill scratch (fp16 X rows padded to 64 elements, 256-byte aligned, then one
// float per token) a matmul of K x N takes.
inline size_t prefill_scratch_bytes(int K, int N) {
    const size_t Kp = (static_cast<size_t>(K) + 63) / 64 * 64;
    return (Kp * 2 * static_cast<size_t>(N) + 255) / 256 * 256 + 4 * static_cast<size_t>(N);
}

// n floats at d (device) into h (pinned host memory) by `*wgs` workgroups (at most max_wgs, kTooLarge
// beyond), each storing seq to done[b] at system scope once its slice is stored: the host reads
// done[0 .. *wgs) until every word holds seq, then h (host_copy.hip).
int launch_copy_to_host(const float *d, float *h, size_t n, int *done, int max_wgs, int seq, hipStream_t stream,
                        int *wgs);

// Compute units of the current device, looked up once (1 when there is no device: the launch
// that follows fails and reports it). Defined in device.cpp.
int device_cu_count();

// ---- scratch memory (scratch.cpp) ---------------------------------------------------------
// Split-K exchange slots (zero between launches) and the prefill X workspace. Eager
// launches use the set of their (device, stream); inside a ScratchScope (graph capture,
// decode engine) the scope's set. Growth under stream capture fails with kHipFailed;
// a fixed set answers a request beyond its preset buffers with kTooLarge.
struct ScratchSet;
int scratch_split_slots(hipStream_t s, size_t nslots, unsigned long long **slots);
int scratch_prefill(hipStream_t s, size_t bytes, void **ws);
ScratchSet *scratch_set_new();
ScratchSet *scratch_set_fixed(void *xws, size_t xws_bytes);
void scratch_set_free(ScratchSet *set);  // the caller has synchronised every launch that used it
void scratch_forget_stream(hipStream_t s);  // the stream is being destroyed (synchronised)
long scratch_live_sets();                    // ScratchSet objects alive (bookkeeping checks)
class ScratchScope {
  public:
    explicit ScratchScope(ScratchSet *set);
    ~ScratchScope();
    ScratchScope(const ScratchScope &) = delete;
    ScratchScope &operator=(const ScratchScope &) = delete;

  private:
    ScratchSet *prev_;
};
struct ScratchStats {
    size_t split_bytes, prefill_bytes;
    int split_captured, prefill_captured, retired;
};
ScratchStats scratch_stats(hipStream_t s);  // the set a launch on s would use now

}  // namespace tqhip
