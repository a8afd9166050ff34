// i4_matmul.hip -- batched-prefill i4 dequant-GEMM for gfx950.
//
// Y[M,N] = W_i4[M,K] * X[K,N] with X and Y column-major (x[n*K+k], y[n*M+m]),
// the contract of the reference's matmul_i4_ref (kernels/matvec/matmul_i4_ref.cpp:53-114).
// Until the MFMA tile kernel lands, every column is one i4 matvec launch.

#include "tq_common.h"

namespace tqhip {

int launch_i4_matmul(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                     hipStream_t stream) {
    if (M < 1 || K < 1 || N < 1) return kBadShape;
    for (int n = 0; n < N; ++n) {
        const int st = launch_i4_matvec(w, x + static_cast<size_t>(n) * K, y + static_cast<size_t>(n) * M, M, K,
                                        group_size, stream);
        if (st != kOk) return st;
    }
    return kOk;
}

}  // namespace tqhip
