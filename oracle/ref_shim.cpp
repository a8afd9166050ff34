// ref_shim.cpp -- C entry points onto the reference's own dispatch API.
//
// TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile (target `ref`) together
// with the reference's unmodified sources, read in place from the reference
// tree: kernels/dispatch.cpp, kernels/*/*_ref.cpp and kernels/biip/biip_rotate.cpp. The result,
// oracle/_ref/libtqref.so, is the compiled reference `ref` path; tests and
// tests/golden/make_golden.py use it to pin the restatement in oracle.cpp.
//
// Every function here selects the reference's "ref" implementation by name
// (dispatch.h:155, :193) and calls the reference's generic entry point, so the
// code under test is exactly what tinyqwen's runtime would call.

#include "dispatch.h"
#include "ref_ops.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>

namespace {
void select_ref() {
    if (!tinyqwen::set_matvec_i4_impl_by_name("ref") || !tinyqwen::set_matvec_vq2_impl_by_name("ref")) {
        std::fprintf(stderr, "ref_shim: reference 'ref' kernels are not registered\n");
        std::abort();
    }
}
}  // namespace

extern "C" {

void tqref_matvec_i4(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size) {
    select_ref();
    tinyqwen::matvec_i4(w, x, y, out_dim, in_dim, group_size);
}

void tqref_matvec_pair_i4(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2,
                          int out_dim, int in_dim, int group_size) {
    select_ref();
    tinyqwen::matvec_pair_i4(w1, w2, x, y1, y2, out_dim, in_dim, group_size);
}

void tqref_matvec_qkv_i4(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq,
                         float *yk, float *yv, int q_dim, int kv_dim, int in_dim, int group_size) {
    select_ref();
    tinyqwen::matvec_qkv_i4(wq, wk, wv, x, yq, yk, yv, q_dim, kv_dim, in_dim, group_size);
}

void tqref_matvec_vq2(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim) {
    select_ref();
    tinyqwen::matvec_vq2(w, x, y, out_dim, in_dim);
}

void tqref_matmul_i4(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size) {
    // Only "ref" is registered in this build, so it is the current matmul_i4.
    tinyqwen::matmul_i4(w, x, y, M, K, N, group_size);
}

void tqref_matmul_vq2(const uint8_t *w, const float *x, float *y, int M, int K, int N) {
    select_ref();
    tinyqwen::matmul_vq2(w, x, y, M, K, N);
}

void tqref_dequant_i4_row(const uint8_t *embed, int row, int dim, int group_size, float *out) {
    tinyqwen::dequant_i4_row(embed, row, dim, group_size, out);
}

float tqref_half_to_float(uint16_t h) { return tinyqwen::half_to_float(h); }

// Array form, so NaN payloads reach the caller bit-exact (a float return
// value widened to a Python float would quiet signalling NaNs).
void tqref_half_to_float_n(const uint16_t *h, float *f, long long n) {
    for (long long i = 0; i < n; ++i) f[i] = tinyqwen::half_to_float(h[i]);
}
void tqref_float_to_half_n(const float *f, uint16_t *h, long long n) {
    for (long long i = 0; i < n; ++i) h[i] = tinyqwen::float_to_half(f[i]);
}
uint16_t tqref_float_to_half(float f) { return tinyqwen::float_to_half(f); }

int tqref_unknown_i4_name_rejected(void) {
    return tinyqwen::set_matvec_i4_impl_by_name("no_such_impl") ? 0 : 1;
}

// The reference's generic BiIP entry with its ops registry on "ref"
// (dispatch.cpp:880-889 falls back to biip_rotate_activation_ref).
void tqref_biip_rotate(const float *x, float *y, int dim, const float *scale, const float *sign, int block_size) {
    if (!tinyqwen::set_ops_impl_by_name("ref")) std::abort();
    tinyqwen::biip_rotate_activation(x, y, dim, scale, sign, block_size);
}

}  // extern "C"
