// ref_shim.cpp -- C entry points onto the reference's own dispatch API.
//
// TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile (target `ref`) together
// with the reference's unmodified sources, read in place from the reference
// tree: kernels/dispatch.cpp, kernels/*/*_ref.cpp, kernels/biip/biip_rotate.cpp,
// runtime/model_loader.cpp, runtime/tensor.cpp and the CPU forward of
// runtime/ (QwenModel and what it links). The result,
// oracle/_ref/libtqref.so, is the compiled reference `ref` path; tests and
// tests/golden/make_golden.py use it to pin the restatement in oracle.cpp.
//
// Every function here selects the reference's "ref" implementation by name
// (dispatch.h:155, :193) and calls the reference's generic entry point, so the
// code under test is exactly what tinyqwen's runtime would call.

#include "dispatch.h"
#include "model_loader.h"
#include "profiler.h"
#include "qwen_model.h"
#include "ref_ops.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>

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

// The reference's own .tqwen loader (ModelFile::load, runtime/model_loader.cpp:267),
// full load without expert offload, as tinyqwen's runtime calls it. One model
// at a time: tqref_model_load replaces the previous one.
static tinyqwen::ModelFile *g_model = nullptr;

int tqref_model_load(const char *path, char *err, int err_len) {
    delete g_model;
    g_model = new tinyqwen::ModelFile;
    std::string msg;
    const bool ok = g_model->load(path, &msg);
    if (err && err_len > 0) {
        std::strncpy(err, msg.c_str(), err_len - 1);
        err[err_len - 1] = 0;
    }
    if (!ok) {
        delete g_model;
        g_model = nullptr;
    }
    return ok ? 1 : 0;
}

int tqref_model_tensor_count(void) { return g_model ? static_cast<int>(g_model->tensor_count()) : 0; }

// Tensor i in file order: name (NUL-terminated, 65 bytes), dtype, ndim,
// shape[4], file offset, nbytes, and the quant group size of the model.
int tqref_model_tensor_at(int i, char *name, int *dtype, int *ndim, uint64_t *shape, uint64_t *offset,
                          uint64_t *nbytes) {
    if (!g_model || i < 0 || i >= static_cast<int>(g_model->tensor_count())) return 0;
    const tinyqwen::TensorView *t = g_model->get(g_model->tensor_names()[i]);
    std::memset(name, 0, 65);
    std::strncpy(name, t->name.c_str(), 64);
    *dtype = static_cast<int>(t->dtype);
    *ndim = t->ndim;
    for (int d = 0; d < 4; ++d) shape[d] = t->shape[d];
    *offset = t->file_offset;
    *nbytes = t->nbytes;
    return 1;
}

int tqref_model_quant_group_size(void) { return g_model ? static_cast<int>(g_model->config().quant_group_size) : -1; }
int tqref_model_type(void) { return g_model ? static_cast<int>(g_model->config().model_type) : -1; }

// The reference's CPU decode (QwenModel::create + forward_token,
// runtime/qwen_model.h:117-149) on a .tqwen file, with the `ref` kernels. One
// model at a time.
static tinyqwen::ModelFile *g_dfile = nullptr;
static tinyqwen::Profiler *g_dprof = nullptr;
static std::unique_ptr<tinyqwen::QwenModel> g_dmodel;

int tqref_decode_create(const char *path, int max_seq_len, char *err, int err_len) {
    select_ref();
    g_dmodel.reset();
    delete g_dfile;
    g_dfile = new tinyqwen::ModelFile;
    if (!g_dprof) g_dprof = new tinyqwen::Profiler(false);
    std::string msg;
    bool ok = g_dfile->load(path, &msg);
    if (ok) ok = tinyqwen::QwenModel::create(*g_dfile, max_seq_len, *g_dprof, &msg, &g_dmodel);
    if (err && err_len > 0) {
        std::strncpy(err, msg.c_str(), err_len - 1);
        err[err_len - 1] = 0;
    }
    return ok ? 1 : 0;
}

int tqref_decode_step(int token) { return g_dmodel->forward_token(token, nullptr, 5, true); }

void tqref_decode_logits(float *out, int n) { std::memcpy(out, g_dmodel->last_logits(), sizeof(float) * n); }

void tqref_decode_reset(void) { g_dmodel->reset(); }

}  // extern "C"
