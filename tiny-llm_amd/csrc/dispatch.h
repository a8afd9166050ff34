// dispatch.h -- the quantized-projection slice of tiny-llm's kernel registry.
//
// Same names, signatures and semantics as the reference's kernels/dispatch.h
// for the i4 / VQ2 / i4-matmul families (dispatch.h:151-175, 187-201, 249-253,
// macros 459-474 and 277-279), so code written against the reference registry
// compiles and behaves the same against this library:
//   * variants self-register from static initialisers (TINYQWEN_*_VARIANT);
//   * set_*_impl_by_name returns false on an unknown name and keeps the
//     current choice;
//   * pair / qkv entry points use a fused variant registered under the current
//     name, else fall back to separate matvec calls;
//   * VQ2 pair / qkv / matmul always decompose into matvec_vq2 calls.
// Differences, all deliberate:
//   * this library contains only the "hip" variants, so the default (nothing
//     selected) is "hip" instead of the reference's "ref";
//   * set_matmul_i4_impl_by_name exists (the reference picks the first
//     registered matmul, which depends on static-init order).
// When the variants are linked into tinyqwen itself, tinyqwen's own
// dispatch.cpp is used instead of this one (see include/tqhip.h).
#pragma once

#include <cstdint>

namespace tinyqwen {

using MatvecI4Fn = void (*)(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size);
using MatvecPairI4Fn = void (*)(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2,
                                int out_dim, int in_dim, int group_size);
using MatvecQkvI4Fn = void (*)(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq,
                               float *yk, float *yv, int q_dim, int kv_dim, int in_dim, int group_size);
using MatvecVQ2Fn = void (*)(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim);
using MatmulI4Fn = void (*)(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size);

void register_matvec_i4_impl(const char *name, MatvecI4Fn fn);
bool set_matvec_i4_impl_by_name(const char *name);
const char *matvec_i4_impl_name();
const char *available_matvec_i4_impls();
void matvec_i4(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size);

void register_matvec_i4_pair_impl(const char *name, MatvecPairI4Fn fn);
void matvec_pair_i4(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2, int out_dim,
                    int in_dim, int group_size);

void register_matvec_qkv_i4_impl(const char *name, MatvecQkvI4Fn fn);
void matvec_qkv_i4(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq, float *yk,
                   float *yv, int q_dim, int kv_dim, int in_dim, int group_size);

void register_matvec_vq2_impl(const char *name, MatvecVQ2Fn fn);
bool set_matvec_vq2_impl_by_name(const char *name);
const char *matvec_vq2_impl_name();
const char *available_matvec_vq2_impls();
void matvec_vq2(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim);
void matvec_pair_vq2(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2, int out_dim,
                     int in_dim);
void matvec_qkv_vq2(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq, float *yk,
                    float *yv, int q_dim, int kv_dim, int in_dim);
void matmul_vq2(const uint8_t *w, const float *x, float *y, int M, int K, int N);

void register_matmul_i4_impl(const char *name, MatmulI4Fn fn);
bool set_matmul_i4_impl_by_name(const char *name);
const char *matmul_i4_impl_name();
void matmul_i4(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size);

// BiIP activation rotation (dispatch.h:220-231 of the reference): one of the
// reference's "ops" (rmsnorm, rope, ... share one selected name,
// dispatch.cpp:777-800). Only the BiIP member of that family is on this
// library's path, so only it is registered here.
using BiipRotateFn = void (*)(const float *x, float *y, int dim, const float *scale, const float *sign,
                              int block_size);
void register_biip_rotate_impl(const char *name, BiipRotateFn fn);
bool set_ops_impl_by_name(const char *name);
const char *ops_impl_name();
void biip_rotate_activation(const float *x, float *y, int dim, const float *scale, const float *sign,
                            int block_size);

}  // namespace tinyqwen

#define TINYQWEN_BIIP_ROTATE_VARIANT(fn, name) \
    [[maybe_unused]] static const bool tqwen_reg_biip_##fn = (tinyqwen::register_biip_rotate_impl(name, fn), true)
#define TINYQWEN_MATVEC_I4_VARIANT(fn, name) \
    [[maybe_unused]] static const bool tqwen_reg_i4_##fn = (tinyqwen::register_matvec_i4_impl(name, fn), true)
#define TINYQWEN_MATVEC_I4_PAIR_VARIANT(fn, name) \
    [[maybe_unused]] static const bool tqwen_reg_i4_pair_##fn = (tinyqwen::register_matvec_i4_pair_impl(name, fn), true)
#define TINYQWEN_MATVEC_QKV_I4_VARIANT(fn, name) \
    [[maybe_unused]] static const bool tqwen_reg_qkv_i4_##fn = (tinyqwen::register_matvec_qkv_i4_impl(name, fn), true)
#define TINYQWEN_MATVEC_VQ2_VARIANT(fn, name) \
    [[maybe_unused]] static const bool tqwen_reg_vq2_##fn = (tinyqwen::register_matvec_vq2_impl(name, fn), true)
#define TINYQWEN_MATMUL_I4_VARIANT(fn, name) \
    [[maybe_unused]] static const bool tqwen_reg_mm_i4_##fn = (tinyqwen::register_matmul_i4_impl(name, fn), true)
