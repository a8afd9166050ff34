// dispatch.cpp -- registry for the i4 / VQ2 / i4-matmul / BiIP-rotation families (see dispatch.h).
//
// Behaviour follows the reference's kernels/dispatch.cpp: i4 (:353-441),
// VQ2 (:465-532), matmul_i4 (:650-660) and biip_rotate_activation (:880-889). Registries are filled by static
// initialisers before main and only read afterwards; the current selection is
// meant to be set once at start-up, as in the reference.

#include "dispatch.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <string>
#include <vector>

namespace tinyqwen {
namespace {

constexpr const char *kDefaultImpl = "hip";

template <typename Fn>
struct Family {
    std::map<std::string, Fn> table;
    Fn current = nullptr;
    std::string current_name;
    std::string joined;

    bool select(const char *name) {
        auto it = table.find(name ? name : "");
        if (it == table.end()) return false;
        current = it->second;
        current_name = it->first;
        return true;
    }
    const char *name() const { return current_name.empty() ? kDefaultImpl : current_name.c_str(); }
    const char *available() {
        std::vector<std::string> names;
        for (const auto &kv : table) names.push_back(kv.first);
        std::sort(names.begin(), names.end());
        joined.clear();
        for (size_t i = 0; i < names.size(); ++i) {
            if (i) joined += ", ";
            joined += names[i];
        }
        return joined.c_str();
    }
    Fn resolve(const char *family) {
        if (current) return current;
        auto it = table.find(kDefaultImpl);
        if (it == table.end()) {
            std::fprintf(stderr, "tqhip: %s '%s' is not registered -- is the variant object linked in?\n", family,
                         kDefaultImpl);
            std::abort();
        }
        return it->second;
    }
};

Family<MatvecI4Fn> &i4() {
    static Family<MatvecI4Fn> f;
    return f;
}
std::map<std::string, MatvecPairI4Fn> &i4_pair() {
    static std::map<std::string, MatvecPairI4Fn> m;
    return m;
}
std::map<std::string, MatvecQkvI4Fn> &i4_qkv() {
    static std::map<std::string, MatvecQkvI4Fn> m;
    return m;
}
Family<MatvecVQ2Fn> &vq2() {
    static Family<MatvecVQ2Fn> f;
    return f;
}
Family<MatmulI4Fn> &mm_i4() {
    static Family<MatmulI4Fn> f;
    return f;
}
Family<BiipRotateFn> &biip() {
    static Family<BiipRotateFn> f;
    return f;
}

}  // namespace

void register_matvec_i4_impl(const char *name, MatvecI4Fn fn) { i4().table[name] = fn; }
bool set_matvec_i4_impl_by_name(const char *name) { return i4().select(name); }
const char *matvec_i4_impl_name() { return i4().name(); }
const char *available_matvec_i4_impls() { return i4().available(); }
void matvec_i4(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size) {
    i4().resolve("matvec_i4")(w, x, y, out_dim, in_dim, group_size);
}

void register_matvec_i4_pair_impl(const char *name, MatvecPairI4Fn fn) { i4_pair()[name] = fn; }
void matvec_pair_i4(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2, int out_dim,
                    int in_dim, int group_size) {
    auto it = i4_pair().find(matvec_i4_impl_name());
    if (it != i4_pair().end()) {
        it->second(w1, w2, x, y1, y2, out_dim, in_dim, group_size);
        return;
    }
    matvec_i4(w1, x, y1, out_dim, in_dim, group_size);
    matvec_i4(w2, x, y2, out_dim, in_dim, group_size);
}

void register_matvec_qkv_i4_impl(const char *name, MatvecQkvI4Fn fn) { i4_qkv()[name] = fn; }
void matvec_qkv_i4(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq, float *yk,
                   float *yv, int q_dim, int kv_dim, int in_dim, int group_size) {
    auto it = i4_qkv().find(matvec_i4_impl_name());
    if (it != i4_qkv().end()) {
        it->second(wq, wk, wv, x, yq, yk, yv, q_dim, kv_dim, in_dim, group_size);
        return;
    }
    matvec_i4(wq, x, yq, q_dim, in_dim, group_size);
    matvec_pair_i4(wk, wv, x, yk, yv, kv_dim, in_dim, group_size);
}

void register_matvec_vq2_impl(const char *name, MatvecVQ2Fn fn) { vq2().table[name] = fn; }
bool set_matvec_vq2_impl_by_name(const char *name) { return vq2().select(name); }
const char *matvec_vq2_impl_name() { return vq2().name(); }
const char *available_matvec_vq2_impls() { return vq2().available(); }
void matvec_vq2(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim) {
    vq2().resolve("matvec_vq2")(w, x, y, out_dim, in_dim);
}
void matvec_pair_vq2(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2, int out_dim,
                     int in_dim) {
    matvec_vq2(w1, x, y1, out_dim, in_dim);
    matvec_vq2(w2, x, y2, out_dim, in_dim);
}
void matvec_qkv_vq2(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq, float *yk,
                    float *yv, int q_dim, int kv_dim, int in_dim) {
    matvec_vq2(wq, x, yq, q_dim, in_dim);
    matvec_vq2(wk, x, yk, kv_dim, in_dim);
    matvec_vq2(wv, x, yv, kv_dim, in_dim);
}
void matmul_vq2(const uint8_t *w, const float *x, float *y, int M, int K, int N) {
    for (int n = 0; n < N; ++n)
        matvec_vq2(w, x + static_cast<size_t>(n) * K, y + static_cast<size_t>(n) * M, M, K);
}

void register_matmul_i4_impl(const char *name, MatmulI4Fn fn) { mm_i4().table[name] = fn; }
bool set_matmul_i4_impl_by_name(const char *name) { return mm_i4().select(name); }
const char *matmul_i4_impl_name() { return mm_i4().name(); }
void matmul_i4(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size) {
    mm_i4().resolve("matmul_i4")(w, x, y, M, K, N, group_size);
}

// The reference accepts "ref" here for every op and falls back to its scalar
// _ref functions (dispatch.cpp:777-800, :880-889); this library has no CPU
// path, so like the other families it accepts only registered names.
void register_biip_rotate_impl(const char *name, BiipRotateFn fn) { biip().table[name] = fn; }
bool set_ops_impl_by_name(const char *name) { return biip().select(name); }
const char *ops_impl_name() { return biip().name(); }
void biip_rotate_activation(const float *x, float *y, int dim, const float *scale, const float *sign,
                            int block_size) {
    biip().resolve("biip_rotate_activation")(x, y, dim, scale, sign, block_size);
}

}  // namespace tinyqwen
