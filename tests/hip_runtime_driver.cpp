// hip_runtime_driver.cpp -- the reference's own runtime, unmodified, on a .tqwen file, with the
// implementation named on the command line selected in its registries the way runtime/main.cpp
// does (set_matvec_i4_impl_by_name / set_matvec_vq2_impl_by_name / set_ops_impl_by_name,
// main.cpp:462-490; the fusion switches on, main.cpp:879-888).
//
// Built twice by oracle/Makefile (target `runtime`), from the reference sources where they lie:
//   oracle/_ref/tqref_runtime  this file + oracle/_ref/libtqref.so: only the reference's
//                              kernels are registered ("ref")
//   oracle/_ref/tqhip_runtime  the integration guide's hip_variants.cpp (linked first) + the
//                              reference's kernels and runtime + this file + libtqhip.so, with
//                              TQ_HIP_BINDING: the "hip" variants are registered too, and every
//                              entry point the binding calls is wrapped (-Wl,--wrap) to count
//                              its calls, which the driver prints
//
// matmul_i4 has no setter in the reference: the first registration becomes the default
// (kernels/dispatch.cpp:651-654). hip_variants.cpp is linked ahead of the reference's kernels,
// so its static initialisers run first and "hip" is the prefill GEMM, as a maintainer's
// set_matmul_i4_impl_by_name("hip") would make it.
//
// usage: <runtime> <model.tqwen> <impl> <logits.bin> <n_decode> <n_prefill> [engine]
//   decode   a fresh QwenModel; forward_token over n_decode fixed tokens ((7i + 3) % vocab)
//   prefill  a fresh QwenModel; forward_prefill over n_prefill tokens ((11i + 5) % vocab),
//            then 4 greedy forward_token steps from its result
//   engine   (hip only) gpu_decode "hip" (the guide's engine adapter): the decode tokens again
// stdout: one line per leg, "<leg> <token> <token> ...", and with TQ_HIP_BINDING a line
// "calls <entry>=<count> ...". logits.bin: every step's logits (vocab floats), legs in order.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "dispatch.h"
#include "model_loader.h"
#include "profiler.h"
#include "qwen_model.h"

#ifdef TQ_HIP_BINDING
#include <hip/hip_runtime_api.h>

// Call counters around the binding's entry points (-Wl,--wrap=<name> sends the binding's calls
// to __wrap_<name>; __real_<name> is libtqhip.so's).
namespace {
enum { kI4, kPair, kQkv, kVq2, kMm, kRot, kStep, kEntries };
const char *const kNames[kEntries] = {"tqhip_matvec_i4", "tqhip_matvec_pair_i4", "tqhip_matvec_qkv_i4",
                                      "tqhip_matvec_vq2", "tqhip_matmul_i4",      "tqhip_biip_rotate",
                                      "tqhip_decode_step"};
long g_calls[kEntries];
}  // namespace

extern "C" {
void __real_tqhip_matvec_i4(const uint8_t *, const float *, float *, int, int, int);
void __real_tqhip_matvec_pair_i4(const uint8_t *, const uint8_t *, const float *, float *, float *, int, int, int);
void __real_tqhip_matvec_qkv_i4(const uint8_t *, const uint8_t *, const uint8_t *, const float *, float *, float *,
                                float *, int, int, int, int);
void __real_tqhip_matvec_vq2(const uint8_t *, const float *, float *, int, int);
void __real_tqhip_matmul_i4(const uint8_t *, const float *, float *, int, int, int, int);
void __real_tqhip_biip_rotate(const float *, float *, int, const float *, const float *, int);
int __real_tqhip_decode_step(void *, int);

void __wrap_tqhip_matvec_i4(const uint8_t *w, const float *x, float *y, int o, int i, int g) {
    ++g_calls[kI4];
    __real_tqhip_matvec_i4(w, x, y, o, i, g);
}
void __wrap_tqhip_matvec_pair_i4(const uint8_t *w1, const uint8_t *w2, const float *x, float *y1, float *y2, int o,
                                 int i, int g) {
    ++g_calls[kPair];
    __real_tqhip_matvec_pair_i4(w1, w2, x, y1, y2, o, i, g);
}
void __wrap_tqhip_matvec_qkv_i4(const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x, float *yq,
                                float *yk, float *yv, int q, int kv, int i, int g) {
    ++g_calls[kQkv];
    __real_tqhip_matvec_qkv_i4(wq, wk, wv, x, yq, yk, yv, q, kv, i, g);
}
void __wrap_tqhip_matvec_vq2(const uint8_t *w, const float *x, float *y, int o, int i) {
    ++g_calls[kVq2];
    __real_tqhip_matvec_vq2(w, x, y, o, i);
}
void __wrap_tqhip_matmul_i4(const uint8_t *w, const float *x, float *y, int m, int k, int n, int g) {
    ++g_calls[kMm];
    __real_tqhip_matmul_i4(w, x, y, m, k, n, g);
}
void __wrap_tqhip_biip_rotate(const float *x, float *y, int d, const float *sc, const float *sg, int b) {
    ++g_calls[kRot];
    __real_tqhip_biip_rotate(x, y, d, sc, sg, b);
}
int __wrap_tqhip_decode_step(void *e, int t) {
    ++g_calls[kStep];
    return __real_tqhip_decode_step(e, t);
}
}
#endif

namespace {

void die(const char *what, const std::string &msg) {
    std::fprintf(stderr, "hip_runtime_driver: %s: %s\n", what, msg.c_str());
    std::exit(1);
}

void put(FILE *f, const float *logits, int vocab) {
    if (std::fwrite(logits, sizeof(float), vocab, f) != static_cast<size_t>(vocab)) die("write", "short write");
}

std::unique_ptr<tinyqwen::QwenModel> make_model(const tinyqwen::ModelFile &file, tinyqwen::Profiler &prof) {
    std::unique_ptr<tinyqwen::QwenModel> m;
    std::string err;
    if (!tinyqwen::QwenModel::create(file, 128, prof, &err, &m)) die("QwenModel::create", err);
    m->set_fuse_gate_up(true);
    m->set_fuse_qkv(true);
    return m;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 6) {
        std::fprintf(stderr, "usage: %s <model.tqwen> <impl> <logits.bin> <n_decode> <n_prefill> [engine]\n", argv[0]);
        return 2;
    }
    const std::string impl = argv[2];
    const int n_decode = std::atoi(argv[4]), n_prefill = std::atoi(argv[5]);
    const bool engine = argc > 6 && std::strcmp(argv[6], "engine") == 0;

    tinyqwen::ModelFile file;
    std::string err;
    if (!file.load(argv[1], &err)) die("ModelFile::load", err);
    const int vocab = static_cast<int>(file.config().vocab_size);
    if (!tinyqwen::set_matvec_i4_impl_by_name(impl.c_str()) || !tinyqwen::set_matvec_vq2_impl_by_name(impl.c_str()) ||
        !tinyqwen::set_ops_impl_by_name(impl.c_str()))
        die("select", "no implementation named " + impl + " (i4: " + tinyqwen::available_matvec_i4_impls() + ")");
    std::printf("impl i4=%s vq2=%s\n", tinyqwen::matvec_i4_impl_name(), tinyqwen::matvec_vq2_impl_name());

    FILE *out = std::fopen(argv[3], "wb");
    if (!out) die("open", argv[3]);
    tinyqwen::Profiler prof(false);

    {
        auto m = make_model(file, prof);
        std::printf("decode");
        for (int i = 0; i < n_decode; ++i) {
            std::printf(" %d", m->forward_token((7 * i + 3) % vocab, nullptr, 5, true));
            put(out, m->last_logits(), vocab);
        }
        std::printf("\n");
    }
    {
        auto m = make_model(file, prof);
        std::vector<int> prompt(n_prefill);
        for (int i = 0; i < n_prefill; ++i) prompt[i] = (11 * i + 5) % vocab;
        int tok = m->forward_prefill(prompt.data(), n_prefill);
        std::printf("prefill %d", tok);
        put(out, m->last_logits(), vocab);
        for (int i = 0; i < 4; ++i) {
            tok = m->forward_token(tok, nullptr, 5, true);
            std::printf(" %d", tok);
            put(out, m->last_logits(), vocab);
        }
        std::printf("\n");
    }
#ifdef TQ_HIP_BINDING
    if (engine) {
        if (!tinyqwen::set_gpu_decode_impl_by_name("hip")) die("gpu_decode", "no engine named hip");
        tinyqwen::GpuDecodeEngine *e = nullptr;
        if (!tinyqwen::gpu_decode_create(&file, 128, &err, &e)) die("gpu_decode_create", err);
        std::vector<float> host(vocab);
        std::printf("engine");
        for (int i = 0; i < n_decode; ++i) {
            std::printf(" %d", tinyqwen::gpu_decode_step(e, (7 * i + 3) % vocab));
            if (hipMemcpy(host.data(), tinyqwen::gpu_decode_logits(e), sizeof(float) * vocab, hipMemcpyDeviceToHost) !=
                hipSuccess)
                die("hipMemcpy", "engine logits");
            put(out, host.data(), vocab);
        }
        std::printf("\n");
        tinyqwen::gpu_decode_destroy(e);
    }
    std::printf("calls");
    for (int k = 0; k < kEntries; ++k) std::printf(" %s=%ld", kNames[k], g_calls[k]);
    std::printf("\n");
#else
    if (engine) die("engine", "this build has no gpu_decode engine registered");
#endif
    if (std::fclose(out) != 0) die("close", argv[3]);
    return 0;
}
