// integration_driver.cpp -- links INTEGRATION.md's hip_variants.cpp (the binding a tiny-llm
// maintainer adds) against the reference's own registry (kernels/dispatch.cpp, compiled into
// oracle/_ref/libtqref.so) and libtqhip.so, then checks that every "hip" variant registered and
// can be selected by name. Registration and selection only: no kernel runs, no GPU is needed.
#include <cstdio>
#include <cstring>
#include <string>

#include "dispatch.h"

static int failures = 0;
static void check(bool ok, const char *what) {
    std::printf("%s %s\n", ok ? "ok" : "FAIL", what);
    if (!ok) ++failures;
}
static bool lists(const char *names, const char *name) {
    const std::string s = std::string(", ") + names + ", ";
    return s.find(std::string(", ") + name + ", ") != std::string::npos;
}

int main() {
    using namespace tinyqwen;
    check(lists(available_matvec_i4_impls(), "hip"), "i4 registry lists hip");
    check(lists(available_matvec_i4_impls(), "ref"), "i4 registry still lists ref");
    check(!set_matvec_i4_impl_by_name("no_such_impl"), "unknown i4 name refused");
    check(set_matvec_i4_impl_by_name("hip") && std::strcmp(matvec_i4_impl_name(), "hip") == 0, "i4 hip selected");
    check(lists(available_matvec_vq2_impls(), "hip"), "vq2 registry lists hip");
    check(set_matvec_vq2_impl_by_name("hip") && std::strcmp(matvec_vq2_impl_name(), "hip") == 0, "vq2 hip selected");
    check(set_ops_impl_by_name("hip"), "ops hip (BiIP rotation) selected");
    check(lists(available_gpu_decode_impls(), "hip"), "gpu_decode registry lists hip");
    check(set_gpu_decode_impl_by_name("hip") && std::strcmp(gpu_decode_impl_name(), "hip") == 0,
          "gpu_decode hip selected");
    check(gpu_decode_available(), "gpu_decode available");
    std::printf(failures ? "FAILED\n" : "all ok\n");
    return failures ? 1 : 0;
}
