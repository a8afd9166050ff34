// tqwen_model.cpp -- .tqwen weight files read, validated and uploaded to HBM.
//
// The file format is the reference's (runtime/tiny_format.h:32-330,
// docs/weight_format.md): a 192-byte header, a table of 120-byte tensor
// entries, then 64-byte aligned tensor data. The checks follow the reference
// loader's stages (runtime/model_loader.cpp:302-740) for the files this library
// can serve -- f32 / f16 / i4 / VQ2 files of the dense Qwen2 and Qwen3.5 model
// types -- so such a file is accepted here exactly when the reference accepts
// it, and the i4 / VQ2 tensors it holds have the byte sizes the kernels assume
// (stages 5 and 5b). GPTQ files and MoE model types are rejected as
// unsupported. After validation, tqhip_model_upload copies the data region to
// one HBM allocation; every tensor keeps its file offset, so its device address
// is base + (offset - data_offset) and stays 64-byte aligned.

#include "../../include/tqhip.h"

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "tq_common.h"

namespace tqhip {
namespace {

constexpr size_t kHeaderBytes = 192, kEntryBytes = 120, kNameBytes = 64, kAlign = 64;
constexpr uint32_t kVersionMin = 1, kVersionMax = 3;
constexpr size_t kUploadChunk = size_t(64) << 20;
enum : uint32_t { kF32 = 0, kF16 = 1, kI8 = 2, kI4 = 3, kVQ2 = 4, kGPTQ4 = 5 };

template <typename T>
T rd(const uint8_t *p) {
    T v;
    std::memcpy(&v, p, sizeof(T));
    return v;
}

struct Tensor {
    std::string name;
    uint32_t dtype = 0, ndim = 0;
    uint64_t shape[4] = {0, 0, 0, 0};
    uint64_t offset = 0, nbytes = 0;
};

struct Model {
    std::string path;                  // empty for an image in memory
    const uint8_t *image = nullptr;    // the caller's copy of the whole file, or null
    tqhip_model_config config{};
    uint64_t file_bytes = 0, data_offset = 0;
    uint32_t version = 0, dtype = 0, model_type = 0, quant_group_size = 0;
    std::vector<Tensor> tensors;  // file order
    std::unordered_map<std::string, size_t> index;
    void *device = nullptr;  // data region [data_offset, file_bytes) once uploaded
};

bool fail(std::string *err, const std::string &msg) {
    *err = msg;
    return false;
}

std::string want_got(uint64_t want, uint64_t got) {
    return ", expected " + std::to_string(want) + " got " + std::to_string(got);
}

// Opens a file and returns its size, as the reference's stat() does.
FILE *open_sized(const std::string &path, uint64_t *bytes, std::string *err) {
    FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) {
        fail(err, "cannot open file: " + path + " (" + std::strerror(errno) + ")");
        return nullptr;
    }
    const bool ok = std::fseek(f, 0, SEEK_END) == 0;
    const long n = ok ? std::ftell(f) : -1;
    if (n < 0 || std::fseek(f, 0, SEEK_SET) != 0) {
        std::fclose(f);
        fail(err, "cannot size file: " + path);
        return nullptr;
    }
    *bytes = static_cast<uint64_t>(n);
    return f;
}

// A file or a caller's in-memory image of one.
struct Source {
    FILE *f = nullptr;
    const uint8_t *mem = nullptr;
};

bool read_at(const Source &src, uint64_t off, size_t n, uint8_t *dst, std::string *err) {
    if (n == 0) return true;
    if (src.mem) {
        std::memcpy(dst, src.mem + off, n);
        return true;
    }
    FILE *f = src.f;
    if (std::fseek(f, static_cast<long>(off), SEEK_SET) != 0 || std::fread(dst, 1, n, f) != n)
        return fail(err, "short read");
    return true;
}

// The checks of the reference loader's stages 1, 2, 4, 4b, 5 and 5b, in its
// order and with its messages (callers match on them), for header and tensor
// fields at their tiny_format.h offsets.
// Only the header and the tensor table are read: no check looks at tensor data.
bool validate(Model &m, const Source &f, std::string *err) {
    // stage 1: header
    if (m.file_bytes < kHeaderBytes) return fail(err, "file too small for header: " + m.path);
    std::vector<uint8_t> b(kHeaderBytes);
    if (!read_at(f, 0, kHeaderBytes, b.data(), err)) return false;
    if (std::memcmp(b.data(), "TINYQWEN", 8) != 0) return fail(err, "bad magic (not a .tqwen file): " + m.path);
    m.version = rd<uint32_t>(&b[8]);
    m.dtype = rd<uint32_t>(&b[12]);
    if (m.version < kVersionMin || m.version > kVersionMax) return fail(err, "unsupported format version: " + std::to_string(m.version) + " (this build supports " +
                                  std::to_string(kVersionMin) + ".." + std::to_string(kVersionMax) + ")");
    if (m.dtype != kF32 && m.dtype != kF16 && m.dtype != kI4 && m.dtype != kVQ2 && m.dtype != kGPTQ4)
        return fail(err, "loader supports dtype f32/f16/i4/vq2/gptq4, got " + std::to_string(m.dtype));
    if (m.dtype == kGPTQ4) return fail(err, "GPTQ-int4 files are not served by this library");
    const uint32_t n_layers = rd<uint32_t>(&b[16]), hidden = rd<uint32_t>(&b[20]), inter = rd<uint32_t>(&b[24]);
    const uint32_t n_heads = rd<uint32_t>(&b[28]), n_kv = rd<uint32_t>(&b[32]), head_dim = rd<uint32_t>(&b[36]);
    const uint32_t vocab = rd<uint32_t>(&b[40]), max_seq = rd<uint32_t>(&b[44]);
    const float eps = rd<float>(&b[56]), theta = rd<float>(&b[60]);
    const uint64_t count = rd<uint64_t>(&b[64]), table = rd<uint64_t>(&b[72]);
    m.data_offset = rd<uint64_t>(&b[80]);
    const uint64_t total = rd<uint64_t>(&b[88]);
    if (total != m.file_bytes)
        return fail(err, "total_bytes mismatch: header=" + std::to_string(total) + " actual=" + std::to_string(m.file_bytes));
    if (table != kHeaderBytes) return fail(err, "tensor_table_offset must be 192 in v1");
    if (count == 0 || count > 100000) return fail(err, "implausible tensor_count: " + std::to_string(count));
    if (table + count * kEntryBytes > m.file_bytes) return fail(err, "tensor table runs past end of file");
    if (m.data_offset % kAlign != 0 || m.data_offset < kHeaderBytes || m.data_offset > m.file_bytes)
        return fail(err, "bad data_offset: " + std::to_string(m.data_offset));
    if (!n_layers || !hidden || !inter || !n_heads || !n_kv || !head_dim || !vocab || !max_seq)
        return fail(err, "model config contains zero fields");
    if (n_heads % n_kv != 0) return fail(err, "n_heads % n_kv_heads != 0");
    if (eps <= 0.0f || theta <= 0.0f) return fail(err, "rms_norm_eps / rope_theta must be positive");
    m.config = tqhip_model_config{static_cast<int>(n_layers), static_cast<int>(hidden), static_cast<int>(inter),
                                  static_cast<int>(n_heads), static_cast<int>(n_kv), static_cast<int>(head_dim),
                                  static_cast<int>(vocab), static_cast<int>(max_seq),
                                  static_cast<int>(rd<uint32_t>(&b[48]) != 0), eps, theta, 0, 0, 0};

    // stage 2: tensor table
    std::vector<uint8_t> entries(count * kEntryBytes);
    if (!read_at(f, table, entries.size(), entries.data(), err)) return false;
    for (uint64_t i = 0; i < count; ++i) {
        const uint8_t *e = &entries[i * kEntryBytes];
        Tensor t;
        const std::string tag = "tensor #" + std::to_string(i) + ": ";
        t.dtype = rd<uint32_t>(e + 64);
        t.ndim = rd<uint32_t>(e + 68);
        for (int d = 0; d < 4; ++d) t.shape[d] = rd<uint64_t>(e + 72 + 8 * d);
        t.offset = rd<uint64_t>(e + 104);
        t.nbytes = rd<uint64_t>(e + 112);
        if (t.ndim < 1 || t.ndim > 4) return fail(err, tag + "bad ndim " + std::to_string(t.ndim));
        if (m.dtype == kI4) {
            if (t.dtype != kI4 && t.dtype != kF32) return fail(err, tag + "i4 file allows only i4/f32 tensors, got dtype " + std::to_string(t.dtype));
        } else if (m.dtype == kVQ2) {
            if (t.dtype != kVQ2 && t.dtype != kF32 && t.dtype != kF16 && t.dtype != kI4)
                return fail(err, tag + "vq2 file allows only vq2/f32/f16/i4 tensors, got dtype " + std::to_string(t.dtype));
        } else if (t.dtype != m.dtype) {
            return fail(err, tag + "dtype " + std::to_string(t.dtype) + " != header dtype " + std::to_string(m.dtype) +
                                 " (uniform-dtype)");
        }
        uint64_t numel = 1;
        for (uint32_t d = 0; d < t.ndim; ++d) {
            if (t.shape[d] == 0) return fail(err, tag + "zero in shape");
            numel *= t.shape[d];
        }
        for (uint32_t d = t.ndim; d < 4; ++d)
            if (t.shape[d] != 0) return fail(err, tag + "trailing shape must be 0");
        if (t.dtype == kI4 || t.dtype == kVQ2) {
            if (t.ndim != 2) return fail(err, tag + "i4/vq2/gptq tensor must be 2D");
        } else if (t.nbytes != numel * (t.dtype == kF32 ? 4u : 2u)) {
            return fail(err, tag + "nbytes mismatch");
        }
        if (t.offset % kAlign != 0 || t.offset < m.data_offset) return fail(err, tag + "unaligned / bad offset");
        if (t.offset + t.nbytes > m.file_bytes) return fail(err, tag + "payload runs past end of file");
        size_t len = 0;
        while (len < kNameBytes && e[len] != 0) ++len;
        t.name.assign(reinterpret_cast<const char *>(e), len);
        if (t.name.empty()) return fail(err, tag + "empty name");
        if (m.index.count(t.name)) return fail(err, "duplicate tensor name: " + t.name);
        m.index[t.name] = m.tensors.size();
        m.tensors.push_back(t);
    }

    // stage 4: the v2 extension (model type, Qwen3.5 hybrid fields, group size)
    if (m.version >= 2) {
        const uint8_t *x = &b[96];
        m.model_type = rd<uint32_t>(x);
        const uint32_t qk_heads = rd<uint32_t>(x + 4), v_heads = rd<uint32_t>(x + 8), qk_dim = rd<uint32_t>(x + 12);
        const uint32_t v_dim = rd<uint32_t>(x + 16), conv = rd<uint32_t>(x + 20), interval = rd<uint32_t>(x + 24);
        const float rotary = rd<float>(x + 28);
        const uint32_t pad = rd<uint32_t>(x + 36);
        m.quant_group_size = rd<uint32_t>(x + 40);
        if (m.model_type > 3) return fail(err, "unknown model_type: " + std::to_string(m.model_type));
        if (pad != 0) return fail(err, "v2 ext pad field must be 0");
        if (m.model_type == 2 || m.model_type == 3) return fail(err, "MoE model types are not served by this library");
        if (m.model_type == 1) {
            if (!qk_heads || !v_heads || !qk_dim || !v_dim || conv < 2)
                return fail(err, "qwen3_5: linear attention shape fields must be set (conv kernel >= 2)");
            if (interval < 2) return fail(err, "qwen3_5: full_attention_interval must be >= 2");
            if (n_layers % interval != 0) return fail(err, "qwen3_5: n_layers must be divisible by full_attention_interval");
            if (rotary <= 0.0f || rotary > 1.0f) return fail(err, "qwen3_5: partial_rotary_factor must be in (0, 1]");
            if (v_heads % qk_heads != 0) return fail(err, "qwen3_5: linear_num_v_heads % linear_num_qk_heads != 0");
        }
    }
    // stage 4b: the v3 extension (MoE and GPTQ fields; dense files keep them unused)
    if (m.version >= 3 && rd<uint32_t>(&b[96 + 64 + 28]) != 0) return fail(err, "v3 ext pad field must be 0");

    // stage 5: i4 files -- group size, and every i4 tensor's bytes
    const int gs = static_cast<int>(m.quant_group_size);
    if (m.dtype == kI4) {
        if (m.quant_group_size == 0 || m.quant_group_size > 1024) return fail(err, "i4 file: quant_group_size must be in [1,1024], got " + std::to_string(m.quant_group_size));
        if (m.quant_group_size % 2 != 0) return fail(err, "i4 file: quant_group_size must be even");
        for (const Tensor &t : m.tensors) {
            if (t.dtype != kI4) continue;
            const uint64_t want = t.shape[0] * i4_row_bytes(static_cast<int>(t.shape[1]), gs);
            if (t.nbytes != want) return fail(err, "tensor '" + t.name + "': i4 nbytes mismatch" + want_got(want, t.nbytes));
        }
    }
    // stage 5b: VQ2 files -- every VQ2 tensor's bytes, and an i4 embedding's
    if (m.dtype == kVQ2) {
        for (const Tensor &t : m.tensors) {
            if (t.dtype != kVQ2) continue;
            if (t.shape[1] % kVq2Dim != 0) return fail(err, "tensor '" + t.name + "': vq2 in_dim must be divisible by " + std::to_string(kVq2Dim));
            const uint64_t want = vq2_bytes(static_cast<int>(t.shape[0]), static_cast<int>(t.shape[1]));
            if (t.nbytes != want) return fail(err, "tensor '" + t.name + "': vq2 nbytes mismatch" + want_got(want, t.nbytes));
        }
        for (const Tensor &t : m.tensors) {
            if (t.dtype != kI4) continue;
            if (gs <= 0) return fail(err, "vq2 file with i4 embed requires quant_group_size > 0");
            const uint64_t want = t.shape[0] * i4_row_bytes(static_cast<int>(t.shape[1]), gs);
            if (t.nbytes != want)
                return fail(err, "tensor '" + t.name + "': i4 embed nbytes mismatch" + want_got(want, t.nbytes));
        }
    }
    m.config.model_type = static_cast<int>(m.model_type);
    m.config.quant_group_size = static_cast<int>(m.quant_group_size);
    m.config.file_dtype = static_cast<int>(m.dtype);
    return true;
}

void copy_err(const std::string &msg, char *err, int err_len) {
    if (!err || err_len <= 0) return;
    const size_t n = std::min(msg.size(), static_cast<size_t>(err_len - 1));
    std::memcpy(err, msg.data(), n);
    err[n] = 0;
}

void fill(const Model &m, const Tensor &t, tqhip_tensor_info *out) {
    std::memset(out, 0, sizeof(*out));
    std::memcpy(out->name, t.name.data(), t.name.size());
    out->dtype = static_cast<int>(t.dtype);
    out->ndim = static_cast<int>(t.ndim);
    for (int d = 0; d < 4; ++d) out->shape[d] = t.shape[d];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->device = m.device ? static_cast<const uint8_t *>(m.device) + (t.offset - m.data_offset) : nullptr;
}

}  // namespace
}  // namespace tqhip

using namespace tqhip;

extern "C" {

int tqhip_model_inspect(const char *path, void **model, char *err, int err_len) {
    if (!path || !model) return kBadFile;
    *model = nullptr;
    std::string msg;
    Model *m = new Model;
    m->path = path;
    FILE *f = open_sized(path, &m->file_bytes, &msg);
    const bool ok = f && validate(*m, Source{f, nullptr}, &msg);
    if (f) std::fclose(f);
    if (!ok) {
        copy_err(msg, err, err_len);
        delete m;
        return kBadFile;
    }
    *model = m;
    return kOk;
}

int tqhip_model_inspect_memory(const void *image, uint64_t bytes, void **model, char *err, int err_len) {
    if (!image || !model) return kBadFile;
    *model = nullptr;
    std::string msg;
    Model *m = new Model;
    m->image = static_cast<const uint8_t *>(image);
    m->file_bytes = bytes;
    if (!validate(*m, Source{nullptr, m->image}, &msg)) {
        copy_err(msg, err, err_len);
        delete m;
        return kBadFile;
    }
    *model = m;
    return kOk;
}

int tqhip_model_config_get(const void *model, tqhip_model_config *out) {
    if (!model || !out) return kBadShape;
    *out = static_cast<const Model *>(model)->config;
    return kOk;
}

int tqhip_model_upload(void *model) {
    Model *m = static_cast<Model *>(model);
    if (!m) return kBadShape;
    if (m->device) return kOk;
    const size_t n = m->file_bytes - m->data_offset;
    if (m->image) {
        void *dev = nullptr;
        if (n > 0 && hipMalloc(&dev, n) != hipSuccess) return kHipFailed;
        if (n > 0 && hipMemcpy(dev, m->image + m->data_offset, n, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipFree(dev);
            return kHipFailed;
        }
        m->device = dev;
        return kOk;
    }
    std::string msg;
    uint64_t bytes = 0;
    FILE *f = open_sized(m->path, &bytes, &msg);
    if (!f) return kBadFile;
    int rc = bytes == m->file_bytes ? kOk : kBadFile;  // the file changed since it was inspected
    void *dev = nullptr;
    if (rc == kOk && n > 0 && hipMalloc(&dev, n) != hipSuccess) rc = kHipFailed;
    // The data region streams through one host chunk; the model may be far
    // larger than what is worth holding twice in host memory.
    std::vector<uint8_t> chunk(std::min<size_t>(n, kUploadChunk));
    for (size_t done = 0; rc == kOk && done < n;) {
        const size_t len = std::min(chunk.size(), n - done);
        if (!read_at(Source{f, nullptr}, m->data_offset + done, len, chunk.data(), &msg)) rc = kBadFile;
        else if (hipMemcpy(static_cast<uint8_t *>(dev) + done, chunk.data(), len, hipMemcpyHostToDevice) != hipSuccess)
            rc = kHipFailed;
        done += len;
    }
    std::fclose(f);
    if (rc != kOk) {
        if (dev) (void)hipFree(dev);
        return rc;
    }
    m->device = dev;
    return kOk;
}

int tqhip_model_tensor_count(const void *model) {
    return model ? static_cast<int>(static_cast<const Model *>(model)->tensors.size()) : 0;
}

int tqhip_model_tensor_at(const void *model, int i, tqhip_tensor_info *out) {
    const Model *m = static_cast<const Model *>(model);
    if (!m || !out || i < 0 || i >= static_cast<int>(m->tensors.size())) return kBadShape;
    fill(*m, m->tensors[i], out);
    return kOk;
}

int tqhip_model_find(const void *model, const char *name, tqhip_tensor_info *out) {
    const Model *m = static_cast<const Model *>(model);
    if (!m || !name || !out) return kBadShape;
    const auto it = m->index.find(name);
    if (it == m->index.end()) return kBadShape;
    fill(*m, m->tensors[it->second], out);
    return kOk;
}

int tqhip_model_quant_group_size(const void *model) {
    return model ? static_cast<int>(static_cast<const Model *>(model)->quant_group_size) : 0;
}

int tqhip_model_file_dtype(const void *model) {
    return model ? static_cast<int>(static_cast<const Model *>(model)->dtype) : -1;
}

int tqhip_model_type(const void *model) {
    return model ? static_cast<int>(static_cast<const Model *>(model)->model_type) : -1;
}

void tqhip_model_free(void *model) {
    Model *m = static_cast<Model *>(model);
    if (!m) return;
    if (m->device) (void)hipFree(m->device);
    delete m;
}

}  // extern "C"
