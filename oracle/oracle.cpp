// oracle.cpp -- CPU restatement of tiny-llm's quantized-projection `ref` kernels.
//
// TEST INFRASTRUCTURE ONLY. This file is the checker for the HIP kernels in
// tiny-llm_amd/csrc. Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg may load it; the product library never links or calls it.
//
// What it restates (paths relative to the reference root):
//   orc_half_to_float     kernels/ref_ops.h:51-74    exact IEEE binary16 -> binary32
//   orc_float_to_half     kernels/ref_ops.h:78-105   binary32 -> binary16, round-to-nearest-even
//   orc_matvec_i4         kernels/matvec/matvec_i4_ref.cpp:45-103
//   orc_matvec_vq2        kernels/matvec/matvec_vq2_ref.cpp:52-81
//   orc_matmul_i4         kernels/matvec/matmul_i4_ref.cpp:53-114
//   orc_dequant_i4_row    kernels/ref_ops.h:183-205
//   orc_i4_row_bytes      runtime/tiny_format.h:73-78
//   orc_vq2_tensor_bytes  runtime/tiny_format.h:100-103
//   orc_quantized_size    quantization/quant.cpp:94-118
//
// Numerics follow the reference exactly: every weight is dequantized in fp32
// as (float(q) - zero) * scale, multiplied with x in double, accumulated in
// double in ascending index order, and the row sum is cast to float once.
// The file must be compiled with -ffp-contract=off so that the double
// multiply-add is not fused; with that flag the results are bit-identical to
// the reference built with g++ (checked against tests/golden fixtures).
//
// The *_mt variants split output rows (or output columns for matmul) over
// threads. Rows are independent, so they are bit-identical to the 1-thread
// versions.

#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr int kI4Header = 4;          // fp16 scale + fp16 zero in front of every group
constexpr int kVq2Dim = 4;            // weights per VQ2 index
constexpr int kVq2Entries = 256;      // codebook rows
constexpr int kVq2CodebookBytes = kVq2Entries * kVq2Dim * 2;

inline uint16_t load_u16(const uint8_t *p) {
    uint16_t v;
    std::memcpy(&v, p, 2);
    return v;
}

float half_bits_to_float(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (m << 13);  // inf / nan, payload kept
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (m << 13);  // rebias 15 -> 127
    } else if (m == 0) {
        bits = sign;
    } else {
        // Subnormal half: value = m * 2^-24, which is a normal float.
        const float mag = std::ldexp(static_cast<float>(m), -24);
        std::memcpy(&bits, &mag, 4);
        bits |= sign;
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t float_to_half_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return static_cast<uint16_t>(sign | 0x7E00u);  // nan
    if (a >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u); // rounds to >= 65520 -> inf
    if (a >= 0x38800000u) {
        // Normal half. Keep 10 mantissa bits, round the dropped 13 bits to even.
        const uint32_t e = (a >> 23) - 112u;
        const uint32_t m = a & 0x7FFFFFu;
        uint32_t r = (e << 10) | (m >> 13);
        const uint32_t rest = m & 0x1FFFu;
        if (rest > 0x1000u || (rest == 0x1000u && (r & 1u))) ++r;  // carry may bump exponent
        return static_cast<uint16_t>(sign | r);
    }
    // Subnormal or zero half: value = round(|f| * 2^24) units of 2^-24.
    // The reference flushes every |f| < 2^-24 to zero (ref_ops.h:94), so
    // (2^-25, 2^-24) gives 0 here where IEEE round-to-nearest would give the
    // smallest subnormal. That quirk is kept on purpose.
    const int exp = static_cast<int>(a >> 23);
    if (exp < 103) return sign;
    const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
    const int shift = 126 - exp;  // 14..24
    uint32_t r = mant >> shift;
    const uint32_t rest = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rest > half || (rest == half && (r & 1u))) ++r;
    return static_cast<uint16_t>(sign | r);
}

size_t i4_row_bytes_impl(int in_dim, int group_size) {
    const size_t groups = static_cast<size_t>((in_dim + group_size - 1) / group_size);
    return groups * static_cast<size_t>(kI4Header + group_size / 2);
}

// One output row of the i4 ref kernel (matvec_i4_ref.cpp:57-102).
float i4_row_dot(const uint8_t *row, const float *x, int in_dim, int group_size) {
    const int groups = (in_dim + group_size - 1) / group_size;
    const int gbytes = kI4Header + group_size / 2;
    double acc = 0.0;
    for (int g = 0; g < groups; ++g) {
        const uint8_t *gp = row + static_cast<size_t>(g) * gbytes;
        const float scale = half_bits_to_float(load_u16(gp));
        const float zero = half_bits_to_float(load_u16(gp + 2));
        const int col = g * group_size;
        const int n = (col + group_size <= in_dim) ? group_size : in_dim - col;
        const uint8_t *codes = gp + kI4Header;
        for (int i = 0; i < n; ++i) {
            const uint8_t b = codes[i >> 1];
            const int q = (i & 1) ? (b >> 4) : (b & 0x0F);
            const float w = (static_cast<float>(q) - zero) * scale;
            acc += static_cast<double>(w) * static_cast<double>(x[col + i]);
        }
    }
    return static_cast<float>(acc);
}

void matvec_i4_rows(const uint8_t *w, const float *x, float *y, int r0, int r1, int in_dim,
                    int group_size) {
    const size_t rb = i4_row_bytes_impl(in_dim, group_size);
    for (int o = r0; o < r1; ++o) y[o] = i4_row_dot(w + static_cast<size_t>(o) * rb, x, in_dim, group_size);
}

struct Codebook {
    float v[kVq2Entries][kVq2Dim];
};

void decode_codebook(const uint8_t *w, Codebook *cb) {
    for (int e = 0; e < kVq2Entries; ++e)
        for (int j = 0; j < kVq2Dim; ++j) cb->v[e][j] = half_bits_to_float(load_u16(w + 2 * (e * kVq2Dim + j)));
}

void matvec_vq2_rows(const Codebook &cb, const uint8_t *idx, const float *x, float *y, int r0,
                     int r1, int in_dim) {
    const int blocks = in_dim / kVq2Dim;
    for (int o = r0; o < r1; ++o) {
        const uint8_t *row = idx + static_cast<size_t>(o) * blocks;
        double acc = 0.0;
        for (int b = 0; b < blocks; ++b) {
            const float *c = cb.v[row[b]];
            for (int j = 0; j < kVq2Dim; ++j)
                acc += static_cast<double>(c[j]) * static_cast<double>(x[b * kVq2Dim + j]);
        }
        y[o] = static_cast<float>(acc);
    }
}

template <typename Fn>
void parallel_rows(int n, int threads, Fn fn) {
    if (threads <= 1 || n < 2) {
        fn(0, n);
        return;
    }
    if (threads > n) threads = n;
    std::vector<std::thread> pool;
    pool.reserve(threads);
    for (int t = 0; t < threads; ++t) {
        const int a = static_cast<int>(static_cast<long long>(n) * t / threads);
        const int b = static_cast<int>(static_cast<long long>(n) * (t + 1) / threads);
        pool.emplace_back([=] { fn(a, b); });
    }
    for (auto &th : pool) th.join();
}

}  // namespace

extern "C" {

float orc_half_to_float(uint16_t h) { return half_bits_to_float(h); }
uint16_t orc_float_to_half(float f) { return float_to_half_bits(f); }

void orc_half_to_float_n(const uint16_t *h, float *f, long long n) {
    for (long long i = 0; i < n; ++i) f[i] = half_bits_to_float(h[i]);
}
void orc_float_to_half_n(const float *f, uint16_t *h, long long n) {
    for (long long i = 0; i < n; ++i) h[i] = float_to_half_bits(f[i]);
}

size_t orc_i4_row_bytes(int in_dim, int group_size) { return i4_row_bytes_impl(in_dim, group_size); }

size_t orc_vq2_tensor_bytes(int rows, int cols) {
    return static_cast<size_t>(kVq2CodebookBytes) + static_cast<size_t>(rows) * (static_cast<size_t>(cols) / kVq2Dim);
}

// type: 0 = f32, 1 = f16, 3 = i4, 4 = vq2 (the .tqwen dtype codes).
size_t orc_quantized_size(int type, int rows, int cols, int group_size) {
    switch (type) {
        case 0: return static_cast<size_t>(rows) * cols * 4;
        case 1: return static_cast<size_t>(rows) * cols * 2;
        case 3: {
            const size_t groups = static_cast<size_t>((cols + group_size - 1) / group_size);
            return static_cast<size_t>(rows) * ((cols + 1) / 2) + static_cast<size_t>(rows) * groups * 4;
        }
        case 4: return orc_vq2_tensor_bytes(rows, cols);
        default: return 0;
    }
}

void orc_matvec_i4(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int group_size) {
    matvec_i4_rows(w, x, y, 0, out_dim, in_dim, group_size);
}

void orc_matvec_i4_mt(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim,
                      int group_size, int threads) {
    parallel_rows(out_dim, threads,
                  [=](int a, int b) { matvec_i4_rows(w, x, y, a, b, in_dim, group_size); });
}

void orc_matvec_vq2(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim) {
    Codebook cb;
    decode_codebook(w, &cb);
    matvec_vq2_rows(cb, w + kVq2CodebookBytes, x, y, 0, out_dim, in_dim);
}

void orc_matvec_vq2_mt(const uint8_t *w, const float *x, float *y, int out_dim, int in_dim, int threads) {
    Codebook cb;
    decode_codebook(w, &cb);
    const uint8_t *idx = w + kVq2CodebookBytes;
    parallel_rows(out_dim, threads, [&, idx](int a, int b) { matvec_vq2_rows(cb, idx, x, y, a, b, in_dim); });
}

// Y[M,N] = W_i4[M,K] * X[K,N]; X and Y are column-major (x[n*K+k], y[n*M+m]).
void orc_matmul_i4(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size) {
    for (int n = 0; n < N; ++n)
        matvec_i4_rows(w, x + static_cast<size_t>(n) * K, y + static_cast<size_t>(n) * M, 0, M, K, group_size);
}

void orc_matmul_i4_mt(const uint8_t *w, const float *x, float *y, int M, int K, int N, int group_size,
                      int threads) {
    // Split the M*N outputs by rows within each column; every output is an
    // independent row dot product, so the split does not change any bit.
    const long long total = static_cast<long long>(M) * N;
    const int chunks = threads > 1 ? threads * 4 : 1;
    parallel_rows(chunks, threads, [=](int a, int b) {
        for (int c = a; c < b; ++c) {
            const long long lo = total * c / chunks, hi = total * (c + 1) / chunks;
            for (long long i = lo; i < hi;) {
                const int n = static_cast<int>(i / M);
                const int m0 = static_cast<int>(i % M);
                const long long col_end = static_cast<long long>(n + 1) * M;
                const int m1 = static_cast<int>((hi < col_end ? hi : col_end) - static_cast<long long>(n) * M);
                matvec_i4_rows(w, x + static_cast<size_t>(n) * K, y + static_cast<size_t>(n) * M, m0, m1, K,
                               group_size);
                i += m1 - m0;
            }
        }
    });
}

void orc_dequant_i4_row(const uint8_t *embed, int row, int dim, int group_size, float *out) {
    const int groups = (dim + group_size - 1) / group_size;
    const int gbytes = kI4Header + group_size / 2;
    const uint8_t *r = embed + static_cast<size_t>(row) * groups * gbytes;
    for (int g = 0; g < groups; ++g) {
        const uint8_t *gp = r + static_cast<size_t>(g) * gbytes;
        const float scale = half_bits_to_float(load_u16(gp));
        const float zero = half_bits_to_float(load_u16(gp + 2));
        const int col = g * group_size;
        const int n = (col + group_size <= dim) ? group_size : dim - col;
        for (int i = 0; i < n; ++i) {
            const uint8_t b = gp[kI4Header + (i >> 1)];
            const int q = (i & 1) ? (b >> 4) : (b & 0x0F);
            out[col + i] = (static_cast<float>(q) - zero) * scale;
        }
    }
}

// BiIP activation rotation (kernels/biip/biip_rotate.cpp:37-68):
// y = blockHadamard((x / scale) * sign), scale == nullptr skipping the division;
// per block of block_size (a power of two) an unnormalised butterfly, stage h
// = 1, 2, 4, ... replacing (a, c) at (j, j + h) by (a + c, a - c), then every
// element times 1 / sqrt(block_size) (computed in float). y may alias x.
void orc_biip_rotate(const float *x, float *y, int dim, const float *scale, const float *sign, int block_size) {
    for (int j = 0; j < dim; ++j) y[j] = scale ? (x[j] / scale[j]) * sign[j] : x[j] * sign[j];
    const float inv_sqrt = 1.0f / std::sqrt(static_cast<float>(block_size));
    for (int b = 0; b < dim / block_size; ++b) {
        float *blk = y + static_cast<size_t>(b) * block_size;
        for (int h = 1; h < block_size; h <<= 1)
            for (int i = 0; i < block_size; i += 2 * h)
                for (int j = i; j < i + h; ++j) {
                    const float a = blk[j], c = blk[j + h];
                    blk[j] = a + c;
                    blk[j + h] = a - c;
                }
        for (int j = 0; j < block_size; ++j) blk[j] *= inv_sqrt;
    }
}

}  // extern "C"
