"""Writes the golden fixtures in tests/golden/*.npz from the compiled reference.

Run in the development container only (it needs the reference tree):

    make -C oracle ref && python tests/golden/make_golden.py

Every expected output comes from oracle/_ref/libtqref.so, i.e. tiny-llm's own
kernels/dispatch.cpp + kernels/*/*_ref.cpp compiled unmodified with g++
-ffp-contract=off, called through the reference's dispatch API (set "ref",
then matvec_i4 / matvec_vq2 / matmul_i4 / ...). Inputs are drawn with numpy's
PCG64 from fixed seeds and stored in the fixture next to the outputs, so the
fixtures are data only: no reference source travels with them.

Cases mirror the reference's own tests (tests/test_matvec_i4.cpp:200-224, 514-536;
tests/test_matvec_vq2.cpp:154-275; tests/test_quant_ops.cpp:62-112) at the same
shapes, plus edge cases the BASELINE contract needs (non-integer fp16 zeros,
subnormal / zero / negative scales, partial last groups, group sizes whose
group stride is odd, one-row and one-group matrices).
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import oracle  # noqa: E402  (test infrastructure)


def _p(a):
    return a.ctypes.data


def ref():
    r = oracle.ref_lib()
    if r is None:
        raise SystemExit("oracle/_ref/libtqref.so missing: run `make -C oracle ref` first")
    return r


def i4_random(rng, out_dim, in_dim, G, scale=(0.002, 0.02), zero=(0.0, 15.0), special=False):
    gb = 4 + G // 2
    groups = (in_dim + G - 1) // G
    w = rng.integers(0, 256, size=(out_dim, groups, gb), dtype=np.uint8)
    s = rng.uniform(scale[0], scale[1], size=(out_dim, groups)).astype(np.float16)
    z = rng.uniform(zero[0], zero[1], size=(out_dim, groups)).astype(np.float16)
    if special:
        flat_s = s.reshape(-1)
        flat_z = z.reshape(-1)
        n = flat_s.size
        picks = rng.choice(n, size=min(n, 12), replace=False)
        specials_s = np.array([0.0, -0.0, 6e-8, 3e-5, -0.013, 65504.0 / 4096, 1.0, -2.5, 1e-7, 0.5, 5.96e-8, -6.1e-5],
                              dtype=np.float16)
        specials_z = np.array([0.0, 15.0, 7.5, -3.0, 16.0, 1e-3, 0.0, 8.25, 3.0, 14.999, -0.0, 100.0],
                              dtype=np.float16)
        flat_s[picks] = specials_s[: len(picks)]
        flat_z[picks] = specials_z[: len(picks)]
    w[:, :, 0:2] = s[:, :, None].view(np.uint8).reshape(out_dim, groups, 2)
    w[:, :, 2:4] = z[:, :, None].view(np.uint8).reshape(out_dim, groups, 2)
    return np.ascontiguousarray(w.reshape(-1))


def ref_matvec_i4(w, x, M, K, G):
    y = np.empty(M, dtype=np.float32)
    ref().tqref_matvec_i4(_p(w), _p(x), _p(y), M, K, G)
    return y


def ref_matvec_vq2(w, x, M, K):
    y = np.empty(M, dtype=np.float32)
    ref().tqref_matvec_vq2(_p(w), _p(x), _p(y), M, K)
    return y


def ref_matmul_i4(w, x, M, K, N, G):
    y = np.empty(M * N, dtype=np.float32)
    ref().tqref_matmul_i4(_p(w), _p(x), _p(y), M, K, N, G)
    return y


def ref_matmul_vq2(w, x, M, K, N):
    y = np.empty(M * N, dtype=np.float32)
    ref().tqref_matmul_vq2(_p(w), _p(x), _p(y), M, K, N)
    return y


def save(name, **arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    print(f"{name}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in arrays.items()))


def make_i4(rng):
    # Known answer, tests/test_matvec_i4.cpp:200-213: q=[1,2,15,0], s=2, z=1, x=1 -> 28.
    kat = np.zeros(6, dtype=np.uint8)
    kat[0:2] = np.array([2.0], dtype=np.float16).view(np.uint8)
    kat[2:4] = np.array([1.0], dtype=np.float16).view(np.uint8)
    kat[4] = (2 << 4) | 1
    kat[5] = (0 << 4) | 15
    xk = np.ones(4, dtype=np.float32)
    save("i4_kat_1x4_g4", w=kat, x=xk, y=ref_matvec_i4(kat, xk, 1, 4, 4), dims=np.array([1, 4, 4]))

    cases = [
        ("i4_64x256_g128", 64, 256, 128, False),   # tests/test_matvec_i4.cpp:218
        ("i4_64x256_g64", 64, 256, 64, False),     # :219
        ("i4_32x200_g64", 32, 200, 64, False),     # :224, partial last group
        ("i4_96x384_g64", 96, 384, 64, True),      # special scales/zeros
        ("i4_40x192_g64", 40, 192, 64, False),
        ("i4_17x520_g40", 17, 520, 40, False),     # smallest G on the MFMA path, 24-byte groups
        ("i4_9x1000_g256", 9, 1000, 256, True),
        ("i4_5x100_g32", 5, 100, 32, False),       # G=32: portable kernel
        ("i4_3x70_g6", 3, 70, 6, False),           # odd group stride (7 bytes)
        ("i4_1x64_g64", 1, 64, 64, False),
        ("i4_130x896_g64", 130, 896, 64, False),   # Qwen2.5 hidden size, ragged tile
        ("i4_33x2560_g64", 33, 2560, 64, True),    # Qwen3.5-4B hidden size
    ]
    for name, M, K, G, special in cases:
        w = i4_random(rng, M, K, G, special=special)
        x = rng.standard_normal(K).astype(np.float32)
        if special:
            x[:: max(1, K // 7)] = 0.0
            x[1] = 1e-30
            x[2] = -3e4
        save(name, w=w, x=x, y=ref_matvec_i4(w, x, M, K, G), dims=np.array([M, K, G]))

    # pair / qkv decomposition through the reference's generic entry points
    K, G = 256, 64
    wq = i4_random(rng, 48, K, G)
    wk = i4_random(rng, 16, K, G)
    wv = i4_random(rng, 16, K, G)
    x = rng.standard_normal(K).astype(np.float32)
    yq = np.empty(48, np.float32)
    yk = np.empty(16, np.float32)
    yv = np.empty(16, np.float32)
    ref().tqref_matvec_qkv_i4(_p(wq), _p(wk), _p(wv), _p(x), _p(yq), _p(yk), _p(yv), 48, 16, K, G)
    save("i4_qkv_48_16x256_g64", wq=wq, wk=wk, wv=wv, x=x, yq=yq, yk=yk, yv=yv, dims=np.array([48, 16, K, G]))
    y1 = np.empty(16, np.float32)
    y2 = np.empty(16, np.float32)
    ref().tqref_matvec_pair_i4(_p(wk), _p(wv), _p(x), _p(y1), _p(y2), 16, K, G)
    save("i4_pair_16x256_g64", w1=wk, w2=wv, x=x, y1=y1, y2=y2, dims=np.array([16, K, G]))


def make_matmul(rng):
    cases = [
        ("mm_i4_48x128x2_g64", 48, 128, 2, 64),    # tests/test_matvec_i4.cpp:514-536
        ("mm_i4_40x192x5_g64", 40, 192, 5, 64),
        ("mm_i4_24x200x3_g64", 24, 200, 3, 64),    # partial last group
        ("mm_i4_64x256x33_g128", 64, 256, 33, 128),
        ("mm_i4_70x320x40_g64", 70, 320, 40, 64),  # >= 32 tokens: the MFMA prefill path
    ]
    for name, M, K, N, G in cases:
        w = i4_random(rng, M, K, G)
        x = rng.standard_normal(K * N).astype(np.float32)
        save(name, w=w, x=x, y=ref_matmul_i4(w, x, M, K, N, G), dims=np.array([M, K, N, G]))


def vq2_random(rng, out_dim, in_dim, cb_std=1.0):
    cb = (rng.standard_normal(1024) * cb_std).astype(np.float16)
    idx = rng.integers(0, 256, size=out_dim * (in_dim // 4), dtype=np.uint8)
    return np.concatenate([cb.view(np.uint8), idx])


def make_vq2(rng):
    # Known answer, tests/test_matvec_vq2.cpp:154-164: codebook[5] = 5s, index 5, x = 1s -> 20.
    cb = np.zeros(1024, dtype=np.float16)
    cb[20:24] = 5.0
    w = np.concatenate([cb.view(np.uint8), np.array([5], dtype=np.uint8)])
    x = np.ones(4, dtype=np.float32)
    save("vq2_kat_1x4", w=w, x=x, y=ref_matvec_vq2(w, x, 1, 4), dims=np.array([1, 4]))
    for name, M, K, std in [("vq2_32x128", 32, 128, 1.0), ("vq2_96x384", 96, 384, 1.0),
                            ("vq2_33x200", 33, 200, 1.0), ("vq2_100x52", 100, 52, 1.0),
                            ("vq2_64x1024", 64, 1024, 0.02), ("vq2_513x896", 513, 896, 0.02)]:
        w = vq2_random(rng, M, K, std)
        x = rng.standard_normal(K).astype(np.float32)
        save(name, w=w, x=x, y=ref_matvec_vq2(w, x, M, K), dims=np.array([M, K]))
    M, K, N = 48, 192, 5  # tests/test_matvec_vq2.cpp:254-275
    w = vq2_random(rng, M, K)
    x = rng.standard_normal(K * N).astype(np.float32)
    save("mm_vq2_48x192x5", w=w, x=x, y=ref_matmul_vq2(w, x, M, K, N), dims=np.array([M, K, N]))


def make_scalar(rng):
    # fp16 -> fp32 for every bit pattern, and fp32 -> fp16 on specials and randoms.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = np.empty(h.size, dtype=np.float32)
    ref().tqref_half_to_float_n(_p(h), _p(f), h.size)
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 70000.0, np.inf, -np.inf, np.nan,
                         6.1035156e-05, 6.0e-05, 5.96e-08, 5.9604645e-08, 2.98e-08, 2.9802322e-08, 1.0e-08,
                         1.00048828125, 1.000732421875, 0.1, 0.2, 1e-3, 2048.5, 4097.0],
                        dtype=np.float32)
    rand = np.concatenate([rng.standard_normal(2000).astype(np.float32),
                           (rng.standard_normal(2000) * 1e-5).astype(np.float32),
                           (rng.standard_normal(1000) * 3e4).astype(np.float32)])
    fin = np.concatenate([specials, rand])
    fout = np.empty(fin.size, dtype=np.uint16)
    ref().tqref_float_to_half_n(_p(fin), _p(fout), fin.size)
    save("fp16_conversions", half_bits=h, half_to_float=f, floats=fin, float_to_half=fout)

    # dequant_i4_row: the known answers of tests/test_quant_ops.cpp:62-112 plus a random embed table
    embed = np.zeros(12, dtype=np.uint8)
    embed[0:2] = np.array([0.5], np.float16).view(np.uint8)
    embed[2:4] = np.array([8.0], np.float16).view(np.uint8)
    embed[4] = (8 << 4) | 0
    embed[5] = (3 << 4) | 15
    embed[6:8] = np.array([0.25], np.float16).view(np.uint8)
    embed[8:10] = np.array([4.0], np.float16).view(np.uint8)
    embed[10] = (4 << 4) | 4
    embed[11] = (4 << 4) | 4
    out = np.zeros(8, dtype=np.float32)
    ref().tqref_dequant_i4_row(_p(embed), 0, 8, 4, _p(out))
    table = i4_random(rng, 7, 200, 64)
    rows = np.zeros((7, 200), dtype=np.float32)
    for r in range(7):
        ref().tqref_dequant_i4_row(_p(table), r, 200, 64, _p(rows[r]))
    save("dequant_i4_row", kat_embed=embed, kat_out=out, table=table, table_rows=rows, dims=np.array([7, 200, 64]))


def main():
    rng = np.random.Generator(np.random.PCG64(20261201))
    make_i4(rng)
    make_matmul(rng)
    make_vq2(rng)
    make_scalar(rng)
    assert ref().tqref_unknown_i4_name_rejected() == 1


if __name__ == "__main__":
    main()
