"""CPU-side checks of the product library: it loads, exports the C ABI, and its
host-only parts (registry, byte accounting, synthetic generator) behave.
No kernel is launched here."""
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import REPO


def header_functions():
    text = open(os.path.join(REPO, "include", "tqhip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(tqhip_\w+|tq_\w+)\s*\(", text))
    return sorted(n for n in names if not n.startswith("tqhip_op"))


def test_library_exports_every_header_symbol(tqa):
    lib_path = tqa.LIB_PATH
    assert os.path.exists(lib_path)
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True, check=True).stdout
    exported = set(line.split()[-1] for line in out.splitlines() if line.strip())
    missing = [n for n in header_functions() if n not in exported]
    assert not missing, missing
    lib = tqa.lib()
    for n in header_functions():
        assert hasattr(lib, n)


def test_library_exports_only_the_c_abi(tqa):
    """The tinyqwen registry copy inside the library is not exported (it would
    interpose on tiny-llm's own registry when linked into it)."""
    out = subprocess.run(["nm", "-D", "--defined-only", tqa.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    names = [line.split()[-1] for line in out.splitlines() if line.strip() and line.split()[-2] in "TtDdBbRrVvWw"]
    assert names and all(n.startswith(("tqhip_", "tq_")) for n in names), [n for n in names
                                                                           if not n.startswith(("tqhip_", "tq_"))]


def test_python_bindings_cover_the_header(tqa):
    assert set(header_functions()) <= set(tqa.EXPORTED)


def test_registry_names_and_unknown_name(tqa):
    # tests/test_matvec_i4.cpp:544-548 and tests/test_matvec_vq2.cpp:169-171
    assert not tqa.set_matvec_i4_impl_by_name("no_such_impl")
    assert tqa.set_matvec_i4_impl_by_name("hip")
    assert tqa.matvec_i4_impl_name() == "hip"
    assert "hip" in tqa.available_matvec_i4_impls().split(", ")
    assert not tqa.set_matvec_vq2_impl_by_name("definitely_not_a_real_impl")
    assert tqa.set_matvec_vq2_impl_by_name("hip")
    assert "hip" in tqa.available_matvec_vq2_impls()
    assert tqa.set_matmul_i4_impl_by_name("hip")
    assert not tqa.set_matmul_i4_impl_by_name("ref")  # the oracle is not part of the product


def test_byte_accounting_matches_oracle(tqa, orc):
    lib = tqa.lib()
    for K, G in [(896, 64), (2560, 64), (200, 64), (70, 6), (1000, 256), (9728, 64)]:
        assert lib.tqhip_i4_row_bytes(K, G) == orc.i4_row_bytes(K, G) == tqa.i4_row_bytes(K, G)
    for M, K in [(3072, 1024), (1, 4), (33, 200)]:
        assert lib.tqhip_vq2_tensor_bytes(M, K) == orc.vq2_tensor_bytes(M, K) == tqa.vq2_tensor_bytes(M, K)


def test_synth_i4_distributions_and_determinism(tqa):
    M, K, G = 512, 2560, 64
    w = tqa.synth_i4(M, K, G, seed=0)
    assert np.array_equal(w, tqa.synth_i4(M, K, G, seed=0))
    assert not np.array_equal(w, tqa.synth_i4(M, K, G, seed=1))
    g = w.reshape(M, K // G, 4 + G // 2)
    s = g[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    z = g[:, :, 2:4].copy().view(np.float16).astype(np.float32)
    assert s.min() >= np.float16(0.002) and s.max() <= np.float16(0.02)
    assert z.min() >= 0.0 and z.max() <= 15.0
    assert abs(float(s.mean()) - 0.011) < 5e-4 and abs(float(z.mean()) - 7.5) < 0.1
    codes = g[:, :, 4:]
    q = np.concatenate([(codes & 15).ravel(), (codes >> 4).ravel()])
    counts = np.bincount(q, minlength=16)
    assert counts.min() > 0.95 * q.size / 16 and counts.max() < 1.05 * q.size / 16


def test_synth_normal_and_vq2(tqa):
    x = tqa.synth_normal(1 << 16, seed=3)
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1.0) < 0.02
    assert np.array_equal(x, tqa.synth_normal(1 << 16, seed=3))
    v = tqa.synth_vq2(300, 1024, seed=4)
    cb = v[:2048].view(np.float16).astype(np.float32)
    assert abs(float(cb.std()) - 0.02) < 0.002
    idx = v[2048:]
    assert idx.size == 300 * 256 and np.bincount(idx, minlength=256).min() > 200


def test_synth_fp16_encoder_is_ieee_rne(tqa):
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(3000) * s for s in (1e-6, 1e-3, 1.0, 1e3, 3e4)]).astype(np.float32)
    vals = np.concatenate([vals, np.array([0.0, -0.0, 65504, 65520, 7e4, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -24],
                                          np.float32)])
    lib = tqa.lib()
    got = np.array([lib.tq_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, vals.astype(np.float16).view(np.uint16))


def test_synth_seed_mixes_layer_and_name(tqa):
    a = tqa.synth_seed(0, 3, "q_proj")
    assert a == tqa.synth_seed(0, 3, "q_proj")
    assert a != tqa.synth_seed(0, 4, "q_proj") and a != tqa.synth_seed(0, 3, "k_proj")
