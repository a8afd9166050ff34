import glob
import importlib.util
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(REPO, "tests", "golden")
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


def load_package():
    """Imports tiny-llm_amd/ (its directory name is not a module name) as tiny_llm_amd."""
    if "tiny_llm_amd" in sys.modules:
        return sys.modules["tiny_llm_amd"]
    spec = importlib.util.spec_from_file_location("tiny_llm_amd", os.path.join(REPO, "tiny-llm_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["tiny_llm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def tqa():
    return load_package()


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture
def gpu(tqa):
    """The HIP library with a visible device; a GPU test without a device fails loudly.

    The host-pointer entry points cache device copies of weights by host
    pointer (the reference contract: weights live for the whole process).
    Tests free their arrays, so the cache is dropped after every test.
    """
    n = tqa.device_count()
    if n < 1:
        pytest.fail("no HIP device visible: GPU tests must run on the MI355X box")
    yield tqa
    tqa.lib().tqhip_release_weights()


def golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def golden_names(prefix):
    return sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, prefix + "*.npz")))


def rel_l2(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def max_abs_rel(got, ref):
    """max |got - ref| / max |ref| (the BASELINE 'relative to the fp32 output scale' measure)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (scale if scale > 0 else 1.0))


def extreme_x(K, seed):
    """Per group of 64: one activation 1e4 times larger, one 1e6 times smaller; group 2 all zero."""
    x = np.random.default_rng(seed).standard_normal(K).astype(np.float32)
    x[::64] *= 1e4
    x[1::64] *= 1e-6
    x[2 * 64:3 * 64] = 0.0
    return x


def special_headers(w, M, K, seed, G=64):
    """Overwrites about 3% of the group headers with special finite fp16 values."""
    w = w.copy()
    groups = (K + G - 1) // G
    hdr = w.reshape(M, groups, 4 + G // 2)[:, :, 0:4].view(np.uint16)  # [..., 0] scale, [..., 1] zero
    rng = np.random.default_rng(seed)
    pick = rng.random((M, groups)) < 0.03
    specials = [(0x0001, 0x4700), (0x03FF, 0x0000), (0x8000 | 0x2148, 0x4880), (0x0000, 0x4B00),
                (0x2148, 0xC200), (0x2148, 0x5640), (0x0400, 0x0001)]
    # (smallest subnormal scale, zero 7), (largest subnormal, 0), (negative scale, 9), (zero scale, 14),
    # (0.01, zero -3), (0.01, zero 100), (smallest normal, subnormal zero)
    kinds = rng.integers(0, len(specials), size=(M, groups))
    for i, (sc, z) in enumerate(specials):
        sel = pick & (kinds == i)
        hdr[..., 0][sel] = sc
        hdr[..., 1][sel] = z
    return w


def fp16_operand_bound_ok(got, want, orc, w, x, M, K, N, G):
    """Every output of an i4 matmul with fp16 operands within 1e-3 of the size of its own terms,
    sum_k |w_mk * x_nk| (rounding both operands to fp16 moves a product by at most 2 * 2^-11 of
    itself): the check for a handful of outputs, where one near-cancelled output decides the
    relative L2 and max measures."""
    wd = np.abs(orc.dequant_i4_matrix_f64(w, M, K, G))
    bound = 1e-3 * (np.abs(np.asarray(x, np.float64)).reshape(N, K) @ wd.T).reshape(-1)
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    return bool(np.all(err <= bound))
