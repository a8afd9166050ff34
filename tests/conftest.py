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
