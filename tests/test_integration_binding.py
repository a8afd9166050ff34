"""The reference-side binding, compiled and linked for real (CPU only).

The repository's integration guide carries the translation unit a tiny-llm maintainer adds
(kernels/matvec/hip_variants.cpp: the six TINYQWEN_*_VARIANT registrations and the gpu_decode
engine adapter). This test extracts those C++ blocks from that file, compiles them with g++
against the reference's own headers (kernels/dispatch.h, runtime/model_loader.h), links
them with the reference's registry (kernels/dispatch.cpp and the rest of the reference,
compiled unmodified into oracle/_ref/libtqref.so) and with libtqhip.so, and runs a driver
(tests/integration_driver.cpp) that selects every "hip" variant by name. It also shows
that libtqhip.so's own copy of the registry does not interpose on tiny-llm's. Nothing
runs on a GPU. It needs the reference tree, so it runs in the development container only.
"""
import os
import shutil
import subprocess

import pytest

from conftest import REPO

REF = "/root/reference"
REF_LIB = os.path.join(REPO, "oracle", "_ref", "libtqref.so")
TQ_DIR = os.path.join(REPO, "tiny-llm_amd")

pytestmark = pytest.mark.skipif(
    not (os.path.isfile(os.path.join(REF, "kernels", "dispatch.h")) and os.path.isfile(REF_LIB)
         and shutil.which("g++")),
    reason="needs the reference tree, oracle/_ref (make -C oracle ref) and g++ (development container)")


def binding_source():
    """The C++ blocks of the integration guide that make up hip_variants.cpp (its sections 1 and 4)."""
    from oracle.extract_binding import binding_source as extract
    return extract(open(os.path.join(REPO, "INTEGRATION.md")).read())


def test_binding_compiles_links_and_selects(tmp_path):
    src = tmp_path / "hip_variants.cpp"
    src.write_text(binding_source())
    exe = tmp_path / "integration_driver"
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Wno-unused-variable", f"-I{REF}/kernels", f"-I{REF}/runtime",
           str(src), os.path.join(REPO, "tests", "integration_driver.cpp"), "-o", str(exe),
           f"-L{os.path.dirname(REF_LIB)}", "-ltqref", f"-L{TQ_DIR}", "-ltqhip",
           f"-Wl,-rpath,{os.path.dirname(REF_LIB)}", f"-Wl,-rpath,{TQ_DIR}", "-pthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120,
                         env=dict(os.environ, HIP_VISIBLE_DEVICES="-1"))
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.endswith("all ok\n"), out.stdout


def test_reference_runtime_driver_on_ref(tmp_path):
    """oracle/_ref/tqref_runtime (the reference's QwenModel with its own kernels, driven by
    tests/hip_runtime_driver.cpp) runs the three legs the GPU test compares against."""
    exe = os.path.join(REPO, "oracle", "_ref", "tqref_runtime")
    if not os.access(exe, os.X_OK):
        pytest.skip("make -C oracle runtime")
    from conftest import load_package
    img, cfg, _ = load_package().tqwen_synth.dense_i4_model(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64,
                                                           inter=512, vocab=300, layers=2, seed=2)
    model, out = tmp_path / "m.tqwen", tmp_path / "l.bin"
    model.write_bytes(bytes(img))
    res = subprocess.run([exe, str(model), "ref", str(out), "5", "33"], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    lines = res.stdout.splitlines()
    assert lines[0] == "impl i4=ref vq2=ref"
    assert lines[1].startswith("decode ") and len(lines[1].split()) == 6
    assert lines[2].startswith("prefill ") and len(lines[2].split()) == 6
    import numpy as np
    logits = np.fromfile(out, dtype=np.float32).reshape(-1, cfg["vocab_size"])
    assert logits.shape[0] == 5 + 5 and np.all(np.isfinite(logits))
    # the returned tokens are the argmax of the logits written for the same step
    toks = [int(t) for t in lines[1].split()[1:]] + [int(t) for t in lines[2].split()[1:]]
    assert toks == [int(np.argmax(r)) for r in logits]
    res = subprocess.run([exe, str(model), "no_such_impl", str(out), "1", "2"], capture_output=True, text=True)
    assert res.returncode == 1 and "no implementation named no_such_impl" in res.stderr
