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
import re
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
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    blocks = [re.sub(r"^  ", "", b, flags=re.M) for b in re.findall(r"```cpp\n(.*?)```", text, flags=re.S)]
    parts = [b for b in blocks if "TINYQWEN_" in b and "VARIANT" in b]
    assert len(parts) == 2, "expected the registry block and the gpu_decode block"
    return "\n".join(parts)


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
