"""Scratch lifetimes of the launches (tiny-llm_amd/csrc/scratch.cpp), on the CPU.

The split-K exchange slots and the prefill X copy are scratch the library owns.
The rules: eager calls use their own (device, stream) set; a graph or decode
engine owns its set for its whole life; nothing grows under capture; a buffer a
graph recorded is retired, never freed; the allocation-free set never allocates.
tests/scratch_harness.cpp checks each rule against recording mocks of the HIP
calls scratch.cpp makes; this test compiles it with g++ and runs it.

The second test checks the other half of the device-pointer contract: with no
device at all, the _dev entry points return an error code instead of aborting.
"""
import os
import shutil
import subprocess
import sys
import textwrap

import pytest

from conftest import REPO

HIP_INCLUDE = "/opt/rocm/include"


@pytest.mark.skipif(not shutil.which("g++") or not os.path.isdir(HIP_INCLUDE), reason="needs g++ and the HIP headers")
def test_scratch_bookkeeping(tmp_path):
    exe = tmp_path / "scratch_harness"
    csrc = os.path.join(REPO, "tiny-llm_amd", "csrc")
    cmd = ["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I", HIP_INCLUDE, "-I", csrc,
           os.path.join(csrc, "scratch.cpp"), os.path.join(REPO, "tests", "scratch_harness.cpp"), "-o", str(exe),
           "-lpthread"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    for name in ("eager_alloc", "reuse", "per_stream", "capture_fit", "capture_grow", "retire", "free_on_grow",
                 "scope", "fixed", "alloc_failure", "forget", "per_device"):
        assert f"ok {name}\n" in out.stdout, out.stdout
    assert out.stdout.endswith("all ok\n")


def test_dev_entry_points_return_errors_without_a_device(tqa):
    """Run in a child process with no GPU visible: every _dev call that needs
    scratch or a kernel must come back with a negative TQHIP_E* code (an abort
    would kill the child)."""
    code = textwrap.dedent(f"""
        import importlib.util, os, sys
        os.environ["HIP_VISIBLE_DEVICES"] = "-1"
        spec = importlib.util.spec_from_file_location("tq", {os.path.join(REPO, "tiny-llm_amd", "__init__.py")!r})
        tq = importlib.util.module_from_spec(spec); spec.loader.exec_module(tq)
        lib = tq.lib()
        # non-null stand-ins for device pointers (no device is visible, so nothing can run on
        # them): the calls get past the operand checks to the scratch allocation and the launch
        p = 1 << 20
        res = [lib.tqhip_matmul_i4_dev(p, p, p, 9728, 2560, 32, 64, None),
               lib.tqhip_matmul_i4_dev(p, p, p, 64, 100, 3, 6, None),
               lib.tqhip_matvec_i4_dev(p, p, p, 2560, 9728, 64, None),
               lib.tqhip_matvec_vq2_dev(p, p, p, 3072, 1024, None)]
        print("codes", res)
        sys.exit(0 if all(r < 0 for r in res) else 3)
    """)
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300, env=env)
    assert out.returncode == 0, (out.returncode, out.stdout, out.stderr)
