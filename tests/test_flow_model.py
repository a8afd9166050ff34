"""The data-flow decode step's protocol (tiny-llm_amd/csrc/decode_flow.h, decode_flow.hip), on the
CPU: tests/flow_model.cpp runs the kernel's phases and tasks on threads, from the same plan and
read/write tables, with tagged atomics for the tagged vectors and random delays. Every token
must equal a sequential run; a stalled task must end the step with an error, not a hang; and a
planted mistake (one hidden-state buffer instead of two) must end in a wait that runs out,
never in a wrong result. Compiled with g++ here; no GPU involved."""
import os
import shutil
import subprocess

import pytest

from conftest import REPO


@pytest.mark.skipif(not shutil.which("g++"), reason="needs g++")
def test_flow_protocol_model(tmp_path):
    exe = tmp_path / "flow_model"
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-I", os.path.join(REPO, "tiny-llm_amd", "csrc"),
           os.path.join(REPO, "tests", "flow_model.cpp"), "-o", str(exe), "-lpthread"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    for name in ("tokens", "timeout", "planted"):
        assert f"ok {name}\n" in out.stdout, out.stdout
