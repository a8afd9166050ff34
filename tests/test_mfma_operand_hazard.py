"""The prefill kernels' gfx950 assembly holds no write to an MFMA's A or B source registers within
the 8 instructions after that MFMA.

An instruction schedule that interleaved the next k-block's dequantization with the MFMAs
(sched_group_barrier) put such writes directly behind the MFMAs reading those registers, and the
results came out wrong on the GPU. The compiler's own hazard handling did not guard that
sequence, so this CPU test compiles i4_matmul.hip for gfx950 and scans the assembly: a schedule
or compiler change that brings the pattern back fails here, before it reaches a GPU.
"""
import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(REPO, "tiny-llm_amd", "csrc", "i4_matmul.hip")
WINDOW = 8


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    return None


def vgprs(operand):
    m = re.match(r"v\[(\d+):(\d+)\]$", operand)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", operand)
    return {int(m.group(1))} if m else set()


def source_overwrites(asm):
    """(kernel, MFMA line, offending line, distance) for every VGPR write within WINDOW
    instructions after an MFMA that targets one of the MFMA's A/B source registers."""
    hits = []
    for name in re.findall(r"^(_Z\S+):\s*$", asm, re.M):
        start = asm.find(name + ":")
        end = asm.find("s_endpgm", start)
        lines = [ln.strip() for ln in asm[start:end].split("\n")]
        lines = [ln for ln in lines if ln and not ln.startswith((".", ";")) and not ln.endswith(":")]
        for k, line in enumerate(lines):
            if not line.startswith("v_mfma"):
                continue
            ops = [o.strip() for o in line.split(None, 1)[1].split(",")]
            src = vgprs(ops[1]) | vgprs(ops[2])
            for d in range(1, WINDOW + 1):
                if k + d >= len(lines):
                    break
                parts = lines[k + d].split(None, 1)
                if len(parts) < 2 or parts[0].startswith("v_mfma"):
                    continue
                if not parts[0].startswith(("v_", "ds_read", "buffer_load", "global_load")):
                    continue
                if vgprs(parts[1].split(",")[0].strip()) & src:
                    hits.append((name, line, lines[k + d], d))
                    break
    return hits


def test_scanner_flags_the_pattern():
    asm = "_Zk:\n\tv_mfma_f32_32x32x16_f16 a[0:15], v[10:13], v[34:37], a[0:15]\n\tv_cvt_f32_ubyte1 v34, v59\n\ts_endpgm\n"
    assert len(source_overwrites(asm)) == 1
    asm_ok = "_Zk:\n\tv_mfma_f32_32x32x16_f16 a[0:15], v[10:13], v[34:37], a[0:15]\n\tv_cvt_f32_ubyte1 v40, v59\n\ts_endpgm\n"
    assert source_overwrites(asm_ok) == []


@pytest.mark.skipif(hipcc() is None, reason="needs hipcc")
def test_prefill_kernels_keep_mfma_sources(tmp_path):
    out = tmp_path / "i4_matmul.s"
    cmd = [hipcc(), "-std=c++17", "-O3", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", SRC, "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    asm = out.read_text()
    assert "v_mfma_f32_32x32x16_f16" in asm
    hits = source_overwrites(asm)
    assert not hits, "\n".join(f"{n[:60]}: +{d} after '{m}': '{o}'" for n, m, o, d in hits[:5])
