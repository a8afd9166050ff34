"""The reference's own runtime, unmodified, on the GPU through the "hip" variants.

oracle/_ref/tqhip_runtime is tiny-llm's QwenModel (runtime/qwen_model.cpp, qwen_forward_token.cpp,
qwen_forward_prefill.cpp, backend_cpu.cpp, kernels/dispatch.cpp: compiled from the reference
sources as they are) linked with the integration guide's hip_variants.cpp and libtqhip.so;
oracle/_ref/tqref_runtime is the same driver (tests/hip_runtime_driver.cpp) with only the
reference's "ref" kernels. Both run forward_token over 12 fixed tokens, forward_prefill over a
40-token prompt followed by 4 greedy steps, and the hip build also steps the gpu_decode "hip"
engine over the 12 tokens. Every step's logits and token of the hip build are compared with the
ref build's, and the binding's call counts show which entry points the runtime reached.

Tolerances: the decode steps and the engine go through the exact-integer i4 matvecs and the
fp32 VQ2 ones (relative L2 <= 1e-4 on the logits); the prefill's GEMM rounds both operands to
fp16 with fp32 accumulation (relative error of one projection about 1e-3 on random data), so the
prefill logits and the decode steps that follow them are held to 5e-3.

Both binaries are built in the development container (make -C oracle runtime, which needs the
reference tree); the GPU box runs the prebuilt files.
"""
import os
import subprocess

import numpy as np
import pytest

from conftest import REPO, load_package, rel_l2

pytestmark = pytest.mark.gpu

tf = load_package().tqwen_synth
REF_RT = os.path.join(REPO, "oracle", "_ref", "tqref_runtime")
HIP_RT = os.path.join(REPO, "oracle", "_ref", "tqhip_runtime")
N_DECODE, N_PREFILL, N_AFTER = 12, 40, 4
DECODE_TOL, PREFILL_TOL = 1e-4, 5e-3

CASES = {
    # Qwen2.5-0.5B layer shapes (q/k/v biases), two layers
    "qwen25_i4": dict(hidden=896, n_heads=14, n_kv_heads=2, head_dim=64, inter=4864, vocab=2000, layers=2),
    # Qwen3-style q/k norms, head_dim 128, BiIP rotations on every projection, untied lm_head
    "qwen3_i4_rotated": dict(hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, inter=1024, vocab=1200, layers=2,
                             biases=False, qk_norm=True, rotated=True, tied=False),
    # VQ2 projections with BiIP rotations and a VQ2 lm_head
    "vq2_rotated": dict(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, inter=1024, vocab=1000, layers=2,
                        vq2=True, rotated=True, tied=False),
}


def run(binary, model, impl, out, engine=False):
    args = [binary, model, impl, out, str(N_DECODE), str(N_PREFILL)] + (["engine"] if engine else [])
    res = subprocess.run(args, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    lines = dict(line.split(" ", 1) for line in res.stdout.strip().splitlines())
    legs = {k: [int(t) for t in lines[k].split()] for k in ("decode", "prefill", "engine") if k in lines}
    calls = {}
    if "calls" in lines:
        calls = {k: int(v) for k, v in (kv.split("=") for kv in lines["calls"].split())}
    return lines["impl"], legs, calls


@pytest.fixture(scope="module")
def binaries():
    for b in (REF_RT, HIP_RT):
        if not os.access(b, os.X_OK):
            pytest.skip(f"{os.path.relpath(b, REPO)} is not built (make -C oracle runtime, development container)")


@pytest.mark.parametrize("case", sorted(CASES))
def test_reference_runtime_on_hip_variants(gpu, binaries, tmp_path, case):
    print(f"[runtime] {case}", flush=True)
    img, cfg, _ = tf.dense_i4_model(seed=11, **CASES[case])
    model = str(tmp_path / "m.tqwen")
    with open(model, "wb") as f:
        f.write(bytes(img))
    vocab = cfg["vocab_size"]
    impl_r, ref, _ = run(REF_RT, model, "ref", str(tmp_path / "ref.bin"))
    impl_h, hip, calls = run(HIP_RT, model, "hip", str(tmp_path / "hip.bin"), engine=True)
    assert impl_r == "i4=ref vq2=ref" and impl_h == "i4=hip vq2=hip", (impl_r, impl_h)
    lr = np.fromfile(tmp_path / "ref.bin", dtype=np.float32).reshape(-1, vocab)
    lh = np.fromfile(tmp_path / "hip.bin", dtype=np.float32).reshape(-1, vocab)
    assert lr.shape[0] == N_DECODE + 1 + N_AFTER and lh.shape[0] == 2 * N_DECODE + 1 + N_AFTER
    assert np.all(np.isfinite(lh))

    dec = [rel_l2(lh[i], lr[i]) for i in range(N_DECODE)]
    pre = [rel_l2(lh[N_DECODE + i], lr[N_DECODE + i]) for i in range(1 + N_AFTER)]
    eng = [rel_l2(lh[N_DECODE + 1 + N_AFTER + i], lr[i]) for i in range(N_DECODE)]
    print(f"[runtime] {case} rel L2 max: decode {max(dec):.2e} prefill {max(pre):.2e} engine {max(eng):.2e}; "
          f"calls {calls}", flush=True)
    assert max(dec) <= DECODE_TOL, dec
    assert max(eng) <= DECODE_TOL, eng
    assert max(pre) <= PREFILL_TOL, pre
    assert hip["decode"] == ref["decode"]
    assert hip["engine"] == ref["decode"]
    assert hip["prefill"] == ref["prefill"]

    # Which entry points the runtime reached through the binding, counted per call. Decode steps
    # (12 + the 4 after the prefill) make one call per projection (forward_token,
    # runtime/qwen_forward_token.cpp:388-421, 458, 633-658; rotated files rotate and project each
    # matrix on its own) plus the lm_head; the prefill makes one GEMM per projection
    # (qwen_forward_prefill.cpp:207-212; VQ2: a matvec per token column, dispatch.cpp:527-532)
    # and one lm_head matvec for its last token.
    L, steps = cfg["n_layers"], N_DECODE + N_AFTER
    c = CASES[case]
    assert calls["tqhip_decode_step"] == N_DECODE
    if c.get("vq2"):
        assert calls["tqhip_matvec_vq2"] == (7 * L + 1) * steps + 7 * L * N_PREFILL + 1
        assert calls["tqhip_matvec_i4"] == calls["tqhip_matmul_i4"] == 0
    elif c.get("rotated"):
        assert calls["tqhip_matvec_i4"] == (7 * L + 1) * steps + 1
        assert calls["tqhip_matvec_qkv_i4"] == calls["tqhip_matvec_pair_i4"] == 0
        assert calls["tqhip_matmul_i4"] == 7 * L
    else:
        assert calls["tqhip_matvec_qkv_i4"] == L * steps   # fused q/k/v
        assert calls["tqhip_matvec_pair_i4"] == L * steps  # fused gate/up
        assert calls["tqhip_matvec_i4"] == (2 * L + 1) * steps + 1  # o, down, lm_head
        assert calls["tqhip_matmul_i4"] == 7 * L
    # BiIP: one rotation per rotated projection call, per token column in the prefill
    assert calls["tqhip_biip_rotate"] == (7 * L * (steps + N_PREFILL) if c.get("rotated") else 0)
