"""The decode-step restatement (oracle/decode.py) against the reference's own CPU
decode (QwenModel::forward_token, compiled from the reference tree into oracle/_ref):
the same logits and the same next token, step after step, on dense i4 files of
several shapes (biases, Qwen3 q/k norms, fp32 embedding with separate lm_head,
group 128, GQA ratios 1 / 2 / 4 / 7, and VQ2 files with fp16 vectors, tied to
the compact-i4 embedding or with a VQ2 lm_head)."""
import ctypes

import numpy as np
import pytest

from conftest import load_package, rel_l2

tf = load_package().tqwen_synth  # synthetic .tqwen images

CASES = {
    "qwen2_gqa7": dict(hidden=256, n_heads=7, n_kv_heads=1, head_dim=64, inter=512, vocab=300, layers=2),
    "qwen2_untied": dict(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=384, vocab=257, layers=1,
                         tied=False),
    "qwen3_qknorm": dict(hidden=256, n_heads=2, n_kv_heads=2, head_dim=128, inter=512, vocab=300, layers=2,
                         biases=False, qk_norm=True),
    "vq2_qwen2": dict(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=512, vocab=300, layers=2, vq2=True),
    "vq2_untied": dict(hidden=256, n_heads=4, n_kv_heads=1, head_dim=64, inter=384, vocab=200, layers=1, vq2=True,
                       tied=False),
    "vq2_rotated": dict(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, inter=384, vocab=300, layers=2,
                        vq2=True, rotated=True),
    "i4_rotated_odd_inter": dict(hidden=256, n_heads=4, n_kv_heads=1, head_dim=64, inter=200, vocab=100, layers=1,
                                 rotated=True),
    "embed_f32_g128": dict(hidden=256, n_heads=4, n_kv_heads=1, head_dim=64, inter=512, vocab=200, layers=1,
                           group_size=128, embed_f32=True, tied=False),
}
TOKENS = [3, 17, 17, 0, 199, 42, 5, 7]


@pytest.fixture(scope="module")
def ref(orc):
    r = orc.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref not built here (it needs the reference tree)")
    return r


@pytest.mark.parametrize("case", sorted(CASES))
def test_restatement_matches_reference_decode(orc, ref, tmp_path, case):
    from oracle.decode import DenseDecoder, argmax
    img, cfg, tensors = tf.dense_i4_model(seed=len(case), **CASES[case])
    path = tmp_path / "m.tqwen"
    path.write_bytes(bytes(img))
    err = ctypes.create_string_buffer(512)
    assert ref.tqref_decode_create(str(path).encode(), 16, err, len(err)), err.value
    dec = DenseDecoder(cfg, tensors, 16)
    want = np.empty(cfg["vocab_size"], np.float32)
    for t in TOKENS:
        t %= cfg["vocab_size"]
        nxt = ref.tqref_decode_step(t)
        ref.tqref_decode_logits(want.ctypes.data, want.size)
        got = dec.step(t)
        assert rel_l2(got, want) <= 1e-6, (case, t)
        assert argmax(got) == nxt
