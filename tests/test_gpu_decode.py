"""The device-resident decode engine (tqhip_decode_*) against the decode-step
restatement (oracle/decode.py, pinned to the reference's CPU forward by
tests/test_decode_oracle.py).

Logits of every step within rel L2 1e-4 of the oracle's (the engine sums in
fp32 where the reference sums in double, and its softmax is two-pass), and the
engine's next token equal to the oracle's argmax wherever the oracle's top two
logits are more than 1e-3 of the logit scale apart. Replays after reset are
bit-identical."""
import numpy as np
import pytest

from conftest import load_package, rel_l2

tf = load_package().tqwen_synth  # synthetic .tqwen images

pytestmark = pytest.mark.gpu

CASES = {
    "qwen25_0p5b_2layers": dict(hidden=896, n_heads=14, n_kv_heads=2, head_dim=64, inter=4864, vocab=2000,
                                layers=2),
    "qwen3_qknorm_hd128": dict(hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, inter=1024, vocab=600,
                               layers=2, biases=False, qk_norm=True),
    # q/k norms on 64-wide heads: the attention's norms and rotation run in wave 0's registers
    "qwen3_qknorm_hd64": dict(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, inter=1024, vocab=600,
                              layers=2, biases=False, qk_norm=True),
    "embed_f32_g128_untied": dict(hidden=512, n_heads=8, n_kv_heads=1, head_dim=64, inter=1024, vocab=500,
                                  layers=1, group_size=128, embed_f32=True, tied=False),
    "vq2_qwen25_shape": dict(hidden=896, n_heads=14, n_kv_heads=2, head_dim=64, inter=4864, vocab=2000, layers=2,
                             vq2=True),
    "vq2_untied_gqa4": dict(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, inter=1024, vocab=500, layers=1,
                            vq2=True, tied=False),
    "vq2_rotated_qwen25_shape": dict(hidden=896, n_heads=14, n_kv_heads=2, head_dim=64, inter=4864, vocab=2000,
                                     layers=2, vq2=True, rotated=True),
    "i4_rotated": dict(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, inter=1200, vocab=300, layers=1,
                       rotated=True),
    "head_dim256": dict(hidden=512, n_heads=2, n_kv_heads=1, head_dim=256, inter=768, vocab=300, layers=1),
    # three layers: the fused layers' hidden state alternates hidden -> hidden2 -> hidden
    "i4_3layers": dict(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, inter=1024, vocab=400, layers=3),
    "vq2_3layers": dict(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, inter=1024, vocab=400, layers=3,
                        vq2=True),
    # rows of more than 1024 elements everywhere (the set kernel's long-row shapes)
    "wide_h1536": dict(hidden=1536, n_heads=12, n_kv_heads=2, head_dim=128, inter=2048, vocab=400, layers=2),
    # a vocabulary past the set kernel's reach: the lm_head takes the register-path kernel, which
    # forms each workgroup's argmax as it stores the logits
    "vocab_70000": dict(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, inter=1024, vocab=70000, layers=1),
}
PROMPT = [11, 257, 3, 3, 0, 199, 42, 5, 123, 7, 64, 99]


def open_model(gpu, tmp_path, case, seed=1, **kw):
    img, cfg, tensors = tf.dense_i4_model(seed=seed, **dict(CASES[case], **kw) if case else kw)
    path = tmp_path / "m.tqwen"
    path.write_bytes(bytes(img))
    return gpu.ModelFile(str(path)), cfg, tensors


def check_step(got_tok, got, want, what):
    err = rel_l2(got, want)
    assert err <= 1e-4, (what, err)
    top = np.sort(want)[-2:]
    if top[1] - top[0] > 1e-3 * np.max(np.abs(want)):
        assert got_tok == int(np.argmax(want)), what
    return err


@pytest.mark.parametrize("case", sorted(CASES))
def test_prompt_logits_match_oracle(gpu, tmp_path, case):
    from oracle.decode import DenseDecoder
    m, cfg, tensors = open_model(gpu, tmp_path, case)
    eng = gpu.DecodeEngine(m, 64)
    dec = DenseDecoder(cfg, tensors, 64)
    worst = 0.0
    for t in PROMPT:
        t %= cfg["vocab_size"]
        tok = eng.step(t)
        worst = max(worst, check_step(tok, eng.logits(), dec.step(t), (case, t)))
    print(f"{case}: worst rel L2 {worst:.2e}")
    assert eng.seq_len == len(PROMPT)
    eng.close()


@pytest.mark.parametrize("case", ["qwen25_0p5b_2layers", "qwen3_qknorm_hd128", "head_dim256",
                                  "vq2_qwen25_shape", "vq2_untied_gqa4", "vq2_rotated_qwen25_shape"])
def test_fused_layers_match_unfused(gpu, tmp_path, monkeypatch, case):
    """i4 files at G 64 without rotations run fused layers: the residual adds, the RMSNorms and
    SwiGLU inside the next projection's set launch (its activation prologue). The same steps
    with TQHIP_DECODE_UNFUSED set (separate add_rmsnorm and swiglu launches) give the same tokens
    and logits within 1e-6: the operations are the same, only the double sum of squares of each
    RMSNorm is added in another order. VQ2 files run the same fused layers through the VQ2
    kernel's staged activations (each workgroup builds them in LDS with the separate kernels'
    operations in their order), which also apply the BiIP rotations of rotated files: every step
    bit-identical to the separate add_rmsnorm, swiglu and rotation launches."""
    m, cfg, _ = open_model(gpu, tmp_path, case)
    fused = gpu.DecodeEngine(m, 32)
    monkeypatch.setenv("TQHIP_DECODE_UNFUSED", "1")
    plain = gpu.DecodeEngine(m, 32)
    monkeypatch.delenv("TQHIP_DECODE_UNFUSED")
    same = 0
    for t in PROMPT:
        t %= cfg["vocab_size"]
        a, b = fused.step(t), plain.step(t)
        la, lb = fused.logits(), plain.logits()
        assert a == b, (case, t)
        assert rel_l2(la, lb) <= 1e-6, (case, t, rel_l2(la, lb))
        same += np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    print(f"{case}: {same} of {len(PROMPT)} steps bit-identical")
    if CASES[case].get("vq2"):
        assert same == len(PROMPT), case
    fused.close()
    plain.close()


@pytest.mark.parametrize("case", ["qwen25_0p5b_2layers", "qwen3_qknorm_hd128", "i4_3layers", "wide_h1536"])
def test_glu_gate_up_matches_separate(gpu, tmp_path, monkeypatch, case):
    """Fused i4 layers run gate/up as one launch that stores silu(gate) * up (each workgroup
    computes a row of gate and the same row of up), and down with no prologue. With
    TQHIP_DECODE_NO_GLU=1 the engine stores gate and up and forms SwiGLU in down's prologue
    instead. The rows and SwiGLU are the same arithmetic either way, so every step's logits must
    be the same bits."""
    m, cfg, _ = open_model(gpu, tmp_path, case)
    glu = gpu.DecodeEngine(m, 32)
    monkeypatch.setenv("TQHIP_DECODE_NO_GLU", "1")
    sep = gpu.DecodeEngine(m, 32)
    monkeypatch.delenv("TQHIP_DECODE_NO_GLU")
    for i, t in enumerate(PROMPT):
        t %= cfg["vocab_size"]
        a, b = glu.step(t), sep.step(t)
        assert a == b, (case, i)
        assert np.array_equal(glu.logits().view(np.uint32), sep.logits().view(np.uint32)), (case, i)
    glu.close()
    sep.close()


@pytest.mark.parametrize("case", ["vocab_70000", "qwen25_0p5b_2layers"])
def test_lm_head_argmax_matches_two_launch_argmax(gpu, tmp_path, monkeypatch, case):
    """Where the i4 lm_head runs on the register-path kernel (vocabularies past the set kernel's
    reach), each of its workgroups keeps the first row of its largest logit and one launch reduces
    the partials; TQHIP_DECODE_NO_AMAX=1 keeps the two argmax launches over the stored logits.
    Both take the first index of the largest value, so every token and every logit must agree
    (at vocab 2000 both engines run the two-launch argmax)."""
    m, cfg, _ = open_model(gpu, tmp_path, case)
    fused = gpu.DecodeEngine(m, 32)
    monkeypatch.setenv("TQHIP_DECODE_NO_AMAX", "1")
    plain = gpu.DecodeEngine(m, 32)
    monkeypatch.delenv("TQHIP_DECODE_NO_AMAX")
    for i, t in enumerate(PROMPT):
        t %= cfg["vocab_size"]
        a, b = fused.step(t), plain.step(t)
        lg = fused.logits()
        assert np.array_equal(lg.view(np.uint32), plain.logits().view(np.uint32)), (case, i)
        assert a == b == int(np.argmax(lg)), (case, i)
    fused.close()
    plain.close()


def test_greedy_generation_and_reset_replay(gpu, tmp_path):
    from oracle.decode import DenseDecoder
    m, cfg, tensors = open_model(gpu, tmp_path, "qwen25_0p5b_2layers", seed=7)
    eng = gpu.DecodeEngine(m, 40)
    dec = DenseDecoder(cfg, tensors, 40)
    tok, first = 5, []
    for _ in range(24):
        nxt = eng.step(tok)
        lg = eng.logits()
        first.append(lg)
        check_step(nxt, lg, dec.step(tok), "greedy")
        tok = int(np.argmax(dec.logits))  # follow the oracle's choice so both stay on one sequence
    eng.reset()
    assert eng.seq_len == 0
    tok = 5
    for i in range(24):
        eng.step(tok)
        assert np.array_equal(eng.logits().view(np.uint32), first[i].view(np.uint32)), i
        tok = int(np.argmax(first[i]))
    eng.close()


def test_positions_past_one_attention_chunk(gpu, tmp_path):
    """4200 positions: the attention kernel's 4096-position chunks and their rescaling."""
    from oracle.decode import DenseDecoder
    m, cfg, tensors = open_model(gpu, tmp_path, None, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64,
                                 inter=256, vocab=100, layers=1, max_seq_len=4300)
    eng = gpu.DecodeEngine(m, 4300)
    dec = DenseDecoder(cfg, tensors, 4300, exact_attention=False)
    rng = np.random.default_rng(3)
    for i, t in enumerate(rng.integers(0, 100, 4200)):
        tok = eng.step(int(t))
        want = dec.step(int(t))
        if i in (0, 4095, 4096, 4097, 4199):
            check_step(tok, eng.logits(), want, i)
    eng.close()


def test_errors(gpu, tmp_path):
    m, cfg, _ = open_model(gpu, tmp_path, "head_dim256")
    with pytest.raises(ValueError, match="max_seq_len"):
        gpu.DecodeEngine(m, cfg["max_seq_len"] + 1)
    eng = gpu.DecodeEngine(m, 2)
    lib = gpu.lib()
    assert lib.tqhip_decode_step(eng._h, cfg["vocab_size"]) == gpu.EBADSHAPE
    assert lib.tqhip_decode_step(eng._h, -1) == gpu.EBADSHAPE
    eng.step(1)
    eng.step(2)
    assert lib.tqhip_decode_step(eng._h, 1) == gpu.EBADSHAPE  # cache full
    eng.close()
    path = tmp_path / "f32.tqwen"
    path.write_bytes(bytes(tf.build([tf.f32_tensor("a", [1.0, 2.0])])))
    with pytest.raises(ValueError, match="i4 and VQ2 files only"):
        gpu.DecodeEngine(gpu.ModelFile(str(path)))
    img, _ = tf.vq2_model(hidden=128, vocab=50)  # a VQ2 file without the layer tensors
    path = tmp_path / "v.tqwen"
    path.write_bytes(bytes(img))
    with pytest.raises(ValueError, match="missing tensor"):
        gpu.DecodeEngine(gpu.ModelFile(str(path)))
    img, _, ts = tf.dense_i4_model(hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, inter=256, vocab=100,
                                   layers=1)
    tf.set_entry_name(img, 3, b"model.layers.0.self_attn.q_proj.weightX")  # q_proj renamed away
    path = tmp_path / "missing.tqwen"
    path.write_bytes(bytes(img))
    with pytest.raises(ValueError, match="missing tensor model.layers.0.self_attn.q_proj.weight"):
        gpu.DecodeEngine(gpu.ModelFile(str(path)))
