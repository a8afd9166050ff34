"""The data-flow decode step (decode_flow.hip) against the engine's graph step.

With TQHIP_DECODE_FLOW=1 at create, an engine of a fused i4 file runs each token's layers as
one cooperative launch whose phases wait for each other's outputs through tagged vectors in
HBM; by default it keeps the graph of separate launches. The flow step computes every value with the graph's own
code (the set kernel's rows, the engine's attention and norms), so the logits must be the
same bits on every step, for every workgroup count (fewer workgroups than tasks: each runs
several tasks of a phase), layer count (odd and even: the hidden state alternates between two
buffers) and embedding kind. A wait that runs out (forced here with a zero time limit) makes
the engine run the token through its graph and keep to it.
"""
import numpy as np
import pytest

from conftest import load_package, rel_l2

tf = load_package().tqwen_synth  # synthetic .tqwen images

pytestmark = pytest.mark.gpu

CASES = {
    "qwen25_0p5b_2layers": dict(hidden=896, n_heads=14, n_kv_heads=2, head_dim=64, inter=4864, vocab=2000,
                                layers=2),
    "qwen25_0p5b_3layers": dict(hidden=896, n_heads=14, n_kv_heads=2, head_dim=64, inter=4864, vocab=1000,
                                layers=3),
    "qwen3_qknorm_hd128": dict(hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, inter=1024, vocab=600,
                               layers=2, biases=False, qk_norm=True),
    "head_dim256": dict(hidden=512, n_heads=2, n_kv_heads=1, head_dim=256, inter=768, vocab=300, layers=1),
    "embed_f32_untied": dict(hidden=512, n_heads=8, n_kv_heads=1, head_dim=64, inter=1024, vocab=500, layers=2,
                             embed_f32=True, tied=False),
    "wide_h1536": dict(hidden=1536, n_heads=12, n_kv_heads=2, head_dim=128, inter=2048, vocab=400, layers=2),
}
PROMPT = [11, 257, 3, 3, 0, 199, 42, 5, 123, 7, 64, 99]


def open_model(gpu, tmp_path, case, seed=1):
    img, cfg, tensors = tf.dense_i4_model(seed=seed, **CASES[case])
    path = tmp_path / "m.tqwen"
    path.write_bytes(bytes(img))
    return gpu.ModelFile(str(path)), cfg, tensors


def engines(gpu, m, monkeypatch, max_seq=64, **env):
    for k, v in dict(env, TQHIP_DECODE_FLOW="1").items():
        monkeypatch.setenv(k, v)
    flow = gpu.DecodeEngine(m, max_seq)
    for k in env:
        monkeypatch.delenv(k)
    monkeypatch.delenv("TQHIP_DECODE_FLOW")
    graph = gpu.DecodeEngine(m, max_seq)
    return flow, graph


def same_steps(flow, graph, tokens, vocab, what):
    for i, t in enumerate(tokens):
        t %= vocab
        a, b = flow.step(t), graph.step(t)
        la, lb = flow.logits(), graph.logits()
        assert a == b, (what, i)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), \
            (what, i, rel_l2(la, lb), int(np.count_nonzero(la != lb)))


@pytest.mark.parametrize("case", sorted(CASES))
def test_flow_step_bit_identical_to_graph(gpu, tmp_path, monkeypatch, case):
    print(f"[flow] {case}", flush=True)
    m, cfg, _ = open_model(gpu, tmp_path, case)
    flow, graph = engines(gpu, m, monkeypatch)
    assert "flow" in flow.mode and "fused" in flow.mode, flow.mode
    assert "flow" not in graph.mode
    same_steps(flow, graph, PROMPT, cfg["vocab_size"], case)
    assert "flow" in flow.mode  # no wait ran out
    flow.close()
    graph.close()
    m.close()


@pytest.mark.parametrize("wgs", [8, 37, 100])
def test_flow_any_workgroup_count(gpu, tmp_path, monkeypatch, wgs):
    """Fewer workgroups than a phase has tasks (72 q/k/v blocks, 152 gate/up blocks, 56 down
    blocks at this shape): each runs several tasks of a phase, one after the other."""
    print(f"[flow] {wgs} workgroups", flush=True)
    m, cfg, _ = open_model(gpu, tmp_path, "qwen25_0p5b_3layers")
    flow, graph = engines(gpu, m, monkeypatch, TQHIP_FLOW_WGS=str(wgs))
    assert "flow" in flow.mode
    same_steps(flow, graph, PROMPT[:6], cfg["vocab_size"], f"{wgs} workgroups")
    flow.close()
    graph.close()
    m.close()


def test_flow_24_layers_and_reset(gpu, tmp_path, monkeypatch):
    """A Qwen2.5-0.5B-shaped stack of 24 layers (small vocabulary), 20 steps, then a reset and the
    same tokens again: bit-identical to the graph on every step, and to itself after the reset."""
    img, cfg, _ = tf.dense_i4_model(hidden=896, n_heads=14, n_kv_heads=2, head_dim=64, inter=4864, vocab=3000,
                                    layers=24, seed=5)
    m = gpu.ModelFile.from_image(img)
    flow, graph = engines(gpu, m, monkeypatch)
    assert "flow" in flow.mode
    toks = [(7 * i + 3) % 3000 for i in range(20)]
    first = []
    for t in toks:
        a, b = flow.step(t), graph.step(t)
        la, lb = flow.logits(), graph.logits()
        assert a == b and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        first.append(la)
    flow.reset()
    for i, t in enumerate(toks):
        flow.step(t)
        assert np.array_equal(flow.logits().view(np.uint32), first[i].view(np.uint32)), i
    assert "flow" in flow.mode
    flow.close()
    graph.close()
    m.close()


def test_flow_wait_out_of_time_falls_back_to_the_graph(gpu, tmp_path, monkeypatch, capfd):
    """A zero wait limit: the first wait of the first step runs out, the kernel's workgroups leave,
    and the engine runs that token through its graph (it rewrites the position's KV rows) and
    keeps to the graph: the logits are still the graph's."""
    m, cfg, _ = open_model(gpu, tmp_path, "qwen25_0p5b_2layers")
    flow, graph = engines(gpu, m, monkeypatch, TQHIP_FLOW_TIMEOUT_US="0")
    assert "flow" in flow.mode
    same_steps(flow, graph, PROMPT[:4], cfg["vocab_size"], "fallback")
    assert "flow" not in flow.mode
    assert "timed out" in capfd.readouterr().err
    flow.close()
    graph.close()
    m.close()
