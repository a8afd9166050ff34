""".tqwen files uploaded to HBM (tqhip_model_upload) and fed to the kernels.

A small Qwen2.5-0.5B-shaped i4 HQQ@64 file and a VQ2 file are written, validated
and uploaded; every tensor's HBM bytes equal its file bytes, and the matvec,
fused qkv / gate-up and embedding kernels run on the uploaded device addresses
and match the oracle on the file's bytes (rel L2 <= 1e-5, embeddings bit-exact).
"""
import numpy as np
import pytest

from conftest import load_package, rel_l2

tf = load_package().tqwen_synth  # synthetic .tqwen images

pytestmark = pytest.mark.gpu

HIDDEN, INTER, VOCAB, G = 896, 4864, 2000, 64


@pytest.fixture(scope="module")
def i4_file(tmp_path_factory):
    img, ts = tf.i4_model(group_size=G, hidden=HIDDEN, inter=INTER, vocab=VOCAB, layers=2, seed=5)
    path = tmp_path_factory.mktemp("tqwen") / "qwen_i4.tqwen"
    path.write_bytes(bytes(img))
    return str(path), {t["name"]: t for t in ts}


def device_bytes(gpu, info):
    out = np.empty(info.nbytes, np.uint8)
    assert gpu.lib().tqhip_memcpy_d2h(out.ctypes.data, info.device, info.nbytes) == 0
    return out


def test_upload_places_every_tensor(gpu, i4_file):
    path, ts = i4_file
    m = gpu.ModelFile(path)
    assert all(m.tensor_at(k).device is None for k in range(m.tensor_count()))
    m.upload()
    m.upload()  # a second call keeps the first copy
    first = m.tensor_at(0)
    for k in range(m.tensor_count()):
        info = m.tensor_at(k)
        t = ts[info.name.decode()]
        assert info.device % 64 == 0
        assert info.device - first.device == info.offset - first.offset
        assert np.array_equal(device_bytes(gpu, info), np.frombuffer(t["data"], np.uint8)), info.name
    m.close()


def test_matvec_on_uploaded_weights(gpu, orc, i4_file):
    path, ts = i4_file
    m = gpu.ModelFile(path)
    m.upload()
    gs = m.quant_group_size
    x = gpu.synth_normal(INTER, seed=11)
    dx = gpu.DeviceBuffer.from_array(x)
    for name, t in ts.items():
        if t["dtype"] != tf.I4 or name == "model.embed_tokens.weight":
            continue
        info = m.get(name)
        M, K = int(info.shape[0]), int(info.shape[1])
        dy = gpu.DeviceBuffer(4 * M)
        gpu.matvec_i4_dev(info.device, dx, dy, M, K, gs)
        gpu.synchronize()
        got = dy.download(np.float32, M)
        want = orc.matvec_i4(np.frombuffer(t["data"], np.uint8), x[:K], M, K, gs, threads=8)
        assert rel_l2(got, want) <= 1e-5, name
    m.close()


def test_fused_projections_on_uploaded_weights(gpu, orc, i4_file):
    path, ts = i4_file
    m = gpu.ModelFile(path)
    m.upload()
    p = "model.layers.1."
    q, k, v = (m.get(p + f"self_attn.{n}_proj.weight") for n in "qkv")
    x = gpu.synth_normal(HIDDEN, seed=12)
    dx = gpu.DeviceBuffer.from_array(x)
    qd, kvd = int(q.shape[0]), int(k.shape[0])
    ys = [gpu.DeviceBuffer(4 * n) for n in (qd, kvd, kvd)]
    gpu.matvec_qkv_i4_dev(q.device, k.device, v.device, dx, *ys, qd, kvd, HIDDEN, G)
    gate, up = m.get(p + "mlp.gate_proj.weight"), m.get(p + "mlp.up_proj.weight")
    yg, yu = gpu.DeviceBuffer(4 * INTER), gpu.DeviceBuffer(4 * INTER)
    gpu.matvec_pair_i4_dev(gate.device, up.device, dx, yg, yu, INTER, HIDDEN, G)
    gpu.synchronize()
    for info, y, n in [(q, ys[0], qd), (k, ys[1], kvd), (v, ys[2], kvd), (gate, yg, INTER), (up, yu, INTER)]:
        want = orc.matvec_i4(np.frombuffer(ts[info.name.decode()]["data"], np.uint8), x, n, HIDDEN, G, threads=8)
        assert rel_l2(y.download(np.float32, n), want) <= 1e-5, info.name
    m.close()


def test_embedding_rows_from_uploaded_table(gpu, orc, i4_file):
    path, ts = i4_file
    m = gpu.ModelFile(path)
    m.upload()
    emb = m.get("model.embed_tokens.weight")
    rows = np.array([0, 1, VOCAB - 1, 17, 17, 1234], np.int32)
    dr = gpu.DeviceBuffer.from_array(rows)
    dout = gpu.DeviceBuffer(4 * HIDDEN * len(rows))
    gpu.dequant_i4_rows_dev(emb.device, dr, len(rows), HIDDEN, G, dout)
    gpu.synchronize()
    got = dout.download(np.float32, HIDDEN * len(rows)).reshape(len(rows), HIDDEN)
    table = np.frombuffer(ts["model.embed_tokens.weight"]["data"], np.uint8)
    for t, r in enumerate(rows):
        want = orc.dequant_i4_row(table, int(r), HIDDEN, G)
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), r
    m.close()


def test_vq2_file_upload_and_matvec(gpu, orc, tmp_path):
    img, ts = tf.vq2_model(group_size=64, hidden=1024, vocab=300, seed=3)
    path = tmp_path / "vq2.tqwen"
    path.write_bytes(bytes(img))
    m = gpu.ModelFile(str(path))
    m.upload()
    x = gpu.synth_normal(2048, seed=13)
    dx = gpu.DeviceBuffer.from_array(x)
    for t in ts:
        if t["dtype"] != tf.VQ2:
            continue
        info = m.get(t["name"])
        M, K = int(info.shape[0]), int(info.shape[1])
        dy = gpu.DeviceBuffer(4 * M)
        gpu.matvec_vq2_dev(info.device, dx, dy, M, K)
        gpu.synchronize()
        want = orc.matvec_vq2(np.frombuffer(t["data"], np.uint8), x[:K], M, K, threads=8)
        assert rel_l2(dy.download(np.float32, M), want) <= 1e-5, t["name"]
    m.close()


def test_upload_refuses_a_file_changed_since_inspect(gpu, tmp_path):
    img, _ = tf.i4_model(group_size=64, hidden=128, inter=256, vocab=100)
    path = tmp_path / "changed.tqwen"
    path.write_bytes(bytes(img))
    m = gpu.ModelFile(str(path))
    with open(path, "ab") as f:
        f.write(b"\0" * 64)
    assert gpu.lib().tqhip_model_upload(m._h) == gpu.EFILE
    assert m.tensor_at(0).device is None
    m.close()
