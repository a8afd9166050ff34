""".tqwen reader and validator (tqhip_model_inspect) against tiny-llm's own loader.

Two kinds of check, both on the CPU (inspect reads files only):
  * the cases of tiny-llm's tests/test_loader.cpp:166-505, restated with their
    expected values (round trip, bad magic, truncation, duplicates, f16 files,
    mixed dtypes, the v2 extension, the v1 default, a bad interval);
  * a corpus of corrupted files, one field of every validation stage
    (runtime/model_loader.cpp:302-740) per case, each loaded by this library
    and by the compiled reference loader (oracle/_ref): both accept or both
    reject, with the same message, and an accepted file has the same tensor
    table. GPTQ files and the MoE model types are rejected here on purpose
    (this library does not serve them).
"""
import ctypes
import math
import os
import re

import numpy as np
import pytest

from conftest import load_package

tf = load_package().tqwen_synth  # synthetic .tqwen images



def write(tmp_path, image, name="m.tqwen"):
    p = tmp_path / name
    p.write_bytes(bytes(image))
    return str(p)


def ours(tqa, path):
    """(accepted, message, table, (quant_group_size, model_type))."""
    try:
        m = tqa.ModelFile(path)
    except ValueError as e:
        return False, str(e), None, None
    table = [(i.name.decode(), i.dtype, i.ndim, tuple(i.shape), i.offset, i.nbytes)
             for i in (m.tensor_at(k) for k in range(m.tensor_count()))]
    out = True, "", table, (m.quant_group_size, m.model_type)
    m.close()
    return out


def reference(r, path):
    err = ctypes.create_string_buffer(512)
    if not r.tqref_model_load(path.encode(), err, len(err)):
        return False, err.value.decode(), None, None
    table = []
    name = ctypes.create_string_buffer(65)
    dtype, ndim = ctypes.c_int(), ctypes.c_int()
    shape = (ctypes.c_uint64 * 4)()
    off, nb = ctypes.c_uint64(), ctypes.c_uint64()
    for k in range(r.tqref_model_tensor_count()):
        assert r.tqref_model_tensor_at(k, name, ctypes.byref(dtype), ctypes.byref(ndim), shape, ctypes.byref(off),
                                       ctypes.byref(nb))
        table.append((name.value.decode(), dtype.value, ndim.value, tuple(shape), off.value, nb.value))
    return True, "", table, (r.tqref_model_quant_group_size(), r.tqref_model_type())


# ---- tiny-llm's own loader tests (tests/test_loader.cpp), expected values as written there -------

def sample(dtype=tf.F32):
    vals = [("a.weight", (2, 3), [0, 1, 2, 3, 4, 5]), ("b", (4,), [-1, 0.5, 2.25, 7])]
    if dtype == tf.F32:
        return [tf.f32_tensor(n, v, s) for n, s, v in vals]
    return [tf.tensor(n, tf.F16, s, np.asarray(v, np.float16).tobytes()) for n, s, v in vals]


def test_round_trip(tqa, tmp_path):
    img = tf.build(sample())
    m = tqa.ModelFile(write(tmp_path, img))
    assert m.tensor_count() == 2 and m.tensor_names() == ["a.weight", "b"]
    a = m.get("a.weight")
    assert (a.ndim, a.shape[0], a.shape[1], a.dtype) == (2, 2, 3, tf.F32)
    assert a.offset % 64 == 0 and a.device is None
    assert np.array_equal(np.frombuffer(bytes(img[a.offset:a.offset + a.nbytes]), np.float32), np.arange(6))
    b = m.get("b")
    assert np.frombuffer(bytes(img[b.offset:b.offset + b.nbytes]), np.float32)[3] == 7.0
    assert m.get("missing") is None
    assert (m.quant_group_size, m.model_type, m.dtype) == (0, 0, tf.F32)


def test_rejects_bad_magic(tqa, tmp_path):
    img = tf.build(sample())
    img[0] = ord("X")
    with pytest.raises(ValueError, match="magic"):
        tqa.ModelFile(write(tmp_path, img))


def test_rejects_truncated_file(tqa, tmp_path):
    img = tf.build(sample())
    with pytest.raises(ValueError, match="."):
        tqa.ModelFile(write(tmp_path, img[:-64]))


def test_rejects_duplicate_names(tqa, tmp_path):
    ts = sample()
    ts[1]["name"] = "a.weight"
    with pytest.raises(ValueError, match="duplicate"):
        tqa.ModelFile(write(tmp_path, tf.build(ts)))


def test_accepts_f16(tqa, tmp_path):
    img = tf.build(sample(tf.F16), dtype=tf.F16)
    m = tqa.ModelFile(write(tmp_path, img))
    a = m.get("a.weight")
    assert m.dtype == tf.F16 and a.dtype == tf.F16 and a.nbytes == 12
    assert np.array_equal(np.frombuffer(bytes(img[a.offset:a.offset + 12]), np.float16), np.arange(6))


def test_rejects_mixed_dtype(tqa, tmp_path):
    img = tf.build(sample())
    tf.set_entry(img, 0, "dtype", tf.F16)
    with pytest.raises(ValueError, match="dtype"):
        tqa.ModelFile(write(tmp_path, img))


QWEN35 = dict(model_type=1, linear_num_qk_heads=2, linear_num_v_heads=2, linear_qk_head_dim=4, linear_v_head_dim=4,
              linear_conv_kernel_dim=4, full_attention_interval=2, partial_rotary_factor=0.25, eos_token_id=248044)


def test_v2_qwen35_extension(tqa, tmp_path):
    m = tqa.ModelFile(write(tmp_path, tf.build(sample(), **QWEN35)))
    assert m.model_type == 1


def test_v1_defaults_to_qwen2(tqa, tmp_path):
    m = tqa.ModelFile(write(tmp_path, tf.build(sample(), version=1, **QWEN35)))  # v1 ignores the extension
    assert m.model_type == 0


def test_v2_rejects_bad_interval(tqa, tmp_path):
    with pytest.raises(ValueError, match="interval|divisible"):
        tqa.ModelFile(write(tmp_path, tf.build(sample(), **dict(QWEN35, full_attention_interval=3))))


# ---- the corruption corpus, against the compiled reference loader --------------------------------

def i4_base():
    return tf.i4_model(group_size=64, hidden=128, inter=256, vocab=100)[0]


def mutate_header(**kv):
    def f(img):
        for k, v in kv.items():
            tf.set_header(img, k, v)
        return img
    return f


def mutate_entry(i, **kv):
    def f(img):
        for k, v in kv.items():
            tf.set_entry(img, i, k, v)
        return img
    return f


def truncate(n):
    return lambda img: img[:n]


def entry_name(i, name):
    def f(img):
        tf.set_entry_name(img, i, name)
        return img
    return f


def rebuilt(**kw):
    return lambda img: tf.i4_model(group_size=64, hidden=128, inter=256, vocab=100, **kw)[0]


# (case id, mutation of the valid i4 file, how the outcome is compared):
#   False         -- same outcome, message and table as the reference;
#   True          -- rejected here as unsupported (GPTQ, MoE);
#   "any_tensor"  -- several tensors fail the same check: the reference names the
#                    first in its hash-map order, this library the first in file order.
CORPUS = [
    ("valid", lambda img: img, False),
    ("too_small", truncate(100), False),
    ("magic", lambda img: img[:7] + b"M" + img[8:], False),
    ("version0", mutate_header(version=0), False),
    ("version4", mutate_header(version=4), False),
    ("version1_no_group", mutate_header(version=1), False),
    ("version2", mutate_header(version=2), False),
    ("dtype_i8", mutate_header(dtype=tf.I8), False),
    ("dtype_9", mutate_header(dtype=9), False),
    ("dtype_gptq", mutate_header(dtype=tf.GPTQ4), True),
    ("total_plus1", lambda img: mutate_header(total_bytes=len(img) + 1)(img), False),
    ("truncated64", lambda img: img[:-64], False),
    ("table_offset", mutate_header(tensor_table_offset=256), False),
    ("count0", mutate_header(tensor_count=0), False),
    ("count_huge", mutate_header(tensor_count=100001), False),
    ("table_past_end", lambda img: mutate_header(tensor_count=len(img) // 120)(img), False),
    ("data_offset_unaligned", lambda img: mutate_header(data_offset=tf.get_header(img, "data_offset") + 8)(img), False),
    ("data_offset_low", mutate_header(data_offset=128), False),
    ("data_offset_past_end", lambda img: mutate_header(data_offset=len(img) + 64)(img), False),
    ("zero_layers", mutate_header(n_layers=0), False),
    ("zero_vocab", mutate_header(vocab_size=0), False),
    ("zero_seq", mutate_header(max_seq_len=0), False),
    ("gqa", mutate_header(n_heads=3, n_kv_heads=2), False),
    ("eps0", mutate_header(rms_norm_eps=0.0), False),
    ("eps_neg", mutate_header(rms_norm_eps=-1e-6), False),
    ("theta0", mutate_header(rope_theta=0.0), False),
    ("eps_nan", mutate_header(rms_norm_eps=math.nan), False),
    ("ndim0", mutate_entry(1, ndim=0), False),
    ("ndim5", mutate_entry(1, ndim=5), False),
    ("f16_in_i4", mutate_entry(1, dtype=tf.F16), False),
    ("vq2_in_i4", mutate_entry(2, dtype=tf.VQ2), False),
    ("zero_shape", mutate_entry(2, shape1=0), False),
    ("trailing_shape", mutate_entry(1, shape1=5), False),
    ("i4_3d", mutate_entry(2, ndim=3, shape2=1), False),
    ("f32_nbytes", mutate_entry(1, nbytes=4 * 128 + 4), False),
    ("offset_unaligned", lambda img: mutate_entry(2, offset=tf.get_entry(img, 2, "offset") + 32)(img), False),
    ("offset_low", mutate_entry(2, offset=64), False),
    ("payload_past_end", lambda img: mutate_entry(2, nbytes=len(img))(img), False),
    ("empty_name", entry_name(3, b""), False),
    ("duplicate", entry_name(3, b"model.layers.0.self_attn.q_proj.weight"), False),
    ("name_64", entry_name(3, b"n" * 64), False),
    ("name_after_nul", entry_name(3, b"x\0y"), False),
    ("model_type4", mutate_header(model_type=4), False),
    ("model_type_moe", mutate_header(model_type=2), True),
    ("model_type_qwen3moe", mutate_header(model_type=3), True),
    ("moe_valid_for_reference", rebuilt(model_type=3, n_routed_experts=8, num_experts_per_tok=2,
                                        moe_intermediate_size=64, gptq_group_size=128), True),
    ("v2_pad", mutate_header(v2_pad=1), False),
    ("qwen35_valid", rebuilt(n_layers=2, layers=2, **QWEN35), False),
    ("qwen35_zero_heads", rebuilt(n_layers=2, layers=2, **dict(QWEN35, linear_num_qk_heads=0)), False),
    ("qwen35_conv1", rebuilt(n_layers=2, layers=2, **dict(QWEN35, linear_conv_kernel_dim=1)), False),
    ("qwen35_interval1", rebuilt(n_layers=2, layers=2, **dict(QWEN35, full_attention_interval=1)), False),
    ("qwen35_interval3", rebuilt(n_layers=2, layers=2, **dict(QWEN35, full_attention_interval=3)), False),
    ("qwen35_rotary0", rebuilt(n_layers=2, layers=2, **dict(QWEN35, partial_rotary_factor=0.0)), False),
    ("qwen35_rotary_big", rebuilt(n_layers=2, layers=2, **dict(QWEN35, partial_rotary_factor=1.5)), False),
    ("qwen35_rotary_nan", rebuilt(n_layers=2, layers=2, **dict(QWEN35, partial_rotary_factor=math.nan)), False),
    ("qwen35_heads_ratio", rebuilt(n_layers=2, layers=2, **dict(QWEN35, linear_num_v_heads=3)), False),
    ("v3_pad", mutate_header(v3_pad=7), False),
    ("v3_pad_in_v2_file", mutate_header(version=2, v3_pad=7), False),
    ("moe_fields_dense", mutate_header(n_routed_experts=8, gptq_group_size=128), False),
    ("group0", mutate_header(quant_group_size=0), False),
    ("group1025", mutate_header(quant_group_size=1025), False),
    ("group_odd", mutate_header(quant_group_size=63), False),
    ("group32", mutate_header(quant_group_size=32), "any_tensor"),
    ("i4_nbytes", lambda img: mutate_entry(2, nbytes=tf.get_entry(img, 2, "nbytes") - 36)(img), False),
    ("group_128_rebuilt", lambda img: tf.i4_model(group_size=128, hidden=128, inter=256, vocab=100)[0], False),
    ("group_40_ragged", lambda img: tf.i4_model(group_size=40, hidden=100, inter=130, vocab=33)[0], False),
]


def vq2_corpus():
    base = lambda **kw: tf.vq2_model(hidden=128, vocab=50, **kw)[0]
    return [
        ("vq2_valid", base(), False),
        ("vq2_group_odd_embed", tf.vq2_model(hidden=128, vocab=50, group_size=33)[0], False),
        ("vq2_no_group", base(quant_group_size=0), False),
        ("vq2_in_dim", mutate_entry(1, shape1=126)(base()), False),
        ("vq2_nbytes", mutate_entry(2, nbytes=2048 + 128 * 64 - 4)(base()), False),
        ("vq2_embed_nbytes", mutate_entry(0, nbytes=50 * 2 * 36 - 36)(base()), False),
        ("vq2_f32_in_vq2", mutate_entry(3, dtype=tf.F32)(base()), False),
        ("vq2_i8_entry", mutate_entry(3, dtype=tf.I8)(base()), False),
    ]


def f32_corpus():
    return [
        ("f32_valid", tf.build(sample()), False),
        ("f16_valid", tf.build(sample(tf.F16), dtype=tf.F16), False),
        ("f16_entry_in_f32", mutate_entry(0, dtype=tf.F16)(tf.build(sample())), False),
        ("f32_v1", tf.build(sample(), version=1), False),
        ("f32_qwen35_v1_ignored", tf.build(sample(), version=1, model_type=9), False),
    ]


def all_cases():
    cases = [(cid, fn(i4_base()), unsup) for cid, fn, unsup in CORPUS]
    return cases + vq2_corpus() + f32_corpus()


@pytest.fixture(scope="module")
def ref(orc):
    r = orc.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref not built here (it needs the reference tree)")
    return r


@pytest.mark.parametrize("cid,image,unsupported", all_cases(), ids=[c[0] for c in all_cases()])
def test_corpus_matches_reference_loader(tqa, ref, tmp_path, cid, image, unsupported):
    path = write(tmp_path, image)
    got, want = ours(tqa, path), reference(ref, path)
    if unsupported is True:
        assert not got[0]
        assert "not served by this library" in got[1]
        if cid == "moe_valid_for_reference":
            assert want[0], want[1]
        return
    assert got[0] == want[0], (cid, got[1], want[1])
    if unsupported == "any_tensor":
        same_check = lambda msg: re.sub(r"tensor '[^']*'", "tensor '*'", msg).split(", expected")[0]
        assert same_check(got[1]) == same_check(want[1])
    else:
        assert got[1] == want[1]
    assert got[2] == want[2]
    assert got[3] == want[3]


def test_corpus_covers_accepts_and_rejects(tqa, tmp_path):
    """The corpus is only a check if both outcomes occur in it many times over."""
    outcomes = [ours(tqa, write(tmp_path, img, f"{cid}.tqwen"))[0] for cid, img, _ in all_cases()]
    assert sum(outcomes) >= 10 and len(outcomes) - sum(outcomes) >= 40


def test_missing_file_and_find(tqa, tmp_path):
    with pytest.raises(ValueError, match="cannot open file"):
        tqa.ModelFile(str(tmp_path / "absent.tqwen"))
    img, ts = tf.i4_model(group_size=64, hidden=128, inter=256, vocab=100)
    m = tqa.ModelFile(write(tmp_path, img))
    assert m.tensor_names() == [t["name"] for t in ts]
    for t in ts:
        info = m.get(t["name"])
        assert info.nbytes == len(t["data"]) and info.dtype == t["dtype"]
        assert tuple(info.shape[:len(t["shape"])]) == t["shape"]
        assert bytes(img[info.offset:info.offset + info.nbytes]) == t["data"]
    assert m.quant_group_size == 64 and m.dtype == tf.I4


def test_close_refused_while_an_engine_is_open(tqa, tmp_path):
    """ModelFile.close() frees the HBM copy a DecodeEngine's captured step reads: the binding
    refuses it while an engine built on the model is open. (No GPU: the engine here is a
    stand-in object registered the way DecodeEngine.__init__ registers itself.)"""
    import weakref
    img, _ = tf.i4_model(group_size=64, hidden=128, inter=256, vocab=100)
    m = tqa.ModelFile(write(tmp_path, img))
    eng = tqa.DecodeEngine.__new__(tqa.DecodeEngine)
    eng._h = 12345  # an open handle (never passed to the library here)
    m._engines = weakref.WeakSet([eng])
    with pytest.raises(RuntimeError, match="still use this model"):
        m.close()
    assert m._h
    eng._h = None  # the engine was closed
    m.close()
    assert m._h is None
    with pytest.raises(ValueError, match="closed"):
        tqa.DecodeEngine(m)
