"""Writes synthetic .tqwen model images: the models the decode engine is benchmarked and
smoke-tested on (random weights of a named architecture) and the files the loader tests feed.

The layout is runtime/tiny_format.h:219-315 of tiny-llm: a 192-byte header, a
table of 120-byte entries, then tensor payloads at 64-byte aligned offsets; the
file ends at the aligned end of its last payload, as tests/test_loader.cpp:31-104
of tiny-llm writes it. Fields are little-endian at the offsets below.
"""
from __future__ import annotations

import struct

import numpy as np

HEADER_BYTES, ENTRY_BYTES, ALIGN = 192, 120, 64
F32, F16, I8, I4, VQ2, GPTQ4 = 0, 1, 2, 3, 4, 5

# TinyHeader (tiny_format.h:219-237), TinyHeaderV2Ext at 96 (:251-266), TinyHeaderV3Ext at 160 (:277-286)
HEADER_FIELDS = {
    "version": (8, "<I"), "dtype": (12, "<I"), "n_layers": (16, "<I"), "hidden_size": (20, "<I"),
    "intermediate_size": (24, "<I"), "n_heads": (28, "<I"), "n_kv_heads": (32, "<I"), "head_dim": (36, "<I"),
    "vocab_size": (40, "<I"), "max_seq_len": (44, "<I"), "tied_embeddings": (48, "<I"),
    "reserved_u32": (52, "<I"), "rms_norm_eps": (56, "<f"), "rope_theta": (60, "<f"),
    "tensor_count": (64, "<Q"), "tensor_table_offset": (72, "<Q"), "data_offset": (80, "<Q"),
    "total_bytes": (88, "<Q"),
    "model_type": (96, "<I"), "linear_num_qk_heads": (100, "<I"), "linear_num_v_heads": (104, "<I"),
    "linear_qk_head_dim": (108, "<I"), "linear_v_head_dim": (112, "<I"), "linear_conv_kernel_dim": (116, "<I"),
    "full_attention_interval": (120, "<I"), "partial_rotary_factor": (124, "<f"), "eos_token_id": (128, "<I"),
    "v2_pad": (132, "<I"), "quant_group_size": (136, "<I"),
    "n_routed_experts": (160, "<I"), "num_experts_per_tok": (164, "<I"), "moe_intermediate_size": (168, "<I"),
    "shared_expert_intermediate_size": (172, "<I"), "n_shared_experts": (176, "<I"), "moe_topk_norm": (180, "<I"),
    "gptq_group_size": (184, "<I"), "v3_pad": (188, "<I"),
}
# TensorEntry (tiny_format.h:298-305)
ENTRY_FIELDS = {"dtype": (64, "<I"), "ndim": (68, "<I"), "shape0": (72, "<Q"), "shape1": (80, "<Q"),
                "shape2": (88, "<Q"), "shape3": (96, "<Q"), "offset": (104, "<Q"), "nbytes": (112, "<Q")}

DEFAULT_CONFIG = dict(n_layers=2, hidden_size=4, intermediate_size=8, n_heads=2, n_kv_heads=1, head_dim=2,
                      vocab_size=16, max_seq_len=32, tied_embeddings=1, rms_norm_eps=1e-6, rope_theta=1e6)


def align(x: int) -> int:
    return (x + ALIGN - 1) // ALIGN * ALIGN


def tensor(name: str, dtype: int, shape, data) -> dict:
    return {"name": name, "dtype": dtype, "shape": tuple(int(s) for s in shape), "data": bytes(data)}


def f32_tensor(name: str, values, shape=None) -> dict:
    a = np.asarray(values, dtype=np.float32)
    return tensor(name, F32, shape if shape is not None else a.shape, a.tobytes())


def build(tensors: list, *, version: int = 3, dtype: int = F32, **fields) -> bytearray:
    """A complete .tqwen image; `fields` override any HEADER_FIELDS entry."""
    data_offset = align(HEADER_BYTES + len(tensors) * ENTRY_BYTES)
    offsets, off = [], data_offset
    for t in tensors:
        offsets.append(off)
        off = align(off + len(t["data"]))
    total = max(off, data_offset)
    buf = bytearray(total)
    buf[0:8] = b"TINYQWEN"
    values = dict(DEFAULT_CONFIG, version=version, dtype=dtype, tensor_count=len(tensors),
                  tensor_table_offset=HEADER_BYTES, data_offset=data_offset, total_bytes=total)
    values.update(fields)
    for k, v in values.items():
        set_header(buf, k, v)
    for i, t in enumerate(tensors):
        base = HEADER_BYTES + i * ENTRY_BYTES
        name = t["name"].encode()
        assert len(name) <= 64
        buf[base:base + len(name)] = name
        set_entry(buf, i, "dtype", t["dtype"])
        set_entry(buf, i, "ndim", len(t["shape"]))
        for d, s in enumerate(t["shape"]):
            set_entry(buf, i, f"shape{d}", s)
        set_entry(buf, i, "offset", offsets[i])
        set_entry(buf, i, "nbytes", len(t["data"]))
        buf[offsets[i]:offsets[i] + len(t["data"])] = t["data"]
    return buf


def set_header(buf: bytearray, field: str, value) -> None:
    off, fmt = HEADER_FIELDS[field]
    struct.pack_into(fmt, buf, off, value)


def get_header(buf, field: str):
    off, fmt = HEADER_FIELDS[field]
    return struct.unpack_from(fmt, buf, off)[0]


def set_entry(buf: bytearray, i: int, field: str, value) -> None:
    off, fmt = ENTRY_FIELDS[field]
    struct.pack_into(fmt, buf, HEADER_BYTES + i * ENTRY_BYTES + off, value)


def get_entry(buf, i: int, field: str):
    off, fmt = ENTRY_FIELDS[field]
    return struct.unpack_from(fmt, buf, HEADER_BYTES + i * ENTRY_BYTES + off)[0]


def set_entry_name(buf: bytearray, i: int, name: bytes) -> None:
    base = HEADER_BYTES + i * ENTRY_BYTES
    buf[base:base + 64] = name.ljust(64, b"\0")[:64]


def i4_payload(rows: int, cols: int, group_size: int, seed: int) -> bytes:
    """Random i4 rows (runtime/tiny_format.h:58-77): per group fp16 scale, fp16 zero, group_size/2 code bytes."""
    rng = np.random.default_rng(seed)
    groups = (cols + group_size - 1) // group_size
    gb = 4 + group_size // 2
    w = np.zeros((rows, groups, gb), np.uint8)
    w[:, :, 0:2] = rng.uniform(0.002, 0.02, (rows, groups)).astype(np.float16)[..., None].view(np.uint8)
    w[:, :, 2:4] = rng.uniform(6.0, 9.0, (rows, groups)).astype(np.float16)[..., None].view(np.uint8)
    w[:, :, 4:] = rng.integers(0, 256, (rows, groups, gb - 4), dtype=np.uint8)
    return w.tobytes()


def vq2_payload(rows: int, cols: int, seed: int) -> bytes:
    """Random VQ2 tensor (runtime/tiny_format.h:79-103): 256x4 fp16 codebook, then rows x cols/4 indices."""
    rng = np.random.default_rng(seed)
    cb = rng.normal(0.0, 0.02, (256, 4)).astype(np.float16)
    idx = rng.integers(0, 256, (rows, cols // 4), dtype=np.uint8)
    return cb.tobytes() + idx.tobytes()


def i4_model(group_size: int = 64, hidden: int = 256, inter: int = 512, vocab: int = 1000, layers: int = 1,
             seed: int = 0, version: int = 3, **fields) -> tuple:
    """A small dense Qwen2-shaped i4 file (names as the runtime binds them); returns (image, tensors)."""
    ts = [tensor("model.embed_tokens.weight", I4, (vocab, hidden), i4_payload(vocab, hidden, group_size, seed))]
    for layer in range(layers):
        p = f"model.layers.{layer}."
        ts.append(f32_tensor(p + "input_layernorm.weight", np.ones(hidden)))
        for j, (n, o, i) in enumerate([("self_attn.q_proj", hidden, hidden), ("self_attn.k_proj", 64, hidden),
                                       ("self_attn.v_proj", 64, hidden), ("self_attn.o_proj", hidden, hidden),
                                       ("mlp.gate_proj", inter, hidden), ("mlp.up_proj", inter, hidden),
                                       ("mlp.down_proj", hidden, inter)]):
            ts.append(tensor(p + n + ".weight", I4, (o, i), i4_payload(o, i, group_size, seed + 10 * layer + j + 1)))
        ts.append(f32_tensor(p + "self_attn.q_proj.bias", np.linspace(-1, 1, hidden)))
    ts.append(f32_tensor("model.norm.weight", np.ones(hidden)))
    ts.append(tensor("lm_head.weight", I4, (vocab, hidden), i4_payload(vocab, hidden, group_size, seed + 999)))
    cfg = dict(n_layers=layers, hidden_size=hidden, intermediate_size=inter, n_heads=4, n_kv_heads=1,
               head_dim=64, vocab_size=vocab, max_seq_len=128, quant_group_size=group_size)
    cfg.update(fields)
    return build(ts, version=version, dtype=I4, **cfg), ts


def vq2_model(group_size: int = 64, hidden: int = 256, vocab: int = 500, seed: int = 0, **fields) -> tuple:
    """A small VQ2 file: VQ2 projections, f16 and f32 vectors and a compact-i4 embedding."""
    ts = [tensor("model.embed_tokens.weight", I4, (vocab, hidden), i4_payload(vocab, hidden, group_size, seed)),
          tensor("model.layers.0.self_attn.q_proj.weight", VQ2, (hidden, hidden), vq2_payload(hidden, hidden, seed + 1)),
          tensor("model.layers.0.mlp.down_proj.weight", VQ2, (hidden, 2 * hidden),
                 vq2_payload(hidden, 2 * hidden, seed + 2)),
          tensor("model.layers.0.input_layernorm.weight", F16, (hidden,), np.ones(hidden, np.float16).tobytes()),
          f32_tensor("model.norm.weight", np.ones(hidden))]
    cfg = dict(n_layers=1, hidden_size=hidden, intermediate_size=2 * hidden, n_heads=4, n_kv_heads=1, head_dim=64,
               vocab_size=vocab, max_seq_len=128, quant_group_size=group_size)
    cfg.update(fields)
    return build(ts, version=3, dtype=VQ2, **cfg), ts


def dense_i4_model(hidden=896, n_heads=14, n_kv_heads=2, head_dim=64, inter=4864, vocab=2000, layers=2,
                   group_size=64, tied=True, biases=True, qk_norm=False, embed_f32=False, seed=0,
                   max_seq_len=256, vq2=False, rotated=False) -> tuple:
    """A dense Qwen2.x-shaped i4 file with every tensor QwenModel binds (runtime/qwen_model.cpp:437-640):
    embedding (i4, or fp32), per layer two RMSNorm weights, q/k/v/o and gate/up/down (i4), optional
    q/k/v biases and q/k norms, the final norm and, when not tied, lm_head. Norm weights are drawn
    around 1 and biases around 0. vq2=True writes a VQ2 file instead: VQ2 projections, fp16
    norms and biases, the compact-i4 embedding (runtime/model_loader.cpp:394-404, 705-719).
    rotated=True adds BiIP rotation vectors (rot_sign of +-1, rot_scale around 1) to every
    projection (runtime/qwen_model.cpp:427-435, 641-647).
    Returns (image, config dict, {name: (dtype, shape, bytes)})."""
    rng = np.random.default_rng(seed)
    qd, kvd = n_heads * head_dim, n_kv_heads * head_dim
    ts = []

    def vec(name, n, mean, std):
        v = rng.normal(mean, std, n)
        ts.append(tensor(name, F16, (n,), v.astype(np.float16).tobytes()) if vq2 else f32_tensor(name, v))

    def rot(prefix, n):
        if rotated:
            sign = np.where(rng.random(n) < 0.5, -1.0, 1.0)
            ts.append(tensor(prefix + ".rot_sign", F16, (n,), sign.astype(np.float16).tobytes()) if vq2
                      else f32_tensor(prefix + ".rot_sign", sign))
            vec(prefix + ".rot_scale", n, 1.0, 0.2)

    def mat(name, rows, cols, i4=False):
        if vq2 and not i4:
            ts.append(tensor(name, VQ2, (rows, cols), vq2_payload(rows, cols, int(rng.integers(1 << 30)))))
        else:
            ts.append(tensor(name, I4, (rows, cols), i4_payload(rows, cols, group_size, int(rng.integers(1 << 30)))))

    if embed_f32:
        ts.append(f32_tensor("model.embed_tokens.weight", rng.normal(0, 0.05, (vocab, hidden)).astype(np.float32)))
    else:
        mat("model.embed_tokens.weight", vocab, hidden, i4=True)
    for li in range(layers):
        p = f"model.layers.{li}."
        vec(p + "input_layernorm.weight", hidden, 1.0, 0.1)
        vec(p + "post_attention_layernorm.weight", hidden, 1.0, 0.1)
        mat(p + "self_attn.q_proj.weight", qd, hidden)
        mat(p + "self_attn.k_proj.weight", kvd, hidden)
        mat(p + "self_attn.v_proj.weight", kvd, hidden)
        mat(p + "self_attn.o_proj.weight", hidden, qd)
        if biases:
            vec(p + "self_attn.q_proj.bias", qd, 0.0, 0.1)
            vec(p + "self_attn.k_proj.bias", kvd, 0.0, 0.1)
            vec(p + "self_attn.v_proj.bias", kvd, 0.0, 0.1)
        if qk_norm:
            vec(p + "self_attn.q_norm.weight", head_dim, 1.0, 0.1)
            vec(p + "self_attn.k_norm.weight", head_dim, 1.0, 0.1)
        mat(p + "mlp.gate_proj.weight", inter, hidden)
        mat(p + "mlp.up_proj.weight", inter, hidden)
        mat(p + "mlp.down_proj.weight", hidden, inter)
        for n, k in (("self_attn.q_proj", hidden), ("self_attn.k_proj", hidden), ("self_attn.v_proj", hidden),
                     ("self_attn.o_proj", qd), ("mlp.gate_proj", hidden), ("mlp.up_proj", hidden),
                     ("mlp.down_proj", inter)):
            rot(p + n, k)
    vec("model.norm.weight", hidden, 1.0, 0.1)
    if not tied or embed_f32:
        mat("lm_head.weight", vocab, hidden)
    cfg = dict(n_layers=layers, hidden_size=hidden, intermediate_size=inter, n_heads=n_heads,
               n_kv_heads=n_kv_heads, head_dim=head_dim, vocab_size=vocab, max_seq_len=max_seq_len,
               tied_embeddings=int(tied), rms_norm_eps=1e-6, rope_theta=1e6, quant_group_size=group_size)
    img = build(ts, version=3, dtype=VQ2 if vq2 else I4, **cfg)
    return img, cfg, {t["name"]: (t["dtype"], t["shape"], t["data"]) for t in ts}
