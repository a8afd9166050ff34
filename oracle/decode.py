"""CPU restatement of tiny-llm's dense decode step -- TEST INFRASTRUCTURE ONLY.

The checker of the device-resident decode engine. One token through a dense
Qwen2.x / Qwen3 model as QwenModel::forward_token runs it
(runtime/qwen_forward_token.cpp:83-700, the full-attention branch):

  embedding row      dequant_i4_row (kernels/ref_ops.h:183-205) or the fp32 row
  rmsnorm            kernels/rmsnorm/rmsnorm_ref.cpp:14-30
  q/k/v, o, gate/up, down, lm_head projections
                     matvec_i4 / matvec_vq2 by the tensor's dtype (the C restatement
                     in oracle.cpp); fp16 vectors of VQ2 files converted once
  biases, q/k norm   runtime/qwen_forward_token.cpp:338-372
  rope               kernels/rope/rope_ref.cpp:13-56
  KV write           runtime/kv_cache.h:118-129 ([layer][kv_head][max_seq][head_dim])
  attention          kernels/attention/attention_decode_ref.cpp:13-60 (online softmax,
                     positions in order)
  swiglu             kernels/silu/swiglu_ref.cpp:12-19
  argmax             kernels/argmax/argmax_ref.cpp:11-20 (first index of the maximum)
  BiIP rotation      biip_rotate (oracle/__init__.py) ahead of a projection carrying
                     rot_sign / rot_scale (runtime/qwen_model.cpp:229-238)

Every step keeps the reference's fp32 operation order; sums the reference
takes in double are taken in double. tests/test_decode_oracle.py pins this
against the compiled reference forward (oracle/_ref).
"""
from __future__ import annotations

import numpy as np

from . import biip_rotate, dequant_i4_row, halves_to_floats, matvec_i4, matvec_vq2

F32, F16, I4, VQ2 = 0, 1, 3, 4


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, np.float32)
    mean_sq = np.float32(np.sum(x.astype(np.float64) ** 2) / x.size)
    scale = np.float32(1.0) / np.sqrt(mean_sq + np.float32(eps), dtype=np.float32)
    return (x * scale) * np.asarray(w, np.float32)


def rope(x: np.ndarray, n_heads: int, head_dim: int, pos: int, theta: float) -> None:
    half = head_dim // 2
    i = np.arange(half, dtype=np.float32)
    exponent = -(np.float32(2) * i) / np.float32(head_dim)
    inv_freq = np.power(np.float32(theta), exponent, dtype=np.float32)
    angle = np.float32(pos) * inv_freq
    c, s = np.cos(angle, dtype=np.float32), np.sin(angle, dtype=np.float32)
    for h in range(n_heads):
        v = x[h * head_dim:(h + 1) * head_dim]
        x0, x1 = v[:half].copy(), v[half:].copy()
        v[:half] = x0 * c - x1 * s
        v[half:] = x1 * c + x0 * s


def attention(q, kcache, vcache, seq, n_heads, n_kv, head_dim, scale) -> np.ndarray:
    out = np.zeros(n_heads * head_dim, np.float32)
    per_kv = n_heads // n_kv
    scale = np.float32(scale)
    for h in range(n_heads):
        kv = h // per_kv
        qh = q[h * head_dim:(h + 1) * head_dim].astype(np.float64)
        o = np.zeros(head_dim, np.float32)
        m, l = np.float32(-np.inf), np.float32(0)
        for t in range(seq):
            s = np.float32(np.dot(qh, kcache[kv, t].astype(np.float64))) * scale
            m_new = s if s > m else m
            rescale = np.exp(np.float32(m - m_new), dtype=np.float32)
            p = np.exp(np.float32(s - m_new), dtype=np.float32)
            o = o * rescale + p * vcache[kv, t]
            l = l * rescale + p
            m = m_new
        out[h * head_dim:(h + 1) * head_dim] = o * (np.float32(1) / l)
    return out


def attention_f64(q, kcache, vcache, seq, n_heads, n_kv, head_dim, scale) -> np.ndarray:
    """The same attention in float64 with a two-pass softmax: not the reference's rounding, for
    sequences too long for the position-by-position loop (a tolerance check only)."""
    per_kv = n_heads // n_kv
    out = np.empty(n_heads * head_dim, np.float32)
    for h in range(n_heads):
        kv = h // per_kv
        s = kcache[kv, :seq].astype(np.float64) @ q[h * head_dim:(h + 1) * head_dim].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h * head_dim:(h + 1) * head_dim] = (p @ vcache[kv, :seq].astype(np.float64)) / p.sum()
    return out


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.asarray(gate, np.float32)
    return (g / (np.float32(1) + np.exp(-g, dtype=np.float32))) * up


def argmax(x: np.ndarray) -> int:
    return int(np.argmax(x))  # numpy also returns the first index of the maximum


class DenseDecoder:
    """One sequence through a dense i4 model given as {name: (dtype, shape, bytes)} plus its config."""

    def __init__(self, config: dict, tensors: dict, max_seq_len: int, exact_attention: bool = True):
        self.attention = attention if exact_attention else attention_f64
        self.c = config
        self.t = tensors
        self.gs = config["quant_group_size"]
        hd, nkv = config["head_dim"], config["n_kv_heads"]
        self.k = np.zeros((config["n_layers"], nkv, max_seq_len, hd), np.float32)
        self.v = np.zeros_like(self.k)
        self.pos = 0

    def _vec(self, name):
        if name not in self.t:
            return None
        dt, _, data = self.t[name]
        if dt == F16:  # bound as fp32 once (runtime/qwen_model.cpp:182-190)
            return halves_to_floats(np.frombuffer(data, np.uint16))
        return np.frombuffer(data, np.float32)

    def _mv(self, name, x, out_dim, in_dim):
        dt, _, data = self.t[name]
        w = np.frombuffer(data, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        prefix = name[:-len(".weight")]
        sign = self._vec(prefix + ".rot_sign")
        if sign is not None:  # mv_rot (runtime/qwen_model.cpp:229-238), bind_rot's block size (:59-66, 427-435)
            bs = next((b for b in (256, 128, 64, 32, 16, 8, 4, 2) if in_dim % b == 0), 1)
            x = biip_rotate(x, self._vec(prefix + ".rot_scale"), sign, bs)
        if dt == VQ2:
            return matvec_vq2(w, x, out_dim, in_dim, threads=8)
        return matvec_i4(w, x, out_dim, in_dim, self.gs, threads=8)

    def step(self, token: int) -> np.ndarray:
        c = self.c
        H, I, V = c["hidden_size"], c["intermediate_size"], c["vocab_size"]
        nh, nkv, hd, eps = c["n_heads"], c["n_kv_heads"], c["head_dim"], c["rms_norm_eps"]
        qd, kvd = nh * hd, nkv * hd
        dt, _, data = self.t["model.embed_tokens.weight"]
        if dt == I4:
            hidden = dequant_i4_row(np.frombuffer(data, np.uint8), token, H, self.gs).astype(np.float32)
        else:
            hidden = np.frombuffer(data, np.float32)[token * H:(token + 1) * H].copy()
        pos = self.pos
        for li in range(c["n_layers"]):
            p = f"model.layers.{li}."
            normed = rmsnorm(hidden, self._vec(p + "input_layernorm.weight"), eps)
            q = self._mv(p + "self_attn.q_proj.weight", normed, qd, H)
            k = self._mv(p + "self_attn.k_proj.weight", normed, kvd, H)
            v = self._mv(p + "self_attn.v_proj.weight", normed, kvd, H)
            for y, n in ((q, "q"), (k, "k"), (v, "v")):
                b = self._vec(p + f"self_attn.{n}_proj.bias")
                if b is not None:
                    y += b
            qn, kn = self._vec(p + "self_attn.q_norm.weight"), self._vec(p + "self_attn.k_norm.weight")
            if qn is not None:
                for h in range(nh):
                    q[h * hd:(h + 1) * hd] = rmsnorm(q[h * hd:(h + 1) * hd], qn, eps)
                for h in range(nkv):
                    k[h * hd:(h + 1) * hd] = rmsnorm(k[h * hd:(h + 1) * hd], kn, eps)
            rope(q, nh, hd, pos, c["rope_theta"])
            rope(k, nkv, hd, pos, c["rope_theta"])
            self.k[li, :, pos] = k.reshape(nkv, hd)
            self.v[li, :, pos] = v.reshape(nkv, hd)
            attn = self.attention(q, self.k[li], self.v[li], pos + 1, nh, nkv, hd,
                             np.float32(1) / np.sqrt(np.float32(hd)))
            hidden = hidden + self._mv(p + "self_attn.o_proj.weight", attn, H, qd)
            normed = rmsnorm(hidden, self._vec(p + "post_attention_layernorm.weight"), eps)
            g = self._mv(p + "mlp.gate_proj.weight", normed, I, H)
            u = self._mv(p + "mlp.up_proj.weight", normed, I, H)
            hidden = hidden + self._mv(p + "mlp.down_proj.weight", swiglu(g, u), H, I)
        normed = rmsnorm(hidden, self._vec("model.norm.weight"), eps)
        head = "lm_head.weight" if "lm_head.weight" in self.t else "model.embed_tokens.weight"
        self.logits = self._mv(head, normed, V, H)
        self.pos += 1
        return self.logits
