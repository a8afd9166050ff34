"""CPU oracle for tiny-llm's quantized-projection path -- TEST INFRASTRUCTURE ONLY.

Loads the C++ restatement (oracle/liboracle.so, built from oracle.cpp) and,
when it has been built in the development container, the compiled reference
(oracle/_ref/libtqref.so: tiny-llm's own kernels/dispatch.cpp and
kernels/*/*_ref.cpp, built by `make -C oracle ref`).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker; the product library never calls it.

Functions and the reference code they restate:
  matvec_i4      kernels/matvec/matvec_i4_ref.cpp:45-103
  matvec_vq2     kernels/matvec/matvec_vq2_ref.cpp:52-81
  matmul_i4      kernels/matvec/matmul_i4_ref.cpp:53-114
  dequant_i4_row kernels/ref_ops.h:183-205
  biip_rotate    kernels/biip/biip_rotate.cpp:37-68
  half_to_float / float_to_half   kernels/ref_ops.h:51-105
  i4_row_bytes / vq2_tensor_bytes runtime/tiny_format.h:73-78, 100-103
  quantized_size quantization/quant.cpp:94-118
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libtqref.so")

_vp, _i, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
_SIGS = {
    "orc_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
    "orc_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
    "orc_half_to_float_n": (None, [_vp, _vp, ctypes.c_longlong]),
    "orc_float_to_half_n": (None, [_vp, _vp, ctypes.c_longlong]),
    "orc_i4_row_bytes": (_sz, [_i, _i]),
    "orc_vq2_tensor_bytes": (_sz, [_i, _i]),
    "orc_quantized_size": (_sz, [_i, _i, _i, _i]),
    "orc_matvec_i4": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "orc_matvec_i4_mt": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "orc_matvec_vq2": (None, [_vp, _vp, _vp, _i, _i]),
    "orc_matvec_vq2_mt": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "orc_matmul_i4": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "orc_matmul_i4_mt": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "orc_dequant_i4_row": (None, [_vp, _i, _i, _i, _vp]),
    "orc_biip_rotate": (None, [_vp, _vp, _i, _vp, _vp, _i]),
}
_REF_SIGS = {
    "tqref_matvec_i4": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "tqref_matvec_pair_i4": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "tqref_matvec_qkv_i4": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "tqref_matvec_vq2": (None, [_vp, _vp, _vp, _i, _i]),
    "tqref_matmul_i4": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "tqref_matmul_vq2": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "tqref_dequant_i4_row": (None, [_vp, _i, _i, _i, _vp]),
    "tqref_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
    "tqref_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
    "tqref_half_to_float_n": (None, [_vp, _vp, ctypes.c_longlong]),
    "tqref_float_to_half_n": (None, [_vp, _vp, ctypes.c_longlong]),
    "tqref_unknown_i4_name_rejected": (_i, []),
    "tqref_biip_rotate": (None, [_vp, _vp, _i, _vp, _vp, _i]),
    "tqref_model_load": (_i, [ctypes.c_char_p, ctypes.c_char_p, _i]),
    "tqref_model_tensor_count": (_i, []),
    "tqref_model_tensor_at": (_i, [_i, ctypes.c_char_p, _vp, _vp, _vp, _vp, _vp]),
    "tqref_model_quant_group_size": (_i, []),
    "tqref_model_type": (_i, []),
    "tqref_decode_create": (_i, [ctypes.c_char_p, _i, ctypes.c_char_p, _i]),
    "tqref_decode_step": (_i, [_i]),
    "tqref_decode_logits": (None, [_vp, _i]),
    "tqref_decode_reset": (None, []),
}

_LIB = None
_REF = None


def build(ref: bool = False) -> None:
    """make -C oracle (and `ref` when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(ORACLE_SO):
            build()
        cdll = ctypes.CDLL(ORACLE_SO)
        for name, (res, args) in _SIGS.items():
            fn = getattr(cdll, name)
            fn.restype, fn.argtypes = res, args
        _LIB = cdll
    return _LIB


def ref_lib():
    """The compiled reference, or None where it was not built (e.g. on the GPU box)."""
    global _REF
    if _REF is None and os.path.exists(REF_SO):
        cdll = ctypes.CDLL(REF_SO)
        for name, (res, args) in _REF_SIGS.items():
            fn = getattr(cdll, name)
            fn.restype, fn.argtypes = res, args
        _REF = cdll
    return _REF


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def half_to_float(h: int) -> float:
    return float(lib().orc_half_to_float(h))


def float_to_half(f: float) -> int:
    return int(lib().orc_float_to_half(f))


def halves_to_floats(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_half_to_float_n(_p(h), _p(out), h.size)
    return out


def floats_to_halves(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().orc_float_to_half_n(_p(f), _p(out), f.size)
    return out


def i4_row_bytes(in_dim: int, group_size: int) -> int:
    return int(lib().orc_i4_row_bytes(in_dim, group_size))


def vq2_tensor_bytes(rows: int, cols: int) -> int:
    return int(lib().orc_vq2_tensor_bytes(rows, cols))


def quantized_size(type_code: int, rows: int, cols: int, group_size: int) -> int:
    return int(lib().orc_quantized_size(type_code, rows, cols, group_size))


def matvec_i4(w, x, out_dim, in_dim, group_size, threads: int = 1) -> np.ndarray:
    y = np.empty(out_dim, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if threads > 1:
        lib().orc_matvec_i4_mt(_p(w), _p(x), _p(y), out_dim, in_dim, group_size, threads)
    else:
        lib().orc_matvec_i4(_p(w), _p(x), _p(y), out_dim, in_dim, group_size)
    return y


def matvec_vq2(w, x, out_dim, in_dim, threads: int = 1) -> np.ndarray:
    y = np.empty(out_dim, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if threads > 1:
        lib().orc_matvec_vq2_mt(_p(w), _p(x), _p(y), out_dim, in_dim, threads)
    else:
        lib().orc_matvec_vq2(_p(w), _p(x), _p(y), out_dim, in_dim)
    return y


def matmul_i4(w, x, M, K, N, group_size, threads: int = 1) -> np.ndarray:
    y = np.empty(M * N, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if threads > 1:
        lib().orc_matmul_i4_mt(_p(w), _p(x), _p(y), M, K, N, group_size, threads)
    else:
        lib().orc_matmul_i4(_p(w), _p(x), _p(y), M, K, N, group_size)
    return y


def dequant_i4_row(embed, row, dim, group_size) -> np.ndarray:
    out = np.zeros(dim, dtype=np.float32)
    lib().orc_dequant_i4_row(_p(embed), row, dim, group_size, _p(out))
    return out


def biip_rotate(x, scale, sign, block_size) -> np.ndarray:
    """BiIP activation rotation; scale None = the reference's nullptr (no division)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    sc = None if scale is None else np.ascontiguousarray(scale, dtype=np.float32)
    sg = np.ascontiguousarray(sign, dtype=np.float32)
    lib().orc_biip_rotate(_p(x), _p(y), x.size, None if sc is None else _p(sc), _p(sg), block_size)
    return y


def dequant_i4_matrix_f64(w: np.ndarray, out_dim: int, in_dim: int, group_size: int) -> np.ndarray:
    """Independent numpy decode of the i4 layout to float64 (textbook cross-check, not the oracle).

    Decodes scale/zero with numpy's float16 and forms (q - zero) * scale in
    float32 like the layout contract says, then widens to float64.
    """
    gb = 4 + group_size // 2
    groups = (in_dim + group_size - 1) // group_size
    a = np.asarray(w, dtype=np.uint8).reshape(out_dim, groups, gb)
    scale = a[:, :, 0:2].copy().view(np.float16).astype(np.float32)[:, :, 0]
    zero = a[:, :, 2:4].copy().view(np.float16).astype(np.float32)[:, :, 0]
    codes = a[:, :, 4:]
    q = np.empty((out_dim, groups, group_size), dtype=np.float32)
    q[:, :, 0::2] = (codes & 0x0F).astype(np.float32)
    q[:, :, 1::2] = (codes >> 4).astype(np.float32)
    deq = (q - zero[:, :, None]) * scale[:, :, None]
    return deq.reshape(out_dim, groups * group_size)[:, :in_dim].astype(np.float64)
