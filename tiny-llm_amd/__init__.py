"""tiny-llm_amd -- MI355X (gfx950) quantized linear-projection path for tiny-llm.

Python host side of libtqhip.so (HIP kernels + the C ABI in include/tqhip.h).
It mirrors the reference registry's entry points (kernels/dispatch.h:151-253
of tiny-llm) on numpy arrays, plus device-buffer helpers for tests and
benchmarks. There is no CPU fallback: every compute call goes to the HIP
library, and loading fails loudly if the library has not been built.

The directory name is not a valid module name, so load it by path::

    spec = importlib.util.spec_from_file_location("tiny_llm_amd", ".../tiny-llm_amd/__init__.py")
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtqhip.so")


def _load_sibling(name: str):
    """A module file of this directory (the directory is loaded by path, not as a package)."""
    spec = importlib.util.spec_from_file_location(f"tiny_llm_amd_{name}", os.path.join(HERE, name + ".py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


# synthetic .tqwen model images (the decode engine's benchmark and smoke models, the loader tests' files)
tqwen_synth = _load_sibling("tqwen_synth")

OK, EBADSHAPE, EBADGROUP, ETOOLARGE, ELAUNCH, EFILE, EHIP, ENOSCRATCH = 0, -1, -2, -3, -4, -5, -6, -7
NOALLOC_SCRATCH_BYTES = 16 << 20  # TQHIP_NOALLOC_SCRATCH_BYTES
OP_I4_MATVEC, OP_VQ2_MATVEC, OP_I4_MATMUL, OP_I4_PAIR, OP_I4_QKV, OP_BIIP_ROTATE, OP_I4_SET, OP_VQ2_SET = 1, 2, 3, 4, 5, 6, 7, 8

_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t


class Op(ctypes.Structure):
    """tqhip_op: one device-pointer call of a tqhip_run_ops list."""
    _fields_ = [("kind", _i), ("w", _vp), ("x", _vp), ("y", _vp),
                ("out_dim", _i), ("in_dim", _i), ("n", _i), ("group_size", _i),
                ("w2", _vp), ("w3", _vp), ("y2", _vp), ("y3", _vp), ("out_dim2", _i)]


class I4Mat(ctypes.Structure):
    """tqhip_i4_mat: one matrix of a matvec set (device pointers)."""
    _fields_ = [("w", _vp), ("x", _vp), ("y", _vp), ("out_dim", _i), ("in_dim", _i)]


def i4_set(mats: list) -> "ctypes.Array":
    """A tqhip_i4_mat array from (w, x, y, out_dim, in_dim) tuples (DeviceBuffers or addresses)."""
    return (I4Mat * len(mats))(*[I4Mat(_ptr(w), _ptr(x), _ptr(y), m, k) for w, x, y, m, k in mats])


def set_op(mats: "ctypes.Array", group_size: int) -> Op:
    """A TQHIP_OP_I4_SET op over a tqhip_i4_mat array; keep the array alive while the op is used."""
    return Op(OP_I4_SET, ctypes.addressof(mats), None, None, 0, 0, len(mats), group_size)


def vq2_set_op(mats: "ctypes.Array") -> Op:
    """A TQHIP_OP_VQ2_SET op over a tqhip_i4_mat array of VQ2 matrices; keep the array alive."""
    return Op(OP_VQ2_SET, ctypes.addressof(mats), None, None, 0, 0, len(mats), 0)


class TensorInfo(ctypes.Structure):
    """tqhip_tensor_info: one entry of a .tqwen tensor table (plus its HBM address once uploaded)."""
    _fields_ = [("name", ctypes.c_char * 65), ("dtype", _i), ("ndim", _i), ("shape", ctypes.c_uint64 * 4),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64), ("device", _vp)]



class ModelConfig(ctypes.Structure):
    """tqhip_model_config: the header's model configuration."""
    _fields_ = [(n, _i) for n in ("n_layers", "hidden_size", "intermediate_size", "n_heads", "n_kv_heads",
                                  "head_dim", "vocab_size", "max_seq_len", "tied_embeddings")] + \
               [("rms_norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("model_type", _i),
                ("quant_group_size", _i), ("file_dtype", _i)]


_SIGS = {
    # host-pointer entry points (the "hip" variants)
    "tqhip_matvec_i4": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "tqhip_matvec_pair_i4": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "tqhip_matvec_qkv_i4": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "tqhip_matvec_vq2": (None, [_vp, _vp, _vp, _i, _i]),
    "tqhip_matmul_i4": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "tqhip_biip_rotate": (None, [_vp, _vp, _i, _vp, _vp, _i]),
    "tqhip_release_weights": (None, []),
    "tqhip_host_timing": (None, [_i]),
    "tqhip_host_timing_last": (None, [_f32p, _f32p, _f32p]),
    # device-pointer entry points
    "tqhip_matvec_i4_dev": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tqhip_matvec_i4_generic_dev": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tqhip_matvec_vq2_dev": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "tqhip_matvec_pair_i4_dev": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "tqhip_matvec_qkv_i4_dev": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "tqhip_matmul_i4_dev": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "tqhip_matmul_i4_noalloc_dev": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "tqhip_matvec_i4_set_dev": (_i, [_vp, _i, _i, _vp]),
    "tqhip_matvec_vq2_set_dev": (_i, [_vp, _i, _vp]),
    "tqhip_biip_rotate_dev": (_i, [_vp, _vp, _i, _vp, _vp, _i, _vp]),
    "tqhip_dequant_i4_rows_dev": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp]),
    # registry
    "tqhip_set_ops_impl_by_name": (_i, [ctypes.c_char_p]),
    "tqhip_ops_impl_name": (ctypes.c_char_p, []),
    "tqhip_biip_rotate_activation": (None, [_vp, _vp, _i, _vp, _vp, _i]),
    "tqhip_set_matvec_i4_impl_by_name": (_i, [ctypes.c_char_p]),
    "tqhip_matvec_i4_impl_name": (ctypes.c_char_p, []),
    "tqhip_available_matvec_i4_impls": (ctypes.c_char_p, []),
    "tqhip_set_matvec_vq2_impl_by_name": (_i, [ctypes.c_char_p]),
    "tqhip_matvec_vq2_impl_name": (ctypes.c_char_p, []),
    "tqhip_available_matvec_vq2_impls": (ctypes.c_char_p, []),
    "tqhip_set_matmul_i4_impl_by_name": (_i, [ctypes.c_char_p]),
    "tqhip_dispatch_matvec_i4": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "tqhip_dispatch_matvec_pair_i4": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "tqhip_dispatch_matvec_qkv_i4": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "tqhip_dispatch_matvec_vq2": (None, [_vp, _vp, _vp, _i, _i]),
    "tqhip_dispatch_matmul_i4": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "tqhip_dispatch_matmul_vq2": (None, [_vp, _vp, _vp, _i, _i, _i]),
    # byte accounting
    "tqhip_i4_row_bytes": (_sz, [_i, _i]),
    "tqhip_vq2_tensor_bytes": (_sz, [_i, _i]),
    # device plumbing
    "tqhip_device_count": (_i, []),
    "tqhip_device_name": (_i, [ctypes.c_char_p, _i]),
    "tqhip_malloc": (_vp, [_sz]),
    "tqhip_free": (_i, [_vp]),
    "tqhip_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "tqhip_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "tqhip_memcpy_d2d": (_i, [_vp, _vp, _sz]),
    "tqhip_memset": (_i, [_vp, _i, _sz]),
    "tqhip_synchronize": (_i, []),
    "tqhip_stream_create": (_vp, []),
    "tqhip_stream_destroy": (_i, [_vp]),
    "tqhip_stream_synchronize": (_i, [_vp]),
    "tqhip_event_create": (_vp, []),
    "tqhip_event_destroy": (_i, [_vp]),
    "tqhip_event_record": (_i, [_vp, _vp]),
    "tqhip_event_elapsed_ms": (_i, [_vp, _vp, _f32p]),
    "tqhip_run_ops": (_i, [ctypes.POINTER(Op), _i, _i, _vp]),
    "tqhip_run_ops_timed": (_i, [ctypes.POINTER(Op), _i, _i, _vp, _f32p]),
    "tqhip_ops_graph_create": (_i, [ctypes.POINTER(Op), _i, _vp, ctypes.POINTER(_vp)]),
    "tqhip_ops_graph_launch": (_i, [_vp, _vp]),
    "tqhip_ops_graph_destroy": (_i, [_vp]),
    # .tqwen weight files
    "tqhip_model_inspect": (_i, [ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.c_char_p, _i]),
    "tqhip_model_upload": (_i, [_vp]),
    "tqhip_model_tensor_count": (_i, [_vp]),
    "tqhip_model_tensor_at": (_i, [_vp, _i, ctypes.POINTER(TensorInfo)]),
    "tqhip_model_find": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(TensorInfo)]),
    "tqhip_model_quant_group_size": (_i, [_vp]),
    "tqhip_model_file_dtype": (_i, [_vp]),
    "tqhip_model_type": (_i, [_vp]),
    "tqhip_model_free": (None, [_vp]),
    "tqhip_model_inspect_memory": (_i, [_vp, ctypes.c_uint64, ctypes.POINTER(_vp), ctypes.c_char_p, _i]),
    "tqhip_model_config_get": (_i, [_vp, ctypes.POINTER(ModelConfig)]),
    # device-resident decode engine
    "tqhip_decode_create": (_i, [_vp, _i, ctypes.c_char_p, _i, ctypes.POINTER(_vp)]),
    "tqhip_decode_step": (_i, [_vp, _i]),
    "tqhip_decode_reset": (None, [_vp]),
    "tqhip_decode_destroy": (None, [_vp]),
    "tqhip_decode_logits": (_vp, [_vp]),
    "tqhip_decode_seq_len": (_i, [_vp]),
    "tqhip_decode_mode": (_i, [_vp]),
    # synthetic inputs
    "tq_synth_seed": (ctypes.c_uint64, [ctypes.c_uint64, _i, ctypes.c_char_p]),
    "tq_synth_i4": (None, [_vp, _i, _i, _i, ctypes.c_uint64, ctypes.c_float, ctypes.c_float,
                           ctypes.c_float, ctypes.c_float]),
    "tq_synth_normal": (None, [_vp, ctypes.c_longlong, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]),
    "tq_synth_vq2": (None, [_vp, _i, _i, ctypes.c_uint64, ctypes.c_float]),
    "tq_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
}

EXPORTED = tuple(_SIGS)
_LIB = None


def build() -> str:
    """Compiles libtqhip.so in-tree (hipcc, gfx950)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("tiny_llm_amd_build", os.path.join(HERE, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build()


def lib() -> ctypes.CDLL:
    """The loaded HIP library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run tiny-llm_amd/build.py (no CPU fallback exists)")
        cdll = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(cdll, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = cdll
    return _LIB


def _stream(s):
    """None (the default stream), a Stream, or a raw hipStream_t value."""
    if s is None:
        return None
    return s.ptr if isinstance(s, Stream) else int(s)


def _ptr(a) -> "int | None":
    if a is None:
        return None  # a NULL pointer (calls that are refused before they touch it)
    if isinstance(a, DeviceBuffer):
        return a.ptr
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise ValueError("array must be C-contiguous")
        return a.ctypes.data
    return int(a)


def _check(status: int, what: str) -> None:
    if status != OK:
        raise RuntimeError(f"{what} failed with status {status}")


# ---- layout and synthetic inputs -------------------------------------------------------------

def i4_row_bytes(in_dim: int, group_size: int) -> int:
    return ((in_dim + group_size - 1) // group_size) * (4 + group_size // 2)


def vq2_tensor_bytes(rows: int, cols: int) -> int:
    return 2048 + rows * (cols // 4)


def synth_seed(base: int, layer: int, name: str) -> int:
    return int(lib().tq_synth_seed(base, layer, name.encode()))


def synth_i4(out_dim: int, in_dim: int, group_size: int, seed: int, scale=(0.002, 0.02),
             zero=(0.0, 15.0)) -> np.ndarray:
    """i4 weights in the interleaved layout; codes U{0..15}, scale/zero fp16(U[.])."""
    w = np.empty(out_dim * i4_row_bytes(in_dim, group_size), dtype=np.uint8)
    lib().tq_synth_i4(w.ctypes.data, out_dim, in_dim, group_size, seed, scale[0], scale[1], zero[0], zero[1])
    return w


def synth_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    x = np.empty(n, dtype=np.float32)
    lib().tq_synth_normal(x.ctypes.data, n, seed, mean, std)
    return x


def synth_vq2(out_dim: int, in_dim: int, seed: int, cb_std: float = 0.02) -> np.ndarray:
    w = np.empty(vq2_tensor_bytes(out_dim, in_dim), dtype=np.uint8)
    lib().tq_synth_vq2(w.ctypes.data, out_dim, in_dim, seed, cb_std)
    return w


# ---- the reference's dispatch entry points, host arrays ------------------------------------

def matvec_i4(w: np.ndarray, x: np.ndarray, out_dim: int, in_dim: int, group_size: int) -> np.ndarray:
    """tinyqwen::matvec_i4 (kernels/dispatch.h:151-159) through the registry."""
    y = np.empty(out_dim, dtype=np.float32)
    lib().tqhip_dispatch_matvec_i4(_ptr(w), _ptr(x), _ptr(y), out_dim, in_dim, group_size)
    return y


def matvec_pair_i4(w1, w2, x, out_dim: int, in_dim: int, group_size: int):
    y1 = np.empty(out_dim, dtype=np.float32)
    y2 = np.empty(out_dim, dtype=np.float32)
    lib().tqhip_dispatch_matvec_pair_i4(_ptr(w1), _ptr(w2), _ptr(x), _ptr(y1), _ptr(y2), out_dim, in_dim,
                                        group_size)
    return y1, y2


def matvec_qkv_i4(wq, wk, wv, x, q_dim: int, kv_dim: int, in_dim: int, group_size: int):
    yq = np.empty(q_dim, dtype=np.float32)
    yk = np.empty(kv_dim, dtype=np.float32)
    yv = np.empty(kv_dim, dtype=np.float32)
    lib().tqhip_dispatch_matvec_qkv_i4(_ptr(wq), _ptr(wk), _ptr(wv), _ptr(x), _ptr(yq), _ptr(yk), _ptr(yv),
                                       q_dim, kv_dim, in_dim, group_size)
    return yq, yk, yv


def matvec_vq2(w: np.ndarray, x: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
    y = np.empty(out_dim, dtype=np.float32)
    lib().tqhip_dispatch_matvec_vq2(_ptr(w), _ptr(x), _ptr(y), out_dim, in_dim)
    return y


def matmul_i4(w: np.ndarray, x: np.ndarray, M: int, K: int, N: int, group_size: int) -> np.ndarray:
    """Y[M,N] = W[M,K] X[K,N]; x is x[n*K+k] (N columns), result is y[n*M+m]."""
    y = np.empty(M * N, dtype=np.float32)
    lib().tqhip_dispatch_matmul_i4(_ptr(w), _ptr(x), _ptr(y), M, K, N, group_size)
    return y


def biip_rotate(x: np.ndarray, scale, sign: np.ndarray, block_size: int) -> np.ndarray:
    """BiIP activation rotation through the ops registry (host pointers); scale None = no division."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    sc = None if scale is None else np.ascontiguousarray(scale, dtype=np.float32)
    sg = np.ascontiguousarray(sign, dtype=np.float32)
    lib().tqhip_biip_rotate_activation(_ptr(x), _ptr(y), x.size, None if sc is None else _ptr(sc), _ptr(sg),
                                       block_size)
    return y


def biip_rotate_dev(x, y, dim: int, scale, sign, block_size: int, stream: "Stream | None" = None) -> None:
    _check(lib().tqhip_biip_rotate_dev(_ptr(x), _ptr(y), dim, None if scale is None else _ptr(scale), _ptr(sign),
                                       block_size, _stream(stream)), "tqhip_biip_rotate_dev")


def dequant_i4_rows_dev(embed, rows, n: int, dim: int, group_size: int, out, stream: "Stream | None" = None) -> None:
    _check(lib().tqhip_dequant_i4_rows_dev(_ptr(embed), _ptr(rows), n, dim, group_size, _ptr(out), _stream(stream)),
           "tqhip_dequant_i4_rows_dev")


def matmul_vq2(w: np.ndarray, x: np.ndarray, M: int, K: int, N: int) -> np.ndarray:
    y = np.empty(M * N, dtype=np.float32)
    lib().tqhip_dispatch_matmul_vq2(_ptr(w), _ptr(x), _ptr(y), M, K, N)
    return y


def set_matvec_i4_impl_by_name(name: str) -> bool:
    return bool(lib().tqhip_set_matvec_i4_impl_by_name(name.encode()))


def set_matvec_vq2_impl_by_name(name: str) -> bool:
    return bool(lib().tqhip_set_matvec_vq2_impl_by_name(name.encode()))


def set_matmul_i4_impl_by_name(name: str) -> bool:
    return bool(lib().tqhip_set_matmul_i4_impl_by_name(name.encode()))


def matvec_i4_impl_name() -> str:
    return lib().tqhip_matvec_i4_impl_name().decode()


def available_matvec_i4_impls() -> str:
    return lib().tqhip_available_matvec_i4_impls().decode()


def available_matvec_vq2_impls() -> str:
    return lib().tqhip_available_matvec_vq2_impls().decode()


# ---- device buffers ----------------------------------------------------------------------------

class DeviceBuffer:
    """An HBM allocation owned by Python (hipMalloc / hipFree through the library)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = lib().tqhip_malloc(max(1, self.nbytes))
        if not p:
            raise MemoryError(f"hipMalloc({self.nbytes}) failed")
        self.ptr = int(p)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than buffer")
        _check(lib().tqhip_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes), "hipMemcpy H2D")

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("read past buffer end")
        _check(lib().tqhip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "hipMemcpy D2H")
        return out

    def free(self) -> None:
        if self.ptr:
            lib().tqhip_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def device_count() -> int:
    return int(lib().tqhip_device_count())


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    return buf.value.decode() if lib().tqhip_device_name(buf, 256) == 0 else "unknown"


def synchronize() -> None:
    _check(lib().tqhip_synchronize(), "hipDeviceSynchronize")


def matvec_i4_dev(w, x, y, out_dim: int, in_dim: int, group_size: int, stream=None) -> None:
    _check(lib().tqhip_matvec_i4_dev(_ptr(w), _ptr(x), _ptr(y), out_dim, in_dim, group_size, _stream(stream)),
           "tqhip_matvec_i4_dev")


def matvec_i4_generic_dev(w, x, y, out_dim: int, in_dim: int, group_size: int, stream=None) -> None:
    _check(lib().tqhip_matvec_i4_generic_dev(_ptr(w), _ptr(x), _ptr(y), out_dim, in_dim, group_size, _stream(stream)),
           "tqhip_matvec_i4_generic_dev")


def matvec_vq2_dev(w, x, y, out_dim: int, in_dim: int, stream=None) -> None:
    _check(lib().tqhip_matvec_vq2_dev(_ptr(w), _ptr(x), _ptr(y), out_dim, in_dim, _stream(stream)), "tqhip_matvec_vq2_dev")


def matvec_pair_i4_dev(w1, w2, x, y1, y2, out_dim: int, in_dim: int, group_size: int, stream=None) -> None:
    _check(lib().tqhip_matvec_pair_i4_dev(_ptr(w1), _ptr(w2), _ptr(x), _ptr(y1), _ptr(y2), out_dim, in_dim,
                                          group_size, _stream(stream)), "tqhip_matvec_pair_i4_dev")


def matvec_qkv_i4_dev(wq, wk, wv, x, yq, yk, yv, q_dim: int, kv_dim: int, in_dim: int, group_size: int,
                      stream=None) -> None:
    _check(lib().tqhip_matvec_qkv_i4_dev(_ptr(wq), _ptr(wk), _ptr(wv), _ptr(x), _ptr(yq), _ptr(yk), _ptr(yv), q_dim,
                                         kv_dim, in_dim, group_size, _stream(stream)), "tqhip_matvec_qkv_i4_dev")


def matmul_i4_dev(w, x, y, M: int, K: int, N: int, group_size: int, stream=None) -> None:
    _check(lib().tqhip_matmul_i4_dev(_ptr(w), _ptr(x), _ptr(y), M, K, N, group_size, _stream(stream)),
           "tqhip_matmul_i4_dev")


def matvec_i4_set_dev(mats, group_size: int, stream=None) -> None:
    """tqhip_matvec_i4_set_dev over a tqhip_i4_mat array (see i4_set) or a list of tuples."""
    arr = mats if isinstance(mats, ctypes.Array) else i4_set(mats)
    _check(lib().tqhip_matvec_i4_set_dev(ctypes.addressof(arr), len(arr), group_size, _stream(stream)),
           "tqhip_matvec_i4_set_dev")


def matvec_vq2_set_dev(mats, stream=None) -> None:
    """tqhip_matvec_vq2_set_dev over a tqhip_i4_mat array (see i4_set) or a list of tuples."""
    arr = mats if isinstance(mats, ctypes.Array) else i4_set(mats)
    _check(lib().tqhip_matvec_vq2_set_dev(ctypes.addressof(arr), len(arr), _stream(stream)), "tqhip_matvec_vq2_set_dev")


def matmul_i4_noalloc_dev(w, x, y, M: int, K: int, N: int, group_size: int, stream=None) -> int:
    """tqhip_matmul_i4_noalloc_dev: the prefill GEMM with X's fp16 copy in the library's static
    device array (no allocation). Returns the status (ENOSCRATCH when the call needs more than
    NOALLOC_SCRATCH_BYTES)."""
    return int(lib().tqhip_matmul_i4_noalloc_dev(_ptr(w), _ptr(x), _ptr(y), M, K, N, group_size, _stream(stream)))


class Stream:
    def __init__(self):
        p = lib().tqhip_stream_create()
        if not p:
            raise RuntimeError("hipStreamCreate failed")
        self.ptr = int(p)

    def synchronize(self) -> None:
        _check(lib().tqhip_stream_synchronize(self.ptr), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.ptr:
                lib().tqhip_stream_destroy(self.ptr)
        except Exception:
            pass


class Event:
    def __init__(self):
        p = lib().tqhip_event_create()
        if not p:
            raise RuntimeError("hipEventCreate failed")
        self.ptr = int(p)

    def record(self, stream: "Stream | None" = None) -> None:
        _check(lib().tqhip_event_record(self.ptr, stream.ptr if stream else None), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _check(lib().tqhip_event_elapsed_ms(self.ptr, end.ptr, ctypes.byref(ms)), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            if self.ptr:
                lib().tqhip_event_destroy(self.ptr)
        except Exception:
            pass


def run_ops(ops: list, repeats: int, stream: "Stream | None" = None) -> None:
    arr = (Op * len(ops))(*ops)
    _check(lib().tqhip_run_ops(arr, len(ops), repeats, _stream(stream)), "tqhip_run_ops")


class OpsGraph:
    """An op list captured into a HIP graph (tqhip_ops_graph_create) on a created
    stream, replayed with launch() on that stream or on another one (the graph
    owns its scratch)."""

    def __init__(self, ops: list, stream: "Stream"):
        self._arr = (Op * len(ops))(*ops)
        self._stream = stream
        h = _vp()
        _check(lib().tqhip_ops_graph_create(self._arr, len(ops), _stream(stream), ctypes.byref(h)),
               "tqhip_ops_graph_create")
        self._h = h

    def launch(self, stream: "Stream | None" = None) -> None:
        _check(lib().tqhip_ops_graph_launch(self._h, _stream(stream or self._stream)), "tqhip_ops_graph_launch")

    def close(self) -> None:
        if self._h:
            _check(lib().tqhip_ops_graph_destroy(self._h), "tqhip_ops_graph_destroy")
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def run_ops_timed(ops: list, repeats: int, stream: "Stream | None" = None) -> np.ndarray:
    """Runs the list `repeats` times with an event pair around every call; returns mean ms per call."""
    arr = (Op * len(ops))(*ops)
    out = np.zeros(len(ops), np.float32)
    _check(lib().tqhip_run_ops_timed(arr, len(ops), repeats, _stream(stream), out.ctypes.data_as(_f32p)),
           "tqhip_run_ops_timed")
    return out


# ---- .tqwen weight files ----------------------------------------------------------------------

class ModelFile:
    """A validated .tqwen file, optionally resident in HBM.

    Mirrors tinyqwen::ModelFile (runtime/model_loader.h:180-330): ``load`` raises
    ValueError with the reference loader's message where the reference rejects the
    file, ``get`` returns None for an absent name, ``tensor_names`` is in file order.
    ``upload`` copies the data region to HBM; each tensor's ``device`` address then
    feeds the ``*_dev`` entry points directly.
    """

    def __init__(self, path: str):
        handle = _vp()
        err = ctypes.create_string_buffer(512)
        rc = lib().tqhip_model_inspect(os.fsencode(path), ctypes.byref(handle), err, len(err))
        if rc != OK:
            raise ValueError(err.value.decode(errors="replace") or f"tqhip_model_inspect failed ({rc})")
        self._h = handle.value

    load = classmethod(lambda cls, path: cls(path))

    @classmethod
    def from_image(cls, image) -> "ModelFile":
        """A whole .tqwen file held in memory (bytes / bytearray / uint8 array); kept alive by the object."""
        buf = np.frombuffer(image, np.uint8)
        handle = _vp()
        err = ctypes.create_string_buffer(512)
        rc = lib().tqhip_model_inspect_memory(buf.ctypes.data, buf.size, ctypes.byref(handle), err, len(err))
        if rc != OK:
            raise ValueError(err.value.decode(errors="replace") or f"tqhip_model_inspect_memory failed ({rc})")
        obj = cls.__new__(cls)
        obj._h = handle.value
        obj._image = buf
        return obj

    def upload(self) -> None:
        _check(lib().tqhip_model_upload(self._h), "tqhip_model_upload")

    def tensor_count(self) -> int:
        return int(lib().tqhip_model_tensor_count(self._h))

    def tensor_at(self, i: int) -> TensorInfo:
        info = TensorInfo()
        _check(lib().tqhip_model_tensor_at(self._h, i, ctypes.byref(info)), "tqhip_model_tensor_at")
        return info

    def tensor_names(self) -> list:
        return [self.tensor_at(i).name.decode() for i in range(self.tensor_count())]

    def get(self, name: str) -> "TensorInfo | None":
        info = TensorInfo()
        rc = lib().tqhip_model_find(self._h, name.encode(), ctypes.byref(info))
        return info if rc == OK else None

    @property
    def config(self) -> ModelConfig:
        c = ModelConfig()
        _check(lib().tqhip_model_config_get(self._h, ctypes.byref(c)), "tqhip_model_config_get")
        return c

    @property
    def quant_group_size(self) -> int:
        return int(lib().tqhip_model_quant_group_size(self._h))

    @property
    def dtype(self) -> int:
        return int(lib().tqhip_model_file_dtype(self._h))

    @property
    def model_type(self) -> int:
        return int(lib().tqhip_model_type(self._h))

    def close(self) -> None:
        """Frees the handle and the HBM copy. Refused while a DecodeEngine built on this
        model is open: its captured step graph reads the model's HBM copy."""
        if getattr(self, "_h", None):
            live = [e for e in list(getattr(self, "_engines", ())) if getattr(e, "_h", None)]
            if live:
                raise RuntimeError(f"ModelFile.close(): {len(live)} DecodeEngine(s) still use this model; "
                                   "close them first")
            lib().tqhip_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DecodeEngine:
    """Device-resident decode engine over an uploaded i4 ModelFile (the gpu_decode boundary,
    kernels/dispatch.h:337-378): ``step(token)`` returns the argmax next token, ``logits()``
    copies the last step's logits to the host, ``reset()`` returns to position 0."""

    def __init__(self, model: ModelFile, max_seq_len: int = 0):
        if not getattr(model, "_h", None):
            raise ValueError("DecodeEngine: the ModelFile is closed")
        handle = _vp()
        err = ctypes.create_string_buffer(512)
        rc = lib().tqhip_decode_create(model._h, max_seq_len, err, len(err), ctypes.byref(handle))
        if rc != OK:
            raise ValueError(err.value.decode(errors="replace") or f"tqhip_decode_create failed ({rc})")
        self._h = handle.value
        self._model = model  # the engine reads the model's HBM copy
        if not hasattr(model, "_engines"):
            model._engines = weakref.WeakSet()
        model._engines.add(self)  # ModelFile.close() refuses while this engine is open
        self.vocab = model.config.vocab_size

    def step(self, token: int) -> int:
        r = int(lib().tqhip_decode_step(self._h, int(token)))
        if r < 0:
            raise RuntimeError(f"tqhip_decode_step failed with status {r}")
        return r

    def logits(self) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        _check(lib().tqhip_memcpy_d2h(out.ctypes.data, lib().tqhip_decode_logits(self._h), out.nbytes),
               "hipMemcpy D2H")
        return out

    def reset(self) -> None:
        lib().tqhip_decode_reset(self._h)

    @property
    def seq_len(self) -> int:
        return int(lib().tqhip_decode_seq_len(self._h))

    @property
    def mode(self) -> set:
        """How a step runs: a subset of {"fused", "flow", "eager"} (tqhip_decode_mode)."""
        m = int(lib().tqhip_decode_mode(self._h))
        return {name for bit, name in ((1, "fused"), (2, "flow"), (4, "eager")) if m & bit}

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().tqhip_decode_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
