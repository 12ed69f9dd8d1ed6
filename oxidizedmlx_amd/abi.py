"""ctypes mirror of include/mlxhip.h and the loader for the mlx-hip library.

The structures here are byte-for-byte the C structs of the header; the
function table lists every exported entry point with its prototype. Loading
fails loudly (``BackendUnavailable``) when the built library is missing: there
is no fallback path of any kind.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmlxhip.so")

ABI_VERSION = 1

# mlxhip_status_t (MlxError, crates/mlx-core/src/lib.rs:31-50)
OK = 0
ERR_NULL_PTR = 1
ERR_FFI_FAILED = 2
ERR_SHAPE_MISMATCH = 3
ERR_INVALID_ARGUMENT = 4
ERR_BACKEND_UNAVAILABLE = 5
ERR_IO = 6

# mlxhip_dtype_t (crates/mlx-core/src/types.rs:4-11)
F32, F16, BF16, I32, I64 = 0, 1, 2, 3, 4
DTYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", I32: "i32", I64: "i64"}


class MlxError(Exception):
    """Base error; subclasses mirror MlxError's variants."""

    code = -1

    def __init__(self, msg: str = ""):
        super().__init__(msg)
        self.msg = msg


class NullPtr(MlxError):
    code = ERR_NULL_PTR


class FfiFailed(MlxError):
    code = ERR_FFI_FAILED


class ShapeMismatch(MlxError):
    """MlxError::ShapeMismatch{expected, got}; `expected` / `got` carry the
    shapes (from mlxhip_last_shape_mismatch) when the library recorded them."""

    code = ERR_SHAPE_MISMATCH

    def __init__(self, msg: str = "", expected=None, got=None):
        super().__init__(msg)
        self.expected = expected
        self.got = got


class InvalidArgument(MlxError):
    code = ERR_INVALID_ARGUMENT


class BackendUnavailable(MlxError):
    code = ERR_BACKEND_UNAVAILABLE


class IoError(MlxError):
    code = ERR_IO


_ERRORS = {c.code: c for c in (NullPtr, FfiFailed, ShapeMismatch, InvalidArgument,
                               BackendUnavailable, IoError)}


def error_for(code: int, msg: str) -> MlxError:
    return _ERRORS.get(code, MlxError)(msg)


class mlxhip_op_t(C.Structure):
    _fields_ = [
        ("kind", C.c_int32),
        ("axis", C.c_int32),
        ("has_axis", C.c_int32),
        ("causal", C.c_int32),
        ("eps", C.c_float),
        ("scale", C.c_float),
        ("theta", C.c_float),
        ("base", C.c_float),
        ("shape", C.POINTER(C.c_int64)),
        ("shape_len", C.c_size_t),
        ("axes", C.POINTER(C.c_int64)),
        ("axes_len", C.c_size_t),
        ("start", C.c_int64),
        ("length", C.c_int64),
        ("rotary_dim", C.c_uint64),
        ("pos_offset", C.c_uint64),
        ("offset", C.c_uint64),
        ("traditional", C.c_int32),
        ("reserved_", C.c_int32),
    ]


class mlxhip_input_t(C.Structure):
    _fields_ = [
        ("data", C.c_void_p),
        ("len", C.c_size_t),
        ("shape", C.POINTER(C.c_int64)),
        ("ndim", C.c_size_t),
        ("dtype", C.c_int32),
    ]


class mlxhip_meta_t(C.Structure):
    _fields_ = [
        ("shape", C.POINTER(C.c_int64)),
        ("ndim", C.c_size_t),
        ("dtype", C.c_int32),
    ]


class mlxhip_ew_instr_t(C.Structure):
    _fields_ = [("op", C.c_int32), ("operand", C.c_int32)]


class mlxhip_decoder_config_t(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int32),
        ("d_model", C.c_int32),
        ("n_heads", C.c_int32),
        ("hidden", C.c_int32),
        ("vocab", C.c_int32),
        ("max_batch", C.c_int32),
        ("max_seq", C.c_int32),
        ("eps", C.c_float),
    ]


# mlxhip_decoder_param_t
DEC_EMBEDDING, DEC_LM_HEAD = 0, 1
DEC_LAYER_PARAMS = {"wq": 2, "bq": 3, "wk": 4, "bk": 5, "wv": 6, "bv": 7,
                    "wo": 8, "bo": 9, "w1": 10, "b1": 11, "w2": 12, "b2": 13}
DEC_EAGER = 1

EW_MAX_INSTR = 16
EW_MAX_INPUTS = 8

_i = C.c_int
_i32 = C.c_int32
_i64 = C.c_int64
_u64 = C.c_uint64
_sz = C.c_size_t
_f = C.c_float
_vp = C.c_void_p
_fp = C.c_void_p  # float* passed as raw address

# name -> (restype, argtypes); the complete export list of include/mlxhip.h
PROTOTYPES = {
    "mlxhip_abi_version": (_i, []),
    "mlxhip_last_error": (C.c_char_p, []),
    "mlxhip_last_status": (_i, []),
    "mlxhip_last_shape_mismatch": (_i, [C.POINTER(_i64), C.POINTER(_sz), C.POINTER(_i64),
                                        C.POINTER(_sz), _sz]),
    "mlxhip_debug_fail_allocations": (_i, [_i64]),
    "mlxhip_device_count": (_i, []),
    "mlxhip_init": (_i, [_i]),
    "mlxhip_synchronize": (_i, [_vp]),
    "mlxhip_eval_node": (_i, [C.POINTER(mlxhip_op_t), C.POINTER(mlxhip_input_t), _sz,
                              C.POINTER(mlxhip_meta_t), _fp, _sz]),
    "mlxhip_buffer_alloc": (_vp, [_sz]),
    "mlxhip_buffer_free": (None, [_vp]),
    "mlxhip_buffer_ptr": (_vp, [_vp]),
    "mlxhip_buffer_size": (_sz, [_vp]),
    "mlxhip_buffer_upload": (_i, [_vp, _sz, _vp, _sz]),
    "mlxhip_buffer_download": (_i, [_vp, _sz, _vp, _sz]),
    "mlxhip_eval_node_dev": (_i, [C.POINTER(mlxhip_op_t), C.POINTER(mlxhip_input_t), _sz,
                                  C.POINTER(mlxhip_meta_t), _fp, _vp]),
    "mlxhip_stream_new": (_vp, []),
    "mlxhip_stream_free": (None, [_vp]),
    "mlxhip_stream_add_constant": (_u64, [_vp, _fp, _sz, C.POINTER(mlxhip_meta_t)]),
    "mlxhip_stream_add_op": (_u64, [_vp, C.POINTER(mlxhip_op_t), C.POINTER(_u64), _sz,
                                    C.POINTER(mlxhip_meta_t)]),
    "mlxhip_stream_eval": (_i, [_vp, _u64]),
    "mlxhip_stream_get_buffer": (_i, [_vp, _u64, _fp, _sz]),
    "mlxhip_stream_eval_count": (_u64, [_vp]),
    "mlxhip_stream_cache_len": (_sz, [_vp]),
    "mlxhip_stream_launch_count": (_u64, [_vp]),
    "mlxhip_stream_set_fusion": (_i, [_vp, _i]),
    "mlxhip_stream_set_async": (_i, [_vp, _i]),
    "mlxhip_stream_synchronize": (_i, [_vp]),
    "mlxhip_stream_clear": (_i, [_vp]),
    "mlxhip_stream_eval_many": (_i, [_vp, C.POINTER(_u64), _sz]),
    "mlxhip_stream_add_constant_dev": (_u64, [_vp, _vp, _sz, C.POINTER(mlxhip_meta_t)]),
    "mlxhip_stream_add_constant_view": (_u64, [_vp, _vp, _sz, C.POINTER(mlxhip_meta_t)]),
    "mlxhip_stream_grad": (_i, [_vp, _u64, C.POINTER(_u64), _sz, C.POINTER(_u64)]),
    "mlxhip_gemm": (_i, [_i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64,
                         _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp]),
    "mlxhip_gemm_noalloc": (_i, [_i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64,
                                 _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp]),
    "mlxhip_gemm_noalloc_scratch_bytes": (_sz, []),
    "mlxhip_softmax_rows": (_i, [_fp, _fp, _i64, _i64, _vp]),
    "mlxhip_scaled_masked_softmax_rows": (_i, [_fp, _fp, _i64, _i64, _f, _i32, _vp]),
    "mlxhip_layernorm_rows": (_i, [_fp, _fp, _i64, _i64, _f, _vp]),
    "mlxhip_rmsnorm_rows": (_i, [_fp, _fp, _i64, _i64, _f, _vp]),
    "mlxhip_softmax_vjp_rows": (_i, [_fp, _fp, _fp, _i64, _i64, _vp]),
    "mlxhip_layernorm_vjp_rows": (_i, [_fp, _fp, _fp, _i64, _i64, _f, _vp]),
    "mlxhip_rmsnorm_vjp_rows": (_i, [_fp, _fp, _fp, _i64, _i64, _f, _vp]),
    "mlxhip_ew_chain": (_i, [C.POINTER(mlxhip_ew_instr_t), _sz, C.POINTER(_vp), _sz,
                             _fp, _i64, _vp]),
    "mlxhip_attention": (_i, [_fp, _fp, _fp, _fp, _i64, _i64, _i64, _i64, _f, _i32, _vp]),
    "mlxhip_attention_vjp": (_i, [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _i64, _i64, _i64, _f, _i32, _vp]),
    "mlxhip_transpose2d": (_i, [_fp, _fp, _i64, _i64, _vp]),
    "mlxhip_cast": (_i, [_vp, _i32, _vp, _i32, _i64, _vp]),
    "mlxhip_decoder_new": (_vp, [C.POINTER(mlxhip_decoder_config_t)]),
    "mlxhip_decoder_free": (None, [_vp]),
    "mlxhip_decoder_set_param": (_i, [_vp, _i32, _i32, _fp, _sz]),
    "mlxhip_decoder_generate": (_i, [_vp, _vp, _i32, _i32, _i32, _vp, _vp, _fp, _i32]),
    "mlxhip_decoder_last_timing": (_i, [_vp, C.POINTER(_f), C.POINTER(_i32)]),
    "mlxhip_decoder_weight_bytes": (_sz, [_vp]),
    "mlxhip_event_create": (_vp, []),
    "mlxhip_event_destroy": (None, [_vp]),
    "mlxhip_event_record": (_i, [_vp, _vp]),
    "mlxhip_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(_f)]),
    "mlxhip_stream_create_hip": (_vp, []),
    "mlxhip_stream_destroy_hip": (None, [_vp]),
    "mlxhip_graph_begin": (_i, [_vp]),
    "mlxhip_graph_end": (_vp, [_vp]),
    "mlxhip_graph_launch": (_i, [_vp, _vp]),
    "mlxhip_graph_free": (None, [_vp]),
}

_lib = None
_lock = threading.Lock()


def load_library(path: str | None = None) -> C.CDLL:
    """Loads libmlxhip.so (built in-tree by ``__graft_entry__.build()``)."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or os.environ.get("MLXHIP_LIB", LIB_PATH)
        if not os.path.exists(p):
            raise BackendUnavailable(
                f"mlx-hip library not built: {p} is missing (run __graft_entry__.build())")
        lib = C.CDLL(p)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.mlxhip_abi_version() != ABI_VERSION:
            raise BackendUnavailable("mlx-hip ABI version mismatch")
        if path is None:
            _lib = lib
        return lib


def last_shape_mismatch(lib: C.CDLL) -> tuple[list[int], list[int]] | None:
    """(expected, got) of the calling thread's last ShapeMismatch, or None."""
    cap = 16
    e, g = (C.c_int64 * cap)(), (C.c_int64 * cap)()
    ne, ng = C.c_size_t(0), C.c_size_t(0)
    if lib.mlxhip_last_shape_mismatch(e, C.byref(ne), g, C.byref(ng), cap) != OK:
        return None
    return [e[i] for i in range(min(cap, ne.value))], [g[i] for i in range(min(cap, ng.value))]


def check(rc: int, lib: C.CDLL | None = None) -> None:
    """Raises the MlxError subclass matching a non-zero status code."""
    if rc != OK:
        lib = lib or load_library()
        msg = (lib.mlxhip_last_error() or b"").decode(errors="replace")
        if rc == ERR_SHAPE_MISMATCH:
            shapes = last_shape_mismatch(lib)
            raise ShapeMismatch(msg, *(shapes or (None, None)))
        raise error_for(rc, msg)


def int64_array(vals) -> C.Array:
    vals = list(vals)
    arr = (C.c_int64 * max(1, len(vals)))(*vals)
    return arr
