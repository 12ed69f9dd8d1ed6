"""ctypes wrapper of the C oracle (TEST INFRASTRUCTURE ONLY).

``CpuRefBackend().eval_node(op, inputs, meta)`` restates
``CpuRefBackend::eval_node`` (crates/mlx-core/src/cpu_kernels.rs:13-102);
``gen_data`` / ``gen_positive_data`` restate crates/mlx-parity/src/lib.rs:22-39.
The C sources are oracle/mlx_cpu_ref.c; build with ``make -C oracle``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import threading

import numpy as np

from oxidizedmlx_amd import abi
from oxidizedmlx_amd.opkind import NodeInput, Op, TensorMeta, inputs_to_c

HERE = os.path.dirname(os.path.abspath(__file__))
# MLXHIP_ORACLE_LIB selects another build of the same sources (the sanitized
# one, oracle/_sanitize/libmlx_cpu_ref.so).
LIB = os.environ.get("MLXHIP_ORACLE_LIB") or os.path.join(HERE, "libmlx_cpu_ref.so")
SAN_LIB = os.path.join(HERE, "_sanitize", "libmlx_cpu_ref.so")

_lib = None
_lock = threading.Lock()


def build(sanitize: bool = False) -> None:
    """Compiles the oracle with its Makefile (gcc, -ffp-contract=off); with
    ``sanitize`` the ASan + UBSan build (clang) into oracle/_sanitize."""
    subprocess.run(["make", "-s", "-C", HERE, "-B"] + (["sanitize"] if sanitize else []), check=True)


def load() -> C.CDLL:
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB):
                raise RuntimeError(f"oracle not built: {LIB} (run make -C oracle)")
            lib = C.CDLL(LIB)
            lib.oracle_eval_node.restype = C.c_int
            lib.oracle_eval_node.argtypes = [C.POINTER(abi.mlxhip_op_t),
                                             C.POINTER(abi.mlxhip_input_t), C.c_size_t,
                                             C.POINTER(abi.mlxhip_meta_t),
                                             C.POINTER(C.POINTER(C.c_float)),
                                             C.POINTER(C.c_size_t)]
            lib.oracle_free.restype = None
            lib.oracle_free.argtypes = [C.c_void_p]
            lib.oracle_last_error.restype = C.c_char_p
            lib.oracle_last_error.argtypes = []
            for name in ("oracle_gen_data", "oracle_gen_positive_data"):
                getattr(lib, name).restype = None
                getattr(lib, name).argtypes = [C.c_void_p, C.c_size_t, C.c_uint64]
            lib.oracle_matmul_rows.restype = None
            lib.oracle_matmul_rows.argtypes = [C.c_void_p] * 3 + [C.c_size_t] * 5
            lib.oracle_softmax_lastdim.restype = None
            lib.oracle_softmax_lastdim.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t]
            for name in ("oracle_layer_norm", "oracle_rms_norm"):
                getattr(lib, name).restype = None
                getattr(lib, name).argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t,
                                               C.c_float]
            _lib = lib
        return _lib


class CpuRefBackend:
    """The reference CPU backend (the parity oracle)."""

    def eval_node(self, op: Op, inputs, out_meta: TensorMeta) -> np.ndarray:
        lib = load()
        cop, keep_op = op.to_c()
        arr, keep_in = inputs_to_c(inputs)
        cm, keep_m = out_meta.to_c()
        out = C.POINTER(C.c_float)()
        n = C.c_size_t(0)
        rc = lib.oracle_eval_node(C.byref(cop), arr, len(inputs), C.byref(cm), C.byref(out),
                                  C.byref(n))
        if rc != abi.OK:
            raise abi.error_for(rc, lib.oracle_last_error().decode())
        try:
            res = np.ctypeslib.as_array(out, shape=(max(1, n.value),))[: n.value].copy()
        finally:
            lib.oracle_free(out)
        del keep_op, keep_in, keep_m
        return res


def gen_data(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    load().oracle_gen_data(out.ctypes.data, n, seed)
    return out


def gen_positive_data(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    load().oracle_gen_positive_data(out.ctypes.data, n, seed)
    return out


def matmul_rows(a: np.ndarray, b: np.ndarray, c: np.ndarray, row0: int, nrows: int) -> None:
    m, k = a.shape
    n = b.shape[1]
    load().oracle_matmul_rows(a.ctypes.data, b.ctypes.data, c.ctypes.data, m, k, n, row0, nrows)


def softmax_lastdim(x: np.ndarray) -> np.ndarray:
    y = np.empty_like(x)
    load().oracle_softmax_lastdim(x.ctypes.data, y.ctypes.data, x.shape[0], x.shape[1])
    return y


def layer_norm(x: np.ndarray, eps: float) -> np.ndarray:
    y = np.empty_like(x)
    load().oracle_layer_norm(x.ctypes.data, y.ctypes.data, x.shape[0], x.shape[1], eps)
    return y


def rms_norm(x: np.ndarray, eps: float) -> np.ndarray:
    y = np.empty_like(x)
    load().oracle_rms_norm(x.ctypes.data, y.ctypes.data, x.shape[0], x.shape[1], eps)
    return y
