"""Python face of libmlxhip.so: HipBackend, HipStream, device buffers, the
direct kernel entry points and HIP-event timing.

``HipBackend().eval_node(op, inputs, meta)`` is the reference's
``Backend::eval_node`` (crates/mlx-core/src/backend.rs:27-35) with the
host-vector contract; ``HipStream`` is ``Stream`` (backend.rs:37-185) bound to
this backend with HBM-resident buffers (``hip_stream()`` is the drop-in for
``cpu_stream()`` / ``metal_stream()``). Everything goes through the C ABI;
without the built library or without a GPU the calls raise
``BackendUnavailable`` -- there is no fallback.
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np

from . import abi
from .opkind import NodeInput, Op, TensorMeta, inputs_to_c

_inited = False


def lib() -> C.CDLL:
    return abi.load_library()


def init(device: int = 0) -> None:
    """Loads the library and selects/initialises ``device``."""
    global _inited
    L = lib()
    abi.check(L.mlxhip_init(device), L)
    _inited = True


def device_count() -> int:
    return lib().mlxhip_device_count()


def synchronize(stream: int | None = None) -> None:
    abi.check(lib().mlxhip_synchronize(stream))


class HipBackend:
    """Backend::eval_node with host inputs (copies in, runs in HBM, copies out)."""

    def eval_node(self, op: Op, inputs: Sequence[NodeInput], out_meta: TensorMeta) -> np.ndarray:
        L = lib()
        cop, k1 = op.to_c()
        arr, k2 = inputs_to_c(inputs)
        cm, k3 = out_meta.to_c()
        n = out_meta.numel()
        out = np.empty(max(n, 1), dtype=np.float32)
        abi.check(L.mlxhip_eval_node(C.byref(cop), arr, len(inputs), C.byref(cm), out.ctypes.data, n), L)
        del k1, k2, k3
        return out[:n]


class HipStream:
    """Stream bound to mlx-hip: lazy graph, CSE, memoised HBM-resident buffers."""

    def __init__(self, fusion: bool = True, async_eval: bool = False):
        L = lib()
        self._L = L
        self._s = L.mlxhip_stream_new()
        if not self._s:
            raise abi.error_for(L.mlxhip_last_status(), L.mlxhip_last_error().decode())
        self.metas: dict[int, TensorMeta] = {}
        if not fusion:
            self.set_fusion(False)
        if async_eval:
            self.set_async(True)

    def close(self) -> None:
        if getattr(self, "_s", None):
            self._L.mlxhip_stream_free(self._s)
            self._s = None

    def __del__(self):
        self.close()

    def set_fusion(self, enabled: bool) -> None:
        abi.check(self._L.mlxhip_stream_set_fusion(self._s, 1 if enabled else 0), self._L)

    def set_async(self, enabled: bool) -> None:
        """Asynchronous evaluation: eval returns once the kernels are queued;
        get_buffer / synchronize / close wait for them."""
        abi.check(self._L.mlxhip_stream_set_async(self._s, 1 if enabled else 0), self._L)

    def synchronize(self) -> None:
        abi.check(self._L.mlxhip_stream_synchronize(self._s), self._L)

    def clear(self) -> None:
        """Forgets every node (their HBM is reused by this stream's later
        work); node ids handed out before are no longer valid."""
        abi.check(self._L.mlxhip_stream_clear(self._s), self._L)
        self.metas.clear()

    def add_constant(self, data, m: TensorMeta) -> int:
        d = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        cm, keep = m.to_c()
        nid = self._L.mlxhip_stream_add_constant(self._s, d.ctypes.data, d.size, C.byref(cm))
        if nid == 0:
            abi.check(self._L.mlxhip_last_status() or abi.ERR_FFI_FAILED, self._L)
        self.metas[nid] = m
        return nid

    def add_op(self, op: Op, inputs: Sequence[int], m: TensorMeta) -> int:
        cop, k1 = op.to_c()
        cm, k2 = m.to_c()
        ids = (C.c_uint64 * max(1, len(inputs)))(*inputs)
        nid = self._L.mlxhip_stream_add_op(self._s, C.byref(cop), ids, len(inputs), C.byref(cm))
        if nid == 0:
            abi.check(self._L.mlxhip_last_status() or abi.ERR_FFI_FAILED, self._L)
        self.metas[nid] = m
        return nid

    def eval(self, nid: int) -> None:
        abi.check(self._L.mlxhip_stream_eval(self._s, nid), self._L)

    def eval_many(self, nids: Sequence[int]) -> None:
        ids = (C.c_uint64 * max(1, len(nids)))(*nids)
        abi.check(self._L.mlxhip_stream_eval_many(self._s, ids, len(nids)), self._L)

    def add_constant_dev(self, ptr: int, m: TensorMeta) -> int:
        """Constant copied from device memory at ``ptr`` (numel(m) floats),
        which must stay unchanged until the next eval on this stream returns."""
        cm, keep = m.to_c()
        nid = self._L.mlxhip_stream_add_constant_dev(self._s, ptr, m.numel(), C.byref(cm))
        if nid == 0:
            abi.check(self._L.mlxhip_last_status() or abi.ERR_FFI_FAILED, self._L)
        self.metas[nid] = m
        return nid

    def add_constant_view(self, ptr: int, m: TensorMeta) -> int:
        """Constant that reads numel(m) floats at device address ``ptr``
        (256-byte aligned) in place. The memory must stay valid and unchanged
        while a queued kernel may read it: while the node exists and, with
        asynchronous evaluation, until the stream is next synchronized
        (``synchronize``, ``get_buffer``, ``close``), even after ``clear``,
        which does not wait for queued kernels. With synchronous evaluation,
        ``clear`` / ``close`` end it."""
        cm, keep = m.to_c()
        nid = self._L.mlxhip_stream_add_constant_view(self._s, ptr, m.numel(), C.byref(cm))
        if nid == 0:
            abi.check(self._L.mlxhip_last_status() or abi.ERR_FFI_FAILED, self._L)
        self.metas[nid] = m
        return nid

    def grad(self, loss: int, wrt: Sequence[int]) -> list[int]:
        """value_and_grad's backward pass (mlx-autograd lib.rs:30-107) for
        several wrt nodes: returns the (unevaluated) gradient node ids."""
        ids = (C.c_uint64 * max(1, len(wrt)))(*wrt)
        out = (C.c_uint64 * max(1, len(wrt)))()
        abi.check(self._L.mlxhip_stream_grad(self._s, loss, ids, len(wrt), out), self._L)
        res = [int(out[i]) for i in range(len(wrt))]
        for g, w in zip(res, wrt):
            self.metas.setdefault(g, self.metas[w])
        return res

    def get_buffer(self, nid: int) -> np.ndarray:
        n = self.metas[nid].numel()
        out = np.empty(max(n, 1), dtype=np.float32)
        abi.check(self._L.mlxhip_stream_get_buffer(self._s, nid, out.ctypes.data, n), self._L)
        return out[:n]

    def eval_count(self) -> int:
        return self._L.mlxhip_stream_eval_count(self._s)

    def cache_len(self) -> int:
        return self._L.mlxhip_stream_cache_len(self._s)

    def launch_count(self) -> int:
        return self._L.mlxhip_stream_launch_count(self._s)




def hip_stream(fusion: bool = True) -> HipStream:
    """The drop-in for ``cpu_stream()`` / ``metal_stream()``."""
    return HipStream(fusion=fusion)


class DeviceBuffer:
    """HBM buffer owned by Python (freed when collected)."""

    def __init__(self, nbytes: int):
        L = lib()
        self._L = L
        self.nbytes = int(nbytes)
        self._b = L.mlxhip_buffer_alloc(self.nbytes)
        if not self._b:
            raise abi.error_for(abi.ERR_FFI_FAILED, L.mlxhip_last_error().decode())
        self.ptr = L.mlxhip_buffer_ptr(self._b) or 0

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        abi.check(self._L.mlxhip_buffer_upload(self._b, offset, a.ctypes.data, a.nbytes), self._L)

    def download(self, dtype=np.float32, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        abi.check(self._L.mlxhip_buffer_download(self._b, offset, out.ctypes.data, out.nbytes), self._L)
        return out

    def free(self) -> None:
        if getattr(self, "_b", None):
            self._L.mlxhip_buffer_free(self._b)
            self._b = None
            self.ptr = 0

    def __del__(self):
        self.free()


def _p(x) -> int:
    return x.ptr if isinstance(x, DeviceBuffer) else int(x or 0)


def eval_node_dev(op: Op, inputs: Sequence[tuple], out_meta: TensorMeta, out, stream=None) -> None:
    """Backend::eval_node on HBM-resident operands (mlxhip_eval_node_dev):
    ``inputs`` are (device buffer or address, shape) pairs, ``out`` receives
    numel(out_meta) f32 values; asynchronous on ``stream``."""
    L = lib()
    cop, k1 = op.to_c()
    nodes = [NodeInput(np.empty(0, np.float32), tuple(shape)) for _, shape in inputs]
    arr, k2 = inputs_to_c(nodes, [_p(buf) for buf, _ in inputs])
    cm, k3 = out_meta.to_c()
    abi.check(L.mlxhip_eval_node_dev(C.byref(cop), arr, len(inputs), C.byref(cm), _p(out), stream), L)
    del k1, k2, k3


def gemm(ab_dtype: int, c_dtype: int, trans_a: bool, trans_b: bool, m: int, n: int, k: int,
         a, lda: int, b, ldb: int, c, ldc: int, batch: int = 1, stride_a: int = 0,
         stride_b: int = 0, stride_c: int = 0, stream: int | None = None) -> None:
    L = lib()
    abi.check(L.mlxhip_gemm(ab_dtype, c_dtype, int(trans_a), int(trans_b), m, n, k, batch,
                            _p(a), lda, stride_a, _p(b), ldb, stride_b, _p(c), ldc, stride_c,
                            stream), L)


def gemm_noalloc(ab_dtype: int, c_dtype: int, trans_a: bool, trans_b: bool, m: int, n: int,
                 k: int, a, lda: int, b, ldb: int, c, ldc: int, batch: int = 1,
                 stride_a: int = 0, stride_b: int = 0, stride_c: int = 0,
                 stream: int | None = None) -> None:
    """``gemm`` without any device allocation: its workspace comes from the
    library's fixed per-device scratch (``gemm_noalloc_scratch_bytes()``);
    calls that overlap on one device race."""
    L = lib()
    abi.check(L.mlxhip_gemm_noalloc(ab_dtype, c_dtype, int(trans_a), int(trans_b), m, n, k, batch,
                                    _p(a), lda, stride_a, _p(b), ldb, stride_b, _p(c), ldc,
                                    stride_c, stream), L)


def gemm_noalloc_scratch_bytes() -> int:
    return lib().mlxhip_gemm_noalloc_scratch_bytes()


def softmax_rows(x, y, rows: int, cols: int, stream=None) -> None:
    abi.check(lib().mlxhip_softmax_rows(_p(x), _p(y), rows, cols, stream))


def scaled_masked_softmax_rows(x, y, rows, cols, scale, causal, stream=None) -> None:
    abi.check(lib().mlxhip_scaled_masked_softmax_rows(_p(x), _p(y), rows, cols, scale,
                                                      int(causal), stream))


def layernorm_rows(x, y, rows: int, cols: int, eps: float, stream=None) -> None:
    abi.check(lib().mlxhip_layernorm_rows(_p(x), _p(y), rows, cols, eps, stream))


def rmsnorm_rows(x, y, rows: int, cols: int, eps: float, stream=None) -> None:
    abi.check(lib().mlxhip_rmsnorm_rows(_p(x), _p(y), rows, cols, eps, stream))


def softmax_vjp_rows(dy, s, dx, rows, cols, stream=None) -> None:
    abi.check(lib().mlxhip_softmax_vjp_rows(_p(dy), _p(s), _p(dx), rows, cols, stream))


def layernorm_vjp_rows(dy, x, dx, rows, cols, eps, stream=None) -> None:
    abi.check(lib().mlxhip_layernorm_vjp_rows(_p(dy), _p(x), _p(dx), rows, cols, eps, stream))


def rmsnorm_vjp_rows(dy, x, dx, rows, cols, eps, stream=None) -> None:
    abi.check(lib().mlxhip_rmsnorm_vjp_rows(_p(dy), _p(x), _p(dx), rows, cols, eps, stream))


EW = {"add": 0, "sub": 1, "rsub": 2, "mul": 3, "div": 4, "rdiv": 5, "neg": 6, "exp": 7,
      "log": 8, "sqrt": 9, "silu": 10, "gelu": 11, "silu_vjp": 12, "gelu_vjp": 13}


def ew_chain(prog: Sequence[tuple], inputs: Sequence, out, numel: int, stream=None) -> None:
    """prog: sequence of (op_name, operand_index); acc starts as inputs[0]."""
    ins = (abi.mlxhip_ew_instr_t * max(1, len(prog)))()
    for i, (op, operand) in enumerate(prog):
        ins[i].op = EW[op] if isinstance(op, str) else int(op)
        ins[i].operand = int(operand)
    ptrs = (C.c_void_p * max(1, len(inputs)))(*[_p(x) for x in inputs])
    abi.check(lib().mlxhip_ew_chain(ins, len(prog), ptrs, len(inputs), _p(out), numel, stream))


def attention(q, k, v, o, batch: int, tq: int, tk: int, dh: int, scale: float, causal: bool,
              stream=None) -> None:
    """Fused attention of `batch` packed heads (device buffers)."""
    abi.check(lib().mlxhip_attention(_p(q), _p(k), _p(v), _p(o), batch, tq, tk, dh, scale, int(causal), stream))


def attention_vjp(q, k, v, o, do, dq, dk, dv, batch: int, t: int, dh: int, scale: float, causal: bool,
                  stream=None) -> None:
    """dQ, dK, dV of fused attention for `batch` packed heads (device buffers)."""
    abi.check(lib().mlxhip_attention_vjp(_p(q), _p(k), _p(v), _p(o), _p(do), _p(dq), _p(dk), _p(dv), batch, t, dh,
                                         scale, int(causal), stream))


def transpose2d(x, y, rows: int, cols: int, stream=None) -> None:
    abi.check(lib().mlxhip_transpose2d(_p(x), _p(y), rows, cols, stream))


def cast(x, src: int, y, dst: int, n: int, stream=None) -> None:
    abi.check(lib().mlxhip_cast(_p(x), src, _p(y), dst, n, stream))


class Event:
    def __init__(self):
        L = lib()
        self._L = L
        self._e = L.mlxhip_event_create()
        if not self._e:
            raise abi.error_for(abi.ERR_FFI_FAILED, L.mlxhip_last_error().decode())

    def record(self, stream=None) -> None:
        abi.check(self._L.mlxhip_event_record(self._e, stream), self._L)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0)
        abi.check(self._L.mlxhip_event_elapsed_ms(self._e, end._e, C.byref(ms)), self._L)
        return ms.value

    def __del__(self):
        if getattr(self, "_e", None):
            self._L.mlxhip_event_destroy(self._e)
            self._e = None


def create_stream() -> int:
    s = lib().mlxhip_stream_create_hip()
    if not s:
        raise abi.error_for(abi.ERR_FFI_FAILED, lib().mlxhip_last_error().decode())
    return s


def destroy_stream(s: int) -> None:
    lib().mlxhip_stream_destroy_hip(s)


class HipDecoder:
    """Greedy decoder of a decoder-only model built from mlx-nn layers, with
    bf16 parameters, the KV cache and the token loop resident in HBM
    (``mlxhip_decoder_*``). ``cfg`` is an ``nn.DecoderConfig``."""

    def __init__(self, cfg):
        L = lib()
        self._L = L
        self.cfg = cfg
        c = abi.mlxhip_decoder_config_t(cfg.n_layers, cfg.d_model, cfg.n_heads, cfg.hidden, cfg.vocab,
                                        cfg.max_batch, cfg.max_seq, cfg.eps)
        self._d = L.mlxhip_decoder_new(C.byref(c))
        if not self._d:
            raise abi.error_for(L.mlxhip_last_status(), L.mlxhip_last_error().decode())

    def close(self) -> None:
        if getattr(self, "_d", None):
            self._L.mlxhip_decoder_free(self._d)
            self._d = None

    def __del__(self):
        self.close()

    def set_param(self, layer: int, which: int, values: np.ndarray) -> None:
        v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
        abi.check(self._L.mlxhip_decoder_set_param(self._d, layer, which, v.ctypes.data, v.size), self._L)

    def load(self, params: dict) -> None:
        """``params`` as made by ``nn.decoder_params``."""
        self.set_param(0, abi.DEC_EMBEDDING, params["embedding"])
        self.set_param(0, abi.DEC_LM_HEAD, params["lm_head"])
        for l, lp in enumerate(params["layers"]):
            for name, which in abi.DEC_LAYER_PARAMS.items():
                self.set_param(l, which, lp[name])

    def generate(self, prompt: np.ndarray, n_new: int, *, argmax: bool = False, logits: bool = False,
                 eager: bool = False):
        """prompt [batch, prompt_len] int token ids -> tokens [batch, n_new];
        with ``argmax``/``logits`` also the argmax [batch, S] and the logits
        [batch, S, vocab] after each of the S = prompt_len + n_new - 1
        positions (returned as a tuple)."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        if p.ndim != 2:
            raise abi.InvalidArgument(f"prompt must be [batch, prompt_len], got shape {list(p.shape)}")
        b, t = p.shape
        steps = t + n_new - 1
        toks = np.zeros((b, max(n_new, 1)), np.int32)
        am = np.zeros((b, max(steps, 1)), np.int32) if argmax else None
        lg = np.zeros((b, max(steps, 1), self.cfg.vocab), np.float32) if logits else None
        rc = self._L.mlxhip_decoder_generate(
            self._d, p.ctypes.data, b, t, n_new, toks.ctypes.data,
            am.ctypes.data if am is not None else None, lg.ctypes.data if lg is not None else None,
            abi.DEC_EAGER if eager else 0)
        abi.check(rc, self._L)
        out = [toks]
        if argmax:
            out.append(am)
        if logits:
            out.append(lg)
        return out[0] if len(out) == 1 else tuple(out)

    def last_timing(self) -> tuple[float, int]:
        """(device milliseconds, positions) of the last generate."""
        ms, steps = C.c_float(), C.c_int32()
        abi.check(self._L.mlxhip_decoder_last_timing(self._d, C.byref(ms), C.byref(steps)), self._L)
        return ms.value, steps.value

    def weight_bytes(self) -> int:
        return self._L.mlxhip_decoder_weight_bytes(self._d)


class Graph:
    """The direct kernel calls issued on `stream` inside the ``with`` block,
    recorded once and replayed by ``launch`` (mlxhip_graph_*)."""

    def __init__(self, stream: int):
        if not stream:
            raise abi.NullPtr("Graph: record on a created stream, not the null stream")
        self.stream = stream
        self._g = None

    def __enter__(self) -> "Graph":
        abi.check(lib().mlxhip_graph_begin(self.stream))
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        L = lib()
        g = L.mlxhip_graph_end(self.stream)
        if exc_type is None and not g:
            raise abi.error_for(L.mlxhip_last_status(), L.mlxhip_last_error().decode())
        self._g = g

    def launch(self, stream: int | None = None) -> None:
        abi.check(lib().mlxhip_graph_launch(self._g, stream if stream is not None else self.stream))

    def close(self) -> None:
        if getattr(self, "_g", None):
            lib().mlxhip_graph_free(self._g)
            self._g = None

    def __del__(self):
        self.close()
