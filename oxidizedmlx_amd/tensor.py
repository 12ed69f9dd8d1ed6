"""Lazy tensors over a Stream: the part of mlx-core's ``Tensor`` API
(crates/mlx-core/src/tensor.rs) that mlx-nn layers and mlx-autograd use,
plus ``value_and_grad`` (crates/mlx-autograd/src/lib.rs:30-107).

A ``Tensor`` is a node id with its shape on a stream. Every method adds a
lazy node with the output shape and validation of the matching Rust method;
nothing runs until a value is asked for. The stream is any object with the
methods ``add_constant(data, meta)``, ``add_op(op, inputs, meta)``,
``eval_many(ids)``, ``get_buffer(id)`` and ``grad(loss, wrt)``:
``backend.HipStream`` (graph, scheduler and autograd in libmlxhip.so) is the
product; the same graph code also runs on the test oracle's CPU stream.

Constructors without a stream (``from_f32``, ``zeros``, ``ones``,
``from_data_with_dtype``) bind to the process default stream, as the
reference's do (tensor.rs:55-78,127-141 over ``default_stream()``,
crates/mlx-core/src/backend.rs:193-200). The reference's default is fixed to
its CPU backend; here it is selectable: ``set_default_stream(stream)``, or the
environment variable ``MLX_RS_BACKEND`` read when the default is first needed
("hip", the default, makes a ``HipStream``; this package has no other
backend, so any other value raises ``BackendUnavailable``).
"""
from __future__ import annotations

import contextlib
import os
import threading
from typing import Callable, Iterator, Optional, Sequence, Tuple

import numpy as np

from . import abi
from .opkind import Op, OpKind, TensorMeta


def _shape(dims) -> Tuple[int, ...]:
    return tuple(map(int, dims))


_metas: dict = {}


def _meta(shape: Tuple[int, ...], dtype: int) -> TensorMeta:
    """One TensorMeta per (shape, dtype), so its C form is built once."""
    key = (shape, dtype)
    m = _metas.get(key)
    if m is None:
        if len(_metas) > 4096:
            _metas.clear()
        m = _metas[key] = TensorMeta(shape, dtype)
    return m


def _numel(shape: Sequence[int]) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


_default_lock = threading.Lock()
_default_stream = None


def set_default_stream(stream) -> None:
    """Makes ``stream`` the process default for constructors without an
    explicit stream (None: back to ``MLX_RS_BACKEND``'s choice on next use)."""
    global _default_stream
    with _default_lock:
        _default_stream = stream


def default_stream():
    """The process default stream (``default_stream()``, backend.rs:198-200),
    created on first use from ``MLX_RS_BACKEND`` unless one was set."""
    global _default_stream
    with _default_lock:
        if _default_stream is None:
            which = os.environ.get("MLX_RS_BACKEND", "hip").strip().lower()
            if which != "hip":
                raise abi.BackendUnavailable(
                    f"MLX_RS_BACKEND={which!r}: this package provides the 'hip' backend only")
            from .backend import HipStream
            _default_stream = HipStream()
        return _default_stream


@contextlib.contextmanager
def default_stream_scope(stream) -> Iterator[object]:
    """Sets the default stream for the ``with`` body, then restores the
    previous one."""
    global _default_stream
    with _default_lock:
        prev, _default_stream = _default_stream, stream
    try:
        yield stream
    finally:
        with _default_lock:
            _default_stream = prev


class Tensor:
    """Lazy tensor handle: (stream, node id, shape, dtype)."""

    __slots__ = ("stream", "node", "shape", "dtype")

    def __init__(self, stream, node: int, shape: Sequence[int], dtype: int = abi.F32):
        self.stream = stream
        self.node = int(node)
        self.shape = _shape(shape)
        self.dtype = dtype

    # ── creation (tensor.rs:55-141) ──────────────────────────────────────
    @classmethod
    def from_f32_on_stream(cls, data, shape: Sequence[int], stream, dtype: int = abi.F32) -> "Tensor":
        """A Constant on ``stream`` (tensor.rs:81-103)."""
        shape = _shape(shape)
        d = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        if d.size != _numel(shape):
            raise abi.InvalidArgument(
                f"data length {d.size} does not match shape {list(shape)} (expected {_numel(shape)})")
        return cls(stream, stream.add_constant(d, _meta(shape, dtype)), shape, dtype)

    @classmethod
    def from_f32(cls, data, shape: Sequence[int], stream=None) -> "Tensor":
        """A Constant on the default stream (tensor.rs:66-78), or on
        ``stream`` when one is given."""
        return cls.from_f32_on_stream(data, shape, stream if stream is not None else default_stream())

    @classmethod
    def from_data_with_dtype(cls, data, shape: Sequence[int], dtype: int, stream=None) -> "Tensor":
        """f32 data with a logical dtype tag (tensor.rs:105-125)."""
        return cls.from_f32_on_stream(data, shape, stream if stream is not None else default_stream(), dtype)

    @classmethod
    def zeros(cls, shape: Sequence[int], dtype: int = abi.F32, stream=None) -> "Tensor":
        """tensor.rs:55-59."""
        return cls.from_data_with_dtype(np.zeros(_numel(_shape(shape)), np.float32), shape, dtype, stream)

    @classmethod
    def ones(cls, shape: Sequence[int], dtype: int = abi.F32, stream=None) -> "Tensor":
        """tensor.rs:61-65."""
        return cls.from_data_with_dtype(np.ones(_numel(_shape(shape)), np.float32), shape, dtype, stream)

    @classmethod
    def from_device(cls, ptr: int, shape: Sequence[int], stream=None, dtype: int = abi.F32) -> "Tensor":
        """Constant copied from f32 device memory (HipStream only; the
        default stream when none is given)."""
        shape = _shape(shape)
        stream = stream if stream is not None else default_stream()
        return cls(stream, stream.add_constant_dev(ptr, _meta(shape, dtype)), shape, dtype)

    @classmethod
    def view_device(cls, ptr: int, shape: Sequence[int], stream=None, dtype: int = abi.F32) -> "Tensor":
        """Constant that reads f32 device memory in place (HipStream only):
        256-byte aligned, valid and unchanged while the node exists."""
        shape = _shape(shape)
        stream = stream if stream is not None else default_stream()
        return cls(stream, stream.add_constant_view(ptr, _meta(shape, dtype)), shape, dtype)

    def _lazy(self, op: Op, inputs: Sequence["Tensor"], shape: Sequence[int]) -> "Tensor":
        shape = _shape(shape)
        st = self.stream
        for t in inputs:
            if t.stream is not st:
                raise abi.InvalidArgument("tensors on different streams cannot be combined")
        nid = st.add_op(op, [t.node for t in inputs], _meta(shape, self.dtype))
        return Tensor(st, nid, shape, self.dtype)

    # ── elementwise (tensor.rs:167-238): equal shapes only ───────────────
    def _binary(self, op: Op, rhs: "Tensor") -> "Tensor":
        if self.shape != rhs.shape:
            raise abi.ShapeMismatch(f"expected {list(self.shape)}, got {list(rhs.shape)}")
        return self._lazy(op, [self, rhs], self.shape)

    def add(self, rhs: "Tensor") -> "Tensor":
        return self._binary(OpKind.Add, rhs)

    def sub(self, rhs: "Tensor") -> "Tensor":
        return self._binary(OpKind.Sub, rhs)

    def mul(self, rhs: "Tensor") -> "Tensor":
        return self._binary(OpKind.Mul, rhs)

    def div(self, rhs: "Tensor") -> "Tensor":
        return self._binary(OpKind.Div, rhs)

    def neg(self) -> "Tensor":
        return self._lazy(OpKind.Neg, [self], self.shape)

    def exp(self) -> "Tensor":
        return self._lazy(OpKind.Exp, [self], self.shape)

    def sqrt(self) -> "Tensor":
        return self._lazy(OpKind.Sqrt, [self], self.shape)

    def silu(self) -> "Tensor":
        return self._lazy(OpKind.Silu, [self], self.shape)

    def gelu(self) -> "Tensor":
        return self._lazy(OpKind.Gelu, [self], self.shape)

    # ── reductions (tensor.rs:243-269) ───────────────────────────────────
    def sum_axis(self, axis: int) -> "Tensor":
        nd = len(self.shape)
        ax = axis + nd if axis < 0 else axis
        if ax < 0 or ax >= nd:
            raise abi.InvalidArgument(f"axis {axis} out of range for ndim {nd}")
        return self._lazy(OpKind.Sum(ax), [self], self.shape[:ax] + self.shape[ax + 1:])

    def sum_all(self) -> "Tensor":
        return self._lazy(OpKind.Sum(None), [self], ())

    # ── linear algebra (tensor.rs:274-296; rank 3 per
    #    evals/tasks/003_matmul_batch_3d.json) ──────────────────────────────
    def matmul(self, rhs: "Tensor") -> "Tensor":
        a, b = self.shape, rhs.shape
        if not ((len(a) == 2 and len(b) == 2) or (len(a) == 3 and len(b) == 3)):
            raise abi.InvalidArgument("matmul requires 2D tensors (or two 3D batched tensors)")
        if len(a) == 3 and a[0] != b[0]:
            raise abi.ShapeMismatch(f"expected batch {a[0]}, got {b[0]}")
        if a[-1] != b[-2]:
            raise abi.ShapeMismatch(f"expected {list(a)}, got {list(b)}")
        return self._lazy(OpKind.MatMul, [self, rhs], a[:-1] + (b[-1],))

    def embedding_lookup(self, indices: "Tensor") -> "Tensor":
        """Rows of this [num_embeddings, dim] weight at ``indices`` (ids as
        f32, clamped by the kernel); output shape indices.shape + [dim]
        (tensor.rs:301-317)."""
        if len(self.shape) != 2:
            raise abi.InvalidArgument("embedding weight must be 2D [num_embeddings, embedding_dim]")
        return self._lazy(OpKind.Embedding, [self, indices], indices.shape + (self.shape[1],))

    # ── shape ops (tensor.rs:322-374, 769-801) ───────────────────────────
    def reshape(self, shape: Sequence[int]) -> "Tensor":
        shape = _shape(shape)
        if _numel(shape) != _numel(self.shape):
            raise abi.ShapeMismatch(f"expected {list(self.shape)}, got {list(shape)}")
        return self._lazy(OpKind.Reshape(shape), [self], shape)

    def transpose(self, axes: Optional[Sequence[int]] = None) -> "Tensor":
        nd = len(self.shape)
        if axes is None:
            perm = tuple(range(nd - 1, -1, -1))
        else:
            perm = tuple(int(a) for a in axes)
            if len(perm) != nd:
                raise abi.InvalidArgument(f"transpose axes length {len(perm)} does not match ndim {nd}")
            if sorted(perm) != list(range(nd)):
                raise abi.InvalidArgument(f"invalid permutation {list(perm)}")
        return self._lazy(OpKind.Transpose(None if axes is None else perm), [self],
                          tuple(self.shape[p] for p in perm))

    def broadcast_to(self, shape: Sequence[int]) -> "Tensor":
        shape = _shape(shape)
        if shape == self.shape:
            return self
        if len(self.shape) > len(shape):
            raise abi.InvalidArgument(f"cannot broadcast shape {list(self.shape)} to {list(shape)}")
        pad = len(shape) - len(self.shape)
        for i, d in enumerate(self.shape):
            if d != 1 and d != shape[pad + i]:
                raise abi.InvalidArgument(f"cannot broadcast shape {list(self.shape)} to {list(shape)}")
        return self._lazy(OpKind.Broadcast(shape), [self], shape)

    def narrow(self, axis: int, start: int, length: int) -> "Tensor":
        """tensor.rs:584-611."""
        nd = len(self.shape)
        ax = axis + nd if axis < 0 else axis
        if ax < 0 or ax >= nd:
            raise abi.InvalidArgument(f"narrow: axis {axis} out of range for ndim {nd}")
        if start < 0 or start + length > self.shape[ax]:
            raise abi.InvalidArgument(
                f"narrow: start {start} + length {length} exceeds dim size {self.shape[ax]}")
        shape = self.shape[:ax] + (int(length),) + self.shape[ax + 1:]
        return self._lazy(OpKind.Narrow(ax, int(start), int(length)), [self], shape)

    @staticmethod
    def cat(tensors: Sequence["Tensor"], axis: int) -> "Tensor":
        """tensor.rs:614-660."""
        if not tensors:
            raise abi.InvalidArgument("cat requires at least one tensor")
        first = tensors[0]
        nd = len(first.shape)
        ax = axis + nd if axis < 0 else axis
        if ax < 0 or ax >= nd:
            raise abi.InvalidArgument(f"cat: axis {axis} out of range for ndim {nd}")
        total = 0
        for t in tensors:
            if len(t.shape) != nd:
                raise abi.InvalidArgument("cat: all tensors must have same ndim")
            for d, (a, b) in enumerate(zip(first.shape, t.shape)):
                if d != ax and a != b:
                    raise abi.ShapeMismatch(f"expected {list(first.shape)}, got {list(t.shape)}",
                                            list(first.shape), list(t.shape))
            total += t.shape[ax]
        shape = first.shape[:ax] + (total,) + first.shape[ax + 1:]
        return first._lazy(OpKind.Concatenate(ax), list(tensors), shape)

    def attention(self, k: "Tensor", v: "Tensor", scale: float, causal: bool) -> "Tensor":
        """Single-head attention Q [Tq, Dh], K/V [Tk, Dh] -> [Tq, Dh]
        (tensor.rs:664-690)."""
        if len(self.shape) != 2 or len(k.shape) != 2 or len(v.shape) != 2:
            raise abi.InvalidArgument("attention requires 2D tensors [seq, head_dim]")
        if k.shape[1] != self.shape[1]:
            raise abi.ShapeMismatch(f"expected {list(self.shape)}, got {list(k.shape)}",
                                    list(self.shape), list(k.shape))
        if v.shape[1] != self.shape[1] or k.shape[0] != v.shape[0]:
            raise abi.ShapeMismatch(f"expected {list(k.shape)}, got {list(v.shape)}",
                                    list(k.shape), list(v.shape))
        return self._lazy(OpKind.Attention(scale, causal), [self, k, v], self.shape)

    # ── row ops (tensor.rs:379-435) ──────────────────────────────────────
    def head_attention(self, k: "Tensor", v: "Tensor", scale: float, causal: bool,
                       heads: Optional[int] = None) -> "Tensor":
        """Attention of every head: Q [H, Tq, Dh], K/V [H, Tk, Dh] -> [H, Tq, Dh],
        per head the arithmetic of ``attention``. With ``heads`` = H the heads
        sit side by side in each row instead: Q [B, Tq, H*Dh], K/V [B, Tk, H*Dh]
        -> [B, Tq, H*Dh] (a [B*T, d_model] projection viewed as [B, T, d_model],
        so no head split or merge is needed). No reference counterpart;
        unlike ``attention`` it has a VJP (one fused backward op) on a HIP
        stream, so a block can train through the fused kernels."""
        if len(self.shape) != 3 or len(k.shape) != 3 or len(v.shape) != 3:
            raise abi.InvalidArgument("head_attention requires 3D tensors [heads, seq, head_dim]")
        if heads is not None and (heads < 1 or self.shape[2] % heads):
            raise abi.InvalidArgument(f"head_attention: {heads} heads do not divide rows of {self.shape[2]}")
        if k.shape[0] != self.shape[0] or k.shape[2] != self.shape[2]:
            raise abi.ShapeMismatch(f"expected {list(self.shape)}, got {list(k.shape)}",
                                    list(self.shape), list(k.shape))
        if v.shape != k.shape:
            raise abi.ShapeMismatch(f"expected {list(k.shape)}, got {list(v.shape)}", list(k.shape), list(v.shape))
        return self._lazy(OpKind.HeadAttention(scale, causal, heads), [self, k, v], self.shape)

    def softmax(self, axis: int) -> "Tensor":
        nd = len(self.shape)
        ax = axis + nd if axis < 0 else axis
        if ax < 0 or ax >= nd:
            raise abi.InvalidArgument(f"axis {axis} out of range for ndim {nd}")
        return self._lazy(OpKind.Softmax(ax), [self], self.shape)

    def layer_norm(self, eps: float) -> "Tensor":
        return self._lazy(OpKind.LayerNorm(eps), [self], self.shape)

    def rms_norm(self, eps: float) -> "Tensor":
        return self._lazy(OpKind.RmsNorm(eps), [self], self.shape)

    # ── values ───────────────────────────────────────────────────────────
    def numel(self) -> int:
        return _numel(self.shape)

    def eval(self) -> "Tensor":
        self.stream.eval_many([self.node])
        return self

    def to_numpy(self) -> np.ndarray:
        self.eval()
        return np.asarray(self.stream.get_buffer(self.node), np.float32).reshape(self.shape)


def eval_all(tensors: Sequence[Tensor]) -> None:
    """Evaluates several tensors of one stream in one scheduling pass."""
    if tensors:
        tensors[0].stream.eval_many([t.node for t in tensors])


def value_and_grad(loss: Tensor, wrt: Sequence[Tensor]) -> Tuple[Tensor, list]:
    """Gradients of the scalar ``loss`` with respect to each of ``wrt``
    (mlx-autograd lib.rs:30-107; the reference takes one wrt tensor per call).
    Returns the loss and the lazy gradient tensors."""
    if loss.numel() != 1:
        raise abi.InvalidArgument(f"grad requires scalar loss, got {loss.numel()} elements")
    ids = loss.stream.grad(loss.node, [w.node for w in wrt])
    return loss, [Tensor(loss.stream, g, w.shape, w.dtype) for g, w in zip(ids, wrt)]


def grad(f: Callable[[Tensor], Tensor], x: Tensor) -> Tensor:
    """grad(f, x) (mlx-autograd lib.rs:20-27)."""
    return value_and_grad(f(x), [x])[1][0]
