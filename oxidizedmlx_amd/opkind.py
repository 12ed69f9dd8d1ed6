"""OpKind, TensorMeta and NodeInput as Python values, mirroring
crates/mlx-core/src/graph.rs:18-168 and crates/mlx-core/src/backend.rs:16-20.

``OpKind.Add``, ``OpKind.Softmax(axis=-1)``, ``OpKind.LayerNorm(eps=1e-5)``
and so on read like the Rust enum. ``to_c()`` packs a value into the
``mlxhip_op_t`` struct of include/mlxhip.h (keeping referenced arrays alive).
"""
from __future__ import annotations

import functools

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional, Sequence, Tuple

import numpy as np

from . import abi

KIND = {
    "Constant": 0, "Parameter": 1, "Add": 2, "Sub": 3, "Mul": 4, "Div": 5, "Neg": 6,
    "Exp": 7, "Log": 8, "Sum": 9, "Mean": 10, "Max": 11, "MatMul": 12, "Reshape": 13,
    "Transpose": 14, "Softmax": 15, "Silu": 16, "Gelu": 17, "LayerNorm": 18,
    "RmsNorm": 19, "Rope": 20, "Broadcast": 21, "Embedding": 22,
    "ScaledMaskedSoftmax": 23, "Attention": 24, "LayerNormVjp": 25, "RmsNormVjp": 26,
    "SoftmaxVjp": 27, "SiluVjp": 28, "GeluVjp": 29, "Sqrt": 30, "RoPE": 31,
    "Narrow": 32, "Concatenate": 33, "HeadAttention": 34, "HeadAttentionVjp": 35,
}
NAME = {v: k for k, v in KIND.items()}


@dataclass(frozen=True)
class Op:
    """One OpKind value. Fields an op does not use keep their defaults."""

    name: str
    axis: Optional[int] = None
    eps: float = 0.0
    scale: float = 0.0
    causal: bool = False
    shape: Optional[Tuple[int, ...]] = None
    axes: Optional[Tuple[int, ...]] = None
    start: int = 0
    length: int = 0
    rotary_dim: int = 0
    pos_offset: int = 0
    theta: float = 0.0
    base: float = 0.0
    offset: int = 0
    traditional: bool = False

    @property
    def kind(self) -> int:
        return KIND[self.name]

    def to_c(self) -> Tuple[abi.mlxhip_op_t, list]:
        """The C form (and the arrays it points into); built once per Op
        object (kept on it) and per value (shared), the C side only reads it."""
        c = self.__dict__.get("_c")
        if c is None:
            c = _op_to_c(self)
            object.__setattr__(self, "_c", c)
        return c

    def _build_c(self) -> Tuple[abi.mlxhip_op_t, list]:
        keep: list = []
        s = abi.mlxhip_op_t()
        s.kind = self.kind
        s.axis = int(self.axis) if self.axis is not None else 0
        s.has_axis = 1 if self.axis is not None else 0
        s.causal = 1 if self.causal else 0
        s.eps = self.eps
        s.scale = self.scale
        s.theta = self.theta
        s.base = self.base
        if self.shape is not None:
            arr = abi.int64_array(self.shape)
            keep.append(arr)
            s.shape = C.cast(arr, C.POINTER(C.c_int64))
            s.shape_len = len(self.shape)
        if self.axes is not None:
            arr = abi.int64_array(self.axes)
            keep.append(arr)
            s.axes = C.cast(arr, C.POINTER(C.c_int64))
            s.axes_len = len(self.axes)
        s.start = self.start
        s.length = self.length
        s.rotary_dim = self.rotary_dim
        s.pos_offset = self.pos_offset
        s.offset = self.offset
        s.traditional = 1 if self.traditional else 0
        return s, keep

    def __repr__(self) -> str:  # compact, Rust-like
        return f"OpKind::{self.name}"


_ops: dict = {}


def _interned(name: str, **kw) -> Op:
    """One Op object per (variant, payload), so its C form is built once
    (graph building asks for the same reshapes and transposes every step)."""
    key = (name, tuple(sorted(kw.items())))
    op = _ops.get(key)
    if op is None:
        if len(_ops) > 4096:
            _ops.clear()
        op = _ops[key] = Op(name, **kw)
    return op


class OpKind:
    """Constructors named like the variants of the Rust enum."""

    Constant = Op("Constant")
    Parameter = Op("Parameter")
    Add = Op("Add")
    Sub = Op("Sub")
    Mul = Op("Mul")
    Div = Op("Div")
    Neg = Op("Neg")
    Exp = Op("Exp")
    Log = Op("Log")
    MatMul = Op("MatMul")
    Silu = Op("Silu")
    Gelu = Op("Gelu")
    Embedding = Op("Embedding")
    SiluVjp = Op("SiluVjp")
    GeluVjp = Op("GeluVjp")
    Sqrt = Op("Sqrt")

    @staticmethod
    def Sum(axis: Optional[int] = None) -> Op:
        return Op("Sum", axis=axis)

    @staticmethod
    def Mean(axis: Optional[int] = None) -> Op:
        return Op("Mean", axis=axis)

    @staticmethod
    def Max(axis: Optional[int] = None) -> Op:
        return Op("Max", axis=axis)

    @staticmethod
    def Reshape(new_shape: Sequence[int]) -> Op:
        return _interned("Reshape", shape=tuple(map(int, new_shape)))

    @staticmethod
    def Transpose(axes: Optional[Sequence[int]] = None) -> Op:
        return _interned("Transpose", axes=None if axes is None else tuple(map(int, axes)))

    @staticmethod
    def Softmax(axis: int) -> Op:
        return Op("Softmax", axis=axis)

    @staticmethod
    def LayerNorm(eps: float) -> Op:
        return Op("LayerNorm", eps=eps)

    @staticmethod
    def RmsNorm(eps: float) -> Op:
        return Op("RmsNorm", eps=eps)

    @staticmethod
    def Rope(rotary_dim: int, pos_offset: int, theta: float) -> Op:
        return Op("Rope", rotary_dim=rotary_dim, pos_offset=pos_offset, theta=theta)

    @staticmethod
    def Broadcast(target_shape: Sequence[int]) -> Op:
        return _interned("Broadcast", shape=tuple(map(int, target_shape)))

    @staticmethod
    def ScaledMaskedSoftmax(scale: float, causal: bool) -> Op:
        return Op("ScaledMaskedSoftmax", scale=scale, causal=causal)

    @staticmethod
    def Attention(scale: float, causal: bool) -> Op:
        return Op("Attention", scale=scale, causal=causal)

    @staticmethod
    def HeadAttention(scale: float, causal: bool, heads: Optional[int] = None) -> Op:
        """Attention of every head of Q, K, V (no reference counterpart;
        differentiable on a HIP stream): [heads, t, dh], or with ``heads``
        [groups, t, heads * dh] with the heads side by side in each row."""
        return Op("HeadAttention", scale=scale, causal=causal, axis=heads)

    @staticmethod
    def HeadAttentionVjp(scale: float, causal: bool, heads: Optional[int] = None) -> Op:
        return Op("HeadAttentionVjp", scale=scale, causal=causal, axis=heads)

    @staticmethod
    def LayerNormVjp(eps: float) -> Op:
        return Op("LayerNormVjp", eps=eps)

    @staticmethod
    def RmsNormVjp(eps: float) -> Op:
        return Op("RmsNormVjp", eps=eps)

    @staticmethod
    def SoftmaxVjp(axis: int) -> Op:
        return Op("SoftmaxVjp", axis=axis)

    @staticmethod
    def RoPE(base: float, offset: int, traditional: bool) -> Op:
        return Op("RoPE", base=base, offset=offset, traditional=traditional)

    @staticmethod
    def Narrow(axis: int, start: int, length: int) -> Op:
        return Op("Narrow", axis=axis, start=start, length=length)

    @staticmethod
    def Concatenate(axis: int) -> Op:
        return Op("Concatenate", axis=axis)


@dataclass(frozen=True)
class TensorMeta:
    """TensorMeta (graph.rs:18-21)."""

    shape: Tuple[int, ...]
    dtype: int = abi.F32

    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= int(d)
        return n

    def to_c(self) -> Tuple[abi.mlxhip_meta_t, list]:
        """The C form (built once per object and per value, read-only on the
        C side)."""
        c = self.__dict__.get("_c")
        if c is None:
            c = _meta_to_c(self)
            object.__setattr__(self, "_c", c)
        return c

    def _build_c(self) -> Tuple[abi.mlxhip_meta_t, list]:
        arr = abi.int64_array(self.shape)
        m = abi.mlxhip_meta_t()
        m.shape = C.cast(arr, C.POINTER(C.c_int64))
        m.ndim = len(self.shape)
        m.dtype = self.dtype
        return m, [arr]


@functools.lru_cache(maxsize=4096)
def _op_to_c(op: Op):
    return op._build_c()


@functools.lru_cache(maxsize=4096)
def _meta_to_c(m: TensorMeta):
    return m._build_c()


def meta(dims: Sequence[int], dtype: int = abi.F32) -> TensorMeta:
    """The ``meta`` helper of crates/mlx-parity/src/lib.rs:65-71."""
    return TensorMeta(tuple(int(d) for d in dims), dtype)


@dataclass
class NodeInput:
    """NodeInput (backend.rs:16-20): contiguous f32 data, shape and logical dtype."""

    data: np.ndarray
    shape: Tuple[int, ...]
    dtype: int = abi.F32
    _keep: list = field(default_factory=list, repr=False)


def inputs_to_c(inputs: Sequence[NodeInput], device_ptrs: Optional[Sequence[int]] = None):
    """Packs inputs into an ``mlxhip_input_t`` array. With ``device_ptrs`` the
    data fields are those device addresses instead of the host arrays."""
    n = len(inputs)
    arr = (abi.mlxhip_input_t * max(1, n))()
    keep: list = []
    for i, inp in enumerate(inputs):
        shp = abi.int64_array(inp.shape)
        keep.append(shp)
        if device_ptrs is None:
            d = np.ascontiguousarray(inp.data, dtype=np.float32)
            keep.append(d)
            arr[i].data = d.ctypes.data
            arr[i].len = d.size
        else:
            arr[i].data = device_ptrs[i]
            arr[i].len = int(np.prod(inp.shape, dtype=np.int64)) if inp.shape else 1
        arr[i].shape = C.cast(shp, C.POINTER(C.c_int64))
        arr[i].ndim = len(inp.shape)
        arr[i].dtype = inp.dtype
    return arr, keep
