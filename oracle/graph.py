"""CPU restatement of the reference's Stream, Graph and autograd
(TEST INFRASTRUCTURE ONLY: imported by tests/ and nowhere in the product).

``OracleStream`` follows Stream (crates/mlx-core/src/backend.rs:37-185) and
Graph (crates/mlx-core/src/graph.rs:170-305): Constants are never
deduplicated, other nodes are interned by (op, inputs, meta) with the two
inputs of Add/Mul ordered by node id (graph.rs:213-256, 495-515), evaluation
walks the depth-first post-order of the requested outputs (graph.rs:268-294)
and evaluates each node once with the C oracle's eval_node
(``CpuRefBackend``, the restatement of crates/mlx-core/src/cpu_kernels.rs).

``OracleStream.grad`` restates backward (crates/mlx-autograd/src/lib.rs:
51-107) and the VJP table (crates/mlx-autograd/src/vjp.rs:8-178) as the
reference builds them: every node on the loss's path with a gradient gets
its full VJP (no pruning). It returns the gradients of several wrt nodes
from one pass; the table the pass builds does not depend on wrt, so each is
what the reference's single-wrt call returns. Rank-3 MatMul (the batched
form of evals/tasks/003_matmul_batch_3d.json) swaps its matrix axes with
Transpose [0,2,1] where rank 2 uses Transpose(None).

Usable with ``oxidizedmlx_amd.tensor.Tensor`` (same stream interface as
``HipStream``).
"""
from __future__ import annotations

from typing import Dict, List, Sequence, Tuple

import numpy as np

from oxidizedmlx_amd import abi
from oxidizedmlx_amd.opkind import NodeInput, Op, OpKind, TensorMeta

from .cpu_ref import CpuRefBackend


class OracleStream:
    def __init__(self):
        self.nodes: Dict[int, Tuple[Op, Tuple[int, ...], TensorMeta]] = {}
        self.cse: Dict[tuple, int] = {}
        self.buffers: Dict[int, np.ndarray] = {}
        self.next_id = 1
        self.backend = CpuRefBackend()
        self.metas: Dict[int, TensorMeta] = {}

    # ── graph building ───────────────────────────────────────────────────
    def _add(self, op: Op, inputs: Sequence[int], m: TensorMeta) -> int:
        inputs = tuple(int(i) for i in inputs)
        for i in inputs:
            if i not in self.nodes:
                raise abi.InvalidArgument(f"unknown input node {i}")
        cse_ok = op.name not in ("Constant", "Parameter")
        if cse_ok:
            if op.name in ("Add", "Mul") and len(inputs) == 2 and inputs[0] > inputs[1]:
                inputs = (inputs[1], inputs[0])
            key = (op, inputs, m)
            if key in self.cse:
                return self.cse[key]
        nid = self.next_id
        self.next_id += 1
        self.nodes[nid] = (op, inputs, m)
        self.metas[nid] = m
        if cse_ok:
            self.cse[key] = nid
        return nid

    def add_constant(self, data, m: TensorMeta) -> int:
        d = np.ascontiguousarray(data, dtype=np.float32).reshape(-1).copy()
        if d.size != m.numel():
            raise abi.ShapeMismatch(f"{d.size} values for {m.numel()} elements")
        nid = self._add(OpKind.Constant, (), m)
        self.buffers[nid] = d
        return nid

    def add_op(self, op: Op, inputs: Sequence[int], m: TensorMeta) -> int:
        return self._add(op, inputs, m)

    # ── evaluation ───────────────────────────────────────────────────────
    def topo_sort(self, outputs: Sequence[int]) -> List[int]:
        order, visited = [], set()
        for out in outputs:
            if out in visited:
                continue
            visited.add(out)
            stack = [(out, 0)]
            while stack:
                nid, i = stack[-1]
                ins = self.nodes[nid][1] if nid in self.nodes else ()
                if i < len(ins):
                    stack[-1] = (nid, i + 1)
                    nxt = ins[i]
                    if nxt not in visited:
                        visited.add(nxt)
                        stack.append((nxt, 0))
                else:
                    order.append(nid)
                    stack.pop()
        return order

    def eval_many(self, outputs: Sequence[int]) -> None:
        for nid in self.topo_sort(outputs):
            if nid in self.buffers:
                continue
            op, ins, m = self.nodes[nid]
            inputs = [NodeInput(self.buffers[i], self.nodes[i][2].shape, self.nodes[i][2].dtype) for i in ins]
            self.buffers[nid] = self.backend.eval_node(op, inputs, m)

    def eval(self, nid: int) -> None:
        self.eval_many([nid])

    def get_buffer(self, nid: int) -> np.ndarray:
        if nid not in self.buffers:
            raise abi.InvalidArgument("node not materialised")
        return self.buffers[nid]

    # ── autograd ─────────────────────────────────────────────────────────
    def _shape(self, nid: int) -> Tuple[int, ...]:
        return self.nodes[nid][2].shape

    def _dtype(self, nid: int) -> int:
        return self.nodes[nid][2].dtype

    def _op(self, op: Op, inputs: Sequence[int], shape: Sequence[int]) -> int:
        return self._add(op, inputs, TensorMeta(tuple(int(s) for s in shape), self._dtype(inputs[0])))

    def _transpose(self, a: int, perm) -> int:
        sh = self._shape(a)
        p = tuple(range(len(sh) - 1, -1, -1)) if perm is None else tuple(perm)
        return self._op(OpKind.Transpose(perm), [a], [sh[i] for i in p])

    def _matmul(self, a: int, b: int) -> int:
        sa, sb = self._shape(a), self._shape(b)
        return self._op(OpKind.MatMul, [a, b], sa[:-1] + (sb[-1],))

    def _broadcast_to(self, a: int, shape) -> int:
        shape = tuple(shape)
        if self._shape(a) == shape:
            return a
        return self._op(OpKind.Broadcast(shape), [a], shape)

    def _sum_axis(self, a: int, ax: int) -> int:
        sh = self._shape(a)
        return self._op(OpKind.Sum(ax), [a], sh[:ax] + sh[ax + 1:])

    def _reshape(self, a: int, shape) -> int:
        return self._op(OpKind.Reshape(tuple(shape)), [a], shape)

    def _vjp(self, nid: int, g: int) -> List[int]:
        op, ins, m = self.nodes[nid]
        name = op.name
        sh = lambda i: self._shape(i)  # noqa: E731
        if name == "Add":
            return [g, g]
        if name == "Sub":
            return [g, self._op(OpKind.Neg, [g], sh(g))]
        if name == "Mul":
            return [self._op(OpKind.Mul, [g, ins[1]], sh(g)), self._op(OpKind.Mul, [g, ins[0]], sh(g))]
        if name == "Div":
            ga = self._op(OpKind.Div, [g, ins[1]], sh(g))
            neg_a = self._op(OpKind.Neg, [ins[0]], sh(ins[0]))
            b_sq = self._op(OpKind.Mul, [ins[1], ins[1]], sh(ins[1]))
            gb = self._op(OpKind.Div, [self._op(OpKind.Mul, [g, neg_a], sh(g)), b_sq], sh(g))
            return [ga, gb]
        if name == "Neg":
            return [self._op(OpKind.Neg, [g], sh(g))]
        if name == "Sum":
            ish = sh(ins[0])
            if op.axis is None:
                return [self._broadcast_to(g, ish)]
            uns = list(sh(g))
            uns.insert(op.axis, 1)
            return [self._broadcast_to(self._reshape(g, uns), ish)]
        if name == "MatMul":
            perm = (0, 2, 1) if len(sh(ins[0])) == 3 else None
            b_t = self._transpose(ins[1], perm)
            a_t = self._transpose(ins[0], perm)
            return [self._matmul(g, b_t), self._matmul(a_t, g)]
        if name == "Reshape":
            return [self._reshape(g, sh(ins[0]))]
        if name == "Transpose":
            nd = len(sh(ins[0]))
            perm = op.axes if op.axes is not None else tuple(range(nd - 1, -1, -1))
            inv = [0] * nd
            for i, p in enumerate(perm):
                inv[p] = i
            return [self._transpose(g, tuple(inv))]
        if name == "LayerNorm":
            return [self._op(OpKind.LayerNormVjp(op.eps), [g, ins[0]], sh(ins[0]))]
        if name == "RmsNorm":
            return [self._op(OpKind.RmsNormVjp(op.eps), [g, ins[0]], sh(ins[0]))]
        if name == "Softmax":
            s = self._op(OpKind.Softmax(op.axis), [ins[0]], sh(ins[0]))
            return [self._op(OpKind.SoftmaxVjp(op.axis), [g, s], sh(s))]
        if name == "Silu":
            return [self._op(OpKind.SiluVjp, [g, ins[0]], sh(ins[0]))]
        if name == "Gelu":
            return [self._op(OpKind.GeluVjp, [g, ins[0]], sh(ins[0]))]
        if name == "Broadcast":
            ish = sh(ins[0])
            gi = g
            for _ in range(len(sh(g)) - len(ish)):
                gi = self._sum_axis(gi, 0)
            for i, d in enumerate(ish):
                if d == 1 and sh(gi)[i] != 1:
                    gi = self._sum_axis(gi, i)
                    dims = list(sh(gi))
                    dims.insert(i, 1)
                    gi = self._reshape(gi, dims)
            return [gi]
        if name == "Sqrt":
            eps = self.add_constant([np.finfo(np.float32).eps], TensorMeta((), m.dtype))
            two = self.add_constant([2.0], TensorMeta((), m.dtype))
            safe = self._op(OpKind.Add, [nid, self._broadcast_to(eps, m.shape)], m.shape)
            den = self._op(OpKind.Mul, [safe, self._broadcast_to(two, m.shape)], m.shape)
            return [self._op(OpKind.Div, [g, den], m.shape)]
        raise abi.InvalidArgument(f"VJP not implemented for OpKind::{name}")

    def grad(self, loss: int, wrt: Sequence[int]) -> List[int]:
        m = self.nodes[loss][2]
        if m.numel() != 1:
            raise abi.InvalidArgument(f"grad requires scalar loss, got {m.numel()} elements")
        self.eval_many([loss])
        seed = self.add_constant(np.ones(1, np.float32), m)
        grads = {loss: seed}
        for nid in reversed(self.topo_sort([loss])):
            g = grads.pop(nid, None)
            if g is None:
                continue
            op, ins, _ = self.nodes[nid]
            if op.name in ("Constant", "Parameter"):
                grads[nid] = g
                continue
            for i, ig in zip(ins, self._vjp(nid, g)):
                grads[i] = self._op(OpKind.Add, [grads[i], ig], self._shape(ig)) if i in grads else ig
        out = []
        for w in wrt:
            if w not in grads:
                raise abi.InvalidArgument("gradient not found — input may not affect the loss")
            out.append(grads[w])
        return out
