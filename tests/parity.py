"""Backend parity harness, restating crates/mlx-parity/src/lib.rs:8-84 and
assert_allclose (crates/mlx-conformance/src/lib.rs:32-48).

``run_parity(build_graph, atol, rtol)`` builds the same graph on a fresh CPU
oracle stream and a fresh mlx-hip stream, evaluates both and asserts
|hip - cpu| <= atol + rtol*|cpu| element-wise, reporting max-abs / max-rel.
"""
from __future__ import annotations

import numpy as np

from oracle.cpu_ref import CpuRefBackend, gen_data, gen_positive_data  # noqa: F401
from oxidizedmlx_amd.opkind import NodeInput, Op, OpKind, TensorMeta, meta  # noqa: F401


class CpuStream:
    """Stream (crates/mlx-core/src/backend.rs:41-185) bound to the CPU oracle:
    memoised topological evaluation, constants pre-materialised, one backend
    call per node. Graph-level CSE is irrelevant to results and omitted."""

    def __init__(self):
        self.backend = CpuRefBackend()
        self.nodes = {}
        self.buffers = {}
        self.next_id = 1
        self.eval_calls = 0

    def add_constant(self, data, m: TensorMeta) -> int:
        nid = self.next_id
        self.next_id += 1
        self.nodes[nid] = (OpKind.Constant, (), m)
        self.buffers[nid] = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        return nid

    def add_op(self, op: Op, inputs, m: TensorMeta) -> int:
        nid = self.next_id
        self.next_id += 1
        self.nodes[nid] = (op, tuple(inputs), m)
        return nid

    def eval(self, out: int) -> None:
        order, seen = [], set()

        def visit(n):
            if n in seen:
                return
            seen.add(n)
            for i in self.nodes[n][1]:
                visit(i)
            order.append(n)

        visit(out)
        for n in order:
            if n in self.buffers:
                continue
            op, ins, m = self.nodes[n]
            inputs = [NodeInput(self.buffers[i], self.nodes[i][2].shape, self.nodes[i][2].dtype)
                      for i in ins]
            self.eval_calls += 1
            self.buffers[n] = self.backend.eval_node(op, inputs, m)

    def get_buffer(self, n: int) -> np.ndarray:
        return self.buffers[n].copy()


def cpu_stream() -> CpuStream:
    return CpuStream()


def hip_stream():
    from oxidizedmlx_amd.backend import HipStream
    return HipStream()


def binary_op(s, op: Op, a, b, m: TensorMeta) -> int:
    na = s.add_constant(a, m)
    nb = s.add_constant(b, m)
    return s.add_op(op, [na, nb], m)


def unary_op(s, op: Op, a, m: TensorMeta) -> int:
    na = s.add_constant(a, m)
    return s.add_op(op, [na], m)


def errors(actual, expected):
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    e = np.asarray(expected, dtype=np.float64).reshape(-1)
    if a.size == 0:
        return 0.0, 0.0
    d = np.abs(a - e)
    max_abs = float(d.max())
    with np.errstate(divide="ignore", invalid="ignore"):
        rel = np.where(e != 0, d / np.abs(e), np.where(d == 0, 0.0, np.inf))
    return max_abs, float(rel.max())


def assert_allclose(actual, expected, atol: float, rtol: float, what: str = "") -> None:
    a = np.asarray(actual, dtype=np.float32).reshape(-1)
    e = np.asarray(expected, dtype=np.float32).reshape(-1)
    assert a.size == e.size, f"length mismatch: hip={a.size} cpu={e.size}"
    diff = np.abs(a.astype(np.float64) - e.astype(np.float64))
    tol = atol + rtol * np.abs(e.astype(np.float64))
    bad = ~(diff <= tol)
    max_abs, max_rel = errors(a, e)
    if bad.any():
        i = int(np.argmax(bad))
        raise AssertionError(
            f"{what} mismatch at [{i}]: hip={a[i]} cpu={e[i]} diff={diff[i]} tol={tol[i]} "
            f"({int(bad.sum())} of {a.size} bad; max_abs={max_abs:.3e} max_rel={max_rel:.3e})")
    print(f"  {what} n={a.size} max_abs={max_abs:.3e} max_rel={max_rel:.3e} "
          f"(atol={atol:g} rtol={rtol:g})", flush=True)


def run_parity(build_graph, atol: float, rtol: float, what: str = ""):
    cpu = cpu_stream()
    hip = hip_stream()
    c_out = build_graph(cpu)
    h_out = build_graph(hip)
    cpu.eval(c_out)
    hip.eval(h_out)
    c = cpu.get_buffer(c_out)
    h = hip.get_buffer(h_out)
    assert_allclose(h, c, atol, rtol, what)
    return h, c
