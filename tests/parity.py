"""Backend parity harness, restating crates/mlx-parity/src/lib.rs:8-84 and
assert_allclose (crates/mlx-conformance/src/lib.rs:32-48).

``run_parity(build_graph, atol, rtol)`` builds the same graph on a fresh CPU
oracle stream and a fresh mlx-hip stream, evaluates both and asserts
|hip - cpu| <= atol + rtol*|cpu| element-wise, reporting max-abs / max-rel.
"""
from __future__ import annotations

import math

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


# ── Rigorous bounds shared by the GPU parity tests and their CPU self-checks ──

U32 = 2.0 ** -24     # unit roundoff of f32 (round to nearest)
U_OUT = {"f32": 0.0, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}  # unit roundoff of the C type (8 / 11 significant bits)


def gamma(k: int) -> float:
    """gamma_k = k*u / (1 - k*u): the bound on the relative error of any
    f32 sum of k+1 products accumulated in any order (Higham, Accuracy and
    Stability of Numerical Algorithms, 2nd ed., eq. 3.4)."""
    return k * U32 / (1.0 - k * U32)


def gemm_full_check(c, a, b, out: str = "f32", what: str = "") -> tuple[float, float]:
    """Every element of C (one product, [M, N]) against float64 A @ B on the
    same (already rounded) inputs a [M, K], b [K, N]:

        |C - AB| <= gamma_K (|A| |B|) + u_out (|AB| + gamma_K (|A| |B|))

    holds for an f32 accumulation in any order followed by one rounding of
    the output to `out`; a dropped k-term, a wrong or shifted tile, or a
    transposed operand gives errors of the order of |AB| itself and fails.
    Returns (max_abs, max error / bound)."""
    a64 = np.asarray(a, np.float64)
    b64 = np.asarray(b, np.float64)
    k = a64.shape[1]
    exact = a64 @ b64
    mag = np.abs(a64) @ np.abs(b64)
    g = gamma(k)
    bound = g * mag + U_OUT[out] * (np.abs(exact) + g * mag)
    # A zero bound (an all-zero row or column of A or B) allows only an exact zero.
    err = np.abs(np.asarray(c, np.float64) - exact)
    bad = ~(err <= bound)
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(bound > 0, err / bound, np.where(err == 0, 0.0, np.inf))
    if bad.any():
        i, j = np.unravel_index(int(np.argmax(bad)), bad.shape)
        raise AssertionError(
            f"{what}: C[{i},{j}]={float(c[i, j])!r} exact={exact[i, j]!r} err={err[i, j]:.3e} "
            f"bound={bound[i, j]:.3e} ({int(bad.sum())} of {bad.size} outside the bound)")
    print(f"  {what} full {c.shape}: max_abs={float(err.max()):.3e} "
          f"max err/bound={float(ratio.max()):.3f}", flush=True)
    return float(err.max()), float(ratio.max())


def tree_sum_bound(x, extra_depth: int = 4) -> float:
    """Bound on |s - sum(x)| for an f32 sum s of x formed by any summation
    tree of depth <= ceil(log2 n) + extra_depth (each value passes through at
    most that many roundings): gamma_depth * sum|x|."""
    n = int(np.asarray(x).size)
    depth = max(1, math.ceil(math.log2(max(n, 2)))) + extra_depth
    return gamma(depth) * float(np.abs(np.asarray(x, np.float64)).sum())


def rope_closed_form_check(fn, head_dim: int, rows: int, offset: int, base: float,
                           traditional: bool, what: str = "") -> float:
    """OpKind::RoPE (cpu_kernels.rs:896-956) on one-hot inputs: for row i at
    position p = offset + i and pair d, theta = p * base^(-2d/head_dim), with
    the pair (2d, 2d+1) when `traditional`, else (d, d + head_dim/2). A one
    at the pair's first index must come out as (cos theta, sin theta) on the
    pair, a one at its second index as (-sin theta, cos theta), and zero at
    every other index. `fn(x, shape)` evaluates RoPE on a [rows, head_dim]
    float32 array. Tolerance: the f32 angle carries a few ulp of |theta|.
    Returns the largest error seen."""
    half = head_dim // 2
    worst = 0.0
    for d in range(half):
        i0, i1 = (2 * d, 2 * d + 1) if traditional else (d, d + half)
        for which, role in ((i0, "first"), (i1, "second")):
            x = np.zeros((rows, head_dim), np.float32)
            x[:, which] = 1.0
            y = np.asarray(fn(x, (rows, head_dim)), np.float64).reshape(rows, head_dim)
            for i in range(rows):
                th = (offset + i) * base ** (-(2.0 * d) / head_dim)
                want = np.zeros(head_dim)
                if role == "first":
                    want[i0], want[i1] = math.cos(th), math.sin(th)
                else:
                    want[i0], want[i1] = -math.sin(th), math.cos(th)
                tol = 1e-6 + 16 * float(np.finfo(np.float32).eps) * max(1.0, abs(th))
                err = float(np.abs(y[i] - want).max())
                worst = max(worst, err)
                if err > tol:
                    raise AssertionError(
                        f"{what}: RoPE one-hot at {which} (pair {d}, {role}), row {i}: got "
                        f"{y[i].tolist()} want {want.tolist()} (err {err:.3e} > {tol:.3e})")
    return worst


def tree_sum_f32(x, blocks: int = 1024, threads: int = 256) -> np.float32:
    """The f32 summation order of the library's whole-tensor Sum above 65536
    values (reduce_partial_kernel / reduce_final_kernel): thread t of block b
    folds x[b*threads + t + j*blocks*threads], j = 0, 1, ..., from -0.0; each
    block halves its threads' values pairwise (t += t + o for o = threads/2
    .. 1); one block then folds partial t, t + threads, ... and halves the
    same way. numpy float32 additions round as the GPU's do, so this gives
    the kernel's bits. A planted reorder or dropped term is a different sum."""
    x = np.asarray(x, np.float32).reshape(-1)
    n = x.size
    stride = blocks * threads
    acc = np.full(stride, -0.0, np.float32)
    for j in range(0, n, stride):
        chunk = x[j:j + stride]
        acc[:chunk.size] = acc[:chunk.size] + chunk

    def halve(v):
        v = v.copy()
        o = v.size // 2
        while o > 0:
            v[:o] = v[:o] + v[o:2 * o]
            o //= 2
        return v[0]

    part = np.array([halve(acc[b * threads:(b + 1) * threads]) for b in range(blocks)], np.float32)
    fin = np.full(threads, -0.0, np.float32)
    for j in range(0, blocks, threads):
        fin = fin + part[j:j + threads]
    return np.float32(halve(fin))


# ── Elementwise chains: float64 value and f32 error bound ────────────────────

F32_MAX = float(np.finfo(np.float32).max)
TINY = 2.0 ** -126  # smallest normal f32: a subnormal result may also come out flushed to zero


def chain_bound(ins, prog, unary, binary):
    """Float64 value v of the chain on the f32 inputs, with a bound E on how
    far an f32 evaluation whose every operation errs by at most a few units
    of roundoff (one for + - * / and sqrt, 8 for exp, log, SiLU and GELU) can
    land from v, and a mask of `uncertain` elements where no bound holds:
    the interval a Log, Sqrt or Div reads reaches zero or below, a value may
    overflow f32, or the bound is not finite. Each step also allows an
    absolute error of the smallest normal f32 (TINY): a result in the
    subnormal range may come out flushed or off by a subnormal unit. prog
    steps are (code, j, left): code < len(unary) applies unary[code];
    otherwise binary[code - len(unary)] with input j as the right
    (left=True) or left operand. Mistakes this pins: a wrong op or operand
    order, a dropped step, a step applied twice (each moves the value far
    beyond E), or an f32 error above the stated few ulp."""
    v = ins[0].astype(np.float64)
    e = np.zeros_like(v)
    unc = np.zeros(v.shape, bool)
    with np.errstate(all="ignore"):
        for code, j, left in prog:
            if code < len(unary):
                op = unary[code].name
                if op == "Neg":
                    v = -v
                elif op == "Exp":
                    nv = np.exp(v)
                    e = nv * np.expm1(e) + 8 * U32 * np.exp(v + e) + TINY
                    v = nv
                elif op == "Log":
                    unc |= v - e <= 0
                    nv = np.log(v)
                    e = -np.log1p(-e / v) + 8 * U32 * np.abs(nv) + TINY
                    v = nv
                elif op == "Sqrt":
                    unc |= v - e < 0
                    nv = np.sqrt(v)
                    e = e / (np.sqrt(np.maximum(v - e, 0.0)) + nv) + U32 * nv + TINY
                    v = nv
                elif op == "Silu":
                    nv = v / (1.0 + np.exp(-v))
                    e = 1.1 * e + 8 * U32 * np.abs(nv) + TINY
                    v = nv
                else:  # Gelu, tanh form
                    nv = 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))
                    e = 1.13 * e + 16 * U32 * (np.abs(v) + np.abs(nv)) + TINY
                    v = nv
            else:
                o = ins[j].astype(np.float64)
                a, ea, b, eb = (v, e, o, 0.0) if left else (o, 0.0, v, e)
                op = binary[code - len(unary)].name
                if op == "Add":
                    v, e = a + b, ea + eb
                elif op == "Sub":
                    v, e = a - b, ea + eb
                elif op == "Mul":
                    v, e = a * b, np.abs(a) * eb + np.abs(b) * ea + ea * eb
                else:  # Div
                    unc |= np.abs(b) <= eb
                    v = a / b
                    e = (ea + np.abs(v) * eb) / (np.abs(b) - eb)
                e = e + U32 * np.abs(v) + TINY
            unc |= ~np.isfinite(e) | (np.abs(v) + e >= F32_MAX) | np.isinf(v)
    return v, e, unc


def assert_chain_within_bound(hip, cpu, v, e, unc):
    """Both f32 results lie within E of v, so they differ by at most 2E;
    where v is NaN (a certain domain error) both must be NaN."""
    h = hip.astype(np.float64)
    c = cpu.astype(np.float64)
    nan = np.isnan(v) & ~unc
    assert np.all(np.isnan(h[nan]) & np.isnan(c[nan])), "a certain NaN is not NaN on both sides"
    ok = ~unc & ~np.isnan(v)
    assert np.all(np.isfinite(h[ok]) & np.isfinite(c[ok])), "a finite value came out non-finite"
    d = np.abs(h[ok] - c[ok])
    lim = 2 * e[ok]
    bad = ~(d <= lim)
    if bad.any():
        i = int(np.flatnonzero(ok)[np.argmax(bad)])
        raise AssertionError(f"chain mismatch at [{i}]: hip={hip[i]} cpu={cpu[i]} exact={v[i]} bound={2 * e[i]}")
    print(f"  chain checked {int(ok.sum())} of {v.size} (certain NaN {int(nan.sum())}, "
          f"max diff / bound {float((d / np.maximum(lim, 1e-300)).max()) if d.size else 0.0:.3f})", flush=True)
