"""Backend parity gate on the GPU: the reference's gate and per-op parity
suites (crates/mlx-parity/tests/{gate,elementwise,activations,matmul,
normalization,transpose,rope,attention}.rs) with the same shapes, seeds and
tolerances, mlx-hip stream vs the CPU oracle stream."""
import math

import numpy as np
import pytest

from oxidizedmlx_amd.opkind import OpKind, meta
from parity import binary_op, cpu_stream, gen_data, gen_positive_data, hip_stream, run_parity, unary_op

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip", "oracle_lib")]


# ── gate.rs:16-228 ──────────────────────────────────────────────────────────

@pytest.mark.parametrize("name,op", [("Add", OpKind.Add), ("Sub", OpKind.Sub), ("Mul", OpKind.Mul)])
def test_gate_binary(name, op):
    a, b = gen_data(1024, 1), gen_data(1024, 2)
    run_parity(lambda s: binary_op(s, op, a, b, meta([1024])), 1e-6, 1e-6, name)


def test_gate_div():
    a, b = gen_data(1024, 1), gen_positive_data(1024, 3)
    run_parity(lambda s: binary_op(s, OpKind.Div, a, b, meta([1024])), 1e-6, 1e-6, "Div")


def test_gate_unary():
    a = gen_data(1024, 1)
    run_parity(lambda s: unary_op(s, OpKind.Neg, a, meta([1024])), 1e-6, 1e-6, "Neg")
    e = gen_data(1024, 4) * np.float32(0.5)
    run_parity(lambda s: unary_op(s, OpKind.Exp, e, meta([1024])), 1e-6, 1e-6, "Exp")
    p = gen_positive_data(1024, 5)
    run_parity(lambda s: unary_op(s, OpKind.Log, p, meta([1024])), 1e-6, 1e-6, "Log")
    # Sqrt (cpu_kernels.rs:85-88, f32::sqrt): correctly rounded on both sides,
    # held to the elementwise tolerance of crates/mlx-parity/tests/elementwise.rs:8-9.
    r = gen_positive_data(1024, 6)
    run_parity(lambda s: unary_op(s, OpKind.Sqrt, r, meta([1024])), 1e-6, 1e-6, "Sqrt")


def test_gate_activations_and_softmax():
    a = gen_data(256, 10)
    run_parity(lambda s: unary_op(s, OpKind.Silu, a, meta([256])), 1e-5, 1e-5, "Silu")
    a = gen_data(256, 11)
    run_parity(lambda s: unary_op(s, OpKind.Gelu, a, meta([256])), 1e-5, 1e-5, "Gelu")
    a = gen_data(32 * 128, 12)
    run_parity(lambda s: unary_op(s, OpKind.Softmax(-1), a, meta([32, 128])), 1e-5, 1e-5, "Softmax")


@pytest.mark.parametrize("m,k,n", [(4, 4, 4), (64, 64, 64), (17, 31, 23)])
def test_gate_matmul(m, k, n):
    a, b = gen_data(m * k, 20), gen_data(k * n, 21)

    def g(s):
        na = s.add_constant(a, meta([m, k]))
        nb = s.add_constant(b, meta([k, n]))
        return s.add_op(OpKind.MatMul, [na, nb], meta([m, n]))

    run_parity(g, 1e-4, 1e-4, f"MatMul {m}x{k}x{n}")


def test_gate_norms():
    a = gen_data(32 * 128, 30)
    run_parity(lambda s: unary_op(s, OpKind.LayerNorm(1e-5), a, meta([32, 128])), 1e-3, 1e-3, "LayerNorm")
    a = gen_data(32 * 128, 31)
    run_parity(lambda s: unary_op(s, OpKind.RmsNorm(1e-5), a, meta([32, 128])), 1e-3, 1e-3, "RmsNorm")


def test_gate_rope():
    a = gen_data(4 * 16, 40)
    run_parity(lambda s: unary_op(s, OpKind.Rope(16, 0, 10000.0), a, meta([4, 16])), 5e-4, 5e-3, "Rope")


def test_gate_attention():
    tq, tk = 4, 8
    a = gen_data(tq * tk, 50)
    scale = 1.0 / math.sqrt(tk)
    run_parity(lambda s: unary_op(s, OpKind.ScaledMaskedSoftmax(scale, True), a, meta([tq, tk])),
               1e-3, 1e-3, "ScaledMaskedSoftmax")
    tq, dh = 4, 16
    q, k, v = gen_data(tq * dh, 51), gen_data(tq * dh, 52), gen_data(tq * dh, 53)

    def g(s):
        nq = s.add_constant(q, meta([tq, dh]))
        nk = s.add_constant(k, meta([tq, dh]))
        nv = s.add_constant(v, meta([tq, dh]))
        return s.add_op(OpKind.Attention(1.0 / math.sqrt(dh), True), [nq, nk, nv], meta([tq, dh]))

    run_parity(g, 1e-3, 1e-3, "Attention")


def test_gate_transpose():
    a = gen_data(64 * 128, 60)

    def g(s):
        na = s.add_constant(a, meta([64, 128]))
        return s.add_op(OpKind.Transpose(None), [na], meta([128, 64]))

    run_parity(g, 0.0, 0.0, "Transpose")


# ── per-op parity files ─────────────────────────────────────────────────────

@pytest.mark.parametrize("m,k,n", [(4, 4, 4), (64, 64, 64), (128, 4096, 128), (17, 31, 23)])
def test_parity_matmul(m, k, n):
    # crates/mlx-parity/tests/matmul.rs:12-52 (seeds 70+m, 80+n; 1e-4)
    a, b = gen_data(m * k, 70 + m), gen_data(k * n, 80 + n)

    def g(s):
        na = s.add_constant(a, meta([m, k]))
        nb = s.add_constant(b, meta([k, n]))
        return s.add_op(OpKind.MatMul, [na, nb], meta([m, n]))

    run_parity(g, 1e-4, 1e-4, f"MatMul {m}x{k}x{n}")


@pytest.mark.parametrize("rows,cols,seed_ln,seed_rms", [(4, 8, 90, 93), (32, 128, 91, 94),
                                                        (128, 256, 92, 95)])
def test_parity_normalization(rows, cols, seed_ln, seed_rms):
    # crates/mlx-parity/tests/normalization.rs:14-80 (1e-3)
    a = gen_data(rows * cols, seed_ln)
    run_parity(lambda s: unary_op(s, OpKind.LayerNorm(1e-5), a, meta([rows, cols])), 1e-3, 1e-3, "LN")
    a = gen_data(rows * cols, seed_rms)
    run_parity(lambda s: unary_op(s, OpKind.RmsNorm(1e-5), a, meta([rows, cols])), 1e-3, 1e-3, "RMS")


def test_parity_activations():
    # crates/mlx-parity/tests/activations.rs:91-155 (1e-5)
    for op, n, shp, seed in [(OpKind.Silu, 256, [256], 60), (OpKind.Silu, 2048, [32, 64], 61),
                             (OpKind.Gelu, 256, [256], 62), (OpKind.Gelu, 2048, [32, 64], 63),
                             (OpKind.Softmax(-1), 32, [4, 8], 64),
                             (OpKind.Softmax(-1), 4096, [32, 128], 65)]:
        a = gen_data(n, seed)
        run_parity(lambda s: unary_op(s, op, a, meta(shp)), 1e-5, 1e-5, repr(op))


def test_parity_elementwise():
    # crates/mlx-parity/tests/elementwise.rs:168-231 (1e-6)
    cases = [(OpKind.Add, 1024, 42, 43), (OpKind.Add, 4096, 44, 45), (OpKind.Sub, 1024, 46, 47),
             (OpKind.Mul, 1024, 48, 49)]
    for op, n, sa, sb in cases:
        a, b = gen_data(n, sa), gen_data(n, sb)
        run_parity(lambda s: binary_op(s, op, a, b, meta([n])), 1e-6, 1e-6, repr(op))
    a, b = gen_data(1024, 50), gen_positive_data(1024, 51)
    run_parity(lambda s: binary_op(s, OpKind.Div, a, b, meta([1024])), 1e-6, 1e-6, "Div")
    a = gen_data(1024, 52)
    run_parity(lambda s: unary_op(s, OpKind.Neg, a, meta([1024])), 1e-6, 1e-6, "Neg")
    a = gen_data(1024, 53) * np.float32(0.5)
    run_parity(lambda s: unary_op(s, OpKind.Exp, a, meta([1024])), 1e-6, 1e-6, "Exp")
    a = gen_positive_data(1024, 54)
    run_parity(lambda s: unary_op(s, OpKind.Log, a, meta([1024])), 1e-6, 1e-6, "Log")
    a = gen_positive_data(4096, 55)
    h, c = run_parity(lambda s: unary_op(s, OpKind.Sqrt, a, meta([4096])), 1e-6, 1e-6, "Sqrt")
    np.testing.assert_array_equal(h, c)  # IEEE square root: correctly rounded, so bit for bit
    # Special values: sqrt(+0) = +0, sqrt(-0) = -0, sqrt(+inf) = +inf, negatives and NaN give NaN.
    sp = np.array([0.0, -0.0, np.inf, -1.0, np.nan, 1e-40, 4.0, 2.0], np.float32)
    got = []
    for st in (hip_stream(), cpu_stream()):
        out = unary_op(st, OpKind.Sqrt, sp, meta([8]))
        st.eval(out)
        got.append(st.get_buffer(out))
    h, c = got
    np.testing.assert_array_equal(np.signbit(h[:3]), np.signbit(c[:3]))
    np.testing.assert_array_equal(h, c)


@pytest.mark.parametrize("rows,cols,seed", [(4, 8, 130), (64, 128, 131), (1000, 777, 132)])
def test_parity_transpose_exact(rows, cols, seed):
    # crates/mlx-parity/tests/transpose.rs (exact)
    a = gen_data(rows * cols, seed)

    def g(s):
        na = s.add_constant(a, meta([rows, cols]))
        return s.add_op(OpKind.Transpose(None), [na], meta([cols, rows]))

    h, c = run_parity(g, 0.0, 0.0, "Transpose")
    np.testing.assert_array_equal(h, c)


def test_parity_transpose_nd_exact():
    x = gen_data(2 * 3 * 4 * 5, 133)
    for perm in [(3, 2, 1, 0), (1, 0, 2, 3), (0, 2, 3, 1)]:
        shp = (2, 3, 4, 5)

        def g(s, perm=perm):
            na = s.add_constant(x, meta(shp))
            return s.add_op(OpKind.Transpose(perm), [na], meta([shp[p] for p in perm]))

        run_parity(g, 0.0, 0.0, f"Transpose{perm}")


def test_parity_reductions_bitexact():
    x = gen_data(6 * 7 * 33, 140).reshape(6, 7, 33)
    for op, out in [(OpKind.Sum(0), [7, 33]), (OpKind.Sum(1), [6, 33]), (OpKind.Sum(-1), [6, 7]),
                    (OpKind.Mean(1), [6, 33]), (OpKind.Max(2), [6, 7]), (OpKind.Sum(None), []),
                    (OpKind.Max(None), []), (OpKind.Mean(None), [])]:
        h, c = run_parity(lambda s: s.add_op(op, [s.add_constant(x, meta(x.shape))], meta(out)),
                          0.0, 0.0, repr(op))
        np.testing.assert_array_equal(h, c)


def test_parity_broadcast_narrow_concat_embedding_rope_mlx():
    x = gen_data(12, 150)
    run_parity(lambda s: s.add_op(OpKind.Broadcast((5, 3, 4)), [s.add_constant(x, meta([3, 4]))],
                                  meta([5, 3, 4])), 0.0, 0.0, "Broadcast")
    y = gen_data(2 * 6 * 4, 151)
    run_parity(lambda s: s.add_op(OpKind.Narrow(1, 2, 3), [s.add_constant(y, meta([2, 6, 4]))],
                                  meta([2, 3, 4])), 0.0, 0.0, "Narrow")
    z = gen_data(2 * 2 * 4, 152)
    run_parity(lambda s: s.add_op(OpKind.Concatenate(1), [s.add_constant(y, meta([2, 6, 4])),
                                                         s.add_constant(z, meta([2, 2, 4]))],
                                  meta([2, 8, 4])), 0.0, 0.0, "Concatenate")
    w = gen_data(10 * 8, 153)
    idx = np.array([0, 9, 3, 12, -1, 2.7], np.float32)
    run_parity(lambda s: s.add_op(OpKind.Embedding, [s.add_constant(w, meta([10, 8])),
                                                     s.add_constant(idx, meta([6]))],
                                  meta([6, 8])), 0.0, 0.0, "Embedding")
    r = gen_data(6 * 16, 154)
    for trad in (True, False):
        run_parity(lambda s: unary_op(s, OpKind.RoPE(10000.0, 3, trad), r, meta([6, 16])),
                   5e-4, 5e-3, f"RoPE traditional={trad}")


def test_reductions_over_all_large_input():
    # More than 65536 values take the tree reduction (1024 blocks of 256
    # threads, then one folding block): depth <= ceil(log2 n) + 4 roundings
    # per value, so |sum - exact| <= gamma_depth * sum|x| (tree_sum_bound:
    # 0.21 here, against a true sum of -138.7). Against the oracle's
    # sequential fold the bound grows by that fold's own error. The kernel's
    # order is also restated in numpy float32 (tree_sum_f32), which must give
    # the same bits. tests/test_checkers.py shows that dropping block 0's
    # partial (|partial| = 8.2) or nearly any other block's fails the bound.
    from parity import tree_sum_bound, tree_sum_f32
    n = 300_001
    for name, x in (("signed", gen_data(n, 160)),
                    ("positive", (np.float32(0.5) + np.float32(0.5) * np.abs(gen_data(n, 161))).astype(np.float32))):
        x64 = x.astype(np.float64)
        exact = float(x64.sum())
        bound = tree_sum_bound(x)
        if name == "positive":
            assert float(x.min()) > bound  # any one value left out would fail
        for op, scale in ((OpKind.Sum(None), 1.0), (OpKind.Mean(None), 1.0 / n)):
            hip = hip_stream()
            hid = hip.add_op(op, [hip.add_constant(x, meta([n]))], meta([]))
            hip.eval(hid)
            h = float(hip.get_buffer(hid)[0])
            cpu = cpu_stream()
            cid = cpu.add_op(op, [cpu.add_constant(x, meta([n]))], meta([]))
            cpu.eval(cid)
            c = float(cpu.get_buffer(cid)[0])
            # Mean divides once more in f32: one more rounding of the result.
            tol = (bound + 2.0 ** -23 * (abs(exact) + bound)) * scale if scale != 1.0 else bound
            print(f"  {name} {op!r}: hip={h!r} cpu={c!r} exact={exact * scale!r} bound={tol:.3e}", flush=True)
            assert abs(h - exact * scale) <= tol, (name, op, h, exact * scale, tol)
            assert abs(h - c) <= tol + abs(c - exact * scale), (name, op, h, c)
            if scale == 1.0:
                assert np.float32(h) == tree_sum_f32(x), (name, h, float(tree_sum_f32(x)))
    h, c = run_parity(lambda s: s.add_op(OpKind.Max(None), [s.add_constant(x, meta([n]))], meta([])),
                      0.0, 0.0, "Max(None)")
    assert float(h[0]) == float(x.max())
    # A sum of negative zeros is -0.0 on both paths (sign bit checked).
    z = np.full(n, -0.0, np.float32)
    h, c = run_parity(lambda s: s.add_op(OpKind.Sum(None), [s.add_constant(z, meta([n]))], meta([])),
                      0.0, 0.0, "Sum(-0.0)")
    assert np.signbit(h[0]) and np.signbit(c[0])
