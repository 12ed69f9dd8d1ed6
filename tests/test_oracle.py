"""Pins the CPU oracle (oracle/mlx_cpu_ref.c) before it is trusted.

Each check comes from outside the oracle's own formula: the reference's
known-answer tests (cited file:line), exact integer arithmetic, float64 numpy
re-derivations with rounding bounds, invariants, finite differences, or the
committed golden vectors in tests/golden/.
"""
import math

import numpy as np
import pytest

from oracle.cpu_ref import CpuRefBackend, gen_data, gen_positive_data
from oxidizedmlx_amd import abi
from oxidizedmlx_amd.opkind import NodeInput, OpKind, meta

pytestmark = pytest.mark.usefixtures("oracle_lib")

B = CpuRefBackend()
F32_EPS = float(np.finfo(np.float32).eps)


def ev(op, *ins, out_shape=None):
    inputs = [NodeInput(np.asarray(d, np.float32).reshape(-1), tuple(s)) for d, s in ins]
    shp = out_shape if out_shape is not None else ins[0][1]
    return B.eval_node(op, inputs, meta(shp))


# ── gen_data (crates/mlx-parity/src/lib.rs:22-39, tests :90-118) ───────────

def _gen_data_py(n, seed):
    state, out = seed, []
    for _ in range(n):
        state = (state * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        out.append(np.float32((state >> 33) / float(1 << 31) * 2.0 - 1.0))
    return np.array(out, np.float32)


def test_gen_data_matches_integer_lcg():
    for seed in (0, 1, 42, 70 + 128, 2**63 + 5):
        np.testing.assert_array_equal(gen_data(257, seed), _gen_data_py(257, seed))


def test_gen_data_deterministic_range_and_seed():
    a, b = gen_data(100, 42), gen_data(100, 42)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(gen_data(100, 42), gen_data(100, 43))
    d = gen_data(10000, 1)
    assert np.all((d >= -1.0) & (d <= 1.0))
    assert np.all(gen_positive_data(1000, 1) > 0.0)


# ── MatMul (cpu_kernels.rs:197-230) ─────────────────────────────────────────

def test_matmul_known_answer():
    # cpu_kernels.rs:995-1008, tensor.rs:905-910
    r = ev(OpKind.MatMul, ([1, 2, 3, 4], (2, 2)), ([5, 6, 7, 8], (2, 2)))
    np.testing.assert_array_equal(r, [19.0, 22.0, 43.0, 50.0])


def test_matmul_4x4_c00():
    # crates/mlx-conformance/tests/parity_gate.rs:71-83: C[0,0] = 9.0
    a = np.arange(1, 17, dtype=np.float32)
    b = (np.arange(1, 17, dtype=np.float32)) * np.float32(0.1)
    r = ev(OpKind.MatMul, (a, (4, 4)), (b, (4, 4)))
    assert abs(r[0] - 9.0) <= 1e-4 + 1e-4 * 9.0


def test_matmul_exact_on_integers():
    # Small integers: every partial sum is exact in f32, so any summation order
    # gives the float64 answer bit for bit.
    rng = np.random.default_rng(7)
    for m, k, n in [(17, 31, 23), (1, 64, 128), (5, 1, 3)]:
        a = rng.integers(-8, 9, size=(m, k)).astype(np.float32)
        b = rng.integers(-8, 9, size=(k, n)).astype(np.float32)
        r = ev(OpKind.MatMul, (a, (m, k)), (b, (k, n)), out_shape=(m, n))
        np.testing.assert_array_equal(r.reshape(m, n), (a.astype(np.float64) @ b).astype(np.float32))


def test_matmul_random_within_sequential_bound():
    # |fl(sum) - sum| <= k*eps*sum|a||b| for sequential f32 accumulation.
    rng = np.random.default_rng(8)
    m, k, n = 33, 257, 19
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    r = ev(OpKind.MatMul, (a, (m, k)), (b, (k, n)), out_shape=(m, n)).reshape(m, n)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    bound = k * F32_EPS * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(r - exact) <= bound)


def test_matmul_sequential_order_detectable():
    # The oracle sums left to right from 0.0: 1e8 + 1 - 1e8 ... ordering shows.
    a = np.array([[1e8, 1.0, -1e8, 1.0]], np.float32)
    b = np.ones((4, 1), np.float32)
    r = ev(OpKind.MatMul, (a, (1, 4)), (b, (4, 1)), out_shape=(1, 1))
    # ((((0+1e8)+1)-1e8)+1) in f32 = 1.0 (the first +1 is absorbed)
    assert r[0] == 1.0


def test_matmul_errors():
    with pytest.raises(abi.InvalidArgument):
        ev(OpKind.MatMul, ([1, 2, 3], (3,)), ([1, 2, 3], (3,)))
    with pytest.raises(abi.ShapeMismatch):
        ev(OpKind.MatMul, (np.ones(6), (2, 3)), (np.ones(8), (4, 2)), out_shape=(2, 2))


# ── Elementwise (cpu_kernels.rs:24-35,85-88) ────────────────────────────────

def test_elementwise_known_answers():
    np.testing.assert_array_equal(ev(OpKind.Add, ([1, 2, 3], (3,)), ([4, 5, 6], (3,))), [5, 7, 9])
    np.testing.assert_array_equal(ev(OpKind.Neg, ([1, -2, 3], (3,))), [-1, 2, -3])
    a = gen_data(1024, 1)
    b = gen_positive_data(1024, 3)
    np.testing.assert_array_equal(ev(OpKind.Sub, (a, (1024,)), (b, (1024,))), a - b)
    np.testing.assert_array_equal(ev(OpKind.Mul, (a, (1024,)), (b, (1024,))), a * b)
    np.testing.assert_array_equal(ev(OpKind.Div, (a, (1024,)), (b, (1024,))), a / b)
    with pytest.raises(abi.ShapeMismatch):
        ev(OpKind.Add, ([1, 2, 3], (3,)), ([1, 2], (2,)))


def test_unary_libm_within_ulps():
    x = gen_data(4096, 9) * np.float32(4.0)
    xp = np.abs(x) + np.float32(0.01)
    for op, f, data in [(OpKind.Exp, np.exp, x), (OpKind.Log, np.log, xp),
                        (OpKind.Sqrt, np.sqrt, xp)]:
        r = ev(op, (data, (4096,))).astype(np.float64)
        ref = f(data.astype(np.float64))
        assert np.all(np.abs(r - ref) <= 2 * F32_EPS * np.abs(ref) + 1e-30), op


def test_silu_known_and_f64():
    # cpu_kernels.rs:1081-1091
    r = ev(OpKind.Silu, ([0.0, 1.0, -1.0], (3,)))
    assert r[0] == 0.0 and abs(r[1] - 0.7311) < 1e-3 and abs(r[2] + 0.2689) < 1e-3
    x = gen_data(4096, 10).astype(np.float64) * 6
    r = ev(OpKind.Silu, (x, (4096,))).astype(np.float64)
    ref = x / (1 + np.exp(-x.astype(np.float32).astype(np.float64)))
    assert np.all(np.abs(r - ref) <= 4 * F32_EPS * np.abs(ref) + 1e-7)


def test_gelu_f64():
    x = (gen_data(4096, 11) * 5).astype(np.float32).astype(np.float64)
    r = ev(OpKind.Gelu, (x, (4096,))).astype(np.float64)
    ref = 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    assert np.all(np.abs(r - ref) <= 8 * F32_EPS * np.abs(x) + 1e-7)
    # gelu(0) = 0, odd-symmetric part: gelu(x) - gelu(-x) = x
    r0 = ev(OpKind.Gelu, ([0.0, 2.0, -2.0], (3,)))
    assert r0[0] == 0.0 and abs((r0[1] - r0[2]) - 2.0) < 1e-6


# ── Softmax (cpu_kernels.rs:276-315) ────────────────────────────────────────

def test_softmax_closed_form():
    # crates/mlx-conformance/tests/parity_gate.rs:107-132
    r = ev(OpKind.Softmax(1), ([1, 2, 3, 1, 1, 1], (2, 3)))
    e = np.exp(np.array([1, 2, 3], np.float32))
    exp = [e[0] / e.sum(), e[1] / e.sum(), e[2] / e.sum(), 1 / 3, 1 / 3, 1 / 3]
    np.testing.assert_allclose(r, exp, atol=1e-5, rtol=1e-5)
    assert abs(r[:3].sum() - 1) < 1e-5 and abs(r[3:].sum() - 1) < 1e-5
    r = ev(OpKind.Softmax(0), ([1, 2, 3], (3,)))
    assert abs(r.sum() - 1) < 1e-6 and r[0] < r[1] < r[2]  # cpu_kernels.rs:1010-1025


def test_softmax_f64_and_axes():
    x = gen_data(3 * 5 * 7, 12).reshape(3, 5, 7) * np.float32(8)
    for axis in (0, 1, 2, -1):
        r = ev(OpKind.Softmax(axis), (x, x.shape)).reshape(x.shape)
        xd = x.astype(np.float64)
        ref = np.exp(xd - xd.max(axis=axis, keepdims=True))
        ref /= ref.sum(axis=axis, keepdims=True)
        np.testing.assert_allclose(r, ref, rtol=2e-6, atol=1e-9)
    with pytest.raises(abi.InvalidArgument):
        ev(OpKind.Softmax(3), (x, x.shape))


# ── LayerNorm / RmsNorm (cpu_kernels.rs:338-363, 647-669) ───────────────────

def test_layer_norm_known_answers():
    r = ev(OpKind.LayerNorm(1e-5), ([1, 2, 3], (1, 3)))  # mlx-nn/src/lib.rs:81-91
    np.testing.assert_allclose(r, [-1.2247, 0, 1.2247], atol=1e-3, rtol=1e-3)
    r = ev(OpKind.LayerNorm(1e-5), ([2, 4, 6, 8], (4,)))  # parity_gate.rs:157-169
    np.testing.assert_allclose(r, (np.array([2, 4, 6, 8]) - 5) / np.sqrt(5), atol=1e-4, rtol=1e-4)
    r = ev(OpKind.LayerNorm(1e-5), ([1, 2, 3, 4, 5, 6], (2, 3)))  # cpu_kernels.rs:1037-1051
    assert abs(r[:3].mean()) < 1e-5
    np.testing.assert_array_equal(ev(OpKind.LayerNorm(1e-5), ([3.5], ())), [3.5])  # rank 0


def test_rms_norm_known_answers():
    r = ev(OpKind.RmsNorm(1e-5), ([1, 2, 3, 4], (4,)))  # parity_gate.rs:144-151
    np.testing.assert_allclose(r, np.array([1, 2, 3, 4]) / np.sqrt(7.5), atol=1e-4, rtol=1e-4)
    r = ev(OpKind.RmsNorm(1e-5), ([1, 2, 3], (1, 3)))  # mlx-nn/src/lib.rs:173-183
    np.testing.assert_allclose(r, np.array([1, 2, 3]) / np.sqrt(14 / 3), atol=1e-4, rtol=1e-4)
    r = ev(OpKind.RmsNorm(1e-5), (np.ones(64), (2, 32)))  # mlx-metal/tests/norm_test.rs:7-29
    np.testing.assert_allclose(r, 1 / np.sqrt(1 + 1e-5), rtol=1e-6)


def test_norms_f64_and_invariants():
    x = gen_data(16 * 300, 13).reshape(16, 300) * np.float32(2)
    xd = x.astype(np.float64)
    r = ev(OpKind.LayerNorm(1e-5), (x, x.shape)).reshape(x.shape)
    mu = xd.mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(1, keepdims=True) + 1e-5)
    np.testing.assert_allclose(r, ref, rtol=1e-5, atol=2e-6)
    assert np.all(np.abs(r.astype(np.float64).mean(1)) < 1e-5)
    r = ev(OpKind.RmsNorm(1e-5), (x, x.shape)).reshape(x.shape)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-5)
    np.testing.assert_allclose(r, ref, rtol=1e-5, atol=1e-7)


# ── Transpose / Broadcast / Reshape / Narrow / Concatenate ─────────────────

def test_transpose_known_and_nd():
    r = ev(OpKind.Transpose(None), ([1, 2, 3, 4, 5, 6], (2, 3)), out_shape=(3, 2))
    np.testing.assert_array_equal(r, [1, 4, 2, 5, 3, 6])  # tensor.rs:957-969
    x = gen_data(2 * 3 * 4 * 5, 14).reshape(2, 3, 4, 5)
    for perm in [(3, 2, 1, 0), (1, 0, 2, 3), (0, 2, 3, 1), (2, 0, 3, 1)]:
        r = ev(OpKind.Transpose(perm), (x, x.shape), out_shape=tuple(x.shape[p] for p in perm))
        np.testing.assert_array_equal(r, np.transpose(x, perm).reshape(-1))
    r = ev(OpKind.Transpose(None), (x, x.shape), out_shape=x.shape[::-1])
    np.testing.assert_array_equal(r, np.transpose(x).reshape(-1))
    with pytest.raises(abi.InvalidArgument):
        ev(OpKind.Transpose((1, 0)), (x, x.shape))


def test_broadcast_numpy_rules():
    x = gen_data(12, 15)
    for ish, osh in [((3, 1), (2, 3, 4)), ((4,), (3, 4)), ((1, 4), (5, 4)), ((3, 4), (3, 4)),
                     ((), (2, 2))]:
        n = int(np.prod(ish)) if ish else 1
        r = ev(OpKind.Broadcast(osh), (x[:n], ish), out_shape=osh)
        np.testing.assert_array_equal(r, np.broadcast_to(x[:n].reshape(ish), osh).reshape(-1))


def test_reshape_narrow_concatenate():
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    np.testing.assert_array_equal(ev(OpKind.Reshape((4, 6)), (x, x.shape), out_shape=(4, 6)),
                                  x.reshape(-1))
    r = ev(OpKind.Narrow(1, 1, 2), (x, x.shape), out_shape=(2, 2, 4))
    np.testing.assert_array_equal(r, x[:, 1:3, :].reshape(-1))
    r = ev(OpKind.Narrow(-1, 0, 3), (x, x.shape), out_shape=(2, 3, 3))
    np.testing.assert_array_equal(r, x[..., :3].reshape(-1))
    with pytest.raises(abi.InvalidArgument):
        ev(OpKind.Narrow(1, 2, 2), (x, x.shape))
    y = np.arange(16, dtype=np.float32).reshape(2, 2, 4) + 100
    r = ev(OpKind.Concatenate(1), (x, x.shape), (y, y.shape), out_shape=(2, 5, 4))
    np.testing.assert_array_equal(r, np.concatenate([x, y], 1).reshape(-1))
    with pytest.raises(abi.ShapeMismatch):
        ev(OpKind.Concatenate(0), (x, x.shape), (y, y.shape))


# ── Reductions (cpu_kernels.rs:130-195) ─────────────────────────────────────

def test_reductions_known_answers():
    d = ([1, 2, 3, 4, 5, 6], (2, 3))
    np.testing.assert_array_equal(ev(OpKind.Sum(0), d, out_shape=(3,)), [5, 7, 9])
    np.testing.assert_array_equal(ev(OpKind.Sum(1), d, out_shape=(2,)), [6, 15])
    np.testing.assert_array_equal(ev(OpKind.Sum(None), ([1, 2, 3], (3,)), out_shape=()), [6])
    np.testing.assert_array_equal(ev(OpKind.Mean(1), d, out_shape=(2,)), [2, 5])
    np.testing.assert_array_equal(ev(OpKind.Max(0), d, out_shape=(3,)), [4, 5, 6])
    np.testing.assert_array_equal(ev(OpKind.Max(None), d, out_shape=()), [6])
    with pytest.raises(abi.InvalidArgument):
        ev(OpKind.Sum(2), d)


# ── VJPs (cpu_kernels.rs:403-606): finite differences of the forward oracle ─

def _fd_grad(op_fwd, x, dy, shape, h=1e-2):
    """d/dx sum(dy * f(x)) by central differences in float64 of f32 forwards."""
    g = np.zeros(x.size)
    for i in range(x.size):
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        fp = ev(op_fwd, (xp, shape)).astype(np.float64)
        fm = ev(op_fwd, (xm, shape)).astype(np.float64)
        g[i] = float(np.dot(dy, (fp - fm))) / (2 * h)
    return g


@pytest.mark.parametrize("fwd,vjp", [
    (OpKind.LayerNorm(1e-5), OpKind.LayerNormVjp(1e-5)),
    (OpKind.RmsNorm(1e-5), OpKind.RmsNormVjp(1e-5)),
    (OpKind.Silu, OpKind.SiluVjp),
    (OpKind.Gelu, OpKind.GeluVjp),
])
def test_vjp_finite_differences(fwd, vjp):
    shape = (3, 8)
    x = gen_data(24, 21).astype(np.float64) * 2
    dy = gen_data(24, 22).astype(np.float64)
    g = ev(vjp, (dy, shape), (x, shape)).astype(np.float64)
    np.testing.assert_allclose(g, _fd_grad(fwd, x, dy, shape), atol=1e-2, rtol=1e-2)


def test_softmax_vjp_finite_differences():
    shape = (3, 8)
    x = gen_data(24, 23).astype(np.float64) * 2
    dy = gen_data(24, 24).astype(np.float64)
    s = ev(OpKind.Softmax(-1), (x, shape))
    g = ev(OpKind.SoftmaxVjp(-1), (dy, shape), (s, shape)).astype(np.float64)
    np.testing.assert_allclose(g, _fd_grad(OpKind.Softmax(-1), x, dy, shape), atol=1e-2, rtol=1e-2)


def test_layer_norm_vjp_rows_sum_to_zero():
    # crates/mlx-autograd/src/vjp.rs:236-261
    x = gen_data(4 * 64, 25) * 3
    dy = gen_data(4 * 64, 26)
    g = ev(OpKind.LayerNormVjp(1e-5), (dy, (4, 64)), (x, (4, 64))).reshape(4, 64)
    assert np.all(np.abs(g.astype(np.float64).sum(1)) < 1e-4)
    with pytest.raises(abi.ShapeMismatch):
        ev(OpKind.LayerNormVjp(1e-5), (dy, (4, 64)), (x, (64, 4)))


# ── Attention / ScaledMaskedSoftmax / Rope / Embedding ─────────────────────

def test_scaled_masked_softmax_and_attention_f64():
    tq, tk, dh = 4, 8, 16
    s = gen_data(tq * tk, 50).reshape(tq, tk)
    scale = 1 / math.sqrt(tk)
    r = ev(OpKind.ScaledMaskedSoftmax(scale, True), (s, (tq, tk))).reshape(tq, tk)
    z = s.astype(np.float64) * np.float32(scale)
    z[np.triu_indices(tq, 1, tk)] = -1e9
    ref = np.exp(z - z.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    np.testing.assert_allclose(r, ref, rtol=1e-5, atol=1e-9)
    q, k, v = (gen_data(tq * dh, 51 + i).reshape(tq, dh) for i in range(3))
    k = gen_data(tq * dh, 52).reshape(tq, dh)
    sc = 1 / math.sqrt(dh)
    y = ev(OpKind.Attention(sc, True), (q, (tq, dh)), (k, (tq, dh)), (v, (tq, dh)))
    sd = (q.astype(np.float64) @ k.T.astype(np.float64)) * sc
    sd[np.triu_indices(tq, 1)] = -1e9
    p = np.exp(sd - sd.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(y.reshape(tq, dh), p @ v.astype(np.float64), rtol=1e-4, atol=1e-5)
    with pytest.raises(abi.InvalidArgument):
        ev(OpKind.Attention(sc, True), (q, (tq, dh)), (k, (tq, dh)))


def test_rope_known_answer():
    # cpu_kernels.rs:1093-1127
    r = ev(OpKind.Rope(4, 100, 10000.0), ([1, 0, 0, 1], (1, 4)))
    np.testing.assert_allclose(r, [math.cos(100), math.sin(100), -math.sin(1), math.cos(1)],
                               atol=1e-5)
    r = ev(OpKind.RoPE(10000.0, 0, True), (np.ones(8), (2, 4)))
    assert r.size == 8 and r[0] == 1.0  # position 0 is the identity


@pytest.mark.parametrize("traditional", [True, False])
@pytest.mark.parametrize("hd,rows,offset,base", [(8, 4, 0, 10000.0), (16, 6, 5, 10000.0),
                                                 (4, 3, 17, 500.0), (2, 2, 1, 10.0)])
def test_rope_mlx_closed_form(traditional, hd, rows, offset, base):
    # OpKind::RoPE (cpu_kernels.rs:896-956) on one-hot inputs: each pair
    # rotates by theta = (offset + row) * base^(-2d/hd), the pair being
    # (2d, 2d+1) when traditional, else (d, d + hd/2). A swapped pairing, a
    # wrong exponent or a sign error fails (tests/test_checkers.py plants each).
    from parity import rope_closed_form_check

    def fn(x, shape):
        return ev(OpKind.RoPE(base, offset, traditional), (x, shape))

    rope_closed_form_check(fn, hd, rows, offset, base, traditional, f"oracle RoPE trad={traditional}")


@pytest.mark.parametrize("rd,hd,off,theta", [(4, 4, 0, 10000.0), (4, 8, 3, 10000.0), (6, 6, 11, 100.0)])
def test_rope_closed_form(rd, hd, off, theta):
    # OpKind::Rope (cpu_rope, cpu_kernels.rs:608-645): token t, pair i < rd/2
    # at (2i, 2i+1) rotates by (off + t) * theta^(-2i/rd); dims >= rd pass
    # through unchanged.
    tokens = 4
    for col in range(hd):
        x = np.zeros((tokens, hd), np.float32)
        x[:, col] = 1.0
        y = ev(OpKind.Rope(rd, off, theta), (x, (tokens, hd))).reshape(tokens, hd).astype(np.float64)
        for t in range(tokens):
            want = np.zeros(hd)
            if col >= rd:
                want[col] = 1.0
            else:
                i = col // 2
                a = (off + t) * theta ** (-2.0 * i / rd)
                if col % 2 == 0:
                    want[col], want[col + 1] = math.cos(a), math.sin(a)
                else:
                    want[col - 1], want[col] = -math.sin(a), math.cos(a)
            tol = 1e-6 + 16 * F32_EPS * max(1.0, (off + t))
            assert np.abs(y[t] - want).max() <= tol, (col, t, y[t], want)


def test_embedding_clamps():
    w = np.arange(12, dtype=np.float32).reshape(4, 3)
    idx = np.array([0, 3, 7, -2, 1.9], np.float32)
    r = ev(OpKind.Embedding, (w, (4, 3)), (idx, (5,)), out_shape=(5, 3))
    np.testing.assert_array_equal(r.reshape(5, 3), w[[0, 3, 3, 0, 1]])


def test_constant_rejected():
    with pytest.raises(abi.InvalidArgument):
        ev(OpKind.Constant, ([1.0], (1,)))
