"""The parity checkers can fail: each is run on a correct CPU result (must
pass) and on copies with one planted mistake (must raise). The mistakes are
planted in CPU-side results only; no GPU is involved.

Checkers covered: the full-output float64 GEMM bound (gemm_full_check), the
tree-sum bound of the whole-tensor Sum/Mean (tree_sum_bound, tree_sum_f32),
the closed-form RoPE pin (rope_closed_form_check) and the error bound of
random elementwise chains (chain_bound, assert_chain_within_bound).
"""
import math

import numpy as np
import pytest

from oracle.cpu_ref import CpuRefBackend, gen_data
from oxidizedmlx_amd import synth
from oxidizedmlx_amd.opkind import NodeInput, OpKind, meta
from parity import (assert_chain_within_bound, chain_bound, cpu_stream, gemm_full_check, rope_closed_form_check,
                    tree_sum_bound, tree_sum_f32)

pytestmark = pytest.mark.usefixtures("oracle_lib")


# ── GEMM: full output against float64 with the accumulation bound ─────────

M, N, K = 256, 192, 512


@pytest.fixture(scope="module")
def ab():
    a = synth.round_bf16(synth.normal(101, (M, K)))
    b = synth.round_bf16(synth.normal(102, (K, N)))
    return a, b


def _f32_product(a, b):
    return (a.astype(np.float32) @ b.astype(np.float32)).astype(np.float32)


def test_gemm_check_accepts_f32_and_bf16_results(ab):
    a, b = ab
    c = _f32_product(a, b)
    gemm_full_check(c, a, b, "f32", "correct f32")
    gemm_full_check(synth.round_bf16(c), a, b, "bf16", "correct bf16")
    gemm_full_check(synth.round_f16(c), a, b, "f16", "correct f16")


def _planted(a, b):
    c = _f32_product(a, b)
    out = {}
    x = c.copy()  # one k-term left out of one 32x32 tile
    x[32:64, 64:96] -= np.outer(a[32:64, 300], b[300, 64:96]).astype(np.float32)
    out["dropped k-term in one tile"] = x
    x = c.copy()  # two 64x64 tiles stored in each other's place
    x[0:64, 64:128], x[64:128, 0:64] = c[64:128, 0:64].copy(), c[0:64, 64:128].copy()
    out["swapped tiles"] = x
    x = c.copy()  # one tile never written
    x[192:256, 128:192] = 0.0
    out["unwritten edge tile"] = x
    x = c.copy()  # one K tile (32 k) of one row panel lost
    x[128:160, :] -= (a[128:160, 32:64].astype(np.float64) @ b[32:64, :]).astype(np.float32)
    out["dropped K tile"] = x
    x = c.copy()  # rows shifted by one inside a tile
    x[0:32, 0:64] = np.roll(c[0:32, 0:64], 1, axis=0)
    out["row shift"] = x
    out["f32 product rounded to bf16"] = synth.round_bf16(c)
    return out


@pytest.mark.parametrize("mistake", ["dropped k-term in one tile", "swapped tiles", "unwritten edge tile",
                                     "dropped K tile", "row shift", "f32 product rounded to bf16"])
def test_gemm_check_rejects_planted_mistakes(ab, mistake):
    a, b = ab
    with pytest.raises(AssertionError):
        gemm_full_check(_planted(a, b)[mistake], a, b, "f32", mistake)


def test_gemm_check_rejects_transposed_operand():
    a = synth.round_bf16(synth.normal(103, (128, 128)))
    b = synth.round_bf16(synth.normal(104, (128, 128)))
    with pytest.raises(AssertionError):
        gemm_full_check(_f32_product(a, b.T.copy()), a, b, "f32", "B transposed")


# ── Whole-tensor Sum/Mean: tree bound ─────────────────────────────────────

def test_tree_sum_in_bound_and_dropped_partial_detected():
    n = 300_001
    x = gen_data(n, 160)
    exact = float(x.astype(np.float64).sum())
    bound = tree_sum_bound(x)
    s = float(tree_sum_f32(x))
    assert abs(s - exact) <= bound
    # A sequential f32 fold (the oracle's order) is not held to this bound:
    # its own error is what the GPU test adds to the bound when it compares
    # with the oracle.
    # The bound is small against one block's share of the sum: dropping the
    # partial of block 0 (threads 0..255 over x[0:256] and x[262144:262400])
    # moves the sum by far more, and so does dropping nearly any block.
    idx = np.arange(n)
    blk = (idx % (1024 * 256)) // 256
    partials = np.bincount(blk, weights=x.astype(np.float64), minlength=1024)
    print(f"bound {bound:.4f}; |partial 0| {abs(partials[0]):.3f}; "
          f"median |partial| {np.median(np.abs(partials)):.3f}")
    assert abs(partials[0]) > bound
    assert (np.abs(partials) > bound).mean() > 0.95
    planted = float(tree_sum_f32(np.where(blk == 0, np.float32(0), x)))
    assert abs(planted - exact) > bound
    # The numpy restatement of the kernel's order is itself a different sum
    # from the sequential fold, so a bit-exact check against it pins the order.
    seq = np.float32(-0.0)
    for v in x[:70000]:
        seq = np.float32(seq + v)
    assert tree_sum_f32(x[:70000]) != seq


def test_tree_sum_positive_input_detects_any_single_dropped_value():
    n = 300_001
    x = (np.float32(0.5) + np.float32(0.5) * np.abs(gen_data(n, 161))).astype(np.float32)
    bound = tree_sum_bound(x)
    assert float(x.min()) > bound  # so leaving out any one value is outside the bound
    exact = float(x.astype(np.float64).sum())
    assert abs(float(tree_sum_f32(x)) - exact) <= bound
    y = x.copy()
    y[123_457] = 0.0
    assert abs(float(tree_sum_f32(y)) - exact) > bound


# ── RoPE: closed form on one-hot inputs ───────────────────────────────────

def _oracle_rope(base, offset, traditional):
    cpu = CpuRefBackend()
    return lambda x, shape: cpu.eval_node(OpKind.RoPE(base, offset, traditional),
                                          [NodeInput(x.reshape(-1), shape)], meta(shape))


def _py_rope(base, offset, traditional, pair_swap=False, exp_scale=2.0, sin_sign=1.0):
    """A float64 RoPE with a knob per plausible mistake."""
    def f(x, shape):
        rows, hd = shape
        half = hd // 2
        x = np.asarray(x, np.float64).reshape(rows, hd)
        y = np.zeros_like(x)
        trad = traditional != pair_swap
        for i in range(rows):
            for d in range(half):
                th = (offset + i) * base ** (-(exp_scale * d) / hd)
                c, s = math.cos(th), sin_sign * math.sin(th)
                i0, i1 = (2 * d, 2 * d + 1) if trad else (d, d + half)
                y[i, i0] = x[i, i0] * c - x[i, i1] * s
                y[i, i1] = x[i, i0] * s + x[i, i1] * c
        return y
    return f


@pytest.mark.parametrize("traditional", [True, False])
def test_rope_closed_form_pins_oracle_and_rejects_mistakes(traditional):
    hd, rows, off, base = 8, 5, 3, 10000.0
    rope_closed_form_check(_py_rope(base, off, traditional), hd, rows, off, base, traditional, "f64")
    for wrong in (dict(pair_swap=True), dict(exp_scale=1.0), dict(sin_sign=-1.0)):
        with pytest.raises(AssertionError):
            rope_closed_form_check(_py_rope(base, off, traditional, **wrong), hd, rows, off, base,
                                   traditional, f"planted {wrong}")


# ── Elementwise chains: the f32 error bound of a random program ─────────────

CHAIN_UNARY = [OpKind.Neg, OpKind.Silu, OpKind.Gelu, OpKind.Exp, OpKind.Log, OpKind.Sqrt]
CHAIN_BINARY = [OpKind.Add, OpKind.Sub, OpKind.Mul, OpKind.Div]


def _oracle_chain(ins, prog, unary=CHAIN_UNARY, binary=CHAIN_BINARY):
    s = cpu_stream()
    n = ins[0].size
    leaves = [s.add_constant(a, meta([n])) for a in ins]
    acc = leaves[0]
    for code, j, left in prog:
        if code < len(unary):
            acc = s.add_op(unary[code], [acc], meta([n]))
        else:
            other = leaves[j]
            acc = s.add_op(binary[code - len(unary)], [acc, other] if left else [other, acc], meta([n]))
    s.eval(acc)
    return s.get_buffer(acc)


def _programs():
    rng = np.random.default_rng(2024)
    for _ in range(60):
        L = int(rng.integers(1, 9))
        yield [(int(rng.integers(0, 10)), int(rng.integers(0, 3)), bool(rng.integers(0, 2))) for _ in range(L)]


def test_chain_bound_holds_for_the_oracle():
    """The oracle's own f32 chain lies within E (half the cross-check's 2E)
    of the float64 value on 60 random programs over every op."""
    n = 2000
    ins = [synth.normal(n * 3 + j, (n,), 0.0, 1.0) for j in range(3)]
    checked = 0
    for prog in _programs():
        out = _oracle_chain(ins, prog)
        v, e, unc = chain_bound(ins, prog, CHAIN_UNARY, CHAIN_BINARY)
        ok = ~unc & np.isfinite(v)
        assert np.all(np.abs(out[ok].astype(np.float64) - v[ok]) <= e[ok]), prog
        assert np.all(np.isnan(out[np.isnan(v) & ~unc])), prog
        checked += int(ok.sum())
    assert checked > 60 * n // 4


@pytest.mark.parametrize("swap", ["exp_for_neg", "div_for_mul", "operand_side", "dropped_step"])
def test_chain_bound_catches_planted_mistakes(swap):
    """One wrong step in the evaluated chain (a different op, swapped
    operands of a Sub, a missing step) moves results far beyond the bound."""
    n = 2000
    ins = [synth.normal(n * 3 + j, (n,), 0.0, 1.0) for j in range(3)]
    prog = [(0, 0, True), (6, 1, True), (8, 2, True), (1, 0, True), (7, 1, False)]  # Neg, Add, Mul, Silu, Sub
    bad = list(prog)
    if swap == "exp_for_neg":
        bad[0] = (3, 0, True)
    elif swap == "div_for_mul":
        bad[2] = (9, 2, True)
    elif swap == "operand_side":
        bad[4] = (7, 1, True)
    else:
        bad = bad[:3] + bad[4:]
    good = _oracle_chain(ins, prog)
    wrong = _oracle_chain(ins, bad)
    bound = chain_bound(ins, prog, CHAIN_UNARY, CHAIN_BINARY)
    assert_chain_within_bound(good, good, *bound)
    with pytest.raises(AssertionError):
        assert_chain_within_bound(wrong, good, *bound)
