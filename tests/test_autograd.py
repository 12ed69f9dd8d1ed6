"""Reverse-mode autograd through the Stream: the HIP product
(``mlxhip_stream_grad`` in libmlxhip.so) and the oracle's restatement
(``oracle/graph.py``), both checked on the reference's own autograd tests
(crates/mlx-autograd/src/lib.rs:180-600: known answers and central-difference
checks with their tolerances), then against each other on a small
transformer block. The GPU half also runs the reference tests through the
HIP path and the config-4 block at full size against torch float32 autograd.

Tolerances: the reference's (assert_allclose semantics, crates/mlx-conformance/
src/lib.rs:32-48: |a - e| <= atol + rtol*|e|).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.graph import OracleStream
from oxidizedmlx_amd import abi, nn, synth
from oxidizedmlx_amd.tensor import Tensor, grad, value_and_grad

# ── the reference's autograd tests, as data ──────────────────────────────
# name, x data, x shape, f(x, const) where const(data, shape) makes a
# Constant on the same stream, expected gradient (None: central difference
# with eps 1e-3), atol = rtol.

EXACT = "exact"


def _c(name, x, shape, f, expected=None, tol=1e-3):
    return pytest.param(x, shape, f, expected, tol, id=name)


REFERENCE_TESTS = [
    # lib.rs:180-249 (known answers)
    _c("identity", [1, 2, 3], [3], lambda x, c: x.sum_all(), [1, 1, 1], EXACT),
    _c("add", [1, 2, 3], [3], lambda x, c: x.add(x).sum_all(), [2, 2, 2], 1e-5),
    _c("mul_self", [1, 2, 3], [3], lambda x, c: x.mul(x).sum_all(), [2, 4, 6], 1e-5),
    _c("neg", [1, 2, 3], [3], lambda x, c: x.neg().sum_all(), [-1, -1, -1], 1e-5),
    _c("sub", [1, 2, 3], [3], lambda x, c: x.sub(c([0.5] * 3, [3])).sum_all(), [1, 1, 1], 1e-5),
    _c("div", [2, 4, 6], [3], lambda x, c: x.div(c([2.0] * 3, [3])).sum_all(), [0.5] * 3, 1e-5),
    _c("matmul", [1, 2, 3, 4], [2, 2], lambda x, c: x.matmul(c([0.5, 0.3, 0.7, 0.1], [2, 2])).sum_all(),
       [0.8] * 4, 1e-5),
    # lib.rs:253-600 (central differences)
    _c("check_mul", [1, 2, 3], [3], lambda x, c: x.mul(c([2, 3, 4], [3])).sum_all()),
    _c("check_div", [2, 4, 6], [3], lambda x, c: x.div(c([2, 3, 4], [3])).sum_all()),
    _c("check_chain", [1, 2, 3], [3], lambda x, c: x.mul(x).add(x).sum_all()),
    _c("check_matmul", [1, 2, 3, 4], [2, 2], lambda x, c: x.matmul(c([0.5, 0.3, 0.7, 0.1], [2, 2])).sum_all()),
    _c("sum_axis", [1, 2, 3, 4, 5, 6], [2, 3], lambda x, c: x.sum_axis(0).sum_all()),
    _c("broadcast_rank_extension", [1, 2, 3], [3], lambda x, c: x.broadcast_to([2, 3]).sum_all()),
    _c("broadcast_dim_expansion", [1, 2, 3], [1, 3], lambda x, c: x.broadcast_to([2, 3]).sum_all()),
    _c("broadcast_combined", [1, 2, 3], [3], lambda x, c: x.broadcast_to([2, 1, 3]).sum_all()),
    _c("layer_norm", [1, 2, 3, 4, 5, 6], [2, 3], lambda x, c: x.layer_norm(1e-5).sum_all()),
    _c("rms_norm", [1, 2, 3, 4, 5, 6], [2, 3], lambda x, c: x.rms_norm(1e-5).sum_all()),
    _c("layer_norm_1d", [1, 3, 5, 7], [4], lambda x, c: x.layer_norm(1e-5).sum_all()),
    _c("rms_norm_1d", [1, 3, 5, 7], [4], lambda x, c: x.rms_norm(1e-5).sum_all()),
    _c("layer_norm_chain", [1, 2, 3], [3], lambda x, c: x.mul(c([2.0] * 3, [3])).layer_norm(1e-5).sum_all(),
       None, 1e-2),
    _c("rms_norm_chain", [1, 2, 3], [3], lambda x, c: x.add(c([1.0] * 3, [3])).rms_norm(1e-5).sum_all(),
       None, 1e-2),
    _c("softmax_1d", [1, 2, 3, 4], [4], lambda x, c: x.softmax(0).sum_all()),
    _c("softmax_2d", [1, 2, 3, 4, 5, 6], [2, 3], lambda x, c: x.softmax(1).sum_all()),
    _c("softmax_3d", list(range(1, 13)), [2, 2, 3], lambda x, c: x.softmax(2).sum_all()),
    # #[ignore]d in the reference (lib.rs:525-536, against a Python reference);
    # the central-difference check itself holds.
    _c("softmax_weighted", [1, 2, 3], [3], lambda x, c: x.softmax(0).mul(c([1, 2, 3], [3])).sum_all()),
    _c("silu_1d", [-2, -1, 0, 1, 2], [5], lambda x, c: x.silu().sum_all()),
    _c("silu_2d", [0.5, -0.5, 1.5, -1.5, 2.5, -2.5], [2, 3], lambda x, c: x.silu().sum_all()),
    _c("gelu_1d", [-2, -1, 0, 1, 2], [5], lambda x, c: x.gelu().sum_all()),
    _c("gelu_2d", [0.5, -0.5, 1.5, -1.5, 2.5, -2.5], [2, 3], lambda x, c: x.gelu().sum_all()),
    _c("silu_chain", [1, 2, 3], [3], lambda x, c: x.mul(c([2.0] * 3, [3])).silu().sum_all(), None, 1e-2),
    _c("gelu_chain", [1, 2, 3], [3], lambda x, c: x.add(c([1.0] * 3, [3])).gelu().sum_all(), None, 1e-2),
]


def hip_stream():
    from oxidizedmlx_amd.backend import HipStream
    return HipStream()


STREAMS = {"oracle": OracleStream, "hip": hip_stream}


def scalar(make, f, x_data, shape) -> float:
    s = make()
    c = lambda d, sh: Tensor.from_f32_on_stream(d, sh, s)  # noqa: E731
    return float(f(Tensor.from_f32_on_stream(x_data, shape, s), c).to_numpy().reshape(-1)[0])


def numerical_grad(make, f, x_data, shape, eps=1e-3):
    """Central differences in f32 (lib.rs:159-177)."""
    x = np.asarray(x_data, np.float32)
    out = np.zeros_like(x)
    for i in range(x.size):
        xp, xm = x.copy(), x.copy()
        xp[i] += np.float32(eps)
        xm[i] -= np.float32(eps)
        out[i] = (np.float32(scalar(make, f, xp, shape)) - np.float32(scalar(make, f, xm, shape))) / np.float32(2 * eps)
    return out


def check_reference_case(make, x_data, shape, f, expected, tol):
    s = make()
    c = lambda d, sh: Tensor.from_f32_on_stream(d, sh, s)  # noqa: E731
    x = Tensor.from_f32_on_stream(x_data, shape, s)
    g = grad(lambda t: f(t, c), x).to_numpy().reshape(-1)
    if tol == EXACT:
        np.testing.assert_array_equal(g, np.asarray(expected, np.float32))
        return
    want = np.asarray(expected if expected is not None else numerical_grad(make, f, x_data, shape),
                      np.float64).reshape(-1)
    err = np.abs(g.astype(np.float64) - want)
    assert np.all(err <= tol + tol * np.abs(want)), f"analytical {g} vs expected {want}"


@pytest.mark.usefixtures("oracle_lib")
@pytest.mark.parametrize("x_data,shape,f,expected,tol", REFERENCE_TESTS)
def test_oracle_reference_autograd(x_data, shape, f, expected, tol):
    check_reference_case(OracleStream, x_data, shape, f, expected, tol)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
@pytest.mark.parametrize("x_data,shape,f,expected,tol", REFERENCE_TESTS)
def test_hip_reference_autograd(x_data, shape, f, expected, tol):
    check_reference_case(hip_stream, x_data, shape, f, expected, tol)


# ── error behaviour (lib.rs:35-40, 104-106; vjp.rs:173-176) ──────────────

@pytest.mark.parametrize("kind", ["oracle", pytest.param("hip", marks=pytest.mark.gpu)])
@pytest.mark.usefixtures("oracle_lib")
def test_grad_errors(kind, request):
    if kind == "hip":
        request.getfixturevalue("hip")
    s = STREAMS[kind]()
    x = Tensor.from_f32_on_stream([1, 2, 3], [3], s)
    with pytest.raises(abi.InvalidArgument, match="scalar loss"):
        value_and_grad(x.mul(x), [x])
    other = Tensor.from_f32_on_stream([1, 2, 3], [3], s)
    with pytest.raises(abi.InvalidArgument, match="gradient not found"):
        value_and_grad(x.sum_all(), [other])
    with pytest.raises(abi.InvalidArgument, match="VJP not implemented"):
        value_and_grad(x.exp().sum_all(), [x])


# ── rank-3 MatMul and its VJP ─────────────────────────────────────────────

@pytest.mark.usefixtures("oracle_lib")
def test_oracle_batched_matmul_grad_central_difference():
    a0 = synth.normal(301, (2, 3, 4))
    b0 = synth.normal(302, (2, 4, 5))
    w0 = synth.normal(303, (2, 3, 5))

    def f(x, c):
        return x.matmul(c(b0, b0.shape)).mul(c(w0, w0.shape)).sum_all()

    check_reference_case(OracleStream, a0.reshape(-1), a0.shape, f, None, 1e-3)

    def fb(x, c):
        return c(a0, a0.shape).matmul(x).mul(c(w0, w0.shape)).sum_all()

    check_reference_case(OracleStream, b0.reshape(-1), b0.shape, fb, None, 1e-3)


# ── a small transformer block ─────────────────────────────────────────────

SMALL = nn.BlockConfig(d_model=32, n_heads=4, seq=8, batch=2)


def block_arrays(cfg: nn.BlockConfig, seed: int = 7):
    """Weights N(0, 0.02^2), biases N(0, 0.02^2), x N(0, 1), and the loss
    weights gy N(0, 1): loss = sum(block(x) * gy)."""
    arrs = {}
    for i, (name, shp) in enumerate(cfg.param_shapes().items()):
        arrs[name] = synth.normal(seed * 100 + i, shp, 0.0, 0.02)
    x = synth.normal(seed * 100 + 50, (cfg.rows, cfg.d_model))
    gy = synth.normal(seed * 100 + 51, (cfg.rows, cfg.d_model))
    return arrs, x, gy


def block_loss(s, cfg, arrs, x, gy):
    params = {k: Tensor.from_f32_on_stream(v, v.shape, s) for k, v in arrs.items()}
    xt = Tensor.from_f32_on_stream(x, x.shape, s)
    y = nn.TransformerBlock(cfg, params)(xt)
    loss = y.mul(Tensor.from_f32_on_stream(gy, gy.shape, s)).sum_all()
    return loss, params, xt


def block_grads(s, cfg, arrs, x, gy):
    loss, params, xt = block_loss(s, cfg, arrs, x, gy)
    names = list(params)
    _, gs = value_and_grad(loss, [params[k] for k in names] + [xt])
    s.eval_many([g.node for g in gs])
    out = {k: g.to_numpy() for k, g in zip(names + ["x"], gs)}
    return float(loss.to_numpy().reshape(-1)[0]), out


@pytest.mark.usefixtures("oracle_lib")
def test_oracle_block_grads_central_difference():
    # A few entries of every gradient against central differences of the
    # oracle's own forward pass (eps 1e-2 on O(1) losses).
    cfg = nn.BlockConfig(d_model=8, n_heads=2, seq=4, batch=2)
    arrs, x, gy = block_arrays(cfg, seed=3)
    _, grads = block_grads(OracleStream(), cfg, arrs, x, gy)
    rng = np.random.default_rng(5)
    eps = 1e-2
    for name in list(arrs) + ["x"]:
        base = x if name == "x" else arrs[name]
        for idx in rng.choice(base.size, size=3, replace=False):
            vals = []
            for sign in (1, -1):
                pert = base.copy().reshape(-1)
                pert[idx] += np.float32(sign * eps)
                pert = pert.reshape(base.shape)
                a2 = dict(arrs)
                x2 = x
                if name == "x":
                    x2 = pert
                else:
                    a2[name] = pert
                loss, _, _ = block_loss(OracleStream(), cfg, a2, x2, gy)
                vals.append(float(loss.to_numpy().reshape(-1)[0]))
            num = (vals[0] - vals[1]) / (2 * eps)
            ana = float(grads[name].reshape(-1)[idx])
            assert abs(ana - num) <= 2e-3 + 2e-2 * abs(num), f"{name}[{idx}]: analytical {ana} numerical {num}"


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib")
def test_hip_block_grads_match_oracle():
    arrs, x, gy = block_arrays(SMALL)
    loss_h, gh = block_grads(hip_stream(), SMALL, arrs, x, gy)
    loss_o, go = block_grads(OracleStream(), SMALL, arrs, x, gy)
    assert abs(loss_h - loss_o) <= 1e-4 * max(1.0, abs(loss_o))
    top = max(float(np.abs(g).max()) for g in go.values())
    bad = []
    for k in go:
        scale = max(float(np.abs(go[k]).max()), 1e-3 * top)  # see the config-4 test
        err = float(np.abs(gh[k].astype(np.float64) - go[k]).max())
        if err > 1e-4 * scale:
            bad.append(f"{k}: max abs err {err:.3e} (scale {scale:.3e})")
    assert not bad, "; ".join(bad)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib")
def test_hip_block_config4_prefix_matches_oracle():
    """Config 4 at full size (d_model 1024, 16 heads, seq 512, batch 4) on
    the GPU against the oracle. The loss weights gy are zero except on the
    first P positions of sequence 0, so the loss, every weight gradient and
    the x gradient depend only on that causal prefix (attention at position i
    sees positions <= i; the norms and the MLP act row by row): the oracle
    runs the same block on x[0:P] with gy[0:P] (batch 1, seq P), and the GPU's
    x gradient is exactly zero on every other row (their cotangents are zero
    and masked attention probabilities are exactly zero)."""
    cfg = nn.BlockConfig()
    P = 64
    arrs, x, gy = block_arrays(cfg, seed=31)
    gy_masked = np.zeros_like(gy)
    gy_masked[:P] = gy[:P]  # rows are [batch][seq]: rows 0..P-1 are sequence 0, positions 0..P-1
    print(f"config 4 on the GPU, loss on the first {P} positions of sequence 0", flush=True)
    loss_h, gh = block_grads(hip_stream(), cfg, arrs, x, gy_masked)
    cfg_p = nn.BlockConfig(d_model=cfg.d_model, n_heads=cfg.n_heads, seq=P, batch=1, eps=cfg.eps)
    print(f"oracle on the {P}-position prefix", flush=True)
    loss_o, go = block_grads(OracleStream(), cfg_p, arrs, x[:P], gy[:P])
    assert abs(loss_h - loss_o) <= 1e-4 * max(1.0, abs(loss_o)), (loss_h, loss_o)
    assert not gh["x"][P:].any(), "x gradient outside the prefix is not zero"
    gh = dict(gh, x=gh["x"][:P])
    top = max(float(np.abs(g).max()) for g in go.values())
    bad = []
    for k in go:
        scale = max(float(np.abs(go[k]).max()), 1e-3 * top)  # see the config-4 test against torch
        err = float(np.abs(gh[k].astype(np.float64) - go[k]).max())
        print(f"  {k}: max abs err {err:.3e} (scale {scale:.3e})", flush=True)
        if err > 1e-4 * scale:
            bad.append(f"{k}: max abs err {err:.3e} (scale {scale:.3e})")
    assert not bad, "; ".join(bad)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib")
def test_hip_block_config4_last_sequence_prefix_matches_oracle():
    """The same check on another part of config 4: the loss weights gy are
    non-zero only on the first P = 256 positions of the last sequence of the
    batch (rows 3*512 .. 3*512+255), so the GPU's full-size block must give
    the gradients the oracle computes on that sequence's prefix alone, and an
    x gradient that is exactly zero on every other row (sequences 0-2 and the
    rest of sequence 3). This covers the batch indexing of every kernel
    (attention rows of another sequence, bias gradients summed over rows that
    mostly carry zero cotangents)."""
    cfg = nn.BlockConfig()
    P, b = 256, cfg.batch - 1
    arrs, x, gy = block_arrays(cfg, seed=47)
    r0 = b * cfg.seq
    gy_masked = np.zeros_like(gy)
    gy_masked[r0:r0 + P] = gy[r0:r0 + P]
    print(f"config 4 on the GPU, loss on the first {P} positions of sequence {b}", flush=True)
    loss_h, gh = block_grads(hip_stream(), cfg, arrs, x, gy_masked)
    cfg_p = nn.BlockConfig(d_model=cfg.d_model, n_heads=cfg.n_heads, seq=P, batch=1, eps=cfg.eps)
    print(f"oracle on the {P}-position prefix of sequence {b}", flush=True)
    loss_o, go = block_grads(OracleStream(), cfg_p, arrs, x[r0:r0 + P], gy[r0:r0 + P])
    outside = np.ones(x.shape[0], bool)
    outside[r0:r0 + P] = False
    assert not gh["x"][outside].any(), "x gradient outside the prefix is not zero"
    compare_block_grads(dict(gh, x=gh["x"][r0:r0 + P]), go, loss_h, loss_o)


def compare_block_grads(gh, go, loss_h, loss_o):
    assert abs(loss_h - loss_o) <= 1e-4 * max(1.0, abs(loss_o)), (loss_h, loss_o)
    top = max(float(np.abs(g).max()) for g in go.values())
    bad = []
    for k in go:
        scale = max(float(np.abs(go[k]).max()), 1e-3 * top)
        err = float(np.abs(gh[k].astype(np.float64) - go[k]).max())
        print(f"  {k}: max abs err {err:.3e} (scale {scale:.3e})", flush=True)
        if err > 1e-4 * scale:
            bad.append(f"{k}: max abs err {err:.3e} (scale {scale:.3e})")
    assert not bad, "; ".join(bad)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib")
def test_hip_block_fused_attention_matches_oracle():
    """The block with its attention as one HeadAttention op (fused forward,
    fused VJP) against the oracle's autograd of the composed graph (MatMul,
    scale, -1e9 mask, Softmax, MatMul): same loss and gradients within the
    block tests' tolerance. Head dim 64, two 64-position blocks."""
    import dataclasses
    cfg = nn.BlockConfig(d_model=128, n_heads=2, seq=128, batch=2)
    arrs, x, gy = block_arrays(cfg, seed=17)
    loss_h, gh = block_grads(hip_stream(), dataclasses.replace(cfg, fused_attention=True), arrs, x, gy)
    loss_o, go = block_grads(OracleStream(), cfg, arrs, x, gy)
    compare_block_grads(gh, go, loss_h, loss_o)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib")
def test_hip_block_fused_attention_config4_prefix_matches_oracle():
    """Config 4 at full size with fused attention on the GPU against the
    oracle's composed block on the causal prefix (as in the composed
    config-4 test above): the x gradient is exactly zero past the prefix."""
    import dataclasses
    cfg = nn.BlockConfig()
    P = 64
    arrs, x, gy = block_arrays(cfg, seed=31)
    gy_masked = np.zeros_like(gy)
    gy_masked[:P] = gy[:P]
    print(f"config 4 with fused attention on the GPU, loss on the first {P} positions of sequence 0", flush=True)
    loss_h, gh = block_grads(hip_stream(), dataclasses.replace(cfg, fused_attention=True), arrs, x, gy_masked)
    cfg_p = nn.BlockConfig(d_model=cfg.d_model, n_heads=cfg.n_heads, seq=P, batch=1, eps=cfg.eps)
    loss_o, go = block_grads(OracleStream(), cfg_p, arrs, x[:P], gy[:P])
    assert not gh["x"][P:].any(), "x gradient outside the prefix is not zero"
    compare_block_grads(dict(gh, x=gh["x"][:P]), go, loss_h, loss_o)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
def test_hip_block_async_eval_matches_sync():
    """Asynchronous evaluation (mlxhip_stream_set_async) changes no result:
    three block steps queued on one asynchronous stream without reading
    anything in between (each step's host constants copied while earlier
    steps still run), then every gradient of every step read, bit for bit
    against a synchronous stream."""
    from oxidizedmlx_amd.backend import HipStream
    arrs, x, gy = block_arrays(SMALL, seed=13)
    _, want = block_grads(HipStream(), SMALL, arrs, x, gy)
    st = HipStream(async_eval=True)
    steps = []
    for _ in range(3):
        loss, params, xt = block_loss(st, SMALL, arrs, x, gy)
        names = list(params)
        _, gs = value_and_grad(loss, [params[k] for k in names] + [xt])
        st.eval_many([g.node for g in gs])
        steps.append(dict(zip(names + ["x"], gs)))
    for got in steps:
        for k, g in got.items():
            np.testing.assert_array_equal(g.to_numpy(), want[k], err_msg=k)
    st.synchronize()
    st.set_async(False)
    st.close()


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
def test_hip_softmax_vjp_reuses_forward_softmax():
    """The Softmax VJP takes the forward Softmax node itself (CSE over the
    same op and input) as its output operand, so a gradient evaluated after
    the forward evaluates no second softmax: evaluating y and then dx costs
    exactly the nodes of evaluating dx alone on a fresh stream (a second
    Softmax node would add one), and both give the same dx."""
    from oxidizedmlx_amd.backend import HipStream
    x0, w0 = synth.normal(71, (6, 37)), synth.normal(72, (6, 37))

    def build(st):
        x = Tensor.from_f32_on_stream(x0.reshape(-1), x0.shape, st)
        w = Tensor.from_f32_on_stream(w0.reshape(-1), w0.shape, st)
        y = x.softmax(-1)
        _, gs = value_and_grad(y.mul(w).sum_all(), [x])
        return y, gs[0]

    a, b = HipStream(fusion=False), HipStream(fusion=False)
    ya, ga = build(a)
    a.eval_many([ya.node])
    a.eval_many([ga.node])
    _, gb = build(b)
    b.eval_many([gb.node])
    assert a.eval_count() == b.eval_count()
    np.testing.assert_array_equal(ga.to_numpy(), gb.to_numpy())
    a.close()
    b.close()


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
def test_hip_block_steps_with_clear_reuse_memory():
    """Block steps on one asynchronous stream, each cleared after its eval
    (mlxhip_stream_clear) so the next step's buffers reuse its HBM while its
    kernels may still be queued: four steps queued back to back, then the
    last one's gradients read, bit for bit against a synchronous stream; an
    old node id is rejected after a clear."""
    from oxidizedmlx_amd.backend import HipStream
    arrs, x, gy = block_arrays(SMALL, seed=17)
    _, want = block_grads(HipStream(), SMALL, arrs, x, gy)
    st = HipStream(async_eval=True)
    for step in range(4):
        loss, params, xt = block_loss(st, SMALL, arrs, x, gy)
        names = list(params)
        _, gs = value_and_grad(loss, [params[k] for k in names] + [xt])
        st.eval_many([g.node for g in gs])
        if step < 3:
            old = gs[0].node
            st.clear()
    got = {k: g.to_numpy() for k, g in zip(names + ["x"], gs)}
    for k in want:
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)
    with pytest.raises(abi.InvalidArgument):
        st.eval(old)
    st.close()


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
def test_hip_block_fusion_off_matches_on():
    from oxidizedmlx_amd.backend import HipStream
    arrs, x, gy = block_arrays(SMALL, seed=11)
    _, g_on = block_grads(HipStream(fusion=True), SMALL, arrs, x, gy)
    _, g_off = block_grads(HipStream(fusion=False), SMALL, arrs, x, gy)
    for k in g_on:
        # Fusion changes no arithmetic (chains round per step; folded
        # transposes only change the GEMM's operand layout).
        np.testing.assert_array_equal(g_on[k], g_off[k], err_msg=k)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
@pytest.mark.parametrize("cfg", [nn.BlockConfig(), nn.BlockConfig(seq=1024, batch=2), SMALL],
                         ids=["config4", "seq1024", "small"])
def test_hip_block_head_views_match_permutes(monkeypatch, cfg):
    """The composed attention's head split and merge without permute kernels:
    at config 4 the thin kernels read the Q, K, V and dO heads in place and
    write O, dQ, dK and dV straight into the merged [B*S, D] layout; the
    small block's products do not fit those kernels, so its permutes run
    after all. Either way every gradient is bit for bit the one of the same
    block with the permutes always run (MLXHIP_HEAD_VIEWS=0), with the same
    eval count, and the thin-kernel blocks (config 4; 2 sequences of 1024)
    take 8 fewer launches (4 splits, 4 merges)."""
    from oxidizedmlx_amd.backend import HipStream
    arrs, x, gy = block_arrays(cfg, seed=23)
    runs = {}
    for views in ("1", "0"):
        monkeypatch.setenv("MLXHIP_HEAD_VIEWS", views)
        st = HipStream()
        loss, g = block_grads(st, cfg, arrs, x, gy)
        runs[views] = (loss, g, st.eval_count(), st.launch_count())
        st.close()
    (l1, g1, e1, n1), (l0, g0, e0, n0) = runs["1"], runs["0"]
    print(f"  head views: {n1} launches, permutes: {n0} launches; eval count {e1} / {e0}", flush=True)
    assert l1 == l0 and e1 == e0
    for k in g0:
        np.testing.assert_array_equal(g1[k], g0[k], err_msg=k)
    assert n0 - n1 == (8 if cfg is not SMALL else 0)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
def test_hip_block_config4_matches_torch_fp32_cpu():
    """Config 4 at full size (d_model 1024, 16 heads, seq 512, batch 4)
    against torch float32 autograd of the same block, run on the host CPU
    (torch carries its own HIP runtime, which does not share this process's
    device with libmlxhip.so)."""
    import torch

    cfg = nn.BlockConfig()
    arrs, x, gy = block_arrays(cfg, seed=21)
    loss_h, gh = block_grads(hip_stream(), cfg, arrs, x, gy)

    dev = torch.device("cpu")
    tp = {k: torch.tensor(v, device=dev, requires_grad=True) for k, v in arrs.items()}
    tx = torch.tensor(x, device=dev, requires_grad=True)
    b, s_, h, d = cfg.batch, cfg.seq, cfg.n_heads, cfg.d_model
    dh = d // h

    def lin(t, w, bias):
        return t @ tp[w].t().contiguous() + tp[bias]

    def rms(t):
        return t / torch.sqrt((t * t).mean(-1, keepdim=True) + cfg.eps)

    def heads(t):
        return t.reshape(b, s_, h, dh).permute(0, 2, 1, 3).reshape(b * h, s_, dh).contiguous()

    h1 = rms(tx)
    q, k, v = heads(lin(h1, "wq", "bq")), heads(lin(h1, "wk", "bk")), heads(lin(h1, "wv", "bv"))
    sc = torch.bmm(q, k.transpose(1, 2).contiguous()) * (1.0 / np.sqrt(dh))
    sc = sc + torch.tensor(nn.causal_mask(s_), device=dev)
    o = torch.bmm(torch.softmax(sc, -1), v).reshape(b, h, s_, dh).permute(0, 2, 1, 3).reshape(b * s_, d)
    hh = tx + lin(o, "wo", "bo")
    u = lin(rms(hh), "w1", "b1")
    y = hh + lin(u * torch.sigmoid(u), "w2", "b2")
    loss = (y * torch.tensor(gy, device=dev)).sum()
    loss.backward()
    assert abs(loss_h - loss.item()) <= 1e-3 * max(1.0, abs(loss.item()))
    refs = {name: (tx.grad if name == "x" else tp[name].grad).detach().cpu().numpy() for name in gh}
    top = max(float(np.abs(r).max()) for r in refs.values())
    bad = []
    for name, ref in refs.items():
        # Each gradient within 2e-3 of its own largest entry; a gradient that
        # is zero in exact arithmetic is held to 2e-3 of 1e-3 * the largest
        # gradient entry of the block instead of its own rounding noise.
        scale = max(float(np.abs(ref).max()), 1e-3 * top)
        err = float(np.abs(gh[name].astype(np.float64) - ref).max())
        if err > 2e-3 * scale:
            bad.append(f"{name}: max abs err {err:.3e} (scale {scale:.3e})")
    assert not bad, "; ".join(bad)
    # Adding the same vector to every key shifts each score row by a
    # constant, which softmax ignores: d(loss)/d(bk) is zero.
    assert float(np.abs(gh["bk"]).max()) <= 1e-5 * float(np.abs(gh["bq"]).max())
