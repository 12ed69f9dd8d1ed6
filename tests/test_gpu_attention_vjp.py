"""Gradient of fused attention (kernels/attention_bwd.hip, mlxhip_attention_vjp).

The reference has no VJP for its Attention op (crates/mlx-autograd/src/vjp.rs:
173-176); what it does differentiate is attention composed from MatMul, Mul by
the scale, Add of the -1e9 causal mask and Softmax (the config-4 block). The
fused gradient is held against two checkers on the same inputs:
  * float64 closed form (dV = P^T dO, dS = P o (dO V^T - rowsum(dO o O)),
    dQ = scale dS K, dK = scale dS^T Q), itself pinned on the CPU by central
    differences of the float64 forward;
  * the oracle's autograd of the composed graph in f32, whose own error
    against float64 sets the bound: the GPU's largest error must stay within
    twice the oracle's, plus 1e-6 of the gradient's largest magnitude."""
import math

import numpy as np
import pytest

from oracle.graph import OracleStream
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd import synth
from oxidizedmlx_amd.nn import causal_mask
from oxidizedmlx_amd.tensor import Tensor, value_and_grad


def f64_forward(q, k, v, scale, causal):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    s = np.einsum("bid,bjd->bij", q, k) * scale
    if causal:
        t = s.shape[-1]
        s = np.where(np.arange(t)[None, None, :] > np.arange(t)[None, :, None], -np.inf, s)
    e = np.exp(s - s.max(-1, keepdims=True))
    p = e / e.sum(-1, keepdims=True)
    return np.einsum("bij,bjd->bid", p, v), p


def f64_vjp(q, k, v, do, scale, causal):
    o, p = f64_forward(q, k, v, scale, causal)
    q, k, v, do = (a.astype(np.float64) for a in (q, k, v, do))
    dv = np.einsum("bij,bid->bjd", p, do)
    dp = np.einsum("bid,bjd->bij", do, v)
    ds = p * (dp - (do * o).sum(-1, keepdims=True))
    return scale * np.einsum("bij,bjd->bid", ds, k), scale * np.einsum("bij,bid->bjd", ds, q), dv


@pytest.mark.parametrize("causal", [True, False])
def test_f64_closed_form_matches_central_differences(causal):
    """Pins the float64 checker: every input element's derivative of
    sum(O o dO), by central differences of the float64 forward."""
    rng = np.random.default_rng(5)
    q, k, v, do = (rng.standard_normal((2, 6, 4)) for _ in range(4))
    scale = 0.7
    grads = f64_vjp(q, k, v, do, scale, causal)
    for idx, (x, g) in enumerate(zip((q, k, v), grads)):
        num = np.zeros_like(x)
        for pos in np.ndindex(x.shape):
            d = np.zeros_like(x)
            d[pos] = 1e-6
            args = [q, k, v]
            args[idx] = x + d
            fp = (f64_forward(*args, scale, causal)[0] * do).sum()
            args[idx] = x - d
            fm = (f64_forward(*args, scale, causal)[0] * do).sum()
            num[pos] = (fp - fm) / 2e-6
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-8, err_msg="qkv"[idx])


def oracle_composed_grads(q, k, v, do, scale, causal):
    """f32 gradients of sum(O o dO) through the oracle's autograd of the
    composed graph (the config-4 block's attention)."""
    st = OracleStream()
    b, t, dh = q.shape
    tq, tk, tv = (Tensor.from_f32_on_stream(a.reshape(-1), a.shape, st) for a in (q, k, v))
    scores = tq.matmul(tk.transpose((0, 2, 1)))
    sc = Tensor.from_f32_on_stream([scale], (), st).broadcast_to(scores.shape)
    x = scores.mul(sc)
    if causal:
        x = x.add(Tensor.from_f32_on_stream(causal_mask(t), (t, t), st).broadcast_to(scores.shape))
    o = x.softmax(-1).matmul(tv)
    loss = o.mul(Tensor.from_f32_on_stream(do.reshape(-1), do.shape, st)).sum_all()
    _, gs = value_and_grad(loss, [tq, tk, tv])
    return [g.to_numpy().reshape(q.shape) for g in gs]


def gpu_grads(q, k, v, do, scale, causal):
    b, t, dh = q.shape
    dq_, dk_, dv_, qd, kd, vd, od, dod = (hb.DeviceBuffer(q.nbytes) for _ in range(8))
    for buf, a in ((qd, q), (kd, k), (vd, v), (dod, do)):
        buf.upload(np.ascontiguousarray(a))
    hb.attention(qd, kd, vd, od, b, t, t, dh, scale, causal)
    hb.attention_vjp(qd, kd, vd, od, dod, dq_, dk_, dv_, b, t, dh, scale, causal)
    hb.synchronize()
    return [x.download(np.float32, q.size).reshape(q.shape) for x in (dq_, dk_, dv_)]


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib")
@pytest.mark.parametrize("heads,t,causal", [(3, 64, True), (2, 128, True), (2, 192, False), (1, 256, True),
                                            (2, 64, False)])
def test_attention_vjp_matches_oracle_and_float64(heads, t, causal):
    print(f"attention vjp heads={heads} t={t} causal={causal}", flush=True)
    dh = 64
    q, k, v, do = (synth.normal(900 + 13 * t + i + heads, (heads, t, dh)) for i in range(4))
    scale = 1.0 / math.sqrt(dh)
    got = gpu_grads(q, k, v, do, scale, causal)
    ora = oracle_composed_grads(q, k, v, do, scale, causal)
    exact = f64_vjp(q, k, v, do, scale, causal)
    for name, g, o, e in zip("qkv", got, ora, exact):
        gpu_err = float(np.abs(g - e).max())
        ora_err = float(np.abs(o - e).max())
        print(f"  d{name}: max |gpu - f64| {gpu_err:.3e}, max |oracle - f64| {ora_err:.3e}", flush=True)
        assert gpu_err <= 2.0 * ora_err + 1e-6 * float(np.abs(e).max()), f"d{name}"


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib")
def test_attention_vjp_config4_heads():
    """Config 4's 64 heads of 512 causal positions. The oracle's error is
    measured on two of the heads (its autograd over all 64 would take
    minutes on one core) and bounds every head."""
    heads, t, dh = 64, 512, 64
    print(f"attention vjp heads={heads} t={t} causal=True", flush=True)
    q, k, v, do = (synth.normal(77 + i, (heads, t, dh)) for i in range(4))
    scale = 1.0 / math.sqrt(dh)
    got = gpu_grads(q, k, v, do, scale, True)
    exact = f64_vjp(q, k, v, do, scale, True)
    ora = oracle_composed_grads(q[:2], k[:2], v[:2], do[:2], scale, True)
    for name, g, o, e in zip("qkv", got, ora, exact):
        gpu_err = float(np.abs(g - e).max())
        ora_err = float(np.abs(o - e[:2]).max())
        print(f"  d{name}: max |gpu - f64| {gpu_err:.3e}, max |oracle - f64| (2 heads) {ora_err:.3e}", flush=True)
        assert gpu_err <= 2.0 * ora_err + 1e-6 * float(np.abs(e).max()), f"d{name}"


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
def test_attention_vjp_rejects_unsupported_shapes():
    buf = hb.DeviceBuffer(4 * 64 * 96)
    with pytest.raises(Exception, match="attention vjp"):
        hb.attention_vjp(buf, buf, buf, buf, buf, buf, buf, buf, 1, 96, 64, 1.0, True)   # t not a multiple of 64
    with pytest.raises(Exception, match="attention vjp"):
        hb.attention_vjp(buf, buf, buf, buf, buf, buf, buf, buf, 1, 64, 32, 1.0, True)   # dh 32
    hb.attention_vjp(buf, buf, buf, buf, buf, buf, buf, buf, 0, 64, 64, 1.0, True)       # no heads: nothing to do


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
@pytest.mark.parametrize("b,t,heads,causal", [(2, 128, 4, True), (1, 192, 2, False), (4, 64, 16, True)])
def test_heads_in_rows_layout_matches_head_major(b, t, heads, causal):
    """HeadAttention with heads side by side in rows ([B, T, H*dh], the
    projections' own layout) gives, forward and through its VJP, exactly the
    values of the head-major form ([B*H, T, dh]) on the permuted inputs: per
    head the same kernels' arithmetic, only the addressing differs."""
    from oxidizedmlx_amd.backend import HipStream
    dh = 64
    d = heads * dh
    print(f"heads in rows b={b} t={t} heads={heads} causal={causal}", flush=True)
    q, k, v, g = (synth.normal(1300 + 7 * t + i + heads, (b, t, d)) for i in range(4))
    scale = 1.0 / math.sqrt(dh)

    def head_major(a):
        return np.ascontiguousarray(a.reshape(b, t, heads, dh).transpose(0, 2, 1, 3).reshape(b * heads, t, dh))

    def run(arrs, heads_arg):
        st = HipStream()
        tq, tk, tv, tg = (Tensor.from_f32_on_stream(a.reshape(-1), a.shape, st) for a in arrs)
        o = tq.head_attention(tk, tv, scale, causal, heads=heads_arg)
        loss = o.mul(tg).sum_all()
        _, grads = value_and_grad(loss, [tq, tk, tv])
        return [o.to_numpy().reshape(arrs[0].shape)] + [x.to_numpy().reshape(arrs[0].shape) for x in grads]

    rows = run((q, k, v, g), heads)
    hm = run(tuple(head_major(a) for a in (q, k, v, g)), None)
    for name, a, e in zip(("O", "dQ", "dK", "dV"), rows, hm):
        np.testing.assert_array_equal(head_major(a), e, err_msg=name)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
@pytest.mark.parametrize("shape,heads", [((4, 64, 32), None), ((2, 96, 64), None), ((2, 64, 96), 3)],
                         ids=["dh32", "t96", "rows_dh32"])
def test_unsupported_gradient_shapes_fail_when_the_gradient_is_built(shape, heads):
    """The fused gradient covers dh = 64 with t a multiple of 64. Other
    shapes still run forward, but asking for their gradient fails at once in
    value_and_grad (InvalidArgument), not later when the gradient is
    evaluated."""
    from oxidizedmlx_amd import abi
    from oxidizedmlx_amd.backend import HipStream
    st = HipStream()
    q, k, v = (synth.normal(1500 + i, shape) for i in range(3))
    tq, tk, tv = (Tensor.from_f32_on_stream(a.reshape(-1), a.shape, st) for a in (q, k, v))
    o = tq.head_attention(tk, tv, 0.25, True, heads=heads)
    assert np.isfinite(o.to_numpy()).all()
    with pytest.raises(abi.InvalidArgument, match="HeadAttention gradient"):
        value_and_grad(o.sum_all(), [tq])
    st.close()
