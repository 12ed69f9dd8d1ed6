"""The process default stream (the selection hook the reference lacks:
its default_stream() is fixed to the CPU backend, crates/mlx-core/src/
backend.rs:193-200) and the reference's MultiHeadAttention graph
(crates/mlx-nn/src/attention.rs:47-111) restated over the Tensor API.

CPU half: constructors without a stream land on the default; MLX_RS_BACKEND
names the backend; streams cannot be mixed; MultiHeadAttention on the oracle
stream against a float64 numpy restatement. GPU half: with the default set to
a HipStream, the reference's autograd tests (crates/mlx-autograd/src/lib.rs:
180-600) built from default-stream constructors only, and forward_causal
against the same graph on the oracle.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle.graph import OracleStream
from oxidizedmlx_amd import abi, nn, synth
from oxidizedmlx_amd import tensor as T
from oxidizedmlx_amd.tensor import Tensor, default_stream_scope, grad
from parity import assert_allclose
from test_autograd import EXACT, REFERENCE_TESTS

pytestmark = pytest.mark.usefixtures("oracle_lib")


def test_constructors_bind_to_the_default_stream():
    s = OracleStream()
    with default_stream_scope(s):
        a = Tensor.from_f32([1, 2, 3], [3])
        z = Tensor.zeros([2, 2])
        o = Tensor.ones([2], abi.BF16)
        assert a.stream is s and z.stream is s and o.stream is s
        assert o.dtype == abi.BF16
        np.testing.assert_array_equal(a.add(Tensor.ones([3])).to_numpy(), [2, 3, 4])
        np.testing.assert_array_equal(z.to_numpy(), np.zeros((2, 2)))
    other = OracleStream()
    with default_stream_scope(other):
        b = Tensor.from_f32([1, 2, 3], [3])
    with pytest.raises(abi.InvalidArgument, match="different streams"):
        a.add(b)


def test_backend_variable_names_hip_only(monkeypatch):
    monkeypatch.setenv("MLX_RS_BACKEND", "metal")
    with default_stream_scope(None):
        with pytest.raises(abi.BackendUnavailable, match="hip"):
            T.default_stream()


def _mha_params(d_model, n_heads, seed):
    w = {k: synth.normal(seed + i, (d_model, d_model), 0.0, 0.1) for i, k in enumerate(("wq", "wk", "wv", "wo"))}
    return w


def _mha(w, n_heads, bias=None):
    lin = {k: nn.Linear(Tensor.from_f32(v, v.shape),
                        None if bias is None else Tensor.from_f32(bias[k], bias[k].shape)) for k, v in w.items()}
    return nn.MultiHeadAttention(lin["wq"], lin["wk"], lin["wv"], lin["wo"], n_heads)


def _mha_f64(x, w, n_heads, bias=None):
    seq, d = x.shape
    dh = d // n_heads
    x = x.astype(np.float64)
    proj = {k: x @ w[k].astype(np.float64).T + (0 if bias is None else bias[k]) for k in ("wq", "wk", "wv")}
    outs = []
    for h in range(n_heads):
        q, k, v = (proj[n][:, h * dh:(h + 1) * dh] for n in ("wq", "wk", "wv"))
        s = (q @ k.T) * (1.0 / math.sqrt(dh))
        s[np.triu_indices(seq, 1)] = -1e9
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        outs.append(p @ v)
    o = np.concatenate(outs, 1)
    return o @ w["wo"].astype(np.float64).T + (0 if bias is None else bias["wo"])


@pytest.mark.parametrize("seq,d,h", [(2, 4, 2), (9, 12, 3), (33, 64, 4)])
def test_mha_forward_causal_on_oracle_against_f64(seq, d, h):
    w = _mha_params(d, h, 700 + d)
    bias = {k: synth.normal(800 + i, (d,), 0.0, 0.1) for i, k in enumerate(w)}
    x = synth.normal(900 + seq, (seq, d))
    with default_stream_scope(OracleStream()):
        y = _mha(w, h, bias).forward_causal(Tensor.from_f32(x, x.shape)).to_numpy()
    ref = _mha_f64(x, w, h, bias)
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5)


def test_mha_reference_case_runs():
    # crates/mlx-nn/src/lib.rs:185-211: 2 heads, [2, 4], all projections share
    # one weight; the reference checks the shape and length only.
    wq = np.array([[0.1 * (i + j) for j in range(4)] for i in range(4)], np.float32)
    w = {"wq": wq, "wk": wq, "wv": wq, "wo": wq}
    x = np.array([[1, 0, 0, 0], [0, 1, 0, 0]], np.float32)
    with default_stream_scope(OracleStream()):
        y = _mha(w, 2).forward_causal(Tensor.from_f32(x, (2, 4))).to_numpy()
    assert y.shape == (2, 4)
    np.testing.assert_allclose(y, _mha_f64(x, w, 2), rtol=1e-5, atol=1e-6)


# ── GPU: the default stream is a HipStream ────────────────────────────────

def _hip():
    from oxidizedmlx_amd.backend import HipStream
    return HipStream()


def _default_grad(make, f, x_data, shape):
    with default_stream_scope(make()):
        x = Tensor.from_f32(x_data, shape)
        return grad(lambda t: f(t, lambda d, sh: Tensor.from_f32(d, sh)), x).to_numpy().reshape(-1)


def _default_scalar(make, f, x_data, shape):
    with default_stream_scope(make()):
        return float(f(Tensor.from_f32(x_data, shape), lambda d, sh: Tensor.from_f32(d, sh))
                     .to_numpy().reshape(-1)[0])


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
@pytest.mark.parametrize("x_data,shape,f,expected,tol", REFERENCE_TESTS)
def test_reference_autograd_on_default_hip_stream(x_data, shape, f, expected, tol):
    g = _default_grad(_hip, f, x_data, shape)
    if tol == EXACT:
        np.testing.assert_array_equal(g, np.asarray(expected, np.float32))
        return
    if expected is None:
        # Central differences (lib.rs:159-177) through the oracle as default.
        x = np.asarray(x_data, np.float32)
        want = np.zeros(x.size)
        for i in range(x.size):
            xp, xm = x.copy(), x.copy()
            xp[i] += np.float32(1e-3)
            xm[i] -= np.float32(1e-3)
            want[i] = (np.float32(_default_scalar(OracleStream, f, xp, shape))
                       - np.float32(_default_scalar(OracleStream, f, xm, shape))) / np.float32(2e-3)
    else:
        want = np.asarray(expected, np.float64)
    assert np.all(np.abs(g - want) <= tol + tol * np.abs(want)), f"{g} vs {want}"
    # The oracle's own autograd on its default stream agrees too.
    np.testing.assert_allclose(g, _default_grad(OracleStream, f, x_data, shape), rtol=1e-4, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip")
@pytest.mark.parametrize("seq,d,h", [(2, 4, 2), (9, 12, 3), (33, 64, 4), (64, 256, 4), (128, 512, 8)])
def test_mha_forward_causal_hip_default_against_oracle(seq, d, h):
    # The reference's per-head Narrow -> Attention -> Concatenate -> Linear
    # graph run whole on the HIP default stream (CSE, fusion and the fused
    # attention kernel for head dims 16..128) against the same graph on the
    # oracle.
    w = _mha_params(d, h, 700 + d)
    bias = {k: synth.normal(800 + i, (d,), 0.0, 0.1) for i, k in enumerate(w)}
    x = synth.normal(900 + seq, (seq, d))
    out = {}
    for name, make in (("hip", _hip), ("oracle", OracleStream)):
        with default_stream_scope(make()):
            out[name] = _mha(w, h, bias).forward_causal(Tensor.from_f32(x, x.shape)).to_numpy()
    print(f"MHA seq={seq} d={d} h={h}", flush=True)
    # Both sides round through two K = d projections and the attention; the
    # tolerance scales with the output (1e-5 of its largest magnitude), and
    # against float64 the HIP graph must be as accurate as the oracle's own
    # f32 arithmetic (within 3x its error plus 1e-7 of the scale). A wrong
    # head order, mask or projection moves outputs by O(scale).
    scale = float(np.abs(out["oracle"]).max())
    assert_allclose(out["hip"], out["oracle"], 1e-5 * max(1.0, scale), 1e-4,
                    f"MHA forward_causal [{seq}, {d}] {h} heads")
    ref = _mha_f64(x, w, h, bias)
    e_hip = float(np.abs(out["hip"] - ref).max())
    e_cpu = float(np.abs(out["oracle"] - ref).max())
    print(f"  vs float64: hip {e_hip:.3e}, oracle {e_cpu:.3e} (scale {scale:.3f})", flush=True)
    assert e_hip <= 3 * e_cpu + 1e-7 * scale
