"""Fused attention (kernels/attention.hip) against the oracle's cpu_attention
(crates/mlx-core/src/cpu_kernels.rs:738-812), through the Stream's Attention
op and the batched mlxhip_attention entry point.

Tolerance: |gpu - cpu| <= 2e-6 * max|V| + 1e-5 * |cpu|. The output is a
convex combination of V rows; the GPU sums the score and P·V products in MFMA
order instead of the reference's sequential order, takes exp on the device,
and normalises with a running max (rescaling by exp(m_old - m_new) when a key
tile raises it) and one division per output instead of the reference's
whole-row max and per-probability division."""
import math

import numpy as np
import pytest

from oracle.cpu_ref import CpuRefBackend
from oxidizedmlx_amd import abi, synth
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd.opkind import NodeInput, OpKind, meta
from parity import assert_allclose, run_parity

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip", "oracle_lib")]


def qkv(tq, tk, dh, seed, batch=None):
    pre = (batch,) if batch else ()
    return (synth.normal(seed, pre + (tq, dh)), synth.normal(seed + 1, pre + (tk, dh)),
            synth.normal(seed + 2, pre + (tk, dh)))


def cpu_attention(q, k, v, scale, causal):
    tq, dh = q.shape
    return CpuRefBackend().eval_node(OpKind.Attention(scale, causal),
                                     [NodeInput(q.ravel(), q.shape), NodeInput(k.ravel(), k.shape),
                                      NodeInput(v.ravel(), v.shape)], meta([tq, dh])).reshape(tq, dh)


@pytest.mark.parametrize("tq,tk,dh,causal", [
    (1, 17, 64, False),      # one decode query over a cache
    (64, 64, 64, True),
    (100, 77, 32, True),     # tq != tk, partial query block and key tile
    (77, 100, 32, True),
    (512, 512, 64, True),    # one head of config 4
    (33, 300, 128, False),
    (5, 2000, 16, True),
    (3, 2540, 32, False),
    (70, 5000, 64, False),   # long key rows, streamed tile by tile
    (200, 3000, 128, True),
    (16, 16, 16, False),
    (1, 1, 32, True),        # a single key
    (129, 129, 64, True),    # one row past two full query blocks
    (40, 24, 48, True),      # head dim without a fused kernel: GEMM + softmax + GEMM
])
def test_attention_op_matches_oracle(tq, tk, dh, causal):
    print(f"attention tq={tq} tk={tk} dh={dh} causal={causal}", flush=True)
    q, k, v = qkv(tq, tk, dh, 7 * tq + tk + dh)
    scale = 1.0 / math.sqrt(dh)

    def g(s):
        nq = s.add_constant(q, meta([tq, dh]))
        nk = s.add_constant(k, meta([tk, dh]))
        nv = s.add_constant(v, meta([tk, dh]))
        return s.add_op(OpKind.Attention(scale, causal), [nq, nk, nv], meta([tq, dh]))

    run_parity(g, 2e-6 * float(np.abs(v).max()), 1e-5, f"Attention {tq}x{tk}x{dh}")


def test_growing_scores_rescale_exactly():
    """Scores that grow along the keys raise the running max in every key
    tile; the rescaled result still matches the oracle. Causal and not."""
    tq, tk, dh = 64, 256, 32
    q = np.ones((tq, dh), np.float32) * 0.05
    k = (np.arange(tk, dtype=np.float32)[:, None] / 8.0 * np.ones((1, dh), np.float32)).astype(np.float32)
    v = synth.normal(11, (tk, dh))
    for causal in (False, True):
        s = hb.HipStream()
        nq, nk, nv = (s.add_constant(a, meta(list(a.shape))) for a in (q, k, v))
        y = s.add_op(OpKind.Attention(1.0, causal), [nq, nk, nv], meta([tq, dh]))
        s.eval(y)
        out = s.get_buffer(y).reshape(tq, dh)
        assert_allclose(out, cpu_attention(q, k, v, 1.0, causal), 2e-6 * float(np.abs(v).max()), 1e-5,
                        f"growing scores causal={causal}")


def test_attention_reference_known_answer():
    """Causal row 0 attends to key 0 only: O[0] = V[0] exactly; with equal
    keys every visible key gets the same weight."""
    tq = tk = 32
    dh = 16
    q = synth.normal(1, (tq, dh))
    k = np.tile(synth.normal(2, (1, dh)), (tk, 1))
    v = synth.normal(3, (tk, dh))
    s = hb.HipStream()
    nq, nk, nv = (s.add_constant(a, meta(list(a.shape))) for a in (q, k, v))
    y = s.add_op(OpKind.Attention(0.25, True), [nq, nk, nv], meta([tq, dh]))
    s.eval(y)
    out = s.get_buffer(y).reshape(tq, dh)
    np.testing.assert_array_equal(out[0], v[0])
    ref = np.cumsum(v.astype(np.float64), axis=0) / np.arange(1, tk + 1)[:, None]
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("batch,t,dh,causal", [(6, 128, 64, True), (3, 50, 32, False), (64, 512, 64, True)])
def test_batched_entry_point(batch, t, dh, causal):
    """mlxhip_attention over packed heads equals the oracle head by head."""
    q, k, v = qkv(t, t, dh, 100 + batch, batch=batch)
    dq, dk, dv = (hb.DeviceBuffer.from_array(a) for a in (q, k, v))
    do = hb.DeviceBuffer(q.nbytes)
    scale = 1.0 / math.sqrt(dh)
    hb.attention(dq, dk, dv, do, batch, t, t, dh, scale, causal)
    hb.synchronize()
    out = do.download(np.float32, q.size).reshape(q.shape)
    heads = range(batch) if batch <= 8 else (0, 1, batch // 2, batch - 1)
    for b in heads:
        ref = cpu_attention(q[b], k[b], v[b], scale, causal)
        assert_allclose(out[b], ref, 2e-6 * float(np.abs(v[b]).max()), 1e-5, f"head {b}")


def test_entry_point_errors():
    q = hb.DeviceBuffer(64 * 48 * 4)
    with pytest.raises(abi.InvalidArgument):
        hb.attention(q, q, q, q, 1, 64, 16, 48, 1.0, False)          # no fused kernel for dh 48
    with pytest.raises(abi.InvalidArgument):
        hb.attention(q, q, q, q, 1, 4, 0, 64, 1.0, False)            # no keys
    L = abi.load_library()
    assert L.mlxhip_attention(None, None, None, None, 1, 4, 4, 16, 1.0, 0, None) == abi.ERR_NULL_PTR
    hb.attention(q, q, q, q, 0, 4, 4, 16, 1.0, False)                # empty batch: nothing to do


@pytest.mark.parametrize("misalign", ["q", "out"])
def test_misaligned_operands_take_the_unfused_path(misalign):
    """The fused kernel needs 16-byte aligned Q, K, V and O rows; an Attention
    node on operands offset by one float (mlxhip_eval_node_dev) runs the GEMM
    + scaled-masked softmax + GEMM sequence and still matches the oracle."""
    tq, tk, dh = 40, 72, 64
    q, k, v = qkv(tq, tk, dh, 31)
    scale = 1.0 / math.sqrt(dh)
    bufs = {}
    for name, a in (("q", q), ("k", k), ("v", v)):
        off = 1 if name == misalign else 0
        b = hb.DeviceBuffer((a.size + 4) * 4)
        b.upload(np.concatenate([np.zeros(off, np.float32), a.ravel(), np.zeros(4 - off, np.float32)]))
        bufs[name] = (b, off)
    out_off = 1 if misalign == "out" else 0
    out = hb.DeviceBuffer((tq * dh + 4) * 4)
    ins = [(bufs[n][0].ptr + 4 * bufs[n][1], a.shape) for n, a in (("q", q), ("k", k), ("v", v))]
    hb.eval_node_dev(OpKind.Attention(scale, True), ins, meta([tq, dh]), out.ptr + 4 * out_off)
    hb.synchronize()
    got = out.download(np.float32, tq * dh, offset=4 * out_off).reshape(tq, dh)
    assert_allclose(got, cpu_attention(q, k, v, scale, True), 2e-6 * float(np.abs(v).max()), 1e-5,
                    f"misaligned {misalign}")


def f64_attention(q, k, v, scale, causal):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    sc = q @ k.T * scale
    if causal:
        sc = np.where(np.arange(k.shape[0])[None, :] > np.arange(q.shape[0])[:, None], -np.inf, sc)
    e = np.exp(sc - sc.max(1, keepdims=True))
    return (e / e.sum(1, keepdims=True)) @ v


@pytest.mark.parametrize("dh,causal", [(128, True), (64, False), (32, True)])
def test_large_scores(dh, causal):
    """Q and K of N(0, 3^2) put scores in the tens. There the reference's own
    f32 rounding of a score (about |s| * 2^-24 per term) moves the output by
    ~1e-5, as much as the usual tolerance, so both are held against float64:
    the GPU's largest error must stay within twice the reference's (plus
    2e-6 * max|V|). A split that lost bits would be off by ~1e-3."""
    tq, tk = 96, 300
    q, k, v = qkv(tq, tk, dh, 53)
    q, k = (q * 3.0).astype(np.float32), (k * 3.0).astype(np.float32)
    scale = 1.0 / math.sqrt(dh)
    s = hb.HipStream()
    nq, nk, nv = (s.add_constant(a, meta(list(a.shape))) for a in (q, k, v))
    y = s.add_op(OpKind.Attention(scale, causal), [nq, nk, nv], meta([tq, dh]))
    s.eval(y)
    got = s.get_buffer(y).reshape(tq, dh).astype(np.float64)
    exact = f64_attention(q, k, v, scale, causal)
    ref_err = float(np.abs(cpu_attention(q, k, v, scale, causal) - exact).max())
    gpu_err = float(np.abs(got - exact).max())
    print(f"dh={dh} causal={causal}: max |gpu - f64| {gpu_err:.3e}, max |oracle - f64| {ref_err:.3e}")
    assert gpu_err <= 2.0 * ref_err + 2e-6 * float(np.abs(v).max())
