"""Prefill and decode behaviour after the reference's
crates/mlx-conformance/tests/ttft_behavior.rs: the same deterministic inputs,
graphs and checks (finite outputs, the prefill within 10 s, decode time per
step growing less than 10x from the first quarter of the loop to the last),
plus parity of every output with the CPU oracle's stream on the same graph
(atol 1e-5, rtol 1e-4: matmul, LayerNorm and attention chains in f32)."""
import time

import numpy as np
import pytest

from oxidizedmlx_amd.opkind import OpKind, meta
from parity import assert_allclose, cpu_stream, hip_stream

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip", "oracle_lib")]


def pattern(n, mod, off, scale):
    return ((np.arange(n) % mod).astype(np.float32) - off) * np.float32(scale)


def prefill(s):
    """ttft_prefill_matmul_dominates (ttft_behavior.rs:17-97)."""
    seq, dim, ff = 64, 32, 64
    c = lambda data, shape: s.add_constant(data, meta(shape))  # noqa: E731
    x = c(pattern(seq * dim, 17, 8, 0.05), [seq, dim])
    wq = c(pattern(dim * dim, 13, 6, 0.02), [dim, dim])
    wk = c(pattern(dim * dim, 11, 5, 0.02), [dim, dim])
    wv = c(pattern(dim * dim, 7, 3, 0.03), [dim, dim])
    w1 = c(pattern(dim * ff, 9, 4, 0.01), [dim, ff])
    w2 = c(pattern(ff * dim, 5, 2, 0.01), [ff, dim])
    sd, sf = meta([seq, dim]), meta([seq, ff])
    normed = s.add_op(OpKind.LayerNorm(1e-5), [x], sd)
    q, k, v = (s.add_op(OpKind.MatMul, [normed, w], sd) for w in (wq, wk, wv))
    attn = s.add_op(OpKind.Attention(1.0 / np.sqrt(dim), True), [q, k, v], sd)
    ffn = s.add_op(OpKind.LayerNorm(1e-5), [attn], sd)
    up = s.add_op(OpKind.MatMul, [ffn, w1], sf)
    act = s.add_op(OpKind.Silu, [up], sf)
    return s.add_op(OpKind.MatMul, [act, w2], sd)


def test_prefill_block():
    cpu, hip = cpu_stream(), hip_stream()
    c_out, h_out = prefill(cpu), prefill(hip)
    cpu.eval(c_out)
    t0 = time.perf_counter()
    hip.eval(h_out)
    h = hip.get_buffer(h_out)
    elapsed = time.perf_counter() - t0
    assert h.size == 64 * 32 and np.all(np.isfinite(h))
    assert elapsed < 10.0, f"prefill took {elapsed:.3f} s"
    assert_allclose(h, cpu.get_buffer(c_out), 1e-5, 1e-4, "prefill block")


def test_decode_loop_incremental_attention():
    """decode_loop_incremental_attention (ttft_behavior.rs:100-216): one new
    token per step, its K/V rows appended to a host-side cache, attention of
    its query over the whole cache."""
    dim, steps, prompt = 16, 32, 4
    wq, wk, wv = pattern(dim * dim, 7, 3, 0.05), pattern(dim * dim, 11, 5, 0.03), pattern(dim * dim, 5, 2, 0.04)
    kv = {"cpu": [pattern(prompt * dim, 13, 6, 0.02), pattern(prompt * dim, 9, 4, 0.03)]}
    kv["hip"] = [a.copy() for a in kv["cpu"]]
    streams = {"cpu": cpu_stream(), "hip": hip_stream()}
    w = {name: [s.add_constant(m, meta([dim, dim])) for m in (wq, wk, wv)] for name, s in streams.items()}
    scale = 1.0 / np.sqrt(dim)
    times = []
    for step in range(steps):
        token = ((np.arange(dim) + step * dim) % 11).astype(np.float32) * np.float32(0.1)
        outs = {}
        for name, s in streams.items():
            t0 = time.perf_counter()
            x = s.add_constant(token, meta([1, dim]))
            q, k, v = (s.add_op(OpKind.MatMul, [x, wm], meta([1, dim])) for wm in w[name])
            for node in (k, v):
                s.eval(node)
            kv[name][0] = np.concatenate([kv[name][0], s.get_buffer(k)])
            kv[name][1] = np.concatenate([kv[name][1], s.get_buffer(v)])
            n = kv[name][0].size // dim
            kf = s.add_constant(kv[name][0], meta([n, dim]))
            vf = s.add_constant(kv[name][1], meta([n, dim]))
            o = s.add_op(OpKind.Attention(scale, False), [q, kf, vf], meta([1, dim]))
            s.eval(o)
            outs[name] = s.get_buffer(o)
            if name == "hip":
                times.append(time.perf_counter() - t0)
        assert outs["hip"].size == dim and np.all(np.isfinite(outs["hip"])), step
        assert_allclose(outs["hip"], outs["cpu"], 1e-5, 1e-4, f"decode step {step}")
    assert sum(times) < 30.0
    q1, q4 = np.mean(times[: steps // 4]), np.mean(times[3 * steps // 4:])
    print(f"decode step time: first quarter {q1 * 1e6:.0f} us, last quarter {q4 * 1e6:.0f} us", flush=True)
    assert q4 / q1 < 10.0
