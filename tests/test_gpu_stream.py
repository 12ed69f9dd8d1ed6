"""HipStream (Stream + Graph bound to mlx-hip, HBM-resident buffers).

Restates the reference's Stream tests (crates/mlx-core/src/backend.rs:202-449)
and checks the scheduler's look-ahead fusion against the unfused graph and
the CPU oracle."""
import threading

import numpy as np
import pytest

from oracle import cpu_ref
from oxidizedmlx_amd import abi
from oxidizedmlx_amd import synth
from oxidizedmlx_amd.backend import HipBackend, HipStream
from oxidizedmlx_amd.opkind import NodeInput, OpKind, meta
from parity import assert_allclose, cpu_stream, gen_data

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip", "oracle_lib")]

M2 = meta([2])


def test_stream_constant_and_add():
    s = HipStream()
    a = s.add_constant([1.0, 2.0, 3.0], meta([3]))
    s.eval(a)
    np.testing.assert_array_equal(s.get_buffer(a), [1, 2, 3])
    a = s.add_constant([1.0, 2.0], M2)
    b = s.add_constant([3.0, 4.0], M2)
    c = s.add_op(OpKind.Add, [a, b], M2)
    s.eval(c)
    np.testing.assert_array_equal(s.get_buffer(c), [4, 6])


@pytest.mark.parametrize("fusion", [False, True])
def test_memoization_repeated_eval(fusion):
    s = HipStream(fusion=fusion)
    a, b = s.add_constant([1.0, 2.0], M2), s.add_constant([3.0, 4.0], M2)
    c = s.add_op(OpKind.Add, [a, b], M2)
    s.eval(c)
    n = s.eval_count()
    assert n > 0
    s.eval(c)
    assert s.eval_count() == n


def test_memoization_shared_subgraph():
    s = HipStream(fusion=False)
    a, b = s.add_constant([1.0, 2.0], M2), s.add_constant([3.0, 4.0], M2)
    c = s.add_op(OpKind.Add, [a, b], M2)
    d = s.add_op(OpKind.Mul, [c, c], M2)
    s.eval(d)
    n = s.eval_count()
    s.eval(d)
    s.eval(c)
    assert s.eval_count() == n
    np.testing.assert_array_equal(s.get_buffer(d), [16, 36])


@pytest.mark.parametrize("fusion", [False, True])
def test_memoization_diamond(fusion):
    s = HipStream(fusion=fusion)
    a = s.add_constant([1.0, 2.0], M2)
    b = s.add_op(OpKind.Add, [a, a], M2)
    c = s.add_op(OpKind.Mul, [a, a], M2)
    d = s.add_op(OpKind.Add, [b, c], M2)
    s.eval(d)
    assert s.eval_count() == 3
    s.eval(d)
    assert s.eval_count() == 3
    np.testing.assert_array_equal(s.get_buffer(d), [3, 8])


def test_cache_len_updates():
    s = HipStream(fusion=False)
    assert s.cache_len() == 0
    a, b = s.add_constant([1.0, 2.0], M2), s.add_constant([3.0, 4.0], M2)
    assert s.cache_len() == 2
    c = s.add_op(OpKind.Add, [a, b], M2)
    s.eval(c)
    assert s.cache_len() == 3


def test_cse_dedupes_ops_not_constants():
    s = HipStream()
    a, b = s.add_constant([1.0, 2.0], M2), s.add_constant([1.0, 2.0], M2)
    assert a != b  # constants are never deduplicated (graph.rs:495-500)
    assert s.add_op(OpKind.Add, [a, b], M2) == s.add_op(OpKind.Add, [b, a], M2)  # commutation
    assert s.add_op(OpKind.Sub, [a, b], M2) != s.add_op(OpKind.Sub, [b, a], M2)
    assert s.add_op(OpKind.Softmax(-1), [a], M2) != s.add_op(OpKind.Softmax(0), [a], M2)


def build_chain(s, x, w, b, m):
    nx, nw, nb = s.add_constant(x, m), s.add_constant(w, m), s.add_constant(b, m)
    xw = s.add_op(OpKind.Mul, [nx, nw], m)
    z = s.add_op(OpKind.Add, [xw, nb], m)
    return s.add_op(OpKind.Silu, [z], m)


def test_cfg2_fused_chain_full_size():
    # Config 2 chain y = SiLU(x*w + b), [4096, 4096], x ~ N(0, 2^2), w, b ~ U(-1, 1).
    shape = (4096, 4096)
    x = synth.normal(0x5EED0003, shape, 0.0, 2.0)
    w = synth.uniform(0x5EED0004, shape, -1.0, 1.0)
    b = synth.uniform(0x5EED0005, shape, -1.0, 1.0)
    m = meta(shape)
    c = cpu_stream()
    yc = build_chain(c, x, w, b, m)
    c.eval(yc)
    ref = c.get_buffer(yc)
    s = HipStream(fusion=True)
    y = build_chain(s, x, w, b, m)
    s.eval(y)
    assert s.launch_count() == 1 and s.eval_count() == 3
    assert_allclose(s.get_buffer(y), ref, 1e-6, 1e-6, "SiLU(x*w+b) fused 4096x4096")
    u = HipStream(fusion=False)
    yu = build_chain(u, x, w, b, m)
    u.eval(yu)
    assert u.launch_count() == 3 and u.eval_count() == 3
    # Fused and unfused kernels do identical f32 arithmetic in the same order.
    np.testing.assert_array_equal(u.get_buffer(yu), s.get_buffer(y))


def test_fusion_long_chain_and_reversed_operands():
    n = 10007  # not a multiple of 4: exercises the scalar tail
    xs = [gen_data(n, 200 + i) for i in range(6)]
    pos = np.abs(gen_data(n, 300)) + np.float32(0.5)

    def g(s):
        m = meta([n])
        c = [s.add_constant(v, m) for v in xs]
        p = s.add_constant(pos, m)
        t = s.add_op(OpKind.Mul, [c[0], c[1]], m)
        t = s.add_op(OpKind.Sub, [c[2], t], m)       # acc on the right: RSUB
        t = s.add_op(OpKind.Exp, [t], m)
        t = s.add_op(OpKind.Div, [p, t], m)          # RDIV
        t = s.add_op(OpKind.Gelu, [t], m)
        t = s.add_op(OpKind.Add, [c[3], t], m)
        t = s.add_op(OpKind.Neg, [t], m)
        t = s.add_op(OpKind.SiluVjp, [c[4], t], m)   # dy = c4, x = t
        return s.add_op(OpKind.Mul, [t, c[5]], m)

    cs = cpu_stream()
    out_c = g(cs)
    cs.eval(out_c)
    hs = HipStream(fusion=True)
    out_h = g(hs)
    hs.eval(out_h)
    assert hs.launch_count() == 1
    assert hs.eval_count() == cs.eval_calls == 9
    assert_allclose(hs.get_buffer(out_h), cs.get_buffer(out_c), 1e-5, 1e-5, "long fused chain")


def test_fusion_respects_shared_intermediates():
    n = 4096
    x, y = gen_data(n, 1), gen_data(n, 2)
    s = HipStream(fusion=True)
    m = meta([n])
    a, b = s.add_constant(x, m), s.add_constant(y, m)
    t = s.add_op(OpKind.Mul, [a, b], m)  # consumed twice: must be materialised
    u = s.add_op(OpKind.Exp, [t], m)
    v = s.add_op(OpKind.Add, [t, u], m)
    s.eval(v)
    np.testing.assert_allclose(s.get_buffer(t), x * y, rtol=0, atol=0)
    ref = (x * y) + np.exp(x * y)
    np.testing.assert_allclose(s.get_buffer(v), ref, rtol=1e-6, atol=1e-6)


def test_transpose_folded_into_gemm():
    # Linear: x . W^T (crates/mlx-nn/src/linear.rs:34-43) and autograd's
    # g . B^T / A^T . g (crates/mlx-autograd/src/vjp.rs:71-80).
    T, I, O = 96, 80, 72
    x, W = gen_data(T * I, 5).reshape(T, I), gen_data(O * I, 6).reshape(O, I)

    def g(s):
        nx = s.add_constant(x, meta([T, I]))
        nw = s.add_constant(W, meta([O, I]))
        wt = s.add_op(OpKind.Transpose(None), [nw], meta([I, O]))
        y = s.add_op(OpKind.MatMul, [nx, wt], meta([T, O]))
        xt = s.add_op(OpKind.Transpose(None), [nx], meta([I, T]))
        return s.add_op(OpKind.MatMul, [xt, y], meta([I, O]))

    cs = cpu_stream()
    oc = g(cs)
    cs.eval(oc)
    hs = HipStream(fusion=True)
    oh = g(hs)
    hs.eval(oh)
    assert hs.launch_count() == 2 and hs.eval_count() == 4
    assert_allclose(hs.get_buffer(oh), cs.get_buffer(oc), 1e-4, 1e-4, "folded transposes")


def test_stream_errors_match_reference():
    s = HipStream()
    a = s.add_constant(np.ones(6, np.float32), meta([2, 3]))
    b = s.add_constant(np.ones(8, np.float32), meta([4, 2]))
    mm = s.add_op(OpKind.MatMul, [a, b], meta([2, 2]))
    with pytest.raises(abi.ShapeMismatch) as ei:
        s.eval(mm)
    # MlxError::ShapeMismatch{expected: [m, k], got: [k2, n]} (cpu_kernels.rs:212-217)
    assert (ei.value.expected, ei.value.got) == ([2, 3], [4, 2])
    v = s.add_constant(np.ones(3, np.float32), meta([3]))
    mm1 = s.add_op(OpKind.MatMul, [v, v], meta([1]))
    with pytest.raises(abi.InvalidArgument):
        s.eval(mm1)
    sm = s.add_op(OpKind.Softmax(5), [a], meta([2, 3]))
    with pytest.raises(abi.InvalidArgument):
        s.eval(sm)
    with pytest.raises(abi.InvalidArgument):
        s.add_op(OpKind.Add, [a, 12345], meta([2, 3]))
    # eval_node with Constant is rejected (cpu_kernels.rs:21-23)
    with pytest.raises(abi.InvalidArgument):
        HipBackend().eval_node(OpKind.Constant, [], meta([1]))


def test_eval_node_host_contract_matches_oracle():
    x = gen_data(64 * 96, 9)
    inp = [NodeInput(x, (64, 96))]
    for op in [OpKind.Softmax(-1), OpKind.LayerNorm(1e-5), OpKind.RmsNorm(1e-5), OpKind.Silu,
               OpKind.Gelu]:
        h = HipBackend().eval_node(op, inp, meta([64, 96]))
        c = cpu_ref.CpuRefBackend().eval_node(op, inp, meta([64, 96]))
        assert_allclose(h, c, 1e-6, 1e-5, repr(op))
    # bf16/f16-tagged MatMul: the tag is logical only (tensor.rs:105-125); the
    # stored f32 values are multiplied unrounded, as the oracle does.
    a, b = gen_data(33 * 40, 10), gen_data(40 * 21, 11)
    for dt in (abi.BF16, abi.F16):
        inp = [NodeInput(a, (33, 40), dt), NodeInput(b, (40, 21), dt)]
        h = HipBackend().eval_node(OpKind.MatMul, inp, meta([33, 21], dt))
        c = cpu_ref.CpuRefBackend().eval_node(OpKind.MatMul, inp, meta([33, 21], dt))
        assert_allclose(h, c, 1e-6 * np.sqrt(40), 1e-5, f"MatMul tagged {dt}")
        # Rounding the operands to 16 bits would move results by ~1e-3.
        r16 = synth.round_bf16(a).reshape(33, 40).astype(np.float64) @ synth.round_bf16(b).reshape(40, 21)
        if dt == abi.BF16:
            assert np.abs(h.reshape(33, 21) - r16).max() > 1e-4


def test_empty_tensors():
    h = HipBackend().eval_node(OpKind.Add, [NodeInput(np.zeros(0, np.float32), (0,)),
                                           NodeInput(np.zeros(0, np.float32), (0,))], meta([0]))
    assert h.size == 0


def test_concurrent_streams_deterministic():
    # crates/mlx-core/tests/concurrency_stress.rs:16-101: threads evaluating the
    # same graph must get bit-identical results.
    x = gen_data(256 * 512, 77)
    results, errors = [None] * 8, []

    def work(i):
        try:
            s = HipStream()
            m = meta([256, 512])
            n = s.add_constant(x, m)
            y = s.add_op(OpKind.LayerNorm(1e-5), [n], m)
            z = s.add_op(OpKind.Silu, [y], m)
            s.eval(z)
            results[i] = s.get_buffer(z)
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    ts = [threading.Thread(target=work, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
    for r in results[1:]:
        np.testing.assert_array_equal(r, results[0])


def test_shared_stream_from_threads():
    s = HipStream()
    m = meta([1024])
    a = s.add_constant(gen_data(1024, 1), m)
    b = s.add_constant(gen_data(1024, 2), m)
    c = s.add_op(OpKind.Mul, [a, b], m)
    outs, errs = [], []

    def work():
        try:
            s.eval(c)
            outs.append(s.get_buffer(c))
        except Exception as e:  # noqa: BLE001
            errs.append(e)

    ts = [threading.Thread(target=work) for _ in range(16)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs
    for o in outs:
        np.testing.assert_array_equal(o, outs[0])
    assert s.eval_count() == 1


@pytest.mark.parametrize("fusion", [False, True])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_batched_matmul_with_transposed_operands(fusion, ta, tb):
    # Rank-3 MatMul ([B,M,K] @ [B,K,N]) whose operands are Transpose [0,2,1]
    # nodes: with fusion the transposes fold into the batched GEMM's operand
    # layout instead of being materialised. Checked against the oracle.
    bt, m, k, n = 3, 37, 29, 41
    a0 = synth.normal(401, (bt, k, m) if ta else (bt, m, k))
    b0 = synth.normal(402, (bt, n, k) if tb else (bt, k, n))
    outs = []
    for s in (HipStream(fusion=fusion), cpu_ref_stream()):
        a = s.add_constant(a0, meta(a0.shape))
        b = s.add_constant(b0, meta(b0.shape))
        if ta:
            a = s.add_op(OpKind.Transpose((0, 2, 1)), [a], meta((bt, m, k)))
        if tb:
            b = s.add_op(OpKind.Transpose((0, 2, 1)), [b], meta((bt, k, n)))
        c = s.add_op(OpKind.MatMul, [a, b], meta((bt, m, n)))
        s.eval(c)
        outs.append(s.get_buffer(c))
    bound = 1e-6 * np.sqrt(k) * np.abs(a0).max() * np.abs(b0).max()
    assert_allclose(outs[0], outs[1], bound, 1e-5, "batched matmul")


def test_batched_matmul_rejects_mismatched_batch():
    s = HipStream()
    a = s.add_constant(np.zeros(2 * 3 * 4, np.float32), meta((2, 3, 4)))
    b = s.add_constant(np.zeros(3 * 4 * 5, np.float32), meta((3, 4, 5)))
    c = s.add_op(OpKind.MatMul, [a, b], meta((2, 3, 5)))
    with pytest.raises(abi.ShapeMismatch):
        s.eval(c)


def cpu_ref_stream():
    from oracle.graph import OracleStream
    return OracleStream()


def test_reshape_aliases_its_input():
    # A Reshape keeps the data: no kernel runs for it, and its value (and a
    # consumer's) is the input's.
    s = HipStream()
    x0 = synth.normal(501, (6, 8))
    x = s.add_constant(x0, meta((6, 8)))
    r = s.add_op(OpKind.Reshape((4, 12)), [x], meta((4, 12)))
    y = s.add_op(OpKind.Neg, [r], meta((4, 12)))
    before = s.launch_count()
    s.eval_many([r, y])
    assert s.launch_count() - before == 1  # the Neg only
    np.testing.assert_array_equal(s.get_buffer(r), x0.reshape(-1))
    np.testing.assert_array_equal(s.get_buffer(y), -x0.reshape(-1))


def _broadcast_graph(s, b, r, c):
    """y = ((x * bcast(scale)) + bcast(mask[r, c])) + bcast(bias[c]) with
    x [b, r, c]: the three broadcasts tile their sources."""
    x0 = synth.normal(511, (b, r, c))
    mask0 = synth.normal(512, (r, c))
    bias0 = synth.normal(513, (c,))
    full = meta((b, r, c))
    x = s.add_constant(x0, full)
    sc = s.add_op(OpKind.Broadcast((b, r, c)), [s.add_constant([0.125], meta(()))], full)
    mk = s.add_op(OpKind.Broadcast((b, r, c)), [s.add_constant(mask0, meta((r, c)))], full)
    bi = s.add_op(OpKind.Broadcast((b, r, c)), [s.add_constant(bias0, meta((c,)))], full)
    y = s.add_op(OpKind.Add, [s.add_op(OpKind.Add, [s.add_op(OpKind.Mul, [x, sc], full), mk], full), bi], full)
    return y, (x0 * np.float32(0.125) + mask0) + bias0


@pytest.mark.parametrize("shape", [(4, 16, 32), (3, 5, 7), (2, 64, 1)])
def test_broadcast_operands_read_in_place(shape):
    # Tiling broadcasts feeding elementwise nodes are read periodically by the
    # chain kernel; the result must equal the unfused graph bit for bit and
    # the oracle, and eval_count must not change.
    res, counts = [], []
    for fusion in (True, False):
        s = HipStream(fusion=fusion)
        y, want = _broadcast_graph(s, *shape)
        s.eval(y)
        res.append(s.get_buffer(y))
        counts.append(s.eval_count())
    np.testing.assert_array_equal(res[0], res[1])
    np.testing.assert_array_equal(res[0], want.reshape(-1))
    assert counts[0] == counts[1]
    o = cpu_ref_stream()
    y, _ = _broadcast_graph(o, *shape)
    o.eval(y)
    np.testing.assert_array_equal(res[0], o.get_buffer(y))


def test_broadcast_requested_later_is_materialised():
    s = HipStream()
    full = meta((3, 8))
    b = s.add_op(OpKind.Broadcast((3, 8)), [s.add_constant(np.arange(8, dtype=np.float32), meta((8,)))], full)
    x = s.add_constant(np.ones(24, np.float32), full)
    y = s.add_op(OpKind.Add, [x, b], full)
    s.eval(y)
    s.eval(b)  # not materialised by the first evaluation; must be now
    np.testing.assert_array_equal(s.get_buffer(b), np.tile(np.arange(8, dtype=np.float32), 3))
    np.testing.assert_array_equal(s.get_buffer(y), np.tile(np.arange(8, dtype=np.float32), 3) + 1)


@pytest.mark.parametrize("shape,axis", [((2048, 1024), 0), ((3, 1000, 7), 1), ((5, 37), 1), ((4096, 3), 0),
                                        ((3, 1300, 48), 1), ((2049, 16), 0), ((256, 4096), 0), ((777, 32), -2)])
@pytest.mark.parametrize("kind", ["sum", "mean", "max"])
def test_sum_axis_matches_sequential_fold_bitwise(shape, axis, kind):
    # Sum / Mean / Max over an axis fold each output in order (Sum from
    # -0.0), like the CPU (cpu_kernels.rs:166-195): bit-identical results,
    # with row counts that leave partial register batches.
    x0 = synth.normal(521, shape)
    ax = axis % len(shape)
    out_shape = tuple(d for i, d in enumerate(shape) if i != ax)
    op = {"sum": OpKind.Sum(axis), "mean": OpKind.Mean(axis), "max": OpKind.Max(axis)}[kind]
    res = []
    for s in (HipStream(), cpu_ref_stream()):
        x = s.add_constant(x0, meta(shape))
        y = s.add_op(op, [x], meta(out_shape))
        s.eval(y)
        res.append(s.get_buffer(y))
    np.testing.assert_array_equal(res[0], res[1])


@pytest.mark.parametrize("async_eval", [False, True])
def test_leaf_reductions_beside_other_work(async_eval):
    """Axis reductions over long axes that no node consumes (a block's bias
    gradients) run on the stream's second queue beside the other kernels:
    several of them, read right after the evaluation, equal the oracle bit
    for bit, and so does the work they overlapped."""
    x0, w0 = synth.normal(541, (1024, 256)), synth.normal(542, (256, 512))
    res = []
    for s in ((HipStream(async_eval=True) if async_eval else HipStream()), cpu_ref_stream()):
        x = s.add_constant(x0, meta((1024, 256)))
        w = s.add_constant(w0, meta((256, 512)))
        y = s.add_op(OpKind.MatMul, [x, w], meta((1024, 512)))
        outs = [y, s.add_op(OpKind.Sum(0), [y], meta((512,))), s.add_op(OpKind.Mean(0), [x], meta((256,))),
                s.add_op(OpKind.Max(-2), [y], meta((512,))), s.add_op(OpKind.Neg, [y], meta((1024, 512)))]
        s.eval_many(outs)
        res.append([s.get_buffer(o) for o in outs])
    for i, (a, b) in enumerate(zip(*res)):
        if i in (0, 4):
            assert_allclose(a, b, 1e-5 * float(np.abs(b).max()), 1e-5, f"output {i}")
        else:
            # the fold of the GPU's own product equals the oracle's fold of it
            src = res[0][0].reshape(1024, 512) if i != 2 else x0
            want = {1: np.add.accumulate(src, axis=0)[-1], 2: (np.add.accumulate(src, axis=0)[-1] / np.float32(1024)),
                    3: src.max(axis=0)}[i]
            np.testing.assert_array_equal(a, want.astype(np.float32), err_msg=f"output {i}")


@pytest.mark.parametrize("fusion", [False, True])
def test_transpose_rewrites_match_unfused(fusion):
    # transpose(transpose(W)) read by a MatMul folds to W itself; a Transpose
    # of a MatMul nothing else reads runs as one product with swapped
    # operands. Results must equal the oracle (and the unfused graph).
    x0, w0 = synth.normal(531, (40, 24)), synth.normal(532, (24, 24))
    g0 = synth.normal(533, (40, 24))
    res = []
    for s in (HipStream(fusion=fusion), cpu_ref_stream()):
        x = s.add_constant(x0, meta((40, 24)))
        w = s.add_constant(w0, meta((24, 24)))
        g = s.add_constant(g0, meta((40, 24)))
        wt = s.add_op(OpKind.Transpose(None), [w], meta((24, 24)))
        y = s.add_op(OpKind.MatMul, [x, wt], meta((40, 24)))                 # x W^T
        wtt = s.add_op(OpKind.Transpose(None), [wt], meta((24, 24)))
        dx = s.add_op(OpKind.MatMul, [g, wtt], meta((40, 24)))               # g W
        xt = s.add_op(OpKind.Transpose(None), [x], meta((24, 40)))
        dwt = s.add_op(OpKind.MatMul, [xt, g], meta((24, 24)))               # x^T g
        dw = s.add_op(OpKind.Transpose((1, 0)), [dwt], meta((24, 24)))      # (x^T g)^T
        s.eval_many([y, dx, dw])
        res.append([s.get_buffer(t) for t in (y, dx, dw)])
    for got, want in zip(*res):
        assert_allclose(got, want, 1e-5, 1e-5, "transpose rewrites")


def test_async_eval_stream_semantics():
    """mlxhip_stream_set_async: evaluations return before their kernels
    finish; a host constant added while kernels still run, a chain of
    evaluations that read each other's results, get_buffer (which waits),
    synchronize and turning the mode off all give the synchronous values."""
    rng = np.random.default_rng(21)
    a = rng.standard_normal((256, 384)).astype(np.float32)
    b = rng.standard_normal((384, 128)).astype(np.float32)
    c = rng.standard_normal((256, 128)).astype(np.float32)

    def run(asyn):
        s = HipStream(async_eval=asyn)
        ai = s.add_constant(a, meta([256, 384]))
        bi = s.add_constant(b, meta([384, 128]))
        mm = s.add_op(OpKind.MatMul, [ai, bi], meta([256, 128]))
        s.eval(mm)
        ci = s.add_constant(c, meta([256, 128]))  # copied while the GEMM may still run
        sm = s.add_op(OpKind.Softmax(1), [mm], meta([256, 128]))
        out = s.add_op(OpKind.Add, [sm, ci], meta([256, 128]))
        s.eval(out)
        second = s.add_op(OpKind.Mul, [out, mm], meta([256, 128]))
        s.eval_many([second])
        res = [s.get_buffer(n) for n in (mm, out, second)]
        if asyn:
            s.synchronize()
            s.set_async(False)
        s.close()
        return res

    for x, y in zip(run(False), run(True)):
        np.testing.assert_array_equal(x, y)


def test_constant_views_read_device_memory_in_place():
    """mlxhip_stream_add_constant_view: a node that reads caller-owned device
    memory without a copy gives the copied constant's results bit for bit,
    leaves the memory untouched through evaluation, clear and close, and
    rejects memory that is not 256-byte aligned."""
    rng = np.random.default_rng(3)
    a = rng.standard_normal((64, 96)).astype(np.float32)
    b = rng.standard_normal((96, 32)).astype(np.float32)
    from oxidizedmlx_amd.backend import DeviceBuffer
    A, B = DeviceBuffer.from_array(a), DeviceBuffer.from_array(b)

    def run(view):
        s = HipStream(async_eval=view)
        add = s.add_constant_view if view else s.add_constant_dev
        ai, bi = add(A.ptr, meta([64, 96])), add(B.ptr, meta([96, 32]))
        mm = s.add_op(OpKind.MatMul, [ai, bi], meta([64, 32]))
        sm = s.add_op(OpKind.Softmax(1), [mm], meta([64, 32]))
        s.eval(sm)
        out = s.get_buffer(sm)
        s.clear()
        s.close()
        return out

    np.testing.assert_array_equal(run(True), run(False))
    np.testing.assert_array_equal(A.download(), a.reshape(-1))
    np.testing.assert_array_equal(B.download(), b.reshape(-1))
    s = HipStream()
    with pytest.raises(abi.InvalidArgument, match="aligned"):
        s.add_constant_view(A.ptr + 4, meta([4]))
    s.close()


@pytest.mark.parametrize("fusion", [False, True])
def test_transpose_rewrites_across_evaluations(fusion):
    # The forward product is evaluated first (as grad does with the loss),
    # then the gradient products: transpose(transpose(W)) still folds to W
    # although the inner Transpose's other consumer ran in the earlier
    # evaluation, so the second evaluation runs its two products only.
    x0, w0 = synth.normal(541, (40, 24)), synth.normal(542, (24, 24))
    g0 = synth.normal(543, (40, 24))
    res, launches = [], []
    for s in (HipStream(fusion=fusion), cpu_ref_stream()):
        x = s.add_constant(x0, meta((40, 24)))
        w = s.add_constant(w0, meta((24, 24)))
        g = s.add_constant(g0, meta((40, 24)))
        wt = s.add_op(OpKind.Transpose(None), [w], meta((24, 24)))
        y = s.add_op(OpKind.MatMul, [x, wt], meta((40, 24)))                 # x W^T
        s.eval(y)
        wtt = s.add_op(OpKind.Transpose(None), [wt], meta((24, 24)))
        dx = s.add_op(OpKind.MatMul, [g, wtt], meta((40, 24)))               # g W
        xt = s.add_op(OpKind.Transpose(None), [x], meta((24, 40)))
        dw = s.add_op(OpKind.MatMul, [xt, g], meta((24, 24)))                # x^T g
        before = s.launch_count() if isinstance(s, HipStream) else 0
        s.eval_many([dx, dw])
        if isinstance(s, HipStream):
            launches.append(s.launch_count() - before)
        res.append([s.get_buffer(t) for t in (y, dx, dw)])
    for got, want in zip(*res):
        assert_allclose(got, want, 1e-5, 1e-5, "transpose rewrites across evaluations")
    if fusion:
        assert launches == [2]


def test_split_f32_planes_reused_across_evaluations_and_dropped_at_clear():
    # Products large enough for the split-f32 GEMM: W's planes, made by the
    # first evaluation, serve the second one's g W; after clear() a view
    # constant over the same device memory holding new values gets new
    # planes (every result against float64 with the f32 accumulation bound).
    from oxidizedmlx_amd.backend import DeviceBuffer
    from parity import gemm_full_check
    T, I, O = 1024, 2048, 1024
    x0, g0 = synth.normal(551, (T, I)), synth.normal(553, (T, O))
    wbuf = DeviceBuffer(O * I * 4)
    s = HipStream()
    for rnd, seed in enumerate((552, 554)):
        w0 = synth.normal(seed, (O, I))
        wbuf.upload(w0)
        x = s.add_constant(x0, meta((T, I)))
        w = s.add_constant_view(wbuf.ptr, meta((O, I)))
        wt = s.add_op(OpKind.Transpose(None), [w], meta((I, O)))
        y = s.add_op(OpKind.MatMul, [x, wt], meta((T, O)))                   # x W^T
        s.eval(y)
        g = s.add_constant(g0, meta((T, O)))
        dx = s.add_op(OpKind.MatMul, [g, w], meta((T, I)))                   # g W
        s.eval(dx)
        gemm_full_check(s.get_buffer(y).reshape(T, O), x0, w0.T, "f32", f"x W^T, round {rnd}")
        gemm_full_check(s.get_buffer(dx).reshape(T, I), g0, w0, "f32", f"g W, round {rnd}")
        s.clear()


@pytest.mark.parametrize("shared", ["A", "B", "none"])
def test_sibling_products_run_as_one_grouped_launch(shared):
    # Three products with one operand in common (x W_i^T, the Q/K/V
    # projections of one input; or dY_i^T X, sharing X) or none (dY_i W_i,
    # the products of the input's gradient) at a size that takes
    # the split-f32 path run as one grouped launch; every output against
    # float64 with the f32 accumulation bound, and against the unfused graph
    # (which runs them one by one) within the same bound.
    from parity import gemm_full_check
    # Shapes whose three products together fill the chip unsplit (384 tiles
    # of 128x128), so the grouped launch runs.
    T, I, O = 1024, 2048, (2048 if shared == "A" else 1024)
    x0 = synth.normal(561, (T, I))
    ws0 = [synth.normal(562 + i, (O, I)) for i in range(3)]
    res = {}
    for fusion in (True, False):
        s = HipStream(fusion=fusion)
        if shared == "A":
            x = s.add_constant(x0, meta((T, I)))
            outs = []
            for w0 in ws0:
                w = s.add_constant(w0, meta((O, I)))
                wt = s.add_op(OpKind.Transpose(None), [w], meta((I, O)))
                outs.append(s.add_op(OpKind.MatMul, [x, wt], meta((T, O))))          # x W_i^T
            refs = [(x0, w0.T) for w0 in ws0]
        elif shared == "none":
            # dY_i W_i: no operand in common (the input gradient's products).
            outs = []
            for i, w0 in enumerate(ws0):
                dy = s.add_constant(synth.normal(571 + i, (T, O)), meta((T, O)))
                w = s.add_constant(w0, meta((O, I)))
                outs.append(s.add_op(OpKind.MatMul, [dy, w], meta((T, I))))
            refs = [(synth.normal(571 + i, (T, O)), w0) for i, w0 in enumerate(ws0)]
        else:
            x = s.add_constant(x0, meta((T, I)))
            outs = []
            for w0 in ws0:
                dy = s.add_constant(np.ascontiguousarray(w0[:, :T].T), meta((T, O)))
                dyt = s.add_op(OpKind.Transpose(None), [dy], meta((O, T)))
                outs.append(s.add_op(OpKind.MatMul, [dyt, x], meta((O, I))))         # dY_i^T X
            refs = [(np.ascontiguousarray(w0[:, :T]), x0) for w0 in ws0]
        before = s.launch_count()
        s.eval_many(outs)
        res[fusion] = ([s.get_buffer(o).reshape(refs[0][0].shape[0], refs[0][1].shape[1]) for o in outs],
                       s.launch_count() - before)
    got, launches = res[True]
    assert launches == 1, f"{launches} launches for three sibling products"
    for i, ((a, b), g, u) in enumerate(zip(refs, got, res[False][0])):
        gemm_full_check(g, a, b, "f32", f"grouped product {i} (shared {shared})")
        gemm_full_check(u, a, b, "f32", f"separate product {i}")


def test_swapped_sibling_products_run_as_one_grouped_launch():
    # Four weight-gradient-shaped products (dY_i^T X)^T, each a Transpose of
    # a MatMul nothing else reads, run as swapped products X^T dY_i, and as
    # one grouped launch; every output against float64 with the f32 bound.
    from parity import gemm_full_check
    T, I, O = 2048, 1024, 1024
    x0 = synth.normal(581, (T, I))
    dys = [synth.normal(582 + i, (T, O)) for i in range(4)]
    s = HipStream()
    x = s.add_constant(x0, meta((T, I)))
    outs = []
    for dy0 in dys:
        dy = s.add_constant(dy0, meta((T, O)))
        dyt = s.add_op(OpKind.Transpose(None), [dy], meta((O, T)))
        prod = s.add_op(OpKind.MatMul, [dyt, x], meta((O, I)))                       # dY^T X
        outs.append(s.add_op(OpKind.Transpose((1, 0)), [prod], meta((I, O))))       # (dY^T X)^T
    before = s.launch_count()
    s.eval_many(outs)
    assert s.launch_count() - before == 1
    for i, (o, dy0) in enumerate(zip(outs, dys)):
        gemm_full_check(s.get_buffer(o).reshape(I, O), np.ascontiguousarray(x0.T), dy0, "f32", f"swapped product {i}")


@pytest.mark.parametrize("early_read", [False, True])
def test_products_wait_for_siblings_whose_operands_come_later(early_read):
    # Four weight-gradient-shaped products (-dY_i^T X)^T whose dY_i come out
    # of separate kernels between them (dQ/dK/dV of a backward pass): the
    # first three wait for the last one's operand and the four run as one
    # grouped launch. When a node reads the first product before the last
    # sibling's operand exists, that product runs alone and the other three
    # group. Every output against float64 with the f32 bound.
    from parity import gemm_full_check
    T, I, O = 2048, 1024, 1024
    x0 = synth.normal(601, (T, I))
    dys = [synth.normal(602 + i, (T, O)) for i in range(4)]
    s = HipStream()
    x = s.add_constant(x0, meta((T, I)))
    outs = []
    for dy0 in dys:
        dy = s.add_op(OpKind.Neg, [s.add_constant(dy0, meta((T, O)))], meta((T, O)))
        dyt = s.add_op(OpKind.Transpose(None), [dy], meta((O, T)))
        prod = s.add_op(OpKind.MatMul, [dyt, x], meta((O, I)))                       # -dY^T X
        outs.append(s.add_op(OpKind.Transpose((1, 0)), [prod], meta((I, O))))
    targets = list(outs)
    if early_read:
        targets[0] = s.add_op(OpKind.Neg, [outs[0]], meta((I, O)))
    before = s.launch_count()
    s.eval_many(targets)
    assert s.launch_count() - before == (4 + 1 + 1 + 1 if early_read else 4 + 1)
    for i, (o, dy0) in enumerate(zip(outs, dys)):
        gemm_full_check(s.get_buffer(o).reshape(I, O), np.ascontiguousarray(x0.T), -dy0, "f32", f"product {i}")
    if early_read:
        assert np.array_equal(s.get_buffer(targets[0]), -s.get_buffer(outs[0]))


def _linear(s, x, t, i, o, w0, b0):
    """x W^T + b with b broadcast over the rows (crates/mlx-nn/src/linear.rs:34-43)."""
    w = s.add_constant(w0, meta((o, i)))
    wt = s.add_op(OpKind.Transpose(None), [w], meta((i, o)))
    y = s.add_op(OpKind.MatMul, [x, wt], meta((t, o)))
    bb = s.add_op(OpKind.Broadcast((t, o)), [s.add_constant(b0, meta((o,)))], meta((t, o)))
    return s.add_op(OpKind.Add, [y, bb], meta((t, o)))


@pytest.mark.parametrize("t,i,o", [(2048, 1024, 1024), (2048, 1024, 4096), (67, 45, 93)])
def test_linear_bias_added_in_the_product_store(t, i, o):
    # A linear layer's MatMul + Add of the broadcast bias runs as one product
    # whose store adds the bias (the split-f32 kernel, or its split-K sum),
    # or, below the split-f32 sizes, the product and one bias launch. The
    # same f32 addition as the unfused graph's Add: identical results, the
    # same eval_count.
    x0 = synth.normal(611, (t, i))
    w0 = synth.normal(612, (o, i))
    b0 = synth.normal(613, (o,))
    res = {}
    for fusion in (True, False):
        s = HipStream(fusion=fusion)
        y = _linear(s, s.add_constant(x0, meta((t, i))), t, i, o, w0, b0)
        before, calls = s.launch_count(), s.eval_count()
        s.eval_many([y])
        res[fusion] = (s.get_buffer(y).reshape(t, o), s.launch_count() - before, s.eval_count() - calls)
    assert res[True][1] == 1
    assert res[True][2] == res[False][2]
    assert np.array_equal(res[True][0], res[False][0])
    # x W^T + b as one product over K + 1: [x | 1] [W^T ; b].
    from parity import gemm_full_check
    gemm_full_check(res[True][0], np.hstack([x0, np.ones((t, 1), np.float32)]), np.vstack([w0.T, b0[None, :]]),
                    "f32", "linear with bias")


def test_grouped_linears_add_their_biases():
    # The Q/K/V projections of one input with their biases: one grouped
    # launch whose store adds each product's own bias; each against float64.
    from parity import gemm_full_check
    t, i, o = 2048, 1024, 1024
    x0 = synth.normal(621, (t, i))
    ws0 = [synth.normal(622 + j, (o, i)) for j in range(3)]
    bs0 = [synth.normal(632 + j, (o,)) for j in range(3)]
    s = HipStream()
    x = s.add_constant(x0, meta((t, i)))
    outs = [_linear(s, x, t, i, o, w0, b0) for w0, b0 in zip(ws0, bs0)]
    before = s.launch_count()
    s.eval_many(outs)
    assert s.launch_count() - before == 1
    xa = np.hstack([x0, np.ones((t, 1), np.float32)])
    for j, (y, w0, b0) in enumerate(zip(outs, ws0, bs0)):
        gemm_full_check(s.get_buffer(y).reshape(t, o), xa, np.vstack([w0.T, b0[None, :]]), "f32", f"projection {j}")


def test_grouped_products_with_non_finite_operand():
    # A grouped launch where one product's weight holds inf and NaN: that
    # product takes the exact f32 path (its flag), giving what an f32 product
    # gives; the others keep the split-f32 result (float64 bound).
    from parity import gemm_full_check
    T, I, O = 2048, 1024, 1024
    x0 = synth.normal(591, (T, I))
    ws0 = [synth.normal(592 + i, (O, I)) for i in range(3)]
    ws0[1][5, 7] = np.inf
    ws0[1][9, 3] = np.nan
    s = HipStream()
    x = s.add_constant(x0, meta((T, I)))
    outs = []
    for w0 in ws0:
        w = s.add_constant(w0, meta((O, I)))
        wt = s.add_op(OpKind.Transpose(None), [w], meta((I, O)))
        outs.append(s.add_op(OpKind.MatMul, [x, wt], meta((T, O))))
    s.eval_many(outs)
    got = [s.get_buffer(o).reshape(T, O) for o in outs]
    with np.errstate(over="ignore", invalid="ignore"):
        ref1 = (x0.astype(np.float64) @ ws0[1].T.astype(np.float64)).astype(np.float32)
    assert np.array_equal(np.isnan(got[1]), np.isnan(ref1))
    assert np.array_equal(np.isposinf(got[1]), np.isposinf(ref1))
    assert np.array_equal(np.isneginf(got[1]), np.isneginf(ref1))
    fin = np.isfinite(ref1)
    mag = np.abs(x0).astype(np.float64) @ np.abs(np.nan_to_num(ws0[1], nan=0, posinf=0, neginf=0)).T
    assert np.all(np.abs(got[1][fin] - ref1[fin]) <= 1e-6 * np.sqrt(I) * mag[fin] + 1e-30)
    for i in (0, 2):
        gemm_full_check(got[i], x0, ws0[i].T, "f32", f"finite product {i} of the group")


def test_async_view_constant_rewritten_after_synchronize():
    """The view-constant contract under asynchronous evaluation: kernels
    queued before clear() may still read the caller's memory, so the caller
    rewrites it only after synchronizing. Two steps on one stream: step 1
    reads the view, is cleared without waiting, the stream is synchronized,
    the memory is rewritten, and step 2 sees the new values while step 1's
    result (taken before the clear) keeps the old ones."""
    from oxidizedmlx_amd import backend as _hb
    x = np.arange(4096, dtype=np.float32).reshape(64, 64) / 7.0
    buf = _hb.DeviceBuffer.from_array(x)
    s = HipStream(async_eval=True)
    v = s.add_constant_view(buf.ptr, meta([64, 64]))
    two = s.add_constant(np.full((64, 64), 2.0, np.float32), meta([64, 64]))
    y = s.add_op(OpKind.Mul, [v, two], meta([64, 64]))
    s.eval(y)
    first = s.get_buffer(y).reshape(64, 64)
    s.clear()
    s.synchronize()
    buf.upload(-x)
    v = s.add_constant_view(buf.ptr, meta([64, 64]))
    two = s.add_constant(np.full((64, 64), 2.0, np.float32), meta([64, 64]))
    y = s.add_op(OpKind.Mul, [v, two], meta([64, 64]))
    s.eval(y)
    second = s.get_buffer(y).reshape(64, 64)
    s.close()
    np.testing.assert_array_equal(first, x * np.float32(2.0))
    np.testing.assert_array_equal(second, -x * np.float32(2.0))


@pytest.mark.parametrize("overflow", [False, True])
def test_chain_writes_the_planes_its_product_reads(overflow):
    # A chain whose result a split-f32 product reads writes that operand's
    # bf16 planes itself (the split pass's arithmetic), so the product skips
    # its split: GELU(x) . W at 1024 x 2048 x 1024 gives the unfused graph's
    # result bit for bit. With a value the planes cannot hold (exp overflow)
    # the chain raises the product's flag and the product forms C from the
    # f32 operands, as after a split. A second product reads the chain's
    # result transposed (g^T . v, the weight-gradient form) from the same
    # planes; it is held to the float64 bound.
    from parity import gemm_full_check
    t, i, o = 1024, 1024, 2048
    x0 = synth.normal(641, (t, i))
    if overflow:
        x0[5, 7] = 100.0  # exp(100) is +inf in f32
    w0 = synth.normal(642, (i, o), 0.0, 0.05)
    v0 = synth.normal(643, (t, o), 0.0, 0.05)
    op = OpKind.Exp if overflow else OpKind.Gelu
    res = {}
    for fusion in (True, False):
        s = HipStream(fusion=fusion)
        x = s.add_constant(x0, meta((t, i)))
        w = s.add_constant(w0, meta((i, o)))
        v = s.add_constant(v0, meta((t, o)))
        g = s.add_op(op, [x], meta((t, i)))
        y = s.add_op(OpKind.MatMul, [g, w], meta((t, o)))
        gt = s.add_op(OpKind.Transpose(None), [g], meta((i, t)))
        z = s.add_op(OpKind.MatMul, [gt, v], meta((i, o)))
        s.eval_many([y, z])
        res[fusion] = (s.get_buffer(y).reshape(t, o), s.get_buffer(z).reshape(i, o), s.get_buffer(g).reshape(t, i))
    np.testing.assert_array_equal(res[True][2], res[False][2])
    np.testing.assert_array_equal(res[True][0], res[False][0])
    if overflow:
        assert not np.isfinite(res[True][0][5]).all()
        assert np.isfinite(np.delete(res[True][0], 5, axis=0)).all()
    else:
        gv = res[True][2]
        gemm_full_check(res[True][0], gv, w0, "f32", "GELU(x) . W from the chain's planes")
        gemm_full_check(res[True][1], np.ascontiguousarray(gv.T), v0, "f32", "GELU(x)^T . v from the chain's planes")
