"""Property-based parity over random shapes, in the manner of the
reference's shape properties (crates/mlx-ops/tests/proptest_shapes.rs:89-262,
broadcastable pairs and axis draws) but applied to the kernels: GEMMs with
ragged extents in every layout and input dtype, row ops over any row length
and alignment, N-d transposes, broadcasts, axis reductions and elementwise
chains through the fusing stream.

hypothesis runs derandomized, so every run draws the same cases. Each case is
checked against the CPU oracle (numpy for pure data movement) at the
tolerance its family uses in the other tests: GEMM 1e-5 rel + the
summation-order bound (1e-2 rel for 16-bit inputs), row ops 1e-5 rel / 1e-6
abs, elementwise 1e-5 rel / 1e-6 abs, data movement and axis sums bit for
bit."""
import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd import synth
from oxidizedmlx_amd.opkind import OpKind, meta
from parity import assert_allclose, assert_chain_within_bound, chain_bound, cpu_stream, hip_stream
from test_gpu_gemm import BF16, F16, F32, check_gemm
from test_gpu_rows import oracle, run_rows

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip", "oracle_lib")]

CASES = settings(max_examples=150, deadline=None, derandomize=True, suppress_health_check=list(HealthCheck))


@CASES
@given(m=st.integers(1, 300), n=st.integers(1, 300), k=st.integers(0, 300), ta=st.booleans(), tb=st.booleans(),
       ab=st.sampled_from([F32, BF16, F16]), batch=st.integers(1, 3))
def test_gemm_any_shape(m, n, k, ta, tb, ab, batch):
    print(f"gemm m={m} n={n} k={k} ta={ta} tb={tb} ab={ab} batch={batch}", flush=True)
    check_gemm(m, n, k, ab, F32, ta, tb, batch=batch, seed=m * 7919 + n * 31 + k)


@settings(max_examples=40, deadline=None, derandomize=True, suppress_health_check=list(HealthCheck))
@given(m=st.integers(200, 1500), n=st.integers(200, 1500), k=st.integers(1, 1200), ta=st.booleans(),
       tb=st.booleans(), ab=st.sampled_from([BF16, F16]), cd=st.sampled_from([F32, BF16]))
def test_gemm16_tiled_shapes(m, n, k, ta, tb, ab, cd):
    """Extents large enough for the direct-to-LDS kernel's tile counts
    (and the padded-copy route when an extent is not a multiple of 8)."""
    print(f"gemm16 m={m} n={n} k={k} ta={ta} tb={tb} ab={ab} cd={cd}", flush=True)
    check_gemm(m, n, k, ab, cd if ab == BF16 else F32, ta, tb, seed=m * 131 + n * 17 + k)


@CASES
@given(rows=st.integers(1, 40), cols=st.integers(1, 5000), offset=st.integers(0, 3),
       op=st.sampled_from(["softmax", "layernorm", "rmsnorm"]))
def test_row_ops_any_shape(rows, cols, offset, op):
    print(f"{op} rows={rows} cols={cols} offset={offset}", flush=True)
    x = synth.normal(rows * 10007 + cols, (rows, cols), 0.0, 2.0)
    fn, kind = {"softmax": (hb.softmax_rows, OpKind.Softmax(-1)),
                "layernorm": (lambda a, b, r, c: hb.layernorm_rows(a, b, r, c, 1e-5), OpKind.LayerNorm(1e-5)),
                "rmsnorm": (lambda a, b, r, c: hb.rmsnorm_rows(a, b, r, c, 1e-5), OpKind.RmsNorm(1e-5))}[op]
    assert_allclose(run_rows(fn, x, offset=offset), oracle(kind, x), 1e-6, 1e-5, f"{op} {rows}x{cols}+{offset}")


@st.composite
def shape_and_perm(draw):
    shape = tuple(draw(st.lists(st.integers(1, 12), min_size=1, max_size=4)))
    perm = tuple(draw(st.permutations(range(len(shape)))))
    return shape, perm


@CASES
@given(sp=shape_and_perm())
def test_transpose_any_rank(sp):
    shape, perm = sp
    print(f"transpose {shape} by {perm}", flush=True)
    x = synth.normal(len(shape) * 101 + sum(shape), shape)
    xb, yb = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(max(x.nbytes, 4))
    out_shape = [shape[p] for p in perm]
    hb.eval_node_dev(OpKind.Transpose(perm), [(xb, shape)], meta(out_shape), yb)
    hb.synchronize()
    np.testing.assert_array_equal(yb.download(count=x.size).reshape(out_shape), x.transpose(perm))


@st.composite
def shape_and_perm_keeping_inner(draw):
    """Up to 8 axes, the innermost kept in place and a multiple of 4 long: the
    layouts the gather moves in 16-byte units."""
    inner = 4 * draw(st.integers(1, 40))
    outer = tuple(draw(st.lists(st.integers(1, 5), min_size=1, max_size=7)))
    perm = tuple(draw(st.permutations(range(len(outer))))) + (len(outer),)
    return outer + (inner,), perm


@settings(max_examples=60, deadline=None, derandomize=True, suppress_health_check=list(HealthCheck))
@given(sp=shape_and_perm_keeping_inner())
def test_transpose_keeping_inner_axis(sp):
    shape, perm = sp
    print(f"transpose {shape} by {perm}", flush=True)
    x = synth.normal(len(shape) * 211 + sum(shape), shape)
    xb, yb = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(x.nbytes)
    out_shape = [shape[p] for p in perm]
    hb.eval_node_dev(OpKind.Transpose(perm), [(xb, shape)], meta(out_shape), yb)
    hb.synchronize()
    np.testing.assert_array_equal(yb.download(count=x.size).reshape(out_shape), x.transpose(perm))


@st.composite
def broadcastable(draw):
    out = draw(st.lists(st.integers(1, 6), min_size=1, max_size=4))
    if draw(st.booleans()):
        out.append(4 * draw(st.integers(1, 16)))  # an innermost axis the gather moves 16 bytes at a time
    keep = draw(st.integers(0, len(out)))  # the input is a suffix of the output shape
    src = [d if draw(st.booleans()) else 1 for d in out[len(out) - keep:]]
    return tuple(src), tuple(out)


@CASES
@given(pair=broadcastable())
def test_broadcast_any_pair(pair):
    src, out = pair
    print(f"broadcast {src} -> {out}", flush=True)
    x = synth.normal(len(src) * 13 + len(out), src if src else (1,)).reshape(src)
    xb, yb = hb.DeviceBuffer.from_array(np.ascontiguousarray(x).reshape(-1)), hb.DeviceBuffer(4 * int(np.prod(out)))
    hb.eval_node_dev(OpKind.Broadcast(out), [(xb, src)], meta(out), yb)
    hb.synchronize()
    np.testing.assert_array_equal(yb.download(count=int(np.prod(out))).reshape(out), np.broadcast_to(x, out))


@st.composite
def shape_and_axis(draw):
    shape = tuple(draw(st.lists(st.integers(1, 40), min_size=1, max_size=3)))
    axis = draw(st.integers(0, len(shape) - 1))
    return shape, axis - len(shape) if draw(st.booleans()) else axis


@CASES
@given(sa=shape_and_axis(), kind=st.sampled_from(["sum", "mean", "max"]))
def test_axis_reduction_any_shape(sa, kind):
    shape, axis = sa
    print(f"{kind} over axis {axis} of {shape}", flush=True)
    op = {"sum": OpKind.Sum(axis), "mean": OpKind.Mean(axis), "max": OpKind.Max(axis)}[kind]
    x = synth.normal(sum(shape) * 17 + len(shape), shape)
    out_shape = [d for i, d in enumerate(shape) if i != axis % len(shape)]
    xb, yb = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(4 * max(1, int(np.prod(out_shape))))
    hb.eval_node_dev(op, [(xb, shape)], meta(out_shape), yb)
    hb.synchronize()
    np.testing.assert_array_equal(yb.download(count=int(np.prod(out_shape))), oracle_reduce(op, x, out_shape))


@pytest.mark.parametrize("shape,axis", [
    ((2048, 1024), 0), ((2048, 4096), 0), ((512, 16), 0), ((600, 20), 0), ((2049, 1028), 0),
    ((3, 700, 36), 1), ((2, 1000, 8), -2), ((1279, 4), 0), ((2, 3, 640, 12), 2)])
@pytest.mark.parametrize("kind", ["sum", "mean", "max"])
def test_long_axis_reduction(shape, axis, kind):
    """Axes of 512 elements and more over float4-aligned rows take the
    chunked LDS fold: ragged last chunks, column blocks that run past the
    row, several outer slices; bit for bit against the oracle's fold."""
    print(f"{kind} over axis {axis} of {shape}", flush=True)
    op = {"sum": OpKind.Sum(axis), "mean": OpKind.Mean(axis), "max": OpKind.Max(axis)}[kind]
    x = synth.normal(sum(shape) * 31 + len(shape), shape, 0.0, 3.0)
    out_shape = [d for i, d in enumerate(shape) if i != axis % len(shape)]
    xb, yb = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(4 * int(np.prod(out_shape)))
    hb.eval_node_dev(op, [(xb, shape)], meta(out_shape), yb)
    hb.synchronize()
    np.testing.assert_array_equal(yb.download(count=int(np.prod(out_shape))), oracle_reduce(op, x, out_shape))


def oracle_reduce(op, x, out_shape):
    from oracle.cpu_ref import CpuRefBackend
    from oxidizedmlx_amd.opkind import NodeInput
    return CpuRefBackend().eval_node(op, [NodeInput(x.reshape(-1), x.shape)], meta(out_shape)).reshape(-1)


UNARY = [OpKind.Neg, OpKind.Silu, OpKind.Gelu, OpKind.Exp, OpKind.Log, OpKind.Sqrt]
BINARY = [OpKind.Add, OpKind.Sub, OpKind.Mul, OpKind.Div]
@CASES
@given(n=st.integers(1, 3000), prog=st.lists(st.tuples(st.integers(0, len(UNARY) + len(BINARY) - 1),
                                                       st.integers(0, 2), st.booleans()),
                                              min_size=1, max_size=8), fusion=st.booleans())
def test_elementwise_chain_any_program(n, prog, fusion):
    """A random chain over three inputs: step i applies a unary op (Neg,
    SiLU, GELU, Exp, Log, Sqrt), or a binary op (Add, Sub, Mul, Div) with
    input j on either side; the fusing stream and the oracle's node-by-node
    evaluation must both lie within the chain's f32 error bound of the
    float64 value, and agree on certain NaNs."""
    print(f"chain n={n} prog={prog} fusion={fusion}", flush=True)
    ins = [synth.normal(n * 3 + j, (n,), 0.0, 1.0) for j in range(3)]

    def build(s):
        leaves = [s.add_constant(a, meta([n])) for a in ins]
        acc = leaves[0]
        for code, j, left in prog:
            if code < len(UNARY):
                acc = s.add_op(UNARY[code], [acc], meta([n]))
            else:
                other = leaves[j]
                acc = s.add_op(BINARY[code - len(UNARY)], [acc, other] if left else [other, acc], meta([n]))
        return acc

    cpu, hip = cpu_stream(), hip_stream()
    hip.set_fusion(fusion)
    c_out, h_out = build(cpu), build(hip)
    cpu.eval(c_out)
    hip.eval(h_out)
    assert_chain_within_bound(hip.get_buffer(h_out), cpu.get_buffer(c_out), *chain_bound(ins, prog, UNARY, BINARY))
