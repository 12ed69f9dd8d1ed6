"""Row kernels (softmax / scaled-masked softmax / LayerNorm / RMSNorm and
their VJPs) through the C ABI vs the CPU oracle.

Tolerances (f32): softmax / LayerNorm / RMSNorm rel 1e-5 with atol 1e-6; the
VJPs rel 1e-4 with atol 1e-5 (they subtract row means, so cancellation
amplifies the summation-order difference). Only the order of the row sums
differs from the reference; max-abs / max-rel errors are printed.
"""
import numpy as np
import pytest

from oracle import cpu_ref
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd import synth
from oxidizedmlx_amd.opkind import NodeInput, OpKind, meta
from parity import assert_allclose

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip", "oracle_lib")]

ORACLE = cpu_ref.CpuRefBackend()


def run_rows(fn, x, *extra, offset=0):
    """Runs a direct row entry point on device copies of x (and extra inputs);
    `offset` floats of padding in front misalign the rows on purpose."""
    rows, cols = x.shape
    bufs = []
    for a in (x,) + extra:
        pad = np.zeros(offset + a.size, np.float32)
        pad[offset:] = a.reshape(-1)
        bufs.append(hb.DeviceBuffer.from_array(pad))
    y = hb.DeviceBuffer((offset + x.size) * 4)
    ptrs = [b.ptr + 4 * offset for b in bufs]
    fn(*ptrs, y.ptr + 4 * offset, rows, cols)
    return y.download(count=x.size, offset=4 * offset).reshape(rows, cols)


def oracle(op, *arrays):
    shape = arrays[0].shape
    return ORACLE.eval_node(op, [NodeInput(a.reshape(-1), shape) for a in arrays],
                            meta(shape)).reshape(shape)


@pytest.fixture(scope="module")
def cfg2_x():
    # Config 2: [4096, 4096] f32, entries N(0, 2^2)
    return synth.normal(0x5EED0003, (4096, 4096), 0.0, 2.0)


def test_softmax_cfg2(cfg2_x):
    y = run_rows(hb.softmax_rows, cfg2_x)
    ref = cpu_ref.softmax_lastdim(cfg2_x)
    assert_allclose(y, ref, 1e-6, 1e-5, "softmax 4096x4096")
    np.testing.assert_allclose(y.astype(np.float64).sum(1), 1.0, atol=1e-5)


def test_layernorm_cfg2(cfg2_x):
    y = run_rows(lambda x, y, r, c: hb.layernorm_rows(x, y, r, c, 1e-5), cfg2_x)
    assert_allclose(y, cpu_ref.layer_norm(cfg2_x, 1e-5), 1e-6, 1e-5, "layernorm 4096x4096")


def test_rmsnorm_cfg2(cfg2_x):
    y = run_rows(lambda x, y, r, c: hb.rmsnorm_rows(x, y, r, c, 1e-5), cfg2_x)
    assert_allclose(y, cpu_ref.rms_norm(cfg2_x, 1e-5), 1e-6, 1e-5, "rmsnorm 4096x4096")


RAGGED = [(3, 1), (5, 3), (7, 5), (9, 63), (4, 64), (4, 65), (3, 255), (3, 257), (5, 1000),
          (5, 2000), (5, 2048), (6, 4095), (3, 4097), (2, 8192), (2, 12000), (2, 16384), (2, 16385),
          (1, 40000)]


@pytest.mark.parametrize("rows,cols", RAGGED)
@pytest.mark.parametrize("offset", [0, 1])
def test_rows_ragged_and_misaligned(rows, cols, offset):
    x = synth.normal(1000 + rows * 7 + cols, (rows, cols), 0.0, 2.0)
    y = run_rows(hb.softmax_rows, x, offset=offset)
    assert_allclose(y, oracle(OpKind.Softmax(-1), x), 1e-6, 1e-5, f"softmax {rows}x{cols}+{offset}")
    y = run_rows(lambda a, b, r, c: hb.layernorm_rows(a, b, r, c, 1e-5), x, offset=offset)
    assert_allclose(y, oracle(OpKind.LayerNorm(1e-5), x), 1e-6, 1e-5, f"layernorm {rows}x{cols}")
    y = run_rows(lambda a, b, r, c: hb.rmsnorm_rows(a, b, r, c, 1e-5), x, offset=offset)
    assert_allclose(y, oracle(OpKind.RmsNorm(1e-5), x), 1e-6, 1e-5, f"rmsnorm {rows}x{cols}")


@pytest.mark.parametrize("rows,cols", [(2048, 1024), (64, 512), (3, 77), (5, 1000), (3, 2048), (2, 6000),
                                       (2, 20000)])
def test_vjp_rows(rows, cols):
    x = synth.normal(7 + cols, (rows, cols), 0.0, 1.0)
    dy = synth.normal(8 + cols, (rows, cols), 0.0, 1.0)
    g = run_rows(lambda d, a, o, r, c: hb.layernorm_vjp_rows(d, a, o, r, c, 1e-5), dy, x)
    assert_allclose(g, oracle(OpKind.LayerNormVjp(1e-5), dy, x), 1e-5, 1e-4, "layernorm_vjp")
    g = run_rows(lambda d, a, o, r, c: hb.rmsnorm_vjp_rows(d, a, o, r, c, 1e-5), dy, x)
    assert_allclose(g, oracle(OpKind.RmsNormVjp(1e-5), dy, x), 1e-5, 1e-4, "rmsnorm_vjp")
    s = oracle(OpKind.Softmax(-1), x)
    g = run_rows(hb.softmax_vjp_rows, dy, s)
    assert_allclose(g, oracle(OpKind.SoftmaxVjp(-1), dy, s), 1e-6, 1e-4, "softmax_vjp")


@pytest.mark.parametrize("n,causal", [(512, True), (512, False), (77, True), (1000, True)])
def test_scaled_masked_softmax(n, causal):
    x = synth.normal(99 + n, (n, n), 0.0, 1.0)
    scale = 1.0 / np.sqrt(64.0)
    y = run_rows(lambda a, b, r, c: hb.scaled_masked_softmax_rows(a, b, r, c, scale, causal), x)
    ref = oracle(OpKind.ScaledMaskedSoftmax(scale, causal), x)
    assert_allclose(y, ref, 1e-6, 1e-5, f"scaled_masked_softmax {n} causal={causal}")
    if causal:
        assert np.all(np.triu(y, 1) == 0.0)


def test_empty_rows_are_noops():
    hb.softmax_rows(0, 0, 0, 4096)
    hb.layernorm_rows(0, 0, 5, 0, 1e-5)


def test_softmax_non_last_axis_via_eval_node():
    x = synth.normal(5, (3, 50, 7), 0.0, 2.0)
    for axis in (0, 1):
        out = hb.HipBackend().eval_node(OpKind.Softmax(axis), [NodeInput(x.reshape(-1), x.shape)],
                                        meta(x.shape))
        ref = ORACLE.eval_node(OpKind.Softmax(axis), [NodeInput(x.reshape(-1), x.shape)], meta(x.shape))
        assert_allclose(out, ref, 1e-6, 1e-5, f"softmax axis {axis}")


@pytest.mark.parametrize("cols", [96, 1000, 4096, 6000])
def test_softmax_non_finite_rows(cols):
    # Rows with -inf entries (masked scores), whole lanes of -inf, a row of
    # all -inf (NaN in the reference: exp(-inf - -inf)), +inf and NaN
    # entries. Each row's merged (max, sum) must give the oracle's values:
    # 0 where the oracle has 0, NaN where it has NaN.
    rows = 8
    x = synth.normal(77 + cols, (rows, cols))
    x[0, : cols // 2] = -np.inf             # half a row masked: whole lanes of -inf
    x[1, 1::2] = -np.inf
    x[2, :] = -np.inf                        # all masked
    x[3, cols // 3] = np.inf
    x[4, 7] = np.nan
    x[5, -1] = -np.inf
    y = run_rows(hb.softmax_rows, x)
    ref = oracle(OpKind.Softmax(-1), x)
    assert np.array_equal(np.isnan(y), np.isnan(ref)), (np.isnan(y).sum(1), np.isnan(ref).sum(1))
    fin = ~np.isnan(ref)
    assert_allclose(y[fin], ref[fin], 1e-6, 1e-5, f"softmax non-finite rows, {cols} cols")
    assert np.all(y[0, : cols // 2] == 0.0) and np.all(y[1, 1::2] == 0.0)


@pytest.mark.parametrize("cols", [96, 4096])
def test_layernorm_large_offset_rows(cols):
    # Rows with a large common offset: the per-lane moments and their merge
    # must keep the variance of the small deviations (a one-pass sum of
    # squares would cancel catastrophically here).
    x = (np.float32(1000.0) + synth.normal(91, (64, cols), 0.0, 0.01)).astype(np.float32)
    y = run_rows(lambda a, b, r, c: hb.layernorm_rows(a, b, r, c, 1e-5), x)
    ref = oracle(OpKind.LayerNorm(1e-5), x)
    # The reference's own mean carries ~1e-4 relative error of the deviations
    # at this offset; hold both to float64.
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    ex = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(1, keepdims=True) + 1e-5)
    e_hip = float(np.abs(y - ex).max())
    e_ref = float(np.abs(ref - ex).max())
    print(f"  layernorm offset 1000: hip {e_hip:.3e}, oracle {e_ref:.3e}", flush=True)
    assert e_hip <= 2 * e_ref + 1e-4
