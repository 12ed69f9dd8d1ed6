"""f32 GEMM through bf16 planes (kernels/gemm16_x6.hip) vs the CPU oracle's
matmul (crates/mlx-core/src/cpu_kernels.rs:197-230) and float64.

Each f32 operand is split into hi + mid + lo bf16 planes and the matrix
cores sum the six plane products that reach f32 precision. The checks:
  * the split is exact and its dropped products stay below 2^-23 |a b|
    (CPU, numpy restatement of the rounding);
  * every layout, padded and odd shapes, batches and split-K settings:
    sampled rows against the oracle (|gpu - cpu| <= 1e-6 sqrt(K) max|A|
    max|B| + 1e-5 |cpu|) and every element against float64 with the f32
    accumulation bound (gemm_full_check);
  * operands holding inf / NaN / values past the bf16 range give what an f32
    product gives (the kernel's direct f32 path), and the next call on
    finite operands runs the planes again.
"""
import math

import numpy as np
import pytest

from oxidizedmlx_amd import abi
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd import synth
from parity import gemm_full_check
from test_gpu_gemm import check_gemm, sample_rows

F32 = abi.F32


def split3(x):
    """hi, mid, lo as the kernel forms them: each rounded to nearest even
    bf16 from what the planes before it leave (numpy restatement)."""
    x = np.asarray(x, np.float32)
    hi = synth.round_bf16(x)
    r1 = (x - hi).astype(np.float32)
    mid = synth.round_bf16(r1)
    r2 = (r1 - mid).astype(np.float32)
    return hi, mid, synth.round_bf16(r2)


def test_split_is_exact_and_dropped_products_are_small():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32),
                        (rng.standard_normal(1000) * 1e30).astype(np.float32),
                        (rng.standard_normal(1000) * 1e-30).astype(np.float32),
                        np.float32([1.0, -1.0, 3.0e38, -3.0e38, 1.17549435e-38, 0.0])])
    hi, mid, lo = split3(x)
    assert np.array_equal((hi.astype(np.float64) + mid + lo), x.astype(np.float64))
    nz = x != 0
    assert np.all(np.abs(mid[nz]) <= 2.0 ** -8 * np.abs(x[nz]))
    assert np.all(np.abs(lo[nz]) <= 2.0 ** -16 * np.abs(x[nz]))
    # The three dropped pairs of a product a * b.
    y = np.roll(x, 7)
    hy, my, ly = split3(y)
    dropped = np.abs(mid.astype(np.float64) * ly) + np.abs(lo.astype(np.float64) * my) + np.abs(
        lo.astype(np.float64) * ly)
    prod = np.abs(x.astype(np.float64) * y)
    assert np.all(dropped <= 2.0 ** -23 * prod)


@pytest.fixture
def x6(monkeypatch):
    monkeypatch.setenv("MLXHIP_GEMM_PATH", "x6")


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib", "x6")
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(67, 45, 93), (128, 256, 64), (300, 200, 520), (256, 512, 1024)])
def test_x6_layouts_full(ta, tb, m, n, k):
    check_gemm(m, n, k, F32, F32, ta=bool(ta), tb=bool(tb), seed=3 * m + k, full=True)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib", "x6")
@pytest.mark.parametrize("setting", ["3,1", "4,2"])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(67, 45, 93), (300, 200, 520)])
def test_x6_interleaved_layouts_full(monkeypatch, setting, ta, tb, m, n, k):
    monkeypatch.setenv("MLXHIP_X6", setting)
    check_gemm(m, n, k, F32, F32, ta=bool(ta), tb=bool(tb), seed=5 * m + k, full=True)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib", "x6")
@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0)])
def test_x6_batched_and_padded(ta, tb):
    check_gemm(200, 136, 160, F32, F32, ta=bool(ta), tb=bool(tb), batch=3, seed=11, ld_pad=5, full=True)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib", "x6")
@pytest.mark.parametrize("setting", ["0,1", "0,3", "1,1", "1,2", "1,5", "1,8", "2,1", "2,3", "3,1", "3,3", "4,1",
                                     "4,2"])
def test_x6_block_and_split_settings(monkeypatch, setting):
    """Every block tile of both kernels (segment by segment: 0-2,
    interleaved: 3-4), and split-K ranges that start and end inside a
    segment (5 splits of 6 segments) or cover less than one."""
    monkeypatch.setenv("MLXHIP_X6", setting)
    check_gemm(520, 300, 352, F32, F32, ta=False, tb=True, seed=5, full=True)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "oracle_lib")
@pytest.mark.parametrize("m,n,k,ta,tb", [
    (2048, 1024, 1024, 0, 1),   # config-4 projection
    (1024, 1024, 2048, 1, 0),   # its weight gradient
    (2048, 4096, 1024, 0, 0),   # feed-forward, 256x256 blocks
    (2048, 1024, 4096, 0, 1),   # feed-forward down projection
])
def test_x6_chosen_for_config4_shapes(m, n, k, ta, tb):
    """The shapes the block's f32 products take through the automatic choice
    (the split-f32 kernel), sampled rows against the oracle; the two
    1024-wide ones also every element against float64."""
    check_gemm(m, n, k, F32, F32, ta=bool(ta), tb=bool(tb), seed=m + n + k + 1, rows=sample_rows(m, 8),
               full=(n == 1024 and k <= 2048))


def run_f32(a, b, ta=False, tb=False):
    m, k = (a.shape[1], a.shape[0]) if ta else a.shape
    n = b.shape[0] if tb else b.shape[1]
    da, db = hb.DeviceBuffer.from_array(a), hb.DeviceBuffer.from_array(b)
    dc = hb.DeviceBuffer(m * n * 4)
    hb.gemm(F32, F32, ta, tb, m, n, k, da, a.shape[1], db, b.shape[1], dc, n)
    return dc.download(np.float32, m * n).reshape(m, n)


@pytest.mark.gpu
@pytest.mark.usefixtures("hip", "x6")
@pytest.mark.parametrize("tb", [False, True])
def test_x6_non_finite_inputs_match_f32(tb):
    m, n, k = 96, 160, 200
    a = synth.normal(21, (m, k))
    b = synth.normal(22, (n, k) if tb else (k, n))
    a[3, 17] = np.inf
    a[10, 5] = -np.inf
    a[40, 100] = np.nan
    a[50, 60] = 3.4e38           # finite in f32, past the bf16 range
    if tb:
        b[7, 33] = np.inf
    else:
        b[33, 7] = np.inf
    got = run_f32(a, b, tb=tb)
    bm = b.T if tb else b
    with np.errstate(over="ignore", invalid="ignore"):
        ref = a.astype(np.float64) @ bm.astype(np.float64)
        ref32 = ref.astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(ref32))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref32))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref32))
    fin = np.isfinite(ref32) & (np.abs(a).max(1) < 1e38)[:, None]
    mag = np.abs(np.nan_to_num(a, posinf=0, neginf=0)).astype(np.float64) @ np.abs(
        np.nan_to_num(bm, posinf=0, neginf=0))
    assert np.all(np.abs(got[fin] - ref[fin]) <= 1e-6 * math.sqrt(k) * mag[fin] + 1e-30)
    # A finite product right after: the planes path again, same workspace.
    a2, b2 = synth.normal(23, (m, k)), synth.normal(24, (n, k) if tb else (k, n))
    got2 = run_f32(a2, b2, tb=tb)
    gemm_full_check(got2, a2, b2.T if tb else b2, "f32", "x6 finite after non-finite")
