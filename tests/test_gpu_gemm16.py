"""The direct-to-LDS 16-bit GEMM kernel (kernels/gemm16_impl.hpp) and the
general MFMA kernel, each forced through MLXHIP_GEMM_PATH, against the CPU
oracle's matmul (crates/mlx-core/src/cpu_kernels.rs:197-230) on the same
RNE-rounded inputs.

Tolerance as in test_gpu_gemm.py: |gpu - cpu| <= atol + rtol*|cpu| with
atol = 1e-6 * sqrt(K) * max|A| * max|B| and rtol 1e-5 (f32 C) or 1e-2
(bf16/f16 C). The shapes exercise what the direct-to-LDS kernel handles
with its out-of-range buffer loads: M and N edges inside a block tile,
K not a multiple of the 32-wide K tile, tiles with no valid rows at all,
and batch strides. Both block configurations of that kernel (256 x 256 with
8 waves, 128 x 128 with 4 waves) are forced in turn ("lds16_256",
"lds16_128").
"""
import os

import numpy as np
import pytest

from oxidizedmlx_amd import abi
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd import synth
from test_gpu_gemm import check_gemm, sample_rows, to_dev

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip", "oracle_lib")]

F32, BF16, F16 = abi.F32, abi.BF16, abi.F16


@pytest.fixture
def gemm_path(request):
    old = os.environ.get("MLXHIP_GEMM_PATH")
    os.environ["MLXHIP_GEMM_PATH"] = request.param
    yield request.param
    if old is None:
        del os.environ["MLXHIP_GEMM_PATH"]
    else:
        os.environ["MLXHIP_GEMM_PATH"] = old


@pytest.mark.parametrize("gemm_path", ["lds16_256", "lds16_128"], indirect=True)
@pytest.mark.parametrize("ab,cd", [(BF16, F32), (BF16, BF16), (F16, F32), (F16, F16)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(256, 256, 32), (300, 264, 520), (64, 40, 8), (520, 776, 1528)])
def test_lds16_layouts(gemm_path, ab, cd, ta, tb, m, n, k):
    check_gemm(m, n, k, ab, cd, ta=bool(ta), tb=bool(tb), seed=m + 3 * n + 7 * k,
               rows=sample_rows(m, 40))


@pytest.mark.parametrize("gemm_path", ["lds16_256", "lds16_128"], indirect=True)
@pytest.mark.parametrize("tb", [False, True])
def test_lds16_batched_strided(gemm_path, tb):
    check_gemm(264, 136, 200, BF16, F32, tb=tb, batch=5, seed=77, rows=sample_rows(264, 16))
    check_gemm(128, 128, 96, F16, F16, tb=tb, batch=3, seed=78, rows=np.arange(128), ld_pad=8)


@pytest.mark.parametrize("gemm_path", ["lds16_256", "lds16_128"], indirect=True)
def test_lds16_headline_shape(gemm_path):
    check_gemm(4096, 4096, 4096, BF16, BF16, seed=12, rows=sample_rows(4096, 10))


@pytest.mark.parametrize("gemm_path", ["general"], indirect=True)
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_general_kernel_headline_shape(gemm_path, ta, tb):
    check_gemm(4096, 4096, 4096, BF16, BF16, ta=bool(ta), tb=bool(tb), seed=13,
               rows=sample_rows(4096, 6))


@pytest.mark.parametrize("gemm_path", ["lds16"], indirect=True)
def test_lds16_falls_back_when_unsupported(gemm_path):
    # K = 1531 is not a multiple of 8: the general kernel must run and agree.
    check_gemm(1000, 777, 1531, BF16, F32, seed=31, rows=sample_rows(1000, 12))
    check_gemm(70, 64, 48, F16, F32, ld_pad=3, seed=32, rows=np.arange(70))


@pytest.mark.parametrize("gemm_path", ["lds16_256", "lds16_128", "general"], indirect=True)
@pytest.mark.parametrize("ab", [BF16, F16])
def test_output_rounding_bit_exact(gemm_path, ab):
    # K = 8 with only k = 0 non-zero: C[m, n] = a[m] * b[n], a product of two
    # 16-bit values and so exact in f32. The 16-bit C must then be that
    # product rounded to nearest even, bit for bit (bf16: synth.bf16_bits;
    # f16: numpy's float16 conversion).
    m, n, k = 300, 264, 8
    a0 = synth.normal(91, (m,)) * np.float32(3.0)
    b0 = synth.normal(92, (n,))
    a0 = synth.round_bf16(a0) if ab == BF16 else synth.round_f16(a0)
    b0 = synth.round_bf16(b0) if ab == BF16 else synth.round_f16(b0)
    A = np.zeros((m, k), np.float32)
    A[:, 0] = a0
    B = np.zeros((k, n), np.float32)
    B[0, :] = b0
    exact = np.outer(a0, b0).astype(np.float32)
    assert np.array_equal(exact.astype(np.float64), np.outer(a0.astype(np.float64), b0.astype(np.float64)))
    da, db = to_dev(A, ab), to_dev(B, ab)
    dc = hb.DeviceBuffer(m * n * 2)
    hb.gemm(ab, ab, False, False, m, n, k, da, k, db, n, dc, n)
    got = dc.download(np.uint16, m * n).reshape(m, n)
    want = synth.bf16_bits(exact) if ab == BF16 else exact.astype(np.float16).view(np.uint16)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[0]}: got {got[tuple(bad[0])]:#06x} want {want[tuple(bad[0])]:#06x}"


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("cd", [F32, BF16])
def test_block_configs_agree_bit_for_bit(ta, tb, cd):
    # Both block configurations accumulate every output element over the same
    # sequence of MFMAs (K tiles in order, two k-steps each), so their results
    # must be identical, edges included.
    m, n, k = 392, 520, 1000
    A = synth.normal(101, (k, m) if ta else (m, k))
    B = synth.normal(102, (n, k) if tb else (k, n))
    da, db = to_dev(A, BF16), to_dev(B, BF16)
    es = 4 if cd == F32 else 2
    outs = []
    for path in ("lds16_256", "lds16_128"):
        os.environ["MLXHIP_GEMM_PATH"] = path
        try:
            dc = hb.DeviceBuffer(m * n * es)
            hb.gemm(BF16, cd, bool(ta), bool(tb), m, n, k, da, A.shape[1], db, B.shape[1], dc, n)
            outs.append(dc.download(np.uint32 if es == 4 else np.uint16, m * n))
        finally:
            del os.environ["MLXHIP_GEMM_PATH"]
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("ab,cd", [(F32, F32), (BF16, F32), (BF16, BF16), (F16, F16)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_split_k(ab, cd, ta, tb):
    # 4 x 3 tiles of 64 x 64 per batch with K = 4096: the general kernel splits
    # K over 8 workgroups and a second kernel sums the f32 partials.
    check_gemm(200, 136, 4096, ab, cd, ta=bool(ta), tb=bool(tb), batch=2, seed=61,
               rows=sample_rows(200, 20))


def test_split_k_is_deterministic():
    A = synth.normal(71, (200, 4096))
    B = synth.normal(72, (4096, 136))
    da, db = to_dev(A, F32), to_dev(B, F32)
    outs = []
    for _ in range(3):
        dc = hb.DeviceBuffer(200 * 136 * 4)
        hb.gemm(F32, F32, False, False, 200, 136, 4096, da, 4096, db, 136, dc, 136)
        outs.append(dc.download(np.float32))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


@pytest.mark.parametrize("ab", [BF16, F16, F32])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_unaligned_operands_are_packed(ab, ta, tb):
    # Odd leading dimensions (and batch strides) are copied into padded,
    # aligned buffers before the aligned kernels run.
    check_gemm(97, 75, 131, ab, F32, ta=bool(ta), tb=bool(tb), batch=3, ld_pad=3, seed=81,
               rows=np.arange(97))
