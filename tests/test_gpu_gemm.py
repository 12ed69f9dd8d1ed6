"""MFMA GEMM through the C ABI vs the CPU oracle's matmul
(crates/mlx-core/src/cpu_kernels.rs:197-230, i-j-p with a sequential f32 sum).

op(A) / op(B) for the transposed layouts are formed on the host by exact
transposition before the oracle runs. 16-bit cases give the oracle the same
RNE-rounded inputs (products of bf16/f16 values are exact in f32).

Tolerance |gpu - cpu| <= atol + rtol*|cpu| with
  atol = 1e-6 * sqrt(K) * max|A| * max|B|   (summation-order bound)
  rtol = 1e-5 for f32 output, 1e-2 for bf16/f16 output (one final rounding).
Large shapes compare sampled rows (all columns) so the oracle finishes in
seconds; the sample always includes the first and last rows.
"""
import math

import numpy as np
import pytest

from oracle import cpu_ref
from oxidizedmlx_amd import abi
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd import synth
from parity import assert_allclose, gemm_full_check

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip", "oracle_lib")]

F32, BF16, F16 = abi.F32, abi.BF16, abi.F16
OUT_NAME = {F32: "f32", BF16: "bf16", F16: "f16"}


def to_dev(x, dt):
    if dt == BF16:
        return hb.DeviceBuffer.from_array(synth.bf16_bits(x))
    if dt == F16:
        return hb.DeviceBuffer.from_array(synth.f16_bits(x))
    return hb.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))


def from_dev(buf, dt, n):
    if dt == BF16:
        return synth.bf16_to_f32(buf.download(np.uint16, n))
    if dt == F16:
        return buf.download(np.float16, n).astype(np.float32)
    return buf.download(np.float32, n)


def rounded(x, dt):
    return synth.round_bf16(x) if dt == BF16 else synth.round_f16(x) if dt == F16 else x


def oracle_rows(a, b, rows):
    """Rows `rows` of a @ b by the oracle's loop (a: [M,K], b: [K,N] f32)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    c = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for r in rows:
        cpu_ref.matmul_rows(a, b, c, int(r), 1)
    return c[rows]


def sample_rows(m, count):
    if m <= count:
        return np.arange(m)
    r = np.unique(np.concatenate([[0, m - 1], np.linspace(0, m - 1, count).astype(int)]))
    return r


def check_gemm(m, n, k, ab, cd, ta=False, tb=False, batch=1, seed=1, rows=None, ld_pad=0, full=False):
    """Runs one (batched) GEMM and checks sampled rows of every batch slice
    against the oracle; with `full`, also every element of every slice
    against float64 with the accumulation bound (gemm_full_check)."""
    A = synth.normal(seed, (batch, k, m) if ta else (batch, m, k))
    B = synth.normal(seed + 1, (batch, n, k) if tb else (batch, k, n))
    Ar, Br = rounded(A, ab), rounded(B, ab)
    lda = (m if ta else k) + ld_pad
    ldb = (k if tb else n) + ld_pad
    # Padded leading dimensions: copy into wider rows.
    Ap = np.zeros(A.shape[:2] + (lda,), np.float32)
    Ap[..., : A.shape[2]] = A
    Bp = np.zeros(B.shape[:2] + (ldb,), np.float32)
    Bp[..., : B.shape[2]] = B
    da, db = to_dev(Ap, ab), to_dev(Bp, ab)
    dc = hb.DeviceBuffer(batch * m * n * (4 if cd == F32 else 2))
    hb.gemm(ab, cd, ta, tb, m, n, k, da, lda, db, ldb, dc, n, batch=batch,
            stride_a=Ap[0].size, stride_b=Bp[0].size, stride_c=m * n)
    C = from_dev(dc, cd, batch * m * n).reshape(batch, m, n)
    rows = sample_rows(m, 12) if rows is None else rows
    rtol = 1e-5 if cd == F32 else 1e-2
    for bi in range(batch):
        opA = Ar[bi].T if ta else Ar[bi]
        opB = Br[bi].T if tb else Br[bi]
        ref = oracle_rows(opA, opB, rows)
        atol = 1e-6 * math.sqrt(k) * float(np.abs(opA).max()) * float(np.abs(opB).max()) if k else 0
        assert_allclose(C[bi][rows], ref, atol, rtol,
                        f"gemm {m}x{n}x{k} ab={ab} c={cd} ta={ta} tb={tb} batch {bi}")
        if full:
            gemm_full_check(C[bi], opA, opB, OUT_NAME[cd],
                            f"gemm {m}x{n}x{k} ab={ab} c={cd} ta={ta} tb={tb} batch {bi}")
    return C


def test_f32_512_cfg1():
    # Config 1: f32 C = A.B, M = N = K = 512, N(0,1); all rows checked.
    check_gemm(512, 512, 512, F32, F32, rows=np.arange(512), seed=0x5EED0001, full=True)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k,batch", [
    (64, 64, 64, 1),      # whole tiles, 8 k per half-wave
    (96, 64, 128, 2),     # 16
    (128, 160, 256, 1),   # 32
    (512, 512, 512, 1),   # 64 (config 1)
    (33, 47, 1, 1),       # ragged: edge tiles, K below one run
    (100, 77, 300, 3),    # ragged K inside the last run, batch
    (31, 65, 129, 1),     # one k past a whole run
])
def test_small_f32_kernel_shapes(ta, tb, m, n, k, batch):
    """The one-launch f32 kernels for small products (32 x 32 tiles): whole
    tiles take the 8-wave kernel that stages MN-contiguous operands through
    LDS (K over 16 half-wave runs), the others the 4-wave kernel (K over 8
    runs) that reads zeros past the matrix edge through the buffer
    descriptor. Every element of every slice against float64 with the
    accumulation bound, and sampled rows against the oracle."""
    check_gemm(m, n, k, F32, F32, ta=bool(ta), tb=bool(tb), batch=batch, seed=m + 3 * n + 7 * k + ta + 2 * tb,
               rows=sample_rows(m, 6), full=True)


@pytest.mark.parametrize("m,n,k,batch,ld_pad", [
    (512, 512, 64, 64, 0),   # config 4's composed attention scores: 64 heads of Q K^T, head dim 64
    (256, 512, 60, 64, 4),   # K not a multiple of 8, padded rows
    (512, 256, 36, 64, 0),   # K = 36: the second half-wave's run is mostly past K
    (256, 256, 32, 128, 0),  # K = 32: 16 per half-wave
    (512, 256, 16, 64, 8),   # K = 16: 8 per half-wave
    (256, 256, 4, 128, 0),   # K = 4: the second half-wave reads only zeros
    (192, 128, 32, 343, 0),  # 1029 blocks: not a multiple of 8 (no XCD ranges), 2-3 blocks per workgroup
])
def test_thin_f32_kernel(m, n, k, batch, ld_pad):
    """The thin kernel for many f32 products C = A B^T with K <= 64 (64 x 128
    blocks staged through LDS, K in two half-wave runs, zeros past K): every
    element of every slice against float64 with the accumulation bound, and
    sampled rows against the oracle."""
    assert (m // 64) * (n // 128) * batch >= 1024  # the thin kernel's range
    check_gemm(m, n, k, F32, F32, tb=True, batch=batch, seed=m + n + k + batch, rows=sample_rows(m, 3),
               ld_pad=ld_pad, full=True)


@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("m,k,batch,ld_pad", [
    (512, 512, 64, 0),   # config 4's composed attention: 64 heads of P V / P^T dO, head dimension 64
    (192, 320, 171, 4),  # five chunks of K, an odd batch, padded rows
    (128, 64, 256, 0),   # one chunk
])
def test_thin_n64_f32_kernel(ta, m, k, batch, ld_pad):
    """The thin kernel for many f32 products with N = 64, C = op(A) B with B
    [K][64] (K through two LDS stages of 64 k, A K-contiguous or
    M-contiguous): every element of every slice against float64 with the
    accumulation bound, and sampled rows against the oracle."""
    assert (m // 64) * batch >= 512  # the kernel's range
    check_gemm(m, 64, k, F32, F32, ta=bool(ta), batch=batch, seed=m + k + batch + ta, rows=sample_rows(m, 3),
               ld_pad=ld_pad, full=True)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_small_f32_kernel_any_alignment(ta, tb):
    """The small f32 kernel on operands one element past a 16-byte boundary,
    with odd leading dimensions and odd batch strides (no K-contiguous run is
    16-byte aligned, so whole tiles take the 4-byte-load variant); each
    slice's last element ends exactly at its descriptor's range."""
    m, n, k, batch = 64, 96, 128, 3
    A = synth.normal(70 + ta, (batch, k, m) if ta else (batch, m, k))
    B = synth.normal(72 + tb, (batch, n, k) if tb else (batch, k, n))
    lda, ldb = A.shape[2] + 1, B.shape[2] + 3
    sa, sb = A.shape[1] * lda + 1, B.shape[1] * ldb + 5

    def packed(x, ld, stride):
        flat = np.zeros(1 + batch * stride, np.float32)
        for bi in range(batch):
            for r in range(x.shape[1]):
                o = 1 + bi * stride + r * ld
                flat[o:o + x.shape[2]] = x[bi, r]
        return flat

    da, db = to_dev(packed(A, lda, sa), F32), to_dev(packed(B, ldb, sb), F32)
    dc = hb.DeviceBuffer(batch * m * n * 4)
    hb.gemm(F32, F32, ta, tb, m, n, k, da.ptr + 4, lda, db.ptr + 4, ldb, dc, n, batch=batch,
            stride_a=sa, stride_b=sb, stride_c=m * n)
    C = from_dev(dc, F32, batch * m * n).reshape(batch, m, n)
    for bi in range(batch):
        opA = A[bi].T if ta else A[bi]
        opB = B[bi].T if tb else B[bi]
        gemm_full_check(C[bi], opA, opB, "f32", f"small f32 ta={ta} tb={tb} batch {bi}")


@pytest.mark.parametrize("cd", [BF16, F32])
def test_bf16_4096_headline(cd):
    # Sampled rows against the oracle, and every element of C against
    # float64 on the same rounded inputs within the accumulation bound, so
    # every 256x256 tile of the product (and the XCD / group ordering that
    # places it) is checked.
    check_gemm(4096, 4096, 4096, BF16, cd, seed=11, rows=sample_rows(4096, 10), full=True)


@pytest.mark.parametrize("ab", [BF16, F16])
@pytest.mark.parametrize("tb", [False, True])
def test_batched_cfg3(ab, tb):
    # Config 3: [32,1024,1024] x [32,1024,1024] with f32 accumulate; tb = transposed-B case.
    # Three rows per slice against the oracle; every element of all 32 slices
    # against float64 within the accumulation bound.
    check_gemm(1024, 1024, 1024, ab, F32, tb=tb, batch=32, seed=21, rows=np.array([0, 511, 1023]),
               full=True)


@pytest.mark.parametrize("ab", [BF16, F16])
@pytest.mark.parametrize("tb", [False, True])
def test_batched_cfg3_c_in_operand_dtype(ab, tb):
    # The config-3 products as bench.py times them: C in the operands' dtype,
    # as the reference's matmul gives its result the left operand's dtype
    # (crates/mlx-core/src/tensor.rs:294), rounded once from the f32
    # accumulator. Three rows per slice against the oracle; every element of
    # all 32 slices against float64 with the accumulation bound plus one
    # rounding to the 16-bit type.
    check_gemm(1024, 1024, 1024, ab, ab, tb=tb, batch=32, seed=22, rows=np.array([0, 511, 1023]),
               full=True)


@pytest.mark.parametrize("ab", [BF16, F16])
def test_odd_cfg3_c_in_operand_dtype(ab):
    # The odd shape as bench.py times it (16-bit C; split over K, so the
    # rounding happens in the partial-sum kernel).
    check_gemm(1000, 777, 1531, ab, ab, seed=32, rows=sample_rows(1000, 24), full=True)


@pytest.mark.parametrize("ab", [BF16, F16, F32])
def test_odd_cfg3(ab):
    # Config 3 odd shape M=1000, N=777, K=1531 (edge tiles; unaligned rows).
    check_gemm(1000, 777, 1531, ab, F32, seed=31, rows=sample_rows(1000, 24), full=True)


@pytest.mark.parametrize("ab", [BF16, F16, F32])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(67, 45, 93), (128, 256, 64), (300, 200, 520)])
def test_all_layouts_full(ab, ta, tb, m, n, k):
    check_gemm(m, n, k, ab, F32, ta=bool(ta), tb=bool(tb), seed=m + n + k, rows=np.arange(m))


@pytest.mark.parametrize("ab,cd", [(BF16, BF16), (F16, F16), (BF16, F32)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_big_tile_layouts(ab, cd, ta, tb):
    # Large enough for the 256x256 tile path, with edge tiles in both M and N.
    check_gemm(4000, 3900, 520, ab, cd, ta=bool(ta), tb=bool(tb), seed=41, rows=sample_rows(4000, 8))


@pytest.mark.parametrize("ab", [BF16, F32])
def test_padded_leading_dims(ab):
    check_gemm(130, 70, 90, ab, F32, ld_pad=8, seed=51, rows=np.arange(130))
    check_gemm(130, 70, 90, ab, F32, ld_pad=3, seed=52, rows=np.arange(130))


def test_edge_sizes():
    check_gemm(1, 1, 1, F32, F32, rows=np.arange(1))
    check_gemm(1, 300, 7, BF16, F32, rows=np.arange(1))
    check_gemm(33, 1, 17, F16, F32, rows=np.arange(33))
    check_gemm(5, 6, 1, BF16, BF16, rows=np.arange(5))
    # K = 0: C is all zeros.
    dc = hb.DeviceBuffer.from_array(np.full(12, 7.0, np.float32))
    hb.gemm(F32, F32, False, False, 3, 4, 0, 0, 1, 0, 4, dc, 4)
    np.testing.assert_array_equal(dc.download(np.float32), np.zeros(12, np.float32))
    # M = 0 / N = 0 are no-ops.
    hb.gemm(BF16, F32, False, False, 0, 4, 8, 0, 8, 0, 4, 0, 4)


def test_gemm_argument_errors():
    with pytest.raises(abi.InvalidArgument):
        hb.gemm(abi.I32, F32, False, False, 2, 2, 2, 1, 2, 1, 2, 1, 2)
    with pytest.raises(abi.InvalidArgument):
        hb.gemm(F32, F32, False, False, 2, 2, 4, 1, 2, 1, 2, 1, 2)  # lda < K
    with pytest.raises(abi.NullPtr):
        hb.gemm(F32, F32, False, False, 2, 2, 2, 0, 2, 0, 2, 0, 2)


@pytest.mark.parametrize("m,n,k,ta,tb", [
    (2048, 1024, 1024, 0, 1),   # 128x128 blocks, K split 4 (config-4 projections)
    (1024, 1024, 2048, 1, 0),   # 128x128 blocks, K split 8 (weight gradients)
    (2048, 4096, 1024, 0, 0),   # 128x128 blocks, no split
    (4096, 4096, 256, 1, 1),    # 256x256 blocks
    (1000, 1100, 700, 0, 1),    # 128x128 blocks with edge tiles, split 2
    (1024, 3072, 2048, 1, 0),   # 192 tiles of 128x128: K split 4 (a power of two)
])
def test_f32_block_and_split_choices(monkeypatch, m, n, k, ta, tb):
    # The f32 shapes of the config-4 block pick 128x128 or 256x256 blocks
    # and split K in the general kernel (which the automatic choice gives
    # the split-f32 kernel instead for the larger ones); sampled rows
    # against the oracle.
    monkeypatch.setenv("MLXHIP_GEMM_PATH", "general")
    check_gemm(m, n, k, F32, F32, ta=bool(ta), tb=bool(tb), seed=m + n + k, rows=sample_rows(m, 10))


@pytest.mark.parametrize("m,n,k,ta,tb,batch", [
    (512, 64, 512, 0, 0, 64),   # config-4 P.V per head: 64x64 blocks (128-wide tiles half empty)
    (512, 64, 512, 1, 0, 64),   # its dV = P^T dY
    (64, 512, 2048, 0, 1, 8),   # narrow M, split over K
])
def test_f32_narrow_products(m, n, k, ta, tb, batch):
    check_gemm(m, n, k, F32, F32, ta=bool(ta), tb=bool(tb), batch=batch, seed=m + n + k + batch,
               rows=sample_rows(m, 6))


@pytest.mark.parametrize("ab,cd", [(BF16, BF16), (F16, F16), (BF16, F32)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_small16_kernel_any_alignment(monkeypatch, ab, cd, ta, tb):
    """The one-launch 64 x 64 kernel (forced for every shape here) on
    operands that start one element past a 4-byte boundary, with odd leading
    dimensions and odd batch strides (so rows and slices alternate between
    even and odd element positions), K not a multiple of its 64-wide K tile
    and edge tiles in M and N; every element of every slice against float64
    with the accumulation bound. The last chunk of each slice ends exactly
    at the descriptor's range."""
    monkeypatch.setenv("MLXHIP_GEMM_PATH", "small16")
    m, n, k, batch = 130, 97, 203, 3
    seed = 60 + 4 * ta + 2 * tb + ab
    A = synth.normal(seed, (batch, k, m) if ta else (batch, m, k))
    B = synth.normal(seed + 1, (batch, n, k) if tb else (batch, k, n))
    Ar, Br = rounded(A, ab), rounded(B, ab)
    lda, ldb = A.shape[2] + 1, B.shape[2] + 1         # odd leading dimensions
    sa, sb = A.shape[1] * lda + 1, B.shape[1] * ldb   # odd slice strides

    def packed(x, ld, stride):
        flat = np.zeros(1 + batch * stride, np.float32)   # element 0: offset by one element
        for bi in range(batch):
            for r in range(x.shape[1]):
                o = 1 + bi * stride + r * ld
                flat[o:o + x.shape[2]] = x[bi, r]
        return flat

    da, db = to_dev(packed(A, lda, sa), ab), to_dev(packed(B, ldb, sb), ab)
    dc = hb.DeviceBuffer(batch * m * n * (4 if cd == F32 else 2))
    hb.gemm(ab, cd, ta, tb, m, n, k, da.ptr + 2, lda, db.ptr + 2, ldb, dc, n, batch=batch,
            stride_a=sa, stride_b=sb, stride_c=m * n)
    C = from_dev(dc, cd, batch * m * n).reshape(batch, m, n)
    for bi in range(batch):
        opA = Ar[bi].T if ta else Ar[bi]
        opB = Br[bi].T if tb else Br[bi]
        gemm_full_check(C[bi], opA, opB, OUT_NAME[cd], f"small16 ab={ab} c={cd} ta={ta} tb={tb} batch {bi}")
