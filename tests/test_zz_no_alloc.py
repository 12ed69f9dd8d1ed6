"""mlxhip_gemm_noalloc (the GEMM entry point that allocates nothing, for
callers that cannot call hipMalloc) against mlxhip_gemm on the same operands.

Both run the same kernels with the same split-K plan, so their outputs must
agree bit for bit. Each case makes two calls in a row, the second on a
smaller product, so the second call reads a fixed scratch that still holds
the first call's partials. The cases cover the two workspace uses: split-K
partials (f32 operands) and the zero-padded copies of unaligned operands
(16-bit and f32, the latter then also split over K).
"""
import numpy as np
import pytest

from oxidizedmlx_amd import abi
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd import synth

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip")]

F32, BF16 = abi.F32, abi.BF16


def _dev(x, dt):
    if dt == BF16:
        return hb.DeviceBuffer.from_array(synth.bf16_bits(x))
    return hb.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))


def _run_both(m, n, k, dt, ld_pad, seed):
    """C from mlxhip_gemm and from mlxhip_gemm_noalloc, as raw bits."""
    lda, ldb = k + ld_pad, n + ld_pad
    A = np.zeros((m, lda), np.float32)
    A[:, :k] = synth.normal(seed, (m, k))
    B = np.zeros((k, ldb), np.float32)
    B[:, :n] = synth.normal(seed + 1, (k, n))
    da, db = _dev(A, dt), _dev(B, dt)
    out = []
    for fn in (hb.gemm, hb.gemm_noalloc):
        dc = hb.DeviceBuffer(m * n * 4)
        fn(dt, F32, False, False, m, n, k, da, lda, db, ldb, dc, n)
        hb.synchronize()
        out.append(dc.download(np.uint32, m * n))
    return out


@pytest.mark.parametrize("dt,ld_pad,shapes", [
    # f32, aligned: split-K partials (8 x 1 MiB x 4 B, then 8 x 256 Ki x 4 B)
    (F32, 0, [(1024, 1024, 2048), (512, 512, 1024)]),
    # bf16, unaligned rows: both operands packed into scratch first
    (BF16, 1, [(1000, 777, 1531), (300, 200, 333)]),
    # f32, unaligned rows: packed copies, then split-K partials after them
    (F32, 1, [(513, 300, 1999), (129, 65, 700)]),
], ids=["f32_splitk", "bf16_packed", "f32_packed_splitk"])
def test_noalloc_matches_gemm_on_two_calls(dt, ld_pad, shapes):
    for i, (m, n, k) in enumerate(shapes):
        print(f"noalloc case dt={dt} pad={ld_pad} call {i}: {m}x{n}x{k}", flush=True)
        ref, got = _run_both(m, n, k, dt, ld_pad, seed=17 + i)
        assert np.array_equal(ref, got), f"call {i} {m}x{n}x{k}: {int((ref != got).sum())} elements differ"


def test_noalloc_rejects_products_beyond_its_scratch():
    cap = hb.gemm_noalloc_scratch_bytes()
    assert cap == 64 << 20
    # Unaligned f32 4097 x 4097 x 4096: its padded copies alone need about
    # 128 MiB. The check runs before any launch and C stays untouched.
    m = n = 4097
    k = 4096
    lda, ldb = k + 1, n
    da = hb.DeviceBuffer(m * lda * 4)
    db = hb.DeviceBuffer(k * ldb * 4)
    sentinel = np.full(16, 7.0, np.float32)
    dc = hb.DeviceBuffer(m * n * 4)
    dc.upload(sentinel)
    with pytest.raises(abi.InvalidArgument, match="scratch"):
        hb.gemm_noalloc(F32, F32, False, False, m, n, k, da, lda, db, ldb, dc, n)
    hb.synchronize()
    assert np.array_equal(dc.download(np.float32, 16), sentinel)


def test_noalloc_f32_planes_beyond_scratch_take_the_direct_kernel():
    """An aligned f32 product whose bf16 planes (72 MiB here) exceed the
    64 MiB fixed scratch runs on the direct f32 MFMA kernel instead of
    failing: checked against float64 with the f32 accumulation bound (the
    result need not match mlxhip_gemm's split-f32 bits)."""
    m, n, k = 2048, 2048, 3072
    A = synth.normal(31, (m, k))
    B = synth.normal(32, (k, n))
    da, db = _dev(A, F32), _dev(B, F32)
    dc = hb.DeviceBuffer(m * n * 4)
    print(f"noalloc f32 direct fallback: {m}x{n}x{k}", flush=True)
    hb.gemm_noalloc(F32, F32, False, False, m, n, k, da, k, db, n, dc, n)
    hb.synchronize()
    got = dc.download(np.float32, m * n).reshape(m, n).astype(np.float64)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    bound = (k * np.finfo(np.float32).eps) * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
    err = np.abs(got - ref)
    assert np.all(err <= bound + 1e-30), float((err / np.maximum(bound, 1e-30)).max())


def test_noalloc_refuses_another_stream_while_the_scratch_is_busy():
    """A noalloc call on a second stream while the first stream's noalloc
    kernels are still queued is refused (InvalidArgument, C untouched)
    instead of sharing the scratch; once the first stream has drained, the
    same call runs and matches mlxhip_gemm. Every buffer is made before the
    work is queued: a blocking copy on the null stream would wait for
    stream 1 to drain."""
    s1, s2 = hb.create_stream(), hb.create_stream()
    try:
        n = 4096
        busy = [hb.DeviceBuffer.from_array(synth.bf16_bits(synth.normal(93 + i, (n, n)))) for i in range(2)]
        busy_c = hb.DeviceBuffer(n * n * 2)
        m, k, nn = 512, 1024, 512
        da, db = _dev(synth.normal(91, (m, k)), F32), _dev(synth.normal(92, (k, nn)), F32)
        c1 = hb.DeviceBuffer(m * nn * 4)
        sentinel = np.full(m * nn, 7.0, np.float32)
        c2 = hb.DeviceBuffer.from_array(sentinel)
        ref = hb.DeviceBuffer(m * nn * 4)
        hb.synchronize()
        # ~3 ms of 4096^3 bf16 products ahead of stream 1's noalloc call.
        for _ in range(24):
            hb.gemm(BF16, BF16, False, False, n, n, n, busy[0], n, busy[1], n, busy_c, n, stream=s1)
        hb.gemm_noalloc(F32, F32, False, False, m, nn, k, da, k, db, nn, c1, nn, stream=s1)
        print("noalloc: second stream while the first is busy", flush=True)
        with pytest.raises(abi.InvalidArgument, match="still in use"):
            hb.gemm_noalloc(F32, F32, False, False, m, nn, k, da, k, db, nn, c2, nn, stream=s2)
        hb.synchronize(s1)
        np.testing.assert_array_equal(c2.download(np.float32, m * nn), sentinel)
        hb.gemm_noalloc(F32, F32, False, False, m, nn, k, da, k, db, nn, c2, nn, stream=s2)
        hb.synchronize(s2)
        hb.gemm(F32, F32, False, False, m, nn, k, da, k, db, nn, ref, nn)
        hb.synchronize()
        got = c2.download(np.uint32, m * nn)
        assert np.array_equal(got, ref.download(np.uint32, m * nn))
        assert np.array_equal(got, c1.download(np.uint32, m * nn))
    finally:
        hb.synchronize(s1)
        hb.synchronize(s2)
        hb.destroy_stream(s1)
        hb.destroy_stream(s2)
