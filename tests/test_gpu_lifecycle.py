"""Lifecycle and stress tests after the reference's
crates/mlx-core/tests/concurrency_stress.rs:145-222 (10k create-eval-drop
cycles, add chains up to 500 ops, 4 threads x 100 softmax evaluations) and
crates/mlx-sys/src/lib.rs:395-417 (null frees are no-ops, 10k alloc/free
cycles). Results stay correct and device memory stays bounded: free device
memory is read with hipMemGetInfo from the HIP runtime the library itself
loaded."""
import ctypes as C
import threading

import numpy as np
import pytest

from oxidizedmlx_amd import abi
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd.opkind import OpKind, meta

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip")]


def free_device_bytes() -> int:
    rt = C.CDLL("libamdhip64.so.7")  # already loaded by the library: the same runtime
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert rt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def create_eval_drop() -> np.ndarray:
    s = hb.HipStream()
    a = s.add_constant(np.array([1.0, 2.0, 3.0, 4.0], np.float32), meta([2, 2]))
    b = s.add_constant(np.full(4, 0.5, np.float32), meta([2, 2]))
    c = s.add_op(OpKind.Add, [a, b], meta([2, 2]))
    s.eval(c)
    out = s.get_buffer(c)
    s.close()
    return out


def test_bounded_memory_10k_eval_cycles():
    np.testing.assert_array_equal(create_eval_drop(), [1.5, 2.5, 3.5, 4.5])
    for _ in range(100):
        create_eval_drop()
    hb.synchronize()
    before = free_device_bytes()
    for _ in range(10_000):
        create_eval_drop()
    hb.synchronize()
    after = free_device_bytes()
    print(f"free device memory {before} -> {after} bytes over 10k cycles", flush=True)
    assert before - after < (64 << 20)


@pytest.mark.parametrize("fusion", [True, False])
def test_bounded_memory_chained_ops(fusion):
    for chain_len in (10, 50, 100, 500):
        s = hb.HipStream(fusion=fusion)
        t = s.add_constant(np.ones(4, np.float32), meta([4]))
        one = s.add_constant(np.ones(4, np.float32), meta([4]))
        for _ in range(chain_len):
            t = s.add_op(OpKind.Add, [t, one], meta([4]))
        s.eval(t)
        np.testing.assert_array_equal(s.get_buffer(t), np.full(4, chain_len + 1, np.float32))
        s.close()


def test_concurrent_eval_stress_4_threads_100_iterations():
    x = np.arange(1, 10, dtype=np.float32)
    errors = []

    def worker():
        try:
            for _ in range(100):
                s = hb.HipStream()
                a = s.add_constant(x, meta([3, 3]))
                y = s.add_op(OpKind.Softmax(1), [a], meta([3, 3]))
                s.eval(y)
                r = s.get_buffer(y).reshape(3, 3)
                s.close()
                assert np.all(np.abs(r.sum(axis=1) - 1.0) < 1e-5), r
        except Exception as e:  # reported on the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


def test_buffer_lifecycle_10k_and_null_frees():
    L = abi.load_library()
    L.mlxhip_buffer_free(None)
    L.mlxhip_stream_free(None)
    hb.synchronize()
    before = free_device_bytes()
    host = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    for i in range(10_000):
        b = hb.DeviceBuffer.from_array(host)
        if i == 0:
            np.testing.assert_array_equal(b.download(count=4), host)
        b.free()
    after = free_device_bytes()
    print(f"free device memory {before} -> {after} bytes over 10k alloc/free", flush=True)
    assert before - after < (64 << 20)


def test_freed_streams_return_their_workspaces():
    """A stream's cached workspaces (split-K partials of a 1024 x 1024 x 2048
    f32 product, the partial sums of a reduction over a 4096-long axis) go
    back to the pool when the stream is freed: free device memory stays
    bounded over many create / evaluate / free cycles. Two streams are
    alive at a time, so queue handles are not simply reused in turn."""
    rng = np.random.default_rng(7)
    a = rng.standard_normal((1024, 2048), dtype=np.float32)
    b = rng.standard_normal((2048, 1024), dtype=np.float32)
    x = rng.standard_normal((4096, 256), dtype=np.float32)
    want_sum = x.astype(np.float64).sum(axis=0)

    def cycle(s):
        ia = s.add_constant(a, meta([1024, 2048]))
        ib = s.add_constant(b, meta([2048, 1024]))
        ix = s.add_constant(x, meta([4096, 256]))
        c = s.add_op(OpKind.MatMul, [ia, ib], meta([1024, 1024]))
        r = s.add_op(OpKind.Sum(0), [ix], meta([256]))
        s.eval(c)
        s.eval(r)
        got = s.get_buffer(r)
        assert np.max(np.abs(got - want_sum)) < 1e-2, np.max(np.abs(got - want_sum))
        assert np.isfinite(s.get_buffer(c)).all()

    keep = hb.HipStream()
    cycle(keep)
    for _ in range(3):
        s = hb.HipStream()
        cycle(s)
        s.close()
    hb.synchronize()
    before = free_device_bytes()
    for i in range(24):
        s = hb.HipStream()
        cycle(s)
        old, keep = keep, s
        old.close()
    keep.close()
    hb.synchronize()
    after = free_device_bytes()
    print(f"free device memory {before} -> {after} bytes over 24 stream cycles", flush=True)
    assert before - after < (64 << 20)
