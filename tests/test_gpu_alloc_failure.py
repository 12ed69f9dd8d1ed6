"""Forced device-allocation failures (mlxhip_debug_fail_allocations): every
allocation point of a stream evaluation, a decoder and a device buffer fails
in turn. Each failure must surface as MlxError::FfiFailed through the C ABI
(the reference's error contract, crates/mlx-core/src/lib.rs:31-50), leave no
crash and no leak, and the library must work again once the hook is reset.
The reference forces its error paths with bad shapes and parameters only
(crates/mlx-core/tests/attention_golden.rs:259-302); running out of device
memory is the failure a HIP backend adds."""
import ctypes as C

import numpy as np
import pytest

from oxidizedmlx_amd import abi, nn
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd.opkind import OpKind, meta

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip")]


@pytest.fixture
def hook():
    L = abi.load_library()
    yield lambda after: L.mlxhip_debug_fail_allocations(after)
    L.mlxhip_debug_fail_allocations(-1)


def free_device_bytes() -> int:
    rt = C.CDLL("libamdhip64.so.7")  # the runtime the library loaded
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert rt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def small_graph():
    """x [64, 96] -> softmax(x @ w) + b, materialising several buffers."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 96)).astype(np.float32)
    w = rng.standard_normal((96, 80)).astype(np.float32)
    b = rng.standard_normal((64, 80)).astype(np.float32)
    s = hb.HipStream()
    xi = s.add_constant(x, meta([64, 96]))
    wi = s.add_constant(w, meta([96, 80]))
    bi = s.add_constant(b, meta([64, 80]))
    mm = s.add_op(OpKind.MatMul, [xi, wi], meta([64, 80]))
    sm = s.add_op(OpKind.Softmax(1), [mm], meta([64, 80]))
    out = s.add_op(OpKind.Add, [sm, bi], meta([64, 80]))
    return s, out


def test_stream_eval_fails_cleanly_at_every_allocation(hook):
    s, out = small_graph()
    s.eval(out)
    want = s.get_buffer(out).copy()
    s.close()
    hb.synchronize()
    before = free_device_bytes()
    failures = 0
    for after in range(0, 40):
        print(f"stream eval, allocation {after} fails", flush=True)
        hook(after)
        try:
            s, out = small_graph()
            s.eval(out)
            got = s.get_buffer(out)
        except abi.FfiFailed as e:
            failures += 1
            assert "alloc" in str(e), str(e)
            hook(-1)
            s.close()
            continue
        hook(-1)
        np.testing.assert_array_equal(got, want)  # enough allocations left: unchanged result
        s.close()
        break
    else:
        pytest.fail("the evaluation never completed with 40 allocations allowed")
    assert failures >= 1
    hook(-1)
    s, out = small_graph()
    s.eval(out)
    np.testing.assert_array_equal(s.get_buffer(out), want)
    s.close()
    hb.synchronize()
    assert before - free_device_bytes() < (64 << 20)


def test_buffer_alloc_forced_failure(hook):
    hook(0)
    with pytest.raises(abi.FfiFailed, match="allocation-failure hook"):
        hb.DeviceBuffer(4096)
    hook(-1)
    b = hb.DeviceBuffer.from_array(np.arange(8, dtype=np.float32))
    np.testing.assert_array_equal(b.download(), np.arange(8, dtype=np.float32))
    b.free()


def test_decoder_fails_cleanly_at_every_allocation(hook):
    cfg = nn.DecoderConfig(n_layers=1, d_model=64, n_heads=4, vocab=100, max_batch=2, max_seq=8)
    hb.synchronize()
    before = free_device_bytes()
    built = None
    for after in range(0, 40):
        print(f"decoder, allocation {after} fails", flush=True)
        hook(after)
        try:
            built = hb.HipDecoder(cfg)
        except abi.FfiFailed as e:
            assert "alloc" in str(e), str(e)
            continue
        finally:
            hook(-1)
        break
    assert built is not None, "the decoder was never created with 40 allocations allowed"
    built.load(nn.decoder_params(cfg, 1))
    toks = built.generate(np.array([[1, 2, 3]]), 2)
    assert toks.shape == (1, 2)
    built.close()
    hb.synchronize()
    assert before - free_device_bytes() < (64 << 20)
