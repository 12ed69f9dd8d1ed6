"""Recorded launch sequences (mlxhip_graph_*): direct kernel calls recorded
on a stream and replayed must give exactly the eager results, on every
replay, with the program's own eager work and synchronisations between
replays (a recorded graph must not hold memset nodes whose effect fades
after the first replay)."""
import math

import numpy as np
import pytest

from oxidizedmlx_amd import abi, synth
from oxidizedmlx_amd import backend as hb

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip")]


def test_recorded_sequence_replays_exactly():
    s = hb.create_stream()
    try:
        n1, mo, no, ko = 512, 300, 277, 531          # split-K f32 GEMM; unaligned bf16 GEMM (pack path)
        A1 = hb.DeviceBuffer.from_array(synth.normal(1, (n1, n1)))
        B1 = hb.DeviceBuffer.from_array(synth.normal(2, (n1, n1)))
        C1 = hb.DeviceBuffer(n1 * n1 * 4)
        Ao = hb.DeviceBuffer.from_array(synth.bf16_bits(synth.normal(3, (mo, ko))))
        Bo = hb.DeviceBuffer.from_array(synth.bf16_bits(synth.normal(4, (ko, no))))
        Co = hb.DeviceBuffer(mo * no * 4)
        x = synth.normal(5, (256, 1000), 0.0, 2.0)
        X = hb.DeviceBuffer.from_array(x)
        Y = hb.DeviceBuffer(x.nbytes)
        Z = hb.DeviceBuffer(x.nbytes)
        q, k, v = (synth.normal(6 + i, (4, 64, 32)) for i in range(3))
        Q, K, V = (hb.DeviceBuffer.from_array(a) for a in (q, k, v))
        O = hb.DeviceBuffer(q.nbytes)
        outs = [(C1, n1 * n1), (Co, mo * no), (Y, x.size), (Z, x.size), (O, q.size)]

        def seq():
            hb.gemm(abi.F32, abi.F32, False, False, n1, n1, n1, A1, n1, B1, n1, C1, n1, stream=s)
            hb.gemm(abi.BF16, abi.F32, False, False, mo, no, ko, Ao, ko, Bo, no, Co, no, stream=s)
            hb.softmax_rows(X, Y, 256, 1000, stream=s)
            hb.ew_chain([("mul", 1), ("silu", 0)], [Y, X], Z, x.size, stream=s)
            hb.attention(Q, K, V, O, 4, 64, 64, 32, 1.0 / math.sqrt(32), True, stream=s)

        seq()
        hb.synchronize(s)
        eager = [b.download(np.float32, n) for b, n in outs]
        with hb.Graph(s) as g:
            seq()
        junk = np.full(max(n for _, n in outs), np.nan, np.float32)
        for rep in range(4):
            for b, n in outs:
                b.upload(junk[:n])
            hb.softmax_rows(X, Y, 256, 1000, stream=s)   # eager work between replays
            hb.synchronize(s)
            g.launch()
            hb.synchronize(s)
            for (b, n), ref in zip(outs, eager):
                np.testing.assert_array_equal(b.download(np.float32, n), ref, err_msg=f"replay {rep}")
        g.close()
    finally:
        hb.destroy_stream(s)


def test_graph_errors():
    with pytest.raises(abi.NullPtr):
        hb.Graph(0)
    L = abi.load_library()
    assert L.mlxhip_graph_begin(None) == abi.ERR_NULL_PTR
    s = hb.create_stream()
    try:
        assert not L.mlxhip_graph_end(s)             # nothing is being recorded
        assert L.mlxhip_last_status() == abi.ERR_FFI_FAILED
        # The failed end of capture is reported once, not again by the next launch.
        x = synth.normal(9, (4, 100))
        X, Y = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(x.nbytes)
        hb.softmax_rows(X, Y, 4, 100, stream=s)
        hb.synchronize(s)
        np.testing.assert_allclose(Y.download(np.float32, x.size).reshape(x.shape).sum(1), 1.0, rtol=1e-5)
        assert L.mlxhip_graph_launch(None, s) == abi.ERR_NULL_PTR
        L.mlxhip_graph_free(None)
    finally:
        hb.destroy_stream(s)


def test_workspace_first_grown_under_capture():
    # A fresh stream has no cached workspace yet: the split-K GEMM, the
    # 16-bit split-K GEMM with packed operands and their tile counters are
    # first allocated while the stream is being recorded. Every replay must
    # match the eager result computed on another stream.
    n1, mo, no, ko = 512, 1000, 777, 1531
    A1 = hb.DeviceBuffer.from_array(synth.normal(11, (n1, n1)))
    B1 = hb.DeviceBuffer.from_array(synth.normal(12, (n1, n1)))
    Ao = hb.DeviceBuffer.from_array(synth.bf16_bits(synth.normal(13, (mo, ko))))
    Bo = hb.DeviceBuffer.from_array(synth.bf16_bits(synth.normal(14, (ko, no))))
    C1, Co = hb.DeviceBuffer(n1 * n1 * 4), hb.DeviceBuffer(mo * no * 4)

    def seq(st):
        hb.gemm(abi.F32, abi.F32, False, False, n1, n1, n1, A1, n1, B1, n1, C1, n1, stream=st)
        hb.gemm(abi.BF16, abi.F32, False, False, mo, no, ko, Ao, ko, Bo, no, Co, no, stream=st)

    e = hb.create_stream()
    s = hb.create_stream()
    try:
        seq(e)
        hb.synchronize(e)
        eager = [C1.download(np.float32, n1 * n1), Co.download(np.float32, mo * no)]
        with hb.Graph(s) as g:
            seq(s)
        for rep in range(3):
            C1.upload(np.full(n1 * n1, np.nan, np.float32))
            Co.upload(np.full(mo * no, np.nan, np.float32))
            g.launch()
            hb.synchronize(s)
            np.testing.assert_array_equal(C1.download(np.float32, n1 * n1), eager[0], err_msg=f"replay {rep}")
            np.testing.assert_array_equal(Co.download(np.float32, mo * no), eager[1], err_msg=f"replay {rep}")
        g.close()
    finally:
        hb.destroy_stream(s)
        hb.destroy_stream(e)
