"""Launch geometry on large tensors.

Row ops split batches of more than 2^22 rows into several launches, and the
per-element kernels cap their grid at 2^18 workgroups and stride over the
rest, so that no dispatch exceeds the 32-bit work-item count whatever the
tensor size. These tests cross both limits and check every element: the rows
on either side of a chunk boundary, and elements past the first grid's worth.
The references are numpy expressions with the same rounding where the result
is exact (bf16 cast, transposition, a two-term sum)."""
import numpy as np
import pytest

from oxidizedmlx_amd import abi
from oxidizedmlx_amd import backend as hb
from oxidizedmlx_amd.opkind import OpKind, meta
from parity import assert_allclose

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip")]

GRID_ELEMS = (1 << 18) * 256  # elements the capped grid covers in one stride


def test_softmax_rows_across_launch_chunks():
    rows, cols = (1 << 22) + 3, 8
    x = np.random.default_rng(11).standard_normal((rows, cols), dtype=np.float32) * 2
    xb, yb = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(x.nbytes)
    print(f"softmax_rows rows={rows} cols={cols}", flush=True)
    hb.softmax_rows(xb, yb, rows, cols)
    hb.synchronize()
    y = yb.download(count=x.size).reshape(rows, cols)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    assert_allclose(y, e / e.sum(axis=1, keepdims=True), 1e-6, 1e-5, "softmax across row chunks")


def test_cast_beyond_one_grid_stride():
    n = GRID_ELEMS + 1000
    x = np.random.default_rng(12).standard_normal(n, dtype=np.float32)
    xb, yb = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(2 * n)
    print(f"cast f32->bf16 n={n}", flush=True)
    hb.cast(xb, abi.F32, yb, abi.BF16, n)
    hb.synchronize()
    u = x.view(np.uint32)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even
    np.testing.assert_array_equal(yb.download(np.uint16, count=n), want)


def test_permute_beyond_one_grid_stride():
    shape = (2, 4097, 8193)  # 67.1 M elements, more than one stride of the capped grid
    assert np.prod(shape) > GRID_ELEMS
    x = np.random.default_rng(13).standard_normal(shape, dtype=np.float32)
    xb, yb = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(x.nbytes)
    print(f"transpose (0,2,1) of {shape}", flush=True)
    hb.eval_node_dev(OpKind.Transpose((0, 2, 1)), [(xb, shape)], meta([2, 8193, 4097]), yb)
    hb.synchronize()
    np.testing.assert_array_equal(yb.download(count=x.size).reshape(2, 8193, 4097), x.transpose(0, 2, 1))


def test_axis_sum_beyond_one_grid_stride():
    # 2^24 + 3 outputs at 64 per workgroup: more outputs than the capped grid
    # has threads. A two-term fold from -0.0 equals numpy's x0 + x1 exactly.
    rows = (1 << 24) + 3
    x = np.random.default_rng(14).standard_normal((rows, 2), dtype=np.float32)
    xb, yb = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(4 * rows)
    print(f"sum(axis=1) of [{rows}, 2]", flush=True)
    hb.eval_node_dev(OpKind.Sum(1), [(xb, (rows, 2))], meta([rows]), yb)
    hb.synchronize()
    np.testing.assert_array_equal(yb.download(count=rows), x[:, 0] + x[:, 1])


def test_broadcast_beyond_32bit_indices():
    # 2^31 + 4096 output elements (8 GiB): past what the 32-bit gather
    # indexes, so the broadcast takes the 64-bit kernel. Rows on either side
    # of element 2^31 and the last row are checked.
    rows, cols = (1 << 19) + 1, 4096
    x = np.random.default_rng(15).standard_normal(cols, dtype=np.float32)
    xb, yb = hb.DeviceBuffer.from_array(x), hb.DeviceBuffer(4 * rows * cols)
    print(f"broadcast [1, {cols}] -> [{rows}, {cols}]", flush=True)
    hb.eval_node_dev(OpKind.Broadcast((rows, cols)), [(xb, (1, cols))], meta([rows, cols]), yb)
    hb.synchronize()
    for r in (0, rows - 2, rows - 1):
        np.testing.assert_array_equal(yb.download(count=cols, offset=4 * r * cols), x)
