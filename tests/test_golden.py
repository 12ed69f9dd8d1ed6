"""The committed golden fixtures (tests/golden/, written by make_golden.py)
against the CPU oracle and, on a GPU, against mlx-hip's eval_node.

* known_answers.json: the reference's own known-answer tests, with the
  tolerance each of them asserts (assert_allclose semantics,
  crates/mlx-conformance/src/lib.rs:32-48: |a - e| <= atol + rtol * |e|).
* parity_vectors.npz: gen_data inputs of the reference's parity suite and
  float64 expected outputs from the textbook formula of each op. Tolerances
  are float32 rounding bounds of the respective op (stated per op below),
  far tighter than the reference's own parity tolerances
  (crates/mlx-parity/tests/*.rs: 1e-4 .. 1e-3).
"""
import json
import os

import numpy as np
import pytest

from oracle.cpu_ref import CpuRefBackend, gen_data
from oxidizedmlx_amd.opkind import NodeInput, OpKind, meta

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")

with open(os.path.join(GOLD, "known_answers.json")) as f:
    KNOWN = json.load(f)
VECTORS = dict(np.load(os.path.join(GOLD, "parity_vectors.npz")))
VECTOR_CASES = sorted({k.split("/")[0] for k in VECTORS})

# op name in the fixtures -> (OpKind, (atol, rtol) for float32 results vs the float64 formula)
F32 = float(np.finfo(np.float32).eps)
VECTOR_OPS = {
    "matmul": (OpKind.MatMul, None),  # K-dependent bound, below
    "silu": (OpKind.Silu, (1e-7, 8 * F32)),
    "gelu": (OpKind.Gelu, (1e-7, 8 * F32)),
    "softmax": (OpKind.Softmax(-1), (1e-8, 16 * F32)),
    "layer_norm": (OpKind.LayerNorm(1e-5), (1e-6, 32 * F32)),
    "rms_norm": (OpKind.RmsNorm(1e-5), (1e-7, 16 * F32)),
    "layer_norm_vjp": (OpKind.LayerNormVjp(1e-5), (1e-5, 1e-5)),
    "rms_norm_vjp": (OpKind.RmsNormVjp(1e-5), (1e-5, 1e-5)),
    "silu_vjp": (OpKind.SiluVjp, (1e-7, 16 * F32)),
    "gelu_vjp": (OpKind.GeluVjp, (1e-7, 32 * F32)),
    "softmax_vjp": (OpKind.SoftmaxVjp(-1), (1e-7, 1e-5)),
}


def known_op(case):
    name = case["op"]
    if name == "Softmax":
        return OpKind.Softmax(case["axis"])
    if name == "LayerNorm":
        return OpKind.LayerNorm(case["eps"])
    if name == "RmsNorm":
        return OpKind.RmsNorm(case["eps"])
    if name == "Transpose":
        return OpKind.Transpose(None)
    return getattr(OpKind, name)


def vector_case(name):
    key = name.rsplit("_", 1)[0]
    op, tol = VECTOR_OPS[key]
    ins = [VECTORS[f"{name}/in{i}"] for i in range(3) if f"{name}/in{i}" in VECTORS]
    exp = VECTORS[f"{name}/expected"]
    if tol is None:  # matmul: sequential f32 sum of K products
        a, b = ins
        k = a.shape[1]
        tol = (2 * k * F32 * float(np.abs(a).max()) * float(np.abs(b).max()), 0.0)
    return op, ins, exp, tol


def check(got, expected, atol, rtol, what):
    got = np.asarray(got, np.float64).reshape(-1)
    expected = np.asarray(expected, np.float64).reshape(-1)
    assert got.shape == expected.shape, what
    err = np.abs(got - expected)
    bound = atol + rtol * np.abs(expected)
    bad = np.flatnonzero(~(err <= bound))
    assert bad.size == 0, (f"{what}: {bad.size} elements out of tolerance; first {bad[0]}: "
                           f"got {got[bad[0]]!r} want {expected[bad[0]]!r} (max abs err {err.max():.3e})")


def run_known(backend, case):
    ins = [NodeInput(np.asarray(d, np.float32), tuple(s)) for d, s in zip(case["inputs"], case["shapes"])]
    out = backend.eval_node(known_op(case), ins, meta(case["out_shape"]))
    n = case.get("check_first", len(out))
    check(out[:n], case["expected"], case["atol"], case["rtol"], f"{case['op']} ({case['source']})")


def run_vector(backend, name):
    op, ins, exp, (atol, rtol) = vector_case(name)
    shape = exp.shape
    nodes = [NodeInput(a.reshape(-1), a.shape) for a in ins]
    out = backend.eval_node(op, nodes, meta(shape))
    check(out, exp, atol, rtol, name)


def test_fixture_inputs_are_gen_data():
    # The fixture's restated gen_data and the oracle's must agree bit for bit
    # (crates/mlx-parity/src/lib.rs:22-34; seeds of crates/mlx-parity/tests/matmul.rs:12-14).
    np.testing.assert_array_equal(VECTORS["matmul_17x31x23/in0"].reshape(-1), gen_data(17 * 31, 70 + 17))
    np.testing.assert_array_equal(VECTORS["matmul_17x31x23/in1"].reshape(-1), gen_data(31 * 23, 80 + 23))


@pytest.mark.usefixtures("oracle_lib")
@pytest.mark.parametrize("case", KNOWN, ids=lambda c: c["op"] + ":" + c["source"].split(" ")[0])
def test_oracle_known_answers(case):
    run_known(CpuRefBackend(), case)


@pytest.mark.usefixtures("oracle_lib")
@pytest.mark.parametrize("name", VECTOR_CASES)
def test_oracle_parity_vectors(name):
    run_vector(CpuRefBackend(), name)


@pytest.mark.gpu
@pytest.mark.parametrize("case", KNOWN, ids=lambda c: c["op"] + ":" + c["source"].split(" ")[0])
def test_hip_known_answers(hip, case):
    run_known(hip.HipBackend(), case)


@pytest.mark.gpu
@pytest.mark.parametrize("name", VECTOR_CASES)
def test_hip_parity_vectors(hip, name):
    run_vector(hip.HipBackend(), name)
