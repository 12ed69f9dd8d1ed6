#!/usr/bin/env python3
"""Writes the committed golden fixtures of this directory.

Two fixtures:

* ``known_answers.json`` -- the reference's own known-answer tests, copied as
  data (inputs, expected outputs and the tolerance the reference asserts),
  each with the file:line of the test it comes from. The reference holds no
  golden-vector files; all of its expected values are inline in its tests.

* ``parity_vectors.npz`` -- inputs for the shapes and seeds of the
  reference's backend-parity suite (crates/mlx-parity/tests/*.rs), generated
  with ``gen_data`` (crates/mlx-parity/src/lib.rs:22-34) restated here in
  integer Python, and the expected outputs computed in float64 numpy from the
  textbook formula of each op (not from this repository's oracle or kernels).
  Softmax / LayerNorm / RmsNorm use the reference's definitions
  (crates/mlx-core/src/cpu_kernels.rs: biased variance, eps inside the
  square root, tanh-approximate GELU); VJPs are the analytic derivatives.

Run from the repository root: ``python tests/golden/make_golden.py``.
Everything is deterministic; re-running rewrites identical files.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def gen_data(n: int, seed: int) -> np.ndarray:
    """crates/mlx-parity/src/lib.rs:22-34: LCG (Numerical Recipes constants),
    (state >> 33) / 2^31 * 2 - 1 in float64, rounded once to float32."""
    state, out = seed % (1 << 64), []
    for _ in range(n):
        state = (state * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        out.append((state >> 33) / float(1 << 31) * 2.0 - 1.0)
    return np.array(out, dtype=np.float64).astype(np.float32)


# ── float64 references of each op ──────────────────────────────────────────

def softmax(x):
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def layer_norm(x, eps):
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps)


def rms_norm(x, eps):
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)


def silu(x):
    return x / (1.0 + np.exp(-x))


GELU_K = math.sqrt(2.0 / math.pi)


def gelu(x):
    return 0.5 * x * (1.0 + np.tanh(GELU_K * (x + 0.044715 * x ** 3)))


def silu_vjp(dy, x):
    s = 1.0 / (1.0 + np.exp(-x))
    return dy * s * (1.0 + x * (1.0 - s))


def gelu_vjp(dy, x):
    t = np.tanh(GELU_K * (x + 0.044715 * x ** 3))
    return dy * (0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * GELU_K * (1.0 + 3.0 * 0.044715 * x * x))


def softmax_vjp(dy, s):
    return s * (dy - (dy * s).sum(axis=-1, keepdims=True))


def layer_norm_vjp(dy, x, eps):
    d = x.shape[-1]
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    inv = 1.0 / np.sqrt(var + eps)
    xh = (x - mu) * inv
    return inv * (dy - dy.sum(-1, keepdims=True) / d - xh * (dy * xh).sum(-1, keepdims=True) / d)


def rms_norm_vjp(dy, x, eps):
    d = x.shape[-1]
    inv = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    y = x * inv
    return inv * (dy - y * (dy * y).sum(-1, keepdims=True) / d)


# ── fixtures ───────────────────────────────────────────────────────────────

def known_answers() -> list[dict]:
    f = np.float32
    e = [math.exp(1.0), math.exp(2.0), math.exp(3.0)]
    s0 = sum(e)
    rms4 = math.sqrt(7.5)
    rms3 = math.sqrt(14.0 / 3.0)
    return [
        {"op": "MatMul", "inputs": [[1, 2, 3, 4], [5, 6, 7, 8]], "shapes": [[2, 2], [2, 2]],
         "out_shape": [2, 2], "expected": [19, 22, 43, 50], "atol": 0.0, "rtol": 0.0,
         "source": "crates/mlx-core/src/cpu_kernels.rs:996-1008 (also tensor.rs:909, "
                   "mlx-conformance/tests/basic.rs:71)"},
        {"op": "MatMul", "inputs": [[i + 1 for i in range(16)], [float(f((i + 1) * f(0.1))) for i in range(16)]],
         "shapes": [[4, 4], [4, 4]], "out_shape": [4, 4], "check_first": 1, "expected": [9.0],
         "atol": 1e-4, "rtol": 1e-4, "source": "crates/mlx-conformance/tests/parity_gate.rs:72-83"},
        {"op": "Softmax", "axis": 1, "inputs": [[1, 2, 3, 1, 1, 1]], "shapes": [[2, 3]], "out_shape": [2, 3],
         "expected": [e[0] / s0, e[1] / s0, e[2] / s0, 1 / 3, 1 / 3, 1 / 3], "atol": 1e-5, "rtol": 1e-5,
         "source": "crates/mlx-conformance/tests/parity_gate.rs:108-133"},
        {"op": "RmsNorm", "eps": 1e-5, "inputs": [[1, 2, 3, 4]], "shapes": [[4]], "out_shape": [4],
         "expected": [1 / rms4, 2 / rms4, 3 / rms4, 4 / rms4], "atol": 1e-4, "rtol": 1e-4,
         "source": "crates/mlx-conformance/tests/parity_gate.rs:144-152"},
        {"op": "LayerNorm", "eps": 1e-5, "inputs": [[2, 4, 6, 8]], "shapes": [[4]], "out_shape": [4],
         "expected": [(v - 5) / math.sqrt(5) for v in (2, 4, 6, 8)], "atol": 1e-4, "rtol": 1e-4,
         "source": "crates/mlx-conformance/tests/parity_gate.rs:157-170"},
        {"op": "LayerNorm", "eps": 1e-5, "inputs": [[1, 2, 3]], "shapes": [[1, 3]], "out_shape": [1, 3],
         "expected": [-1.2247, 0.0, 1.2247], "atol": 1e-3, "rtol": 1e-3,
         "source": "crates/mlx-nn/src/lib.rs:82-92"},
        {"op": "RmsNorm", "eps": 1e-5, "inputs": [[1, 2, 3]], "shapes": [[1, 3]], "out_shape": [1, 3],
         "expected": [1 / rms3, 2 / rms3, 3 / rms3], "atol": 1e-4, "rtol": 1e-4,
         "source": "crates/mlx-nn/src/lib.rs:174-184"},
        {"op": "Silu", "inputs": [[0.0, 1.0, -1.0]], "shapes": [[3]], "out_shape": [3],
         "expected": [0.0, 0.7311, -0.2689], "atol": 1e-3, "rtol": 0.0,
         "source": "crates/mlx-core/src/cpu_kernels.rs:1082-1091"},
        {"op": "Neg", "inputs": [[1.0, -2.0, 3.0]], "shapes": [[3]], "out_shape": [3],
         "expected": [-1.0, 2.0, -3.0], "atol": 0.0, "rtol": 0.0,
         "source": "crates/mlx-core/src/cpu_kernels.rs:1027-1035"},
        {"op": "Transpose", "inputs": [[1, 2, 3, 4, 5, 6]], "shapes": [[2, 3]], "out_shape": [3, 2],
         "expected": [1, 4, 2, 5, 3, 6], "atol": 0.0, "rtol": 0.0,
         "source": "crates/mlx-core/src/tensor.rs:958-969"},
    ]


def parity_vectors() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}

    def put(name, inputs, expected):
        for i, a in enumerate(inputs):
            out[f"{name}/in{i}"] = np.ascontiguousarray(a, np.float32)
        out[f"{name}/expected"] = np.ascontiguousarray(expected, np.float64)

    # MatMul: crates/mlx-parity/tests/matmul.rs:12-52 (a seed 70 + m, b seed 80 + n)
    for m, k, n in [(4, 4, 4), (64, 64, 64), (17, 31, 23)]:
        a = gen_data(m * k, 70 + m).reshape(m, k)
        b = gen_data(k * n, 80 + n).reshape(k, n)
        put(f"matmul_{m}x{k}x{n}", [a, b], a.astype(np.float64) @ b.astype(np.float64))
    # Activations: crates/mlx-parity/tests/activations.rs:12-71
    x = gen_data(32 * 64, 61).reshape(32, 64)
    put("silu_32x64", [x], silu(x.astype(np.float64)))
    x = gen_data(32 * 64, 63).reshape(32, 64)
    put("gelu_32x64", [x], gelu(x.astype(np.float64)))
    x = gen_data(4 * 8, 64).reshape(4, 8)
    put("softmax_4x8", [x], softmax(x.astype(np.float64)))
    x = gen_data(32 * 128, 65).reshape(32, 128)
    put("softmax_32x128", [x], softmax(x.astype(np.float64)))
    # Norms: crates/mlx-parity/tests/normalization.rs:15-76, eps 1e-5
    for seed, (r, c) in [(90, (4, 8)), (91, (32, 128))]:
        x = gen_data(r * c, seed).reshape(r, c)
        put(f"layer_norm_{r}x{c}", [x], layer_norm(x.astype(np.float64), 1e-5))
    for seed, (r, c) in [(93, (4, 8)), (94, (32, 128))]:
        x = gen_data(r * c, seed).reshape(r, c)
        put(f"rms_norm_{r}x{c}", [x], rms_norm(x.astype(np.float64), 1e-5))
    # VJPs: inputs [grad_output, original_input] (graph.rs VJP ops); shapes of
    # the norm tests, seeds of this fixture (the reference has no VJP parity test).
    dy = gen_data(32 * 128, 201).reshape(32, 128)
    x = gen_data(32 * 128, 202).reshape(32, 128)
    d64, x64 = dy.astype(np.float64), x.astype(np.float64)
    put("layer_norm_vjp_32x128", [dy, x], layer_norm_vjp(d64, x64, 1e-5))
    put("rms_norm_vjp_32x128", [dy, x], rms_norm_vjp(d64, x64, 1e-5))
    put("silu_vjp_32x128", [dy, x], silu_vjp(d64, x64))
    put("gelu_vjp_32x128", [dy, x], gelu_vjp(d64, x64))
    s = softmax(x64).astype(np.float32)
    put("softmax_vjp_32x128", [dy, s], softmax_vjp(d64, s.astype(np.float64)))
    return out


def main() -> None:
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(known_answers(), f, indent=1)
    np.savez_compressed(os.path.join(HERE, "parity_vectors.npz"), **parity_vectors())
    print("wrote known_answers.json and parity_vectors.npz")


if __name__ == "__main__":
    main()
