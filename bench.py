#!/usr/bin/env python3
"""Benchmark of the mlx-hip hot path on one MI355X.

One step = one pass of the hot path over one batch of synthetic input:
  * bf16 GEMM C = A.B at M = N = K = 4096, f32 accumulate, bf16 C (headline);
  * row softmax, LayerNorm (eps 1e-5) and RMSNorm (eps 1e-5) over a
    [4096, 4096] f32 tensor, x ~ N(0, 2^2) (config 2);
  * the fused chain y = SiLU(x*w + b), w, b ~ U(-1, 1), same shape (config 2).
``value`` is the GEMM's TFLOP/s. The K timed steps run kernel by kernel: each
kernel's K launches go back to back on one stream between two HIP events, and
its time is the events' interval / K (the launch and event-marker overheads
overlap the previous launch instead of adding to each one). Every kernel's
large operand and output buffers rotate over SETS copies, so between two reads of
one buffer at least (SETS-1) x 96 MiB of other traffic passes (384 MiB for
the GEMM, more for the row kernels), more than the 256 MiB Infinity Cache:
operands come from HBM, not from a cache warmed by the previous launch.
``ms_per_step`` is the sum of the per-kernel times of the five step kernels
(one pass of the hot path).
The CPU baseline is the oracle (the C restatement of the reference's mlx-cpu
kernels, single-threaded) timed on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
IDLE_S = 0.2                   # idle device time before each workload's warmup
BF16_PEAK_TFLOPS = 2516.6      # dense bf16 MFMA
SEEDS = {"A": 0x5EED0006, "B": 0x5EED0007, "x": 0x5EED0003, "w": 0x5EED0004, "b": 0x5EED0005}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo (platform.processor()
    gives only the architecture on Linux)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(target_s: float) -> dict:
    """Oracle timings on bounded samples (rank 0, N = 1 only): the 4096^3
    GEMM on a row sample scaled by flop count, config 1 (f32 512^3), the row
    ops and the SiLU(x*w+b) chain at full size."""
    from oracle import cpu_ref
    from oxidizedmlx_amd import synth
    from oxidizedmlx_amd.opkind import NodeInput, OpKind, meta
    out = {}
    n = 4096
    A = synth.round_bf16(synth.normal(SEEDS["A"], (n, n)))
    B = synth.round_bf16(synth.normal(SEEDS["B"], (n, n)))
    C = np.zeros((n, n), np.float32)
    rows, t0 = 0, time.perf_counter()
    while rows < n and (time.perf_counter() - t0) < target_s:
        cpu_ref.matmul_rows(A, B, C, rows, 4)
        rows += 4
    dt = time.perf_counter() - t0
    out["gemm"] = {"tflops": 2.0 * rows * n * n / dt / 1e12, "rows": rows, "seconds": dt}
    A1 = synth.normal(0x5EED0001, (512, 512))
    B1 = synth.normal(0x5EED0002, (512, 512))
    C1 = np.zeros((512, 512), np.float32)
    t0 = time.perf_counter()
    cpu_ref.matmul_rows(A1, B1, C1, 0, 512)
    dt = time.perf_counter() - t0
    out["gemm_f32_512_cfg1"] = {"tflops": 2.0 * 512 ** 3 / dt / 1e12, "seconds": dt, "sample": "full"}
    x = synth.normal(SEEDS["x"], (n, n), 0.0, 2.0)
    for name, fn in [("softmax", lambda: cpu_ref.softmax_lastdim(x)),
                     ("layernorm", lambda: cpu_ref.layer_norm(x, 1e-5)),
                     ("rmsnorm", lambda: cpu_ref.rms_norm(x, 1e-5))]:
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        out[name] = {"gbs": 2 * x.nbytes / dt / 1e9, "seconds": dt}
    # The reference's unfused graph: Mul, Add, Silu, each its own node.
    w = synth.uniform(SEEDS["w"], (n, n), -1.0, 1.0)
    bb = synth.uniform(SEEDS["b"], (n, n), -1.0, 1.0)
    cpu, m = cpu_ref.CpuRefBackend(), meta([n, n])
    t0 = time.perf_counter()
    y = cpu.eval_node(OpKind.Mul, [NodeInput(x.reshape(-1), (n, n)), NodeInput(w.reshape(-1), (n, n))], m)
    y = cpu.eval_node(OpKind.Add, [NodeInput(y, (n, n)), NodeInput(bb.reshape(-1), (n, n))], m)
    y = cpu.eval_node(OpKind.Silu, [NodeInput(y, (n, n))], m)
    dt = time.perf_counter() - t0
    out["silu_fma_chain"] = {"gbs": 4 * x.nbytes / dt / 1e9, "seconds": dt,
                             "sample": "full, three oracle nodes (Mul, Add, Silu)"}
    return out


def parity_samples(outs: dict) -> dict:
    """The oracle as checker (part of the CPU-baseline leg, after the timed
    region): sampled rows of each timed output against the oracle on the
    same inputs, as max-abs / max-rel error with the test suite's tolerance
    (assert_allclose semantics, crates/mlx-conformance/src/lib.rs:32-48).
    `outs` maps a kernel name to its downloaded output and inputs."""
    from oracle import cpu_ref
    from oxidizedmlx_amd.opkind import NodeInput, OpKind, meta

    def summary(got, ref, atol, rtol, rows):
        got = np.asarray(got, np.float64).reshape(-1)
        ref = np.asarray(ref, np.float64).reshape(-1)
        d = np.abs(got - ref)
        with np.errstate(divide="ignore", invalid="ignore"):
            rel = np.where(ref != 0, d / np.abs(ref), np.where(d == 0, 0.0, np.inf))
        ok = bool(np.all(d <= atol + rtol * np.abs(ref)))
        return {"max_abs": float(d.max()), "max_rel": float(rel.max()), "rows": rows,
                "atol": atol, "rtol": rtol, "pass": ok}

    res = {}
    for name, o in outs.items():
        kind = o["kind"]
        if kind == "gemm":
            a, b, c, rows = o["a"], o["b"], o["c"], o["rows"]
            ref = np.zeros((a.shape[0], b.shape[1]), np.float32)
            for r in rows:
                cpu_ref.matmul_rows(a, b, ref, int(r), 1)
            atol = 1e-6 * np.sqrt(a.shape[1]) * float(np.abs(a).max()) * float(np.abs(b).max())
            res[name] = summary(c[rows], ref[rows], atol, o["rtol"], len(rows))
        elif kind == "batched":
            got, ref, nrows = [], [], 0
            for bi in range(o["a"].shape[0]):
                a, b = o["a"][bi], o["b"][bi]
                r = np.zeros((a.shape[0], b.shape[1]), np.float32)
                for row in o["rows"]:
                    cpu_ref.matmul_rows(a, b, r, int(row), 1)
                got.append(o["c"][bi][o["rows"]])
                ref.append(r[o["rows"]])
                nrows += len(o["rows"])
            atol = 1e-6 * np.sqrt(o["a"].shape[2]) * float(np.abs(o["a"]).max()) * float(np.abs(o["b"]).max())
            res[name] = summary(np.stack(got), np.stack(ref), atol, o["rtol"], nrows)
        elif kind == "rows":
            x = np.ascontiguousarray(o["x"])
            ref = {"softmax": lambda: cpu_ref.softmax_lastdim(x),
                   "layernorm": lambda: cpu_ref.layer_norm(x, 1e-5),
                   "rmsnorm": lambda: cpu_ref.rms_norm(x, 1e-5)}[o["op"]]()
            res[name] = summary(o["y"], ref, 1e-6, 1e-5, x.shape[0])
        elif kind == "chain":
            x, w, bb = (np.ascontiguousarray(o[k]) for k in ("x", "w", "b"))
            shp = x.shape
            cpu, m = cpu_ref.CpuRefBackend(), meta(list(shp))
            y = cpu.eval_node(OpKind.Mul, [NodeInput(x.reshape(-1), shp), NodeInput(w.reshape(-1), shp)], m)
            y = cpu.eval_node(OpKind.Add, [NodeInput(y, shp), NodeInput(bb.reshape(-1), shp)], m)
            y = cpu.eval_node(OpKind.Silu, [NodeInput(y, shp)], m)
            res[name] = summary(o["y"], y, 1e-6, 1e-6, shp[0])
        elif kind == "attention":
            cpu = cpu_ref.CpuRefBackend()
            got, ref = [], []
            for h in o["heads"]:
                q, k, v = o["q"][h], o["k"][h], o["v"][h]
                t, dh = q.shape
                r = cpu.eval_node(OpKind.Attention(o["scale"], True),
                                  [NodeInput(q.reshape(-1), (t, dh)), NodeInput(k.reshape(-1), (t, dh)),
                                   NodeInput(v.reshape(-1), (t, dh))], meta([t, dh]))
                got.append(o["o"][h])
                ref.append(r)
            vmax = float(np.abs(o["v"]).max())
            res[name] = summary(np.stack(got), np.stack(ref), 2e-6 * vmax, 1e-5, len(o["heads"]) * o["q"].shape[1])
    return res


def cpu_decode_baseline(cfg, params, batch: int) -> dict:
    """The oracle's decoder (mlx-nn layers over the oracle stream, C kernels,
    1 thread) on a bounded sample: position 0 of `batch` sequences (one
    decode step without cache reads; parameter upload excluded)."""
    from oracle.graph import OracleStream
    from oxidizedmlx_amd import nn as mnn
    tok = np.random.default_rng(0x5EED0201).integers(0, cfg.vocab, size=(batch, 1))
    model = mnn.DecoderLM(cfg, OracleStream(), params)
    t0 = time.perf_counter()
    model(tok).to_numpy()
    dt = time.perf_counter() - t0
    return {"tokens_per_s": batch / dt, "seconds": dt,
            "sample": f"one decode position of {batch} sequences"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="bounded CPU-baseline sample of the GEMM (seconds)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="", help="comma list of kernels to time (profiling)")
    ap.add_argument("--decode-eager", action="store_true",
                    help="launch the decode step's kernels one by one instead of replaying its HIP graph")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; --gpus must be 1 "
              "(sharding over several GPUs is designed, not built or run).", file=sys.stderr)
        return 2

    from oxidizedmlx_amd import abi
    from oxidizedmlx_amd import backend as hb
    from oxidizedmlx_amd import synth

    hb.init(0)
    n = 4096
    only = set(filter(None, args.only.split(",")))
    want = lambda k: not only or k in only  # noqa: E731

    log("bench: generating inputs")
    A = synth.bf16_bits(synth.normal(SEEDS["A"], (n, n)))
    B = synth.bf16_bits(synth.normal(SEEDS["B"], (n, n)))
    SETS = 5
    dA = [hb.DeviceBuffer.from_array(A) for _ in range(SETS)]
    dB = [hb.DeviceBuffer.from_array(B) for _ in range(SETS)]
    dC = [hb.DeviceBuffer(n * n * 2) for _ in range(SETS)]
    # Config 1: f32 512^3. Config 3: batched [32,1024,1024]^2 bf16/f16, the
    # transposed-B case, and the odd 1000 x 777 x 1531 (edge tiles), each with
    # f32 accumulation and C in the operands' dtype: the reference's matmul
    # gives its result the left operand's dtype (tensor.rs:274-294).
    A1 = hb.DeviceBuffer.from_array(synth.normal(0x5EED0001, (512, 512)))
    B1 = hb.DeviceBuffer.from_array(synth.normal(0x5EED0002, (512, 512)))
    C1 = hb.DeviceBuffer(512 * 512 * 4)
    # The headline shape in f32, the reference's own arithmetic (its
    # matmul is f32, cpu_kernels.rs:197-230): N(0,1) operands, one set
    # (the split-f32 path reads bf16 planes made each call).
    A32 = synth.normal(SEEDS["A"], (n, n)) if want("gemm_f32_4096") else None
    B32 = synth.normal(SEEDS["B"], (n, n)) if want("gemm_f32_4096") else None
    dA32 = hb.DeviceBuffer.from_array(A32) if want("gemm_f32_4096") else None
    dB32 = hb.DeviceBuffer.from_array(B32) if want("gemm_f32_4096") else None
    dC32 = hb.DeviceBuffer(n * n * 4) if want("gemm_f32_4096") else None
    nb, bt = 1024, 32
    Ab = synth.normal(0x5EED0008, (bt, nb, nb))
    Bb = synth.normal(0x5EED0009, (bt, nb, nb))
    Ab16 = [hb.DeviceBuffer.from_array(synth.bf16_bits(Ab)) for _ in range(SETS)]
    Bb16 = [hb.DeviceBuffer.from_array(synth.bf16_bits(Bb)) for _ in range(SETS)]
    Abh = [hb.DeviceBuffer.from_array(synth.f16_bits(Ab)) for _ in range(SETS)]
    Bbh = [hb.DeviceBuffer.from_array(synth.f16_bits(Bb)) for _ in range(SETS)]
    Cb = [hb.DeviceBuffer(bt * nb * nb * 2) for _ in range(SETS)]
    mo, no, ko = 1000, 777, 1531
    # The config-1 and odd-shape operands (a few MiB) stay cache-resident
    # whatever the rotation; they get one buffer set.
    Ao = hb.DeviceBuffer.from_array(synth.bf16_bits(synth.normal(0x5EED000A, (mo, ko))))
    Bo = hb.DeviceBuffer.from_array(synth.bf16_bits(synth.normal(0x5EED000B, (ko, no))))
    Co = hb.DeviceBuffer(mo * no * 2)
    del Ab, Bb
    x = synth.normal(SEEDS["x"], (n, n), 0.0, 2.0)
    w = synth.uniform(SEEDS["w"], (n, n), -1.0, 1.0)
    bb = synth.uniform(SEEDS["b"], (n, n), -1.0, 1.0)
    row_ops = ("softmax", "layernorm", "rmsnorm", "chain")
    xs = {op: [hb.DeviceBuffer.from_array(x) for _ in range(SETS)] for op in row_ops}
    ys = {op: [hb.DeviceBuffer(x.nbytes) for _ in range(SETS)] for op in row_ops}
    ws = [hb.DeviceBuffer.from_array(w) for _ in range(SETS)]
    bs = [hb.DeviceBuffer.from_array(bb) for _ in range(SETS)]
    stream = hb.create_stream()

    # Config 4: one pre-norm transformer block (d_model 1024, 16 heads,
    # seq 512, batch 4, 4x SiLU MLP), f32, forward and backward through the
    # Stream's autograd. Weights N(0, 0.02^2), x N(0, 1); the loss is
    # sum(block(x) * gy) with gy N(0, 1). Inputs stay in HBM; each step builds
    # the whole graph again from them (constants that read them in place), runs the
    # autograd and evaluates every gradient. Consecutive steps share one
    # asynchronous stream (mlxhip_stream_set_async): eval_many returns once a
    # step's kernels are queued, so the host builds the next step's graph
    # while the GPU runs this one; the kernels still run one after another on
    # one queue. After its eval a step's nodes are cleared (mlxhip_stream_clear):
    # the next step's buffers reuse their HBM in queue order.
    from oxidizedmlx_amd import nn as mnn
    bcfg = mnn.BlockConfig()
    blk_host = {name: synth.normal(0x5EED0100 + i, shp, 0.0, 0.02)
                for i, (name, shp) in enumerate(bcfg.param_shapes().items())}
    blk_host["x"] = synth.normal(0x5EED0180, (bcfg.rows, bcfg.d_model))
    blk_host["gy"] = synth.normal(0x5EED0181, (bcfg.rows, bcfg.d_model))
    blk_dev = {k: hb.DeviceBuffer.from_array(v) for k, v in blk_host.items()}
    del blk_host

    blk = {"stream": None}

    # The same step with the attention through the fused HeadAttention op:
    # one kernel for the forward of every head, two for its gradient, instead
    # of the [64, 512, 512] score, probability and gradient tensors.
    bcfg_fused = dataclasses.replace(bcfg, fused_attention=True)

    def block_step(fused: bool = False) -> None:
        from oxidizedmlx_amd.tensor import Tensor, value_and_grad
        if blk["stream"] is None:
            blk["stream"] = hb.HipStream(async_eval=True)
        st = blk["stream"]
        t = {k: Tensor.view_device(b.ptr, (bcfg.rows, bcfg.d_model) if k in ("x", "gy")
                                   else bcfg.param_shapes()[k], st) for k, b in blk_dev.items()}
        params = {k: t[k] for k in bcfg.param_shapes()}
        loss = mnn.TransformerBlock(bcfg_fused if fused else bcfg, params)(t["x"]).mul(t["gy"]).sum_all()
        _, grads = value_and_grad(loss, list(params.values()) + [t["x"]])
        st.eval_many([g.node for g in grads])
        st.clear()

    # Config 5: greedy decoding with a 12-layer decoder (d_model 768, 12
    # heads, vocab 32000, 4x SiLU MLP), bf16 weights N(0, 0.02^2), batch 8,
    # prompt of 16 uniform-random ids, 128 new tokens. One step = one whole
    # generate (143 positions, prompt included), timed by the decoder's own
    # HIP events around its position loop.
    dcfg = mnn.DecoderConfig()
    d_batch, d_prompt, d_new = 8, 16, 128
    dec = dparams = None
    if want("decode_cfg5"):
        log("bench: decoder parameters")
        dparams = mnn.decoder_params(dcfg, 0x5EED0200)
        dec = hb.HipDecoder(dcfg)
        dec.load(dparams)
        dprompt = np.random.default_rng(0x5EED0201).integers(0, dcfg.vocab, size=(d_batch, d_prompt))

    # Fused causal attention over config 4's heads: 64 heads of [512, 64] f32
    # (mlxhip_attention). Algorithmic work counts the unmasked products only:
    # 2 * dh per (query, visible key) for the scores and again for P.V.
    at_bh, at_t, at_dh = bcfg.batch * bcfg.n_heads, bcfg.seq, bcfg.d_model // bcfg.n_heads
    at_flops = 4.0 * at_dh * at_bh * (at_t * (at_t + 1) // 2)
    at_bufs = {}
    if want("attention_fused_cfg4"):
        at_bufs = {nm: hb.DeviceBuffer.from_array(synth.normal(0x5EED0300 + i, (at_bh, at_t, at_dh)))
                   for i, nm in enumerate("qkv")}
        at_bufs["o"] = hb.DeviceBuffer(at_bh * at_t * at_dh * 4)

    kernels = {
        "gemm_bf16_4096": dict(flops=2.0 * n * n * n, bytes=3 * n * n * 2),
        # Calibration only (never part of a step): a plain 64 MiB copy whose HBM
        # bytes are known, for scaling the FETCH_SIZE / WRITE_SIZE counters.
        "copy_64MiB": dict(bytes=2 * n * n * 4, calibration=True),
        # Further configurations, reported under "kernels" (not the headline).
        # Small problems are launch-bound; their figure includes the host's
        # per-call work between back-to-back calls. ("graph": True would time
        # one replay of the K calls recorded with mlxhip_graph_*; measured on
        # this stack, replays were not faster than the eager calls.)
        "gemm_f32_512_cfg1": dict(flops=2.0 * 512 ** 3, bytes=3 * 512 * 512 * 4, peak=157.3),
        # f32 FLOP/s; the product runs as six bf16 MFMA products of a
        # three-plane split, so its ceiling is the bf16 peak / 6.
        "gemm_f32_4096": dict(flops=2.0 * n ** 3, bytes=0, peak=BF16_PEAK_TFLOPS / 6.0),
        "gemm_bf16_batched_32x1024_cfg3": dict(flops=2.0 * bt * nb ** 3, bytes=bt * nb * nb * 6),
        "gemm_f16_batched_32x1024_cfg3": dict(flops=2.0 * bt * nb ** 3, bytes=bt * nb * nb * 6),
        "gemm_bf16_batched_32x1024_nt_cfg3": dict(flops=2.0 * bt * nb ** 3, bytes=bt * nb * nb * 6),
        "gemm_bf16_odd_1000x777x1531_cfg3": dict(flops=2.0 * mo * no * ko,
                                                  bytes=(mo * ko + ko * no + mo * no) * 2),
        "softmax_4096x4096": dict(bytes=2 * n * n * 4),
        "layernorm_4096x4096": dict(bytes=2 * n * n * 4),
        "rmsnorm_4096x4096": dict(bytes=2 * n * n * 4),
        "silu_fma_chain_4096x4096": dict(bytes=4 * n * n * 4),
        # Timed by wall clock around the steps (graph build, autograd and
        # every kernel), with the device synchronised before and after them,
        # not by events. The block's f32 products run as six bf16 MFMA
        # products of an exact three-plane split (and so does the fused
        # attention's arithmetic), so their ceiling is the bf16 peak / 6
        # (419.4 TFLOP/s f32-equivalent), not the f32 MFMA peak.
        "transformer_block_fwd_bwd_cfg4": dict(flops=3.0 * bcfg.forward_flops(), bytes=0,
                                               peak=BF16_PEAK_TFLOPS / 6.0, wall=True),
        "transformer_block_fwd_bwd_cfg4_fused_attention": dict(flops=3.0 * bcfg.forward_flops(), bytes=0,
                                                               peak=BF16_PEAK_TFLOPS / 6.0, wall=True),
        "decode_cfg5": dict(bytes=dcfg.decode_bytes(d_batch, d_prompt, d_new), decoder=True),
        "attention_fused_cfg4": dict(flops=at_flops, bytes=4 * at_bh * at_t * at_dh * 4,
                                     peak=BF16_PEAK_TFLOPS / 6.0),
    }
    chain = [("mul", 1), ("add", 2), ("silu", 0)]

    dec_ms = []

    def launch(name: str, i: int) -> None:
        j = i % SETS
        if name == "attention_fused_cfg4":
            hb.attention(at_bufs["q"], at_bufs["k"], at_bufs["v"], at_bufs["o"], at_bh, at_t, at_t, at_dh,
                         1.0 / np.sqrt(at_dh), True, stream=stream)
        elif name == "decode_cfg5":
            dec.generate(dprompt, d_new, eager=args.decode_eager)
            dec_ms.append(dec.last_timing()[0])
        elif name == "transformer_block_fwd_bwd_cfg4":
            block_step()
        elif name == "transformer_block_fwd_bwd_cfg4_fused_attention":
            block_step(fused=True)
        elif name == "gemm_bf16_4096":
            hb.gemm(abi.BF16, abi.BF16, False, False, n, n, n, dA[j], n, dB[j], n, dC[j], n, stream=stream)
        elif name == "softmax_4096x4096":
            hb.softmax_rows(xs["softmax"][j], ys["softmax"][j], n, n, stream=stream)
        elif name == "layernorm_4096x4096":
            hb.layernorm_rows(xs["layernorm"][j], ys["layernorm"][j], n, n, 1e-5, stream=stream)
        elif name == "rmsnorm_4096x4096":
            hb.rmsnorm_rows(xs["rmsnorm"][j], ys["rmsnorm"][j], n, n, 1e-5, stream=stream)
        elif name == "gemm_f32_4096":
            hb.gemm(abi.F32, abi.F32, False, False, n, n, n, dA32, n, dB32, n, dC32, n, stream=stream)
        elif name == "gemm_f32_512_cfg1":
            hb.gemm(abi.F32, abi.F32, False, False, 512, 512, 512, A1, 512, B1, 512, C1, 512,
                    stream=stream)
        elif name.startswith("gemm_") and "batched" in name:
            f16 = name.startswith("gemm_f16_")
            dt16 = abi.F16 if f16 else abi.BF16
            hb.gemm(dt16, dt16, False, "_nt_" in name, nb, nb, nb,
                    (Abh if f16 else Ab16)[j], nb, (Bbh if f16 else Bb16)[j], nb, Cb[j], nb, batch=bt,
                    stride_a=nb * nb, stride_b=nb * nb, stride_c=nb * nb, stream=stream)
        elif name == "gemm_bf16_odd_1000x777x1531_cfg3":
            hb.gemm(abi.BF16, abi.BF16, False, False, mo, no, ko, Ao, ko, Bo, no, Co, no,
                    stream=stream)
        elif name == "copy_64MiB":
            hb.ew_chain([], [xs["chain"][j]], ys["chain"][j], n * n, stream=stream)
        else:
            hb.ew_chain(chain, [xs["chain"][j], ws[j], bs[j]], ys["chain"][j], n * n, stream=stream)

    names = [k for k in kernels
             if ((k in only) if kernels[k].get("calibration") else want(k))]
    ev = {k: (hb.Event(), hb.Event()) for k in names}

    # Each workload's warmup steps run right before its timed steps, so no
    # workload is timed on a chip that another one's warmup has just heated
    # (the headline GEMM measured 1045 TFLOP/s after the f32 4096^3 warmups
    # against 1170 TFLOP/s after its own). Before its warmup the device sits
    # idle for IDLE_S, so a short workload is not timed while the power
    # management still holds the clock down after the previous one (config 1
    # measured 8.8-11.3 us per call right after the headline's launches,
    # 7.1 us alone).
    log(f"bench: {args.warmup} warmup + {args.steps} timed steps per workload")
    t0 = time.perf_counter()
    wall_ms = {}
    graphs = []
    for k in names:
        time.sleep(IDLE_S)
        for i in range(args.warmup):
            launch(k, i)
        hb.synchronize(None)
        if kernels[k].get("decoder"):
            dec_ms.clear()
            for i in range(args.steps):
                launch(k, i)
            continue
        if kernels[k].get("wall"):
            hb.synchronize(None)
            w0 = time.perf_counter()
            for i in range(args.steps):
                launch(k, i)
            hb.synchronize(None)
            wall_ms[k] = (time.perf_counter() - w0) * 1e3
            continue
        e0, e1 = ev[k]
        if kernels[k].get("graph"):
            with hb.Graph(stream) as graph:
                for i in range(args.steps):
                    launch(k, i)
            graph.launch()  # the first replay uploads the recorded launches; time the next one
            hb.synchronize(stream)
            e0.record(stream)
            graph.launch()
            e1.record(stream)
            graphs.append(graph)
            continue
        e0.record(stream)
        for i in range(args.steps):
            launch(k, i)
        e1.record(stream)
        hb.synchronize(stream)
    hb.synchronize(stream)
    wall = time.perf_counter() - t0
    if blk["stream"] is not None:
        blk["stream"].close()
        blk["stream"] = None

    res = {}
    for k in names:
        if kernels[k].get("decoder"):
            ms = sum(dec_ms) / len(dec_ms)
        elif k in wall_ms:
            ms = wall_ms[k] / args.steps
        else:
            e0, e1 = ev[k]
            ms = e0.elapsed_ms(e1) / args.steps
        r = {"us": ms * 1e3}
        if "flops" in kernels[k]:
            r["tflops"] = kernels[k]["flops"] / (ms * 1e-3) / 1e12
            r["peak_tflops"] = kernels[k].get("peak", BF16_PEAK_TFLOPS)
            r["frac_mfma_peak"] = r["tflops"] / r["peak_tflops"]
        if kernels[k]["bytes"]:
            r["gbs"] = kernels[k]["bytes"] / (ms * 1e-3) / 1e9
            r["frac_hbm_peak"] = r["gbs"] / HBM_PEAK_GBS
        if kernels[k].get("decoder"):
            r["tokens_per_s"] = d_batch * d_new / (ms * 1e-3)
            r["us_per_position"] = ms * 1e3 / (d_prompt + d_new - 1)
        res[k] = r
        log(f"bench: {k}: {json.dumps(r)}")
    step_kernels = ("gemm_bf16_4096", "softmax_4096x4096", "layernorm_4096x4096", "rmsnorm_4096x4096",
                    "silu_fma_chain_4096x4096")

    def collect_outputs() -> dict:
        """Downloads a sample of every timed output with its inputs. Every
        rotating buffer set holds the same inputs, so set 0's output (written
        by the warmup and the timed launches) stands for all of them."""
        outs = {}
        # One row in each 256-row tile row of the 4096^3 product.
        grows = np.array([256 * t + (37 * t + 5) % 256 for t in range(16)])
        if "gemm_bf16_4096" in res:
            c = synth.bf16_to_f32(dC[0].download(np.uint16, n * n)).reshape(n, n)
            outs["gemm_bf16_4096"] = dict(kind="gemm", a=synth.bf16_to_f32(A), b=synth.bf16_to_f32(B),
                                          c=c, rows=grows, rtol=1e-2)
        if "gemm_f32_4096" in res:
            outs["gemm_f32_4096"] = dict(kind="gemm", a=A32, b=B32, c=dC32.download(np.float32, n * n).reshape(n, n),
                                         rows=grows, rtol=1e-5)
        if "gemm_f32_512_cfg1" in res:
            outs["gemm_f32_512_cfg1"] = dict(
                kind="gemm", a=synth.normal(0x5EED0001, (512, 512)), b=synth.normal(0x5EED0002, (512, 512)),
                c=C1.download(np.float32, 512 * 512).reshape(512, 512), rows=np.arange(512), rtol=1e-5)
        for k in ("gemm_bf16_batched_32x1024_cfg3", "gemm_f16_batched_32x1024_cfg3",
                  "gemm_bf16_batched_32x1024_nt_cfg3"):
            if k not in res:
                continue
            f16 = k.startswith("gemm_f16_")
            rnd = synth.round_f16 if f16 else synth.round_bf16
            a = rnd(synth.normal(0x5EED0008, (bt, nb, nb)))
            b = rnd(synth.normal(0x5EED0009, (bt, nb, nb)))
            if "_nt_" in k:
                b = np.ascontiguousarray(b.transpose(0, 2, 1))
            # The output buffers are shared by the three batched products:
            # rerun this one into set 0 before reading it.
            launch(k, 0)
            hb.synchronize(stream)
            bits = Cb[0].download(np.uint16, bt * nb * nb)
            c = (bits.view(np.float16).astype(np.float32) if f16 else synth.bf16_to_f32(bits)).reshape(bt, nb, nb)
            outs[k] = dict(kind="batched", a=a, b=b, c=c, rows=np.array([0, 300, 700, 1023]), rtol=1e-2)
        if "gemm_bf16_odd_1000x777x1531_cfg3" in res:
            outs["gemm_bf16_odd_1000x777x1531_cfg3"] = dict(
                kind="gemm", a=synth.round_bf16(synth.normal(0x5EED000A, (mo, ko))),
                b=synth.round_bf16(synth.normal(0x5EED000B, (ko, no))),
                c=synth.bf16_to_f32(Co.download(np.uint16, mo * no)).reshape(mo, no), rows=np.arange(0, mo, 40),
                rtol=1e-2)
        rsel = np.arange(0, n, 64)
        for op, k in (("softmax", "softmax_4096x4096"), ("layernorm", "layernorm_4096x4096"),
                      ("rmsnorm", "rmsnorm_4096x4096")):
            if k in res:
                y = ys[op][0].download(np.float32, n * n).reshape(n, n)
                outs[k] = dict(kind="rows", op=op, x=x[rsel], y=y[rsel])
        if "silu_fma_chain_4096x4096" in res:
            y = ys["chain"][0].download(np.float32, n * n).reshape(n, n)
            outs["silu_fma_chain_4096x4096"] = dict(kind="chain", x=x[rsel], w=w[rsel], b=bb[rsel], y=y[rsel])
        if "attention_fused_cfg4" in res:
            q, k_, v = (synth.normal(0x5EED0300 + i, (at_bh, at_t, at_dh)) for i in range(3))
            o = at_bufs["o"].download(np.float32, at_bh * at_t * at_dh).reshape(at_bh, at_t, at_dh)
            outs["attention_fused_cfg4"] = dict(kind="attention", q=q, k=k_, v=v, o=o, heads=[0, 37, 63],
                                                scale=float(np.float32(1.0 / np.sqrt(at_dh))))
        return outs
    total_ms = sum(r["us"] for k, r in res.items() if k in step_kernels) / 1e3

    cpu = parity = None
    if not args.no_cpu and not only:
        log(f"bench: CPU baseline (oracle, 1 thread, ~{args.cpu_seconds:.0f}s GEMM sample)")
        cb = cpu_baseline(args.cpu_seconds)
        cpu = {
            "value": cb["gemm"]["tflops"], "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": (f"{cb['gemm']['rows']} of 4096 rows of the 4096^3 product by the oracle's "
                       f"i-j-p f32 loop on bf16-rounded inputs ({cb['gemm']['seconds']:.1f}s), "
                       f"scaled by flop count; host {cpu_model()}, 1 core of {os.cpu_count()}"),
            "kernels": {k: v for k, v in cb.items() if k != "gemm"},
        }
        if dparams is not None:
            cpu["kernels"]["decode_cfg5"] = cpu_decode_baseline(dcfg, dparams, d_batch)
        log("bench: parity of sampled outputs against the oracle")
        parity = parity_samples(collect_outputs())
        for k, v in parity.items():
            log(f"bench: parity {k}: {json.dumps(v)}")

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("gemm_bf16_4096")

    g = res.get("gemm_bf16_4096")
    line = {
        "metric": "GEMM TFLOP/s + %MFMA peak at 4096^3; softmax/norm GB/s as % of HBM peak",
        "value": g["tflops"] if g else None,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": total_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (SplitMix64/Box-Muller N(0,1) GEMM operands; config-2 N(0,4), U(-1,1))",
        "config": {"workload": "bf16 GEMM 4096^3 (f32 acc, bf16 C) + softmax/LayerNorm/RMSNorm "
                               "+ SiLU(x*w+b) over [4096,4096] f32 (config 2)",
                   "M": n, "N": n, "K": n, "rows": n, "cols": n},
        "roofline": ({"bound": "mfma", "achieved": g["tflops"], "peak": BF16_PEAK_TFLOPS,
                      "unit": "TFLOP/s", "frac": g["tflops"] / BF16_PEAK_TFLOPS,
                      "traffic": traffic} if g else None),
        "cpu_baseline": cpu,
        "parity": parity,
        "kernels": res,
        "wall_s": wall,
    }
    print(json.dumps(line), flush=True)
    hb.destroy_stream(stream)
    return 0


if __name__ == "__main__":
    sys.exit(main())
