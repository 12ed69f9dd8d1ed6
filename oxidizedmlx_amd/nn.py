"""mlx-nn layers over lazy tensors (crates/mlx-nn/src): Linear, RmsNorm,
LayerNorm, causal self-attention, the SiLU MLP and a pre-norm transformer
block, built only from ops that have a VJP so that autograd runs through the
whole block.

The reference's MultiHeadAttention works on one [seq, d_model] sequence
with per-head Narrow and a fused Attention op (crates/mlx-nn/src/attention.rs:
47-111), none of which has a VJP (crates/mlx-autograd/src/vjp.rs:173-176).
``CausalSelfAttention`` composes the same computation from differentiable
ops instead: per-head views by Reshape/Transpose, the batched (rank-3)
MatMul, Mul by the 1/sqrt(d_head) scale, Add of a causal mask holding -1e9
above the diagonal (the fill value of cpu_attention, crates/mlx-core/src/
cpu_kernels.rs:786-788), Softmax over the last axis and a second batched
MatMul.
"""
from __future__ import annotations

import functools
import math
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

from . import abi
from .tensor import Tensor


class Linear:
    """y = x @ W^T + b, W [out, in], b [out] (crates/mlx-nn/src/linear.rs:34-43)."""

    def __init__(self, weight: Tensor, bias: Optional[Tensor] = None):
        self.weight = weight
        self.bias = bias

    def forward(self, x: Tensor) -> Tensor:
        y = x.matmul(self.weight.transpose())
        if self.bias is not None:
            y = y.add(self.bias.broadcast_to(y.shape))
        return y

    __call__ = forward


class RmsNorm:
    """x / sqrt(mean(x^2) + eps) over the last axis (crates/mlx-nn/src/norm.rs:43-67)."""

    def __init__(self, dim: int, eps: float = 1e-5):
        self.dim, self.eps = dim, eps

    def forward(self, x: Tensor) -> Tensor:
        if not x.shape:
            raise abi.InvalidArgument("RmsNorm requires at least 1D input")
        if x.shape[-1] != self.dim:
            raise abi.InvalidArgument(f"RmsNorm expected last dim {self.dim}, got {x.shape[-1]}")
        return x.rms_norm(self.eps)

    __call__ = forward


class LayerNorm:
    """(x - mean) / sqrt(var + eps) over the last axis (crates/mlx-nn/src/norm.rs:12-36)."""

    def __init__(self, dim: int, eps: float = 1e-5):
        self.dim, self.eps = dim, eps

    def forward(self, x: Tensor) -> Tensor:
        if not x.shape or x.shape[-1] != self.dim:
            raise abi.InvalidArgument(f"LayerNorm expected last dim {self.dim}")
        return x.layer_norm(self.eps)

    __call__ = forward


MASK_FILL = -1e9


@functools.lru_cache(maxsize=8)
def causal_mask(seq: int) -> np.ndarray:
    """[seq, seq] additive mask: 0 on and below the diagonal, -1e9 above
    (read-only, shared between calls)."""
    m = np.triu(np.full((seq, seq), MASK_FILL, np.float32), 1)
    m.setflags(write=False)
    return m


_DEVICE_CONSTANTS: Dict[tuple, object] = {}


def _fixed_constant(key: tuple, values: np.ndarray, shape, st) -> Tensor:
    """A constant that is the same in every graph (the attention scale, the
    causal mask). On a stream that reads device memory in place (HipStream)
    it is uploaded once per process and each graph takes a view of it, so a
    training step copies nothing from the host; other streams take it as an
    ordinary constant."""
    if not hasattr(st, "add_constant_view"):
        return Tensor.from_f32_on_stream(values, shape, st)
    buf = _DEVICE_CONSTANTS.get(key)
    if buf is None:
        from .backend import DeviceBuffer
        buf = DeviceBuffer.from_array(np.ascontiguousarray(values, dtype=np.float32).reshape(-1))
        _DEVICE_CONSTANTS[key] = buf
    return Tensor.view_device(buf.ptr, shape, st)


class CausalSelfAttention:
    """Causal multi-head self-attention over x [batch*seq, d_model] (rows
    ordered batch-major), with Q/K/V/output projections as Linear layers."""

    def __init__(self, wq: Linear, wk: Linear, wv: Linear, wo: Linear, n_heads: int, batch: int, seq: int,
                 fused: bool = False):
        self.wq, self.wk, self.wv, self.wo = wq, wk, wv, wo
        self.h, self.b, self.s = n_heads, batch, seq
        # fused: the scores, mask, softmax and P.V of every head as one
        # HeadAttention op (fused forward kernel, fused backward through its
        # VJP) instead of MatMul, Mul, Add, Softmax, MatMul. Same function;
        # needs a HIP stream (the oracle has no such op).
        self.fused = fused

    def _heads(self, t: Tensor) -> Tensor:
        # [B*S, D] -> [B, S, H, Dh] -> [B, H, S, Dh] -> [B*H, S, Dh]
        d = t.shape[1]
        dh = d // self.h
        return (t.reshape((self.b, self.s, self.h, dh)).transpose((0, 2, 1, 3))
                .reshape((self.b * self.h, self.s, dh)))

    def forward(self, x: Tensor) -> Tensor:
        bs, d = x.shape
        if bs != self.b * self.s or d % self.h:
            raise abi.InvalidArgument(f"attention input {list(x.shape)} does not match "
                                      f"batch {self.b} x seq {self.s}, {self.h} heads")
        dh = d // self.h
        if self.fused:
            # Heads side by side in the projections' rows: [B*S, D] viewed as
            # [B, S, D], no head split or merge.
            q, k, v = (lin(x).reshape((self.b, self.s, d)) for lin in (self.wq, self.wk, self.wv))
            o = q.head_attention(k, v, 1.0 / math.sqrt(dh), True, heads=self.h)   # [B, S, D]
            return self.wo(o.reshape((bs, d)))
        q, k, v = self._heads(self.wq(x)), self._heads(self.wk(x)), self._heads(self.wv(x))
        scores = q.matmul(k.transpose((0, 2, 1)))                      # [B*H, S, S]
        st = x.stream
        scale = _fixed_constant(("scale", dh), np.array([1.0 / math.sqrt(dh)], np.float32), (), st)
        mask = _fixed_constant(("causal", self.s), causal_mask(self.s), (self.s, self.s), st)
        scale, mask = scale.broadcast_to(scores.shape), mask.broadcast_to(scores.shape)
        p = scores.mul(scale).add(mask).softmax(-1)
        o = p.matmul(v)                                                 # [B*H, S, Dh]
        o = o.reshape((self.b, self.h, self.s, dh)).transpose((0, 2, 1, 3)).reshape((bs, d))
        return self.wo(o)

    __call__ = forward


class MultiHeadAttention:
    """The reference's multi-head causal self-attention over one sequence x
    [seq, model_dim] (crates/mlx-nn/src/attention.rs:12-111): Q/K/V Linear
    projections, [seq, H, Dh] -> [H, seq, Dh] per projection, then per head a
    Narrow of one head, a Reshape to [seq, Dh] and the fused Attention op
    (scale 1/sqrt(Dh), causal), the heads concatenated along axis 1 and the
    output projection. Forward only: Narrow, Attention and Concatenate have
    no VJP in the reference (crates/mlx-autograd/src/vjp.rs:173-176)."""

    def __init__(self, wq: Linear, wk: Linear, wv: Linear, wo: Linear, n_heads: int):
        self.wq, self.wk, self.wv, self.wo = wq, wk, wv, wo
        self.n_heads = n_heads
        self.head_dim = wq.weight.shape[0] // n_heads   # attention.rs:28-31

    def forward_causal(self, x: Tensor) -> Tensor:
        seq = x.shape[0]
        h, dh = self.n_heads, self.head_dim
        scale = float(np.float32(1.0) / np.sqrt(np.float32(dh)))

        def heads(t: Tensor) -> Tensor:
            return t.reshape((seq, h, dh)).transpose((1, 0, 2))

        q, k, v = heads(self.wq(x)), heads(self.wk(x)), heads(self.wv(x))
        outs = []
        for i in range(h):
            qh = q.narrow(0, i, 1).reshape((seq, dh))
            kh = k.narrow(0, i, 1).reshape((seq, dh))
            vh = v.narrow(0, i, 1).reshape((seq, dh))
            outs.append(qh.attention(kh, vh, scale, True))
        return self.wo(Tensor.cat(outs, 1))


class Mlp:
    """down(silu(up(x))), hidden = 4 * d_model in the block below."""

    def __init__(self, up: Linear, down: Linear):
        self.up, self.down = up, down

    def forward(self, x: Tensor) -> Tensor:
        return self.down(self.up(x).silu())

    __call__ = forward


@dataclass
class BlockConfig:
    d_model: int = 1024
    n_heads: int = 16
    seq: int = 512
    batch: int = 4
    mlp_ratio: int = 4
    eps: float = 1e-5
    # Attention through the fused HeadAttention op (forward and VJP kernels)
    # instead of the composed MatMul / Softmax graph; HIP streams only.
    fused_attention: bool = False

    @property
    def hidden(self) -> int:
        return self.mlp_ratio * self.d_model

    @property
    def rows(self) -> int:
        return self.batch * self.seq

    def param_shapes(self) -> Dict[str, tuple]:
        d, h = self.d_model, self.hidden
        return {"wq": (d, d), "bq": (d,), "wk": (d, d), "bk": (d,), "wv": (d, d), "bv": (d,),
                "wo": (d, d), "bo": (d,), "w1": (h, d), "b1": (h,), "w2": (d, h), "b2": (d,)}

    def forward_flops(self) -> int:
        """GEMM flops of one forward pass (backward: twice this)."""
        r, d, h, s, b, nh = self.rows, self.d_model, self.hidden, self.seq, self.batch, self.n_heads
        proj = 2 * r * d * d * 4           # Q, K, V, output projections
        mlp = 2 * r * d * h * 2            # up and down
        attn = 2 * (b * nh) * s * s * (d // nh) * 2   # scores and P.V
        return proj + mlp + attn


class TransformerBlock:
    """Pre-norm block: h = x + attn(rms(x)); y = h + mlp(rms(h))."""

    def __init__(self, cfg: BlockConfig, params: Dict[str, Tensor]):
        p = params
        self.cfg = cfg
        self.norm1 = RmsNorm(cfg.d_model, cfg.eps)
        self.norm2 = RmsNorm(cfg.d_model, cfg.eps)
        self.attn = CausalSelfAttention(Linear(p["wq"], p["bq"]), Linear(p["wk"], p["bk"]),
                                        Linear(p["wv"], p["bv"]), Linear(p["wo"], p["bo"]),
                                        cfg.n_heads, cfg.batch, cfg.seq, fused=cfg.fused_attention)
        self.mlp = Mlp(Linear(p["w1"], p["b1"]), Linear(p["w2"], p["b2"]))

    def forward(self, x: Tensor) -> Tensor:
        h = x.add(self.attn(self.norm1(x)))
        return h.add(self.mlp(self.norm2(h)))

    __call__ = forward


# ── decoder-only language model (greedy decode loop) ─────────────────────────

@dataclass
class DecoderConfig:
    """Decoder-only model from mlx-nn layers: Embedding, n_layers pre-norm
    TransformerBlocks (causal attention, SiLU MLP of ``hidden`` = mlp_ratio x
    d_model), final RmsNorm, LM-head Linear without bias."""
    n_layers: int = 12
    d_model: int = 768
    n_heads: int = 12
    vocab: int = 32000
    mlp_ratio: int = 4
    eps: float = 1e-5
    max_batch: int = 8
    max_seq: int = 144

    @property
    def hidden(self) -> int:
        return self.mlp_ratio * self.d_model

    def block(self, batch: int, seq: int) -> BlockConfig:
        return BlockConfig(self.d_model, self.n_heads, seq, batch, self.mlp_ratio, self.eps)

    def step_weight_bytes(self) -> int:
        """bf16 parameter bytes one decode step reads: every block's
        projections and biases and the LM head (the embedding is gathered,
        one row per sequence)."""
        d, h = self.d_model, self.hidden
        per_layer = 4 * d * d + 2 * d * h + 4 * d + h + d
        return 2 * (self.n_layers * per_layer + self.vocab * d)

    def decode_bytes(self, batch: int, prompt_len: int, n_new: int) -> int:
        """Algorithmic HBM bytes of one greedy generate over S = prompt_len +
        n_new - 1 positions: per position t the bf16 weights of
        ``step_weight_bytes``, the f32 K and V cache rows of positions 0..t
        read by every layer's attention, the new K/V rows written and the
        gathered bf16 embedding rows."""
        steps = prompt_len + n_new - 1
        kv_row = 2 * batch * self.d_model * 4 * self.n_layers
        return (steps * self.step_weight_bytes() + kv_row * steps * (steps + 1) // 2
                + kv_row * steps + steps * batch * self.d_model * 2)


def decoder_params(cfg: DecoderConfig, seed: int, std: float = 0.02) -> dict:
    """Random-init parameters N(0, std^2), rounded to bf16 (the values the
    bf16 decoder holds), as float32 numpy arrays, drawn in the order below
    from numpy's PCG64 generator seeded with ``seed`` (standard normals in
    float32, scaled by ``std``)."""
    from . import synth
    d, h, V = cfg.d_model, cfg.hidden, cfg.vocab
    rng = np.random.default_rng(seed)

    def draw(shape):
        z = rng.standard_normal(shape, dtype=np.float32)
        z *= np.float32(std)
        return synth.round_bf16(z)

    params = {"embedding": draw((V, d)), "lm_head": draw((V, d)), "layers": []}
    shapes = BlockConfig(d, cfg.n_heads, 1, 1, cfg.mlp_ratio, cfg.eps).param_shapes()
    for _ in range(cfg.n_layers):
        params["layers"].append({name: draw(shape) for name, shape in shapes.items()})
    return params


class Embedding:
    """Rows of weight [num_embeddings, dim] at integer ids (crates/mlx-nn/src/embed.rs)."""

    def __init__(self, weight: Tensor):
        self.weight = weight

    def forward(self, ids: Tensor) -> Tensor:
        return self.weight.embedding_lookup(ids)

    __call__ = forward


class DecoderLM:
    """Causal forward of the decoder over token ids [batch, seq] on any
    stream: logits [batch*seq, vocab] (rows batch-major). Row (b, t) is what
    greedy decoding sees after position t of sequence b."""

    def __init__(self, cfg: DecoderConfig, stream, params: dict):
        self.cfg, self.stream = cfg, stream
        V, d = cfg.vocab, cfg.d_model
        self.embed = Embedding(Tensor.from_f32_on_stream(params["embedding"], (V, d), stream))
        self.lm_head = Linear(Tensor.from_f32_on_stream(params["lm_head"], (V, d), stream))
        shapes = cfg.block(1, 1).param_shapes()
        self.layer_params = [{k: Tensor.from_f32_on_stream(lp[k], shapes[k], stream) for k in shapes}
                             for lp in params["layers"]]
        self.norm = RmsNorm(d, cfg.eps)

    def forward(self, tokens: np.ndarray) -> Tensor:
        tokens = np.asarray(tokens)
        b, s = tokens.shape
        ids = Tensor.from_f32_on_stream(tokens.reshape(-1).astype(np.float32), (b * s,), self.stream)
        x = self.embed(ids)
        for lp in self.layer_params:
            x = TransformerBlock(self.cfg.block(b, s), lp)(x)
        return self.lm_head(self.norm(x))

    __call__ = forward
