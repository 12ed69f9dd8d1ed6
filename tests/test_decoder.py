"""The decoder-only model (greedy decode loop of config 5) on the CPU: the
oracle's DecoderLM (mlx-nn layers over the oracle stream) pinned against an
independent float64 restatement that decodes position by position with a
growing KV cache (the loop of crates/mlx-conformance/tests/ttft_behavior.rs:
101-216), causality, and the decoder's host-side validation (no GPU needed)."""
import ctypes as C

import numpy as np
import pytest

from oracle.graph import OracleStream
from oxidizedmlx_amd import abi, nn

SMALL = nn.DecoderConfig(n_layers=2, d_model=64, n_heads=4, vocab=1000, max_batch=8, max_seq=16)


def f64_kv_decode(cfg, P, tok):
    """Logits [B, T, vocab] by decoding one position at a time in float64:
    rms-norm, Q/K/V projections, K/V appended to a per-layer cache, softmax
    attention of the new query over the cache, residuals, SiLU MLP, final
    rms-norm, LM head."""
    B, T = tok.shape
    d, H = cfg.d_model, cfg.n_heads
    hd = d // H
    f = lambda a: np.asarray(a, np.float64)  # noqa: E731
    rms = lambda v: v / np.sqrt(np.mean(v * v) + cfg.eps)  # noqa: E731
    out = np.zeros((B, T, cfg.vocab))
    for b in range(B):
        K = [[] for _ in P["layers"]]
        V = [[] for _ in P["layers"]]
        for t in range(T):
            x = f(P["embedding"][min(max(int(tok[b, t]), 0), cfg.vocab - 1)])
            for l, lp in enumerate(P["layers"]):
                h = rms(x)
                q = f(lp["wq"]) @ h + f(lp["bq"])
                K[l].append(f(lp["wk"]) @ h + f(lp["bk"]))
                V[l].append(f(lp["wv"]) @ h + f(lp["bv"]))
                Km = np.stack(K[l]).reshape(t + 1, H, hd)
                Vm = np.stack(V[l]).reshape(t + 1, H, hd)
                s = np.einsum("hd,jhd->hj", q.reshape(H, hd), Km) / np.sqrt(hd)
                p = np.exp(s - s.max(1, keepdims=True))
                p /= p.sum(1, keepdims=True)
                x = x + (f(lp["wo"]) @ np.einsum("hj,jhd->hd", p, Vm).reshape(d) + f(lp["bo"]))
                u = f(lp["w1"]) @ rms(x) + f(lp["b1"])
                x = x + (f(lp["w2"]) @ (u / (1.0 + np.exp(-u))) + f(lp["b2"]))
            out[b, t] = f(P["lm_head"]) @ rms(x)
    return out


@pytest.fixture(scope="module")
def small_model():
    P = nn.decoder_params(SMALL, 1234)
    tok = np.random.default_rng(0).integers(0, SMALL.vocab, size=(3, 12))
    return P, tok


def test_oracle_decoder_matches_f64_kv_decode(oracle_lib, small_model):
    P, tok = small_model
    lg = nn.DecoderLM(SMALL, OracleStream(), P)(tok).to_numpy().reshape(3, 12, SMALL.vocab)
    ref = f64_kv_decode(SMALL, P, tok)
    scale = np.abs(ref).max()
    err = np.abs(lg - ref).max()
    assert err <= 1e-5 * scale, (err, scale)


def test_oracle_decoder_is_causal(oracle_lib, small_model):
    """Row (b, t) depends on tokens 0..t only: changing later tokens or
    dropping them leaves earlier rows bit-identical."""
    P, tok = small_model
    full = nn.DecoderLM(SMALL, OracleStream(), P)(tok).to_numpy().reshape(3, 12, -1)
    tok2 = tok.copy()
    tok2[:, 7:] = (tok2[:, 7:] + 1) % SMALL.vocab
    alt = nn.DecoderLM(SMALL, OracleStream(), P)(tok2).to_numpy().reshape(3, 12, -1)
    np.testing.assert_array_equal(alt[:, :7], full[:, :7])
    assert not np.array_equal(alt[:, 7:], full[:, 7:])
    pre = nn.DecoderLM(SMALL, OracleStream(), P)(tok[:, :5]).to_numpy().reshape(3, 5, -1)
    np.testing.assert_array_equal(pre, full[:, :5])


def test_params_are_bf16_values():
    P = nn.decoder_params(SMALL, 7)
    for a in [P["embedding"], P["lm_head"], *P["layers"][0].values()]:
        u = a.view(np.uint32)
        assert not (u & 0xFFFF).any()
    assert abs(float(P["layers"][1]["w1"].std()) - 0.02) < 0.002


def test_step_weight_bytes_config5():
    # 12 x (4 d^2 + 2 d h + 4 d + h + d) + V d bf16 values, d = 768, h = 3072, V = 32000
    cfg = nn.DecoderConfig()
    assert cfg.step_weight_bytes() == 2 * (12 * (4 * 768 ** 2 + 2 * 768 * 3072 + 5 * 768 + 3072) + 32000 * 768)


@pytest.mark.parametrize("bad", [
    dict(max_batch=9), dict(max_batch=0), dict(n_heads=5), dict(d_model=48, n_heads=4),
    dict(n_heads=1, d_model=512), dict(max_seq=0), dict(vocab=0), dict(n_layers=0), dict(mlp_ratio=0),
    dict(d_model=4096, n_heads=32),
])
def test_invalid_config_rejected_before_device(bad):
    """Config errors are InvalidArgument with or without a GPU (checked
    before the device is touched)."""
    L = abi.load_library()
    c = nn.DecoderConfig(**{**dict(n_layers=1, d_model=64, n_heads=4, vocab=100, max_batch=8, max_seq=16),
                            **bad})
    cc = abi.mlxhip_decoder_config_t(c.n_layers, c.d_model, c.n_heads, c.hidden, c.vocab, c.max_batch,
                                     c.max_seq, c.eps)
    assert not L.mlxhip_decoder_new(C.byref(cc))
    assert L.mlxhip_last_status() == abi.ERR_INVALID_ARGUMENT, L.mlxhip_last_error()


def test_null_arguments_without_gpu():
    L = abi.load_library()
    assert not L.mlxhip_decoder_new(None)
    assert L.mlxhip_last_status() == abi.ERR_NULL_PTR
    L.mlxhip_decoder_free(None)
    assert L.mlxhip_decoder_weight_bytes(None) == 0
    assert L.mlxhip_decoder_generate(None, None, 1, 1, 1, None, None, None, 0) == abi.ERR_NULL_PTR
    assert L.mlxhip_decoder_set_param(None, 0, 0, None, 0) == abi.ERR_NULL_PTR


def test_valid_config_without_gpu_is_backend_unavailable():
    from oxidizedmlx_amd import backend
    if backend.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(abi.BackendUnavailable):
        backend.HipDecoder(SMALL)
