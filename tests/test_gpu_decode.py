"""Greedy decoding on the GPU (mlxhip_decoder_*, through the C ABI) against
the CPU oracle's decoder (mlx-nn layers over the oracle stream).

Teacher forcing makes the comparison exact in structure: the oracle runs the
causal forward over the very token sequence the GPU consumed (prompt +
its own generated tokens), so every position's logits are compared, and the
GPU's argmax must be the oracle's wherever the oracle's top-two logits are
further apart than the logit tolerance (a closer pair may legitimately
resolve either way under f32 rounding differences).

Logit tolerance: |gpu - oracle| <= 2e-5 * max|oracle logits| + 1e-4 * |oracle|.
The GPU keeps f32 activations (its GEMV splits them into three bf16 terms,
exact to f32 precision) and f32 accumulation, so only summation order
differs from the oracle."""
import numpy as np
import pytest

from oracle.graph import OracleStream
from oxidizedmlx_amd import abi, nn
from oxidizedmlx_amd.backend import HipDecoder, HipStream

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip", "oracle_lib")]

SMALL = nn.DecoderConfig(n_layers=2, d_model=64, n_heads=4, vocab=1000, max_batch=8, max_seq=16)
ATOL, RTOL = 2e-5, 1e-4


def check_logits_and_argmax(gpu_logits, gpu_argmax, ref_logits, what):
    ref = ref_logits.astype(np.float64)
    scale = np.abs(ref).max()
    atol = ATOL * scale
    diff = np.abs(gpu_logits.astype(np.float64) - ref)
    tol = atol + RTOL * np.abs(ref)
    bad = diff > tol
    print(f"  {what}: logits max_abs={diff.max():.3e} (scale {scale:.3e}, atol {atol:.3e})", flush=True)
    assert not bad.any(), f"{what}: {int(bad.sum())} logits out of tolerance, max diff {diff.max():.3e}"
    flat = ref.reshape(-1, ref.shape[-1])
    top2 = np.sort(flat, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * (atol + RTOL * np.abs(top2[:, 1]))
    want = flat.argmax(axis=1)
    got = gpu_argmax.reshape(-1)
    mism = clear & (got != want)
    assert not mism.any(), f"{what}: argmax differs at {np.flatnonzero(mism)[:8]} (clear margin)"
    return int(clear.sum()), got.size


def oracle_logits(cfg, P, tokens):
    b, s = tokens.shape
    return nn.DecoderLM(cfg, OracleStream(), P)(tokens).to_numpy().reshape(b, s, cfg.vocab)


@pytest.fixture(scope="module")
def small():
    P = nn.decoder_params(SMALL, 4321)
    dec = HipDecoder(SMALL)
    dec.load(P)
    return dec, P


@pytest.mark.parametrize("batch,prompt_len,n_new", [(3, 5, 8), (8, 1, 16), (1, 16, 1)])
def test_generate_teacher_forced_parity(small, batch, prompt_len, n_new):
    dec, P = small
    print(f"decode parity batch={batch} prompt={prompt_len} n_new={n_new}", flush=True)
    rng = np.random.default_rng(batch * 100 + prompt_len)
    prompt = rng.integers(0, SMALL.vocab, size=(batch, prompt_len))
    toks, am, lg = dec.generate(prompt, n_new, argmax=True, logits=True)
    steps = prompt_len + n_new - 1
    assert toks.shape == (batch, n_new) and am.shape == (batch, steps) and lg.shape == (batch, steps, SMALL.vocab)
    np.testing.assert_array_equal(toks, am[:, prompt_len - 1:])
    seq = np.concatenate([prompt, toks[:, :-1]], axis=1)  # what the GPU consumed
    ref = oracle_logits(SMALL, P, seq)
    clear, total = check_logits_and_argmax(lg, am, ref, f"b{batch} p{prompt_len} n{n_new}")
    assert clear >= total * 0.9


def test_graph_and_eager_identical(small):
    dec, _ = small
    prompt = np.random.default_rng(5).integers(0, SMALL.vocab, size=(4, 6))
    g = dec.generate(prompt, 7, argmax=True, logits=True)
    e = dec.generate(prompt, 7, argmax=True, logits=True, eager=True)
    for a, b in zip(g, e):
        np.testing.assert_array_equal(a, b)


def test_repeatable_and_sequences_independent(small):
    """Same call twice: identical. Each sequence's result does not depend on
    the others in the batch (bit for bit), and a later smaller call is not
    affected by the state an earlier one left in the cache."""
    dec, _ = small
    prompt = np.random.default_rng(9).integers(0, SMALL.vocab, size=(5, 4))
    a = dec.generate(prompt, 9, logits=True)
    b = dec.generate(prompt, 9, logits=True)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    for i in (0, 3):
        t1, l1 = dec.generate(prompt[i:i + 1, :2], 3, logits=True)
        ta, la = dec.generate(prompt[i:i + 1], 9, logits=True)
        np.testing.assert_array_equal(ta[0], a[0][i])
        np.testing.assert_array_equal(la[0], a[1][i])
        np.testing.assert_array_equal(l1[0][:2], la[0][:2])  # same first two tokens


def test_prompt_ids_clamped(small):
    """Out-of-range ids select the first / last embedding row, as
    embedding_lookup clamps them (crates/mlx-core/src/cpu_kernels.rs:317-336)."""
    dec, _ = small
    base = np.array([[3, 17, 999]])
    odd = np.array([[-5, 17, 5000]])
    fixed = np.array([[0, 17, 999]])
    _, lo = dec.generate(odd, 2, logits=True)
    _, lf = dec.generate(fixed, 2, logits=True)
    np.testing.assert_array_equal(lo, lf)
    _, lb = dec.generate(base, 2, logits=True)
    assert not np.array_equal(lb, lf)


def test_generate_errors(small):
    dec, _ = small
    p = np.zeros((2, 4), np.int32)
    with pytest.raises(abi.InvalidArgument):
        dec.generate(np.zeros((9, 2), np.int32), 1)          # batch > max_batch
    with pytest.raises(abi.InvalidArgument):
        dec.generate(p, 14)                                   # 4 + 14 - 1 > max_seq
    with pytest.raises(abi.InvalidArgument):
        dec.generate(p, 0)
    with pytest.raises(abi.InvalidArgument):
        dec.generate(np.zeros((2, 0), np.int32), 2)
    with pytest.raises(abi.ShapeMismatch):
        dec.set_param(0, abi.DEC_LAYER_PARAMS["wq"], np.zeros(10, np.float32))
    with pytest.raises(abi.InvalidArgument):
        dec.set_param(2, abi.DEC_LAYER_PARAMS["wq"], np.zeros(64 * 64, np.float32))
    fresh = HipDecoder(SMALL)
    fresh.set_param(0, abi.DEC_EMBEDDING, np.zeros((1000, 64), np.float32))
    with pytest.raises(abi.InvalidArgument, match="never set"):
        fresh.generate(p, 1)
    dec.generate(p, 2)  # the decoder still works after the errors


def test_vocab_tail_and_wide_mlp():
    """vocab not a multiple of the 16-feature tile, head_dim 32, hidden 512
    (two k-slices), batch 7."""
    cfg = nn.DecoderConfig(n_layers=1, d_model=128, n_heads=4, vocab=777, mlp_ratio=4, max_batch=8, max_seq=12)
    P = nn.decoder_params(cfg, 99)
    dec = HipDecoder(cfg)
    dec.load(P)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, size=(7, 3))
    toks, am, lg = dec.generate(prompt, 6, argmax=True, logits=True)
    seq = np.concatenate([prompt, toks[:, :-1]], axis=1)
    check_logits_and_argmax(lg, am, oracle_logits(cfg, P, seq), "vocab 777")


def test_wide_lm_head_with_a_partial_last_workgroup():
    """vocab 8200: 513 row tiles, so the LM head takes its wide shape (8 row
    tiles per workgroup) and the last workgroup holds one tile in range; its
    RMS still sums the squares of every step of the activation."""
    cfg = nn.DecoderConfig(n_layers=1, d_model=128, n_heads=4, vocab=8200, mlp_ratio=2, max_batch=8, max_seq=8)
    P = nn.decoder_params(cfg, 515)
    dec = HipDecoder(cfg)
    dec.load(P)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, size=(5, 2))
    toks, am, lg = dec.generate(prompt, 4, argmax=True, logits=True)
    seq = np.concatenate([prompt, toks[:, :-1]], axis=1)
    check_logits_and_argmax(lg, am, oracle_logits(cfg, P, seq), "vocab 8200")


def test_config5_matches_stream_forward():
    """Config 5 at full size (12 layers, d_model 768, 12 heads, vocab 32000,
    batch 8, prompt 16, 128 new tokens): the decoder's logits at all 143
    positions against the causal forward of the same mlx-nn model on the
    HipStream (f32 GEMMs over the bf16-valued weights) on the tokens the
    decoder consumed, and one whole sequence (all 143 positions of sequence
    3, teacher-forced) against the oracle's mlx-nn decoder: every logit and
    every clear-margin argmax decision of the generate the bench times
    (crates/mlx-conformance/tests/ttft_behavior.rs:101-216 loops 128 steps)."""
    cfg = nn.DecoderConfig()
    P = nn.decoder_params(cfg, 2024)
    dec = HipDecoder(cfg)
    dec.load(P)
    assert dec.weight_bytes() >= cfg.step_weight_bytes()
    prompt = np.random.default_rng(16).integers(0, cfg.vocab, size=(8, 16))
    toks, am, lg = dec.generate(prompt, 128, argmax=True, logits=True)
    seq = np.concatenate([prompt, toks[:, :-1]], axis=1)
    st = HipStream()
    ref = nn.DecoderLM(cfg, st, P)(seq).to_numpy().reshape(8, 143, cfg.vocab)
    clear, total = check_logits_and_argmax(lg, am, ref, "config 5")
    print(f"  config 5: {clear} of {total} argmax decisions with a clear margin", flush=True)
    assert clear >= total * 0.9
    print("config 5, oracle on the whole of sequence 3 (143 positions)", flush=True)
    ref3 = oracle_logits(cfg, P, seq[3:4])
    clear3, total3 = check_logits_and_argmax(lg[3:4], am[3:4], ref3, "config 5 sequence 3 vs oracle")
    assert total3 == 143 and clear3 >= total3 * 0.9


def test_config5_full_size_matches_oracle():
    """Config 5 at full size (12 layers, d_model 768, 12 heads, vocab 32000,
    batch 8, prompt 16) for 8 new tokens, teacher-forced against the oracle's
    mlx-nn decoder on sequences 0 and 5 (23 positions each): every logit
    and every clear-margin argmax decision."""
    cfg = nn.DecoderConfig()
    P = nn.decoder_params(cfg, 77)
    dec = HipDecoder(cfg)
    dec.load(P)
    prompt = np.random.default_rng(23).integers(0, cfg.vocab, size=(8, 16))
    toks, am, lg = dec.generate(prompt, 8, argmax=True, logits=True)
    seq = np.concatenate([prompt, toks[:, :-1]], axis=1)
    for b in (0, 5):
        print(f"config 5, oracle on sequence {b}", flush=True)
        ref = oracle_logits(cfg, P, seq[b:b + 1])
        check_logits_and_argmax(lg[b:b + 1], am[b:b + 1], ref, f"config 5 sequence {b}")
