"""Parity of the device sampler (msd_sample_token) with the numpy sampling oracle (GPU).

The sampler reproduces numpy's float arithmetic of generate.py:28-65 with the exponential
correctly rounded, so against ``oracle.sampling`` with ``exp="rounded"`` the probabilities
are bitwise equal, the nucleus keeps the same number of ids and the drawn token is the same.
"""
import numpy as np
import pytest
import torch

from oracle import model as om
from oracle import sampling as osm
from transformer_amd.configs import M306, TINY
from transformer_amd.fused_decode_nlayer import prepare_decode_weights_nlayer
from transformer_amd.generate import Sampler, generate_tokens, run_generation, sample_token, stream_tokens
from transformer_amd.multi_sm_decode import Decoder
from transformer_amd.synthetic import make_params, make_prompt

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _gpu_sample(logits, temperature, top_p, pen, seen_ids, u):
    V = len(logits)
    smp = Sampler(V, "cuda")
    smp.reset(seen_ids)
    lg = torch.as_tensor(np.ascontiguousarray(logits, dtype=np.float32)).cuda()
    ud = torch.tensor([u], dtype=torch.float64, device="cuda")
    probs = torch.full((V,), -1.0, dtype=torch.float32, device="cuda")
    kept = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    tok = smp.launch(lg, temperature, top_p, pen, u=ud, probs_out=probs, kept_out=kept)
    torch.cuda.synchronize()
    return int(tok.item()), probs.cpu().numpy(), int(kept.item()), smp.seen.cpu().numpy()


def _oracle_kept(probs, top_p):
    sp = probs[np.argsort(-probs, kind="stable")]
    return min(int(np.searchsorted(np.cumsum(sp), top_p)) + 1, len(probs))


def _check_case(logits, temperature, top_p, pen, seen_ids, u):
    tok, probs, kept, seen = _gpu_sample(logits, temperature, top_p, pen, seen_ids, u)
    ref = osm.sample_token(logits, temperature, top_p, pen, seen_ids, u, exp="rounded")
    if temperature != 0.0:
        pl = osm.apply_repetition_penalty(logits, pen, seen_ids)
        rp = osm.softmax_probs(pl, temperature, exp="rounded")
        assert np.array_equal(probs.view(np.uint32), rp.view(np.uint32)), "probabilities differ"
        if top_p < 1.0:
            assert kept == _oracle_kept(rp, top_p)
    assert tok == ref, (tok, ref)
    assert seen[tok] == 1
    for t in seen_ids:
        assert seen[t] == 1
    return kept


def _logits(rng, V, scale):
    return (rng.standard_normal(V) * scale).astype(np.float32)


@pytest.mark.parametrize("scale", [0.3, 0.9, 3.0, 8.0])
def test_nucleus_matches_oracle_32000(scale):
    rng = np.random.default_rng(int(scale * 10))
    for trial in range(6):
        lg = _logits(rng, 32000, scale)
        seen = [int(x) for x in rng.integers(0, 32000, int(rng.integers(0, 40)))]
        for top_p in (0.95, 0.5, 0.999):
            u = float(rng.random())
            _check_case(lg, 0.7, top_p, 1.2, seen, u)


def test_full_softmax_and_greedy_paths():
    rng = np.random.default_rng(3)
    for trial in range(5):
        lg = _logits(rng, 32000, 1.0)
        seen = [int(x) for x in rng.integers(0, 32000, 20)]
        _check_case(lg, 1.0, 1.0, 1.0, [], float(rng.random()))      # top_p = 1, temp = 1
        _check_case(lg, 0.7, 1.0, 1.2, seen, float(rng.random()))     # top_p = 1 with penalty
        _check_case(lg, 0.0, 0.9, 1.2, seen, 0.5)                     # temperature 0: argmax
        _check_case(lg, 0.0, 1.0, 1.0, [], 0.5)


def test_vocab_sizes_and_edges():
    rng = np.random.default_rng(4)
    for V in (1, 2, 7, 100, 511, 512, 513, 8191, 8193, 20000, 32768):
        lg = _logits(rng, V, 1.5)
        for top_p in (0.0, 0.3, 0.9, 0.99999):
            _check_case(lg, 0.8, top_p, 1.0, [], float(rng.random()))
        _check_case(lg, 1.3, 1.0, 1.0, [], float(rng.random()))


def test_ties_keep_ascending_id_order():
    rng = np.random.default_rng(5)
    # logits on a coarse grid: many exactly equal probabilities straddle the cutoff
    lg = (np.round(rng.standard_normal(32000) * 4) / 4).astype(np.float32)
    for top_p in (0.1, 0.5, 0.9):
        for u in (0.0, 0.37, 0.999999):
            _check_case(lg, 1.0, top_p, 1.0, [], u)
    flat = np.zeros(32000, np.float32)                                 # all equal
    kept = _check_case(flat, 0.7, 0.5, 1.0, [], 0.7)
    assert 15990 <= kept <= 16010
    spike = np.full(32000, -30.0, np.float32)
    spike[[17, 4000, 31999]] = 5.0                                   # three equal maxima
    assert _check_case(spike, 1.0, 0.3, 1.0, [], 0.99) == 1
    assert _gpu_sample(spike, 1.0, 0.3, 1.0, [], 0.99)[0] == 17


def test_penalty_sign_rule_and_history():
    lg = np.array([2.0, 1.9, -1.0, -0.9, 0.0] * 100, np.float32)
    for seen in ([0], [0, 3], [1, 2, 4], list(range(500))):
        _check_case(lg, 0.0, 1.0, 2.0, seen, 0.5)
        _check_case(lg, 0.5, 0.8, 1.7, seen, 0.25)


def test_reference_signature_sample_token():
    rng = np.random.default_rng(6)
    lg = _logits(rng, 32000, 1.0)
    np.random.seed(123)
    a = sample_token(lg, 0.7, 0.95, 1.2, [5, 6, 7])
    u = np.random.RandomState(123).random_sample()
    assert a == osm.sample_token(lg, 0.7, 0.95, 1.2, [5, 6, 7], u)
    dev = torch.as_tensor(lg).cuda()
    assert sample_token(dev, 0.7, 0.95, 1.2, [5, 6, 7], u=u) == a
    assert sample_token(lg, 0.0, 1.0, 1.0, []) == int(np.argmax(lg))


def _teacher_forced_sampled(params, cfg, prompt, n, temperature, top_p, pen, seed):
    """GPU generation with recorded logits, then: (1) each drawn token equals the oracle
    sampler's on the same logits, history and uniform; (2) the recorded logits match the
    oracle's cached decode step fed the GPU's own tokens."""
    w = prepare_decode_weights_nlayer(params, cfg)
    dec = Decoder(w, cfg)
    us = np.random.RandomState(seed).random_sample(n)
    rec = torch.zeros((n, cfg["vocab_size"]), dtype=torch.float32, device="cuda")
    toks = list(run_generation(dec, prompt, n, temperature, top_p, pen, uniforms=us, record_logits=rec))
    rec = rec.cpu().numpy()
    for i in range(n):
        assert osm.sample_token(rec[i], temperature, top_p, pen, toks[:i], us[i], exp="rounded") == toks[i], i
    # oracle: prefill with bf16 projection inputs (as the matrix-core prefill), then f32 steps
    first, kc, vc = om.prefill_with_kv(params, cfg, prompt)
    rope = om.precompute_rope_table(cfg["context_len"], cfg["d_head"])
    np.testing.assert_allclose(rec[0], first[-1], atol=ATOL, rtol=RTOL)
    worst = float(np.max(np.abs(rec[0] - first[-1])))
    for i, t in enumerate(toks[:-1]):
        lg, _ = om.decode_step(params, cfg, t, len(prompt) + i, kc, vc, rope=rope)
        np.testing.assert_allclose(rec[i + 1], lg, atol=ATOL, rtol=RTOL)
        worst = max(worst, float(np.max(np.abs(rec[i + 1] - lg))))
    return toks, worst


def test_tiny_sampled_generation_teacher_forced():
    params = make_params(TINY, seed=0)
    prompt = make_prompt(16, TINY["vocab_size"], seed=1)
    toks, worst = _teacher_forced_sampled(params, TINY, prompt, 100, 0.7, 0.95, 1.2, seed=7)
    print("tiny sampled: distinct tokens", len(set(toks)), "max |logit diff|", worst)
    assert len(set(toks)) > 50


def test_306m_sampled_generation_teacher_forced():
    """temperature 0.7, top-p 0.95, repetition penalty 1.2, 64-token prompt, 256 new tokens."""
    params = make_params(M306, seed=0, resid_scaled=True)
    prompt = make_prompt(64, M306["vocab_size"], seed=1)
    toks, worst = _teacher_forced_sampled(params, M306, prompt, 256, 0.7, 0.95, 1.2, seed=11)
    print("306M sampled: distinct tokens", len(set(toks)), "max |logit diff|", worst)
    assert len(set(toks)) > 128


def test_stream_and_generate_agree():
    params = make_params(TINY, seed=0)
    prompt = make_prompt(16, TINY["vocab_size"], seed=2)
    a = list(stream_tokens(params, TINY, prompt, 40, temperature=0.8, top_p=0.9, rep_penalty=1.1, seed=3))
    b = generate_tokens(params, TINY, prompt, 40, temperature=0.8, top_p=0.9, rep_penalty=1.1, seed=3)
    assert a == b
    g = generate_tokens(params, TINY, prompt, 40)
    assert g == om.greedy_generate(params, TINY, prompt, 40, prefill="full")
    dec = Decoder(prepare_decode_weights_nlayer(params, TINY), TINY)
    st = list(run_generation(dec, list(prompt), 40, prefill="step"))
    assert st == om.greedy_generate(params, TINY, prompt, 40, prefill="step")
    p = generate_tokens(params, TINY, prompt, 20, temperature=0.0, rep_penalty=1.3)
    assert len(p) == 20
