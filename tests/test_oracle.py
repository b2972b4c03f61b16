"""Pins for the numpy oracle: library cross-checks, closed forms and invariants (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import model as om
from oracle.numerics import bf16_round
from oracle import sampling as osm
from oracle.sampling import sample_token, _choice
from transformer_amd.configs import TINY
from transformer_amd.synthetic import bf16_round_np, make_params, make_prompt


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000).astype(np.float32) * 10.0
    # exact ties: low 16 bits = 0x8000 on both even and odd mantissas
    u = rng.integers(0, 2**31, 1000, dtype=np.uint32) & np.uint32(0xFFFF0000) | np.uint32(0x8000)
    x = np.concatenate([x, u.view(np.float32), np.array([0.0, -0.0, 1e-40, 3.0e38], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(bf16_round(x), ref)
    np.testing.assert_array_equal(bf16_round_np(x), ref)


def test_rms_norm_closed_forms():
    s = np.linspace(0.5, 2.0, 64).astype(np.float32)
    c = np.full(64, -3.0, np.float32)
    # constant vector c: x/rms = sign(c) * |c|/sqrt(c^2+eps)
    exp = s * (-3.0 / np.sqrt(9.0 + 1e-5))
    np.testing.assert_allclose(om.rms_norm(c, s), exp, rtol=1e-6)
    x = np.random.default_rng(1).standard_normal((5, 64)).astype(np.float32)
    y = om.rms_norm(x, np.ones(64, np.float32))
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-5)
    assert np.all(om.rms_norm(np.zeros(64, np.float32), s) == 0)


def test_rope_table_closed_form_and_invariants():
    cos, sin = om.precompute_rope_table(128, 64)
    i = np.arange(32)
    f = 10000.0 ** (-2.0 * i / 64)
    ang = np.arange(128)[:, None] * f[None, :]
    np.testing.assert_allclose(cos, np.cos(ang), atol=2e-5)
    np.testing.assert_allclose(sin, np.sin(ang), atol=2e-5)
    np.testing.assert_allclose(cos ** 2 + sin ** 2, 1.0, atol=1e-6)
    rng = np.random.default_rng(2)
    q = rng.standard_normal(64).astype(np.float64)
    k = rng.standard_normal(64).astype(np.float64)
    c64, s64 = om.precompute_rope_table(128, 64, dtype=np.float64)
    np.testing.assert_array_equal(om.apply_rope(q, c64[0], s64[0]), q)
    np.testing.assert_allclose(np.linalg.norm(om.apply_rope(q, c64[37], s64[37])), np.linalg.norm(q), rtol=1e-12)
    # <R_p q, R_s k> depends only on p - s (rotate-half pairs i, i+32)
    d1 = om.apply_rope(q, c64[50], s64[50]) @ om.apply_rope(k, c64[40], s64[40])
    d2 = om.apply_rope(q, c64[13], s64[13]) @ om.apply_rope(k, c64[3], s64[3])
    assert abs(d1 - d2) < 1e-5
    # the pair (i, i+32) rotates by angle pos*f_i: check one explicit 2D rotation
    e = np.zeros(64); e[5] = 1.0
    r = om.apply_rope(e, c64[9], s64[9])
    assert abs(r[5] - np.cos(9 * f[5])) < 1e-6 and abs(r[37] - np.sin(9 * f[5])) < 1e-6


def test_causal_attention_matches_torch_sdpa():
    rng = np.random.default_rng(3)
    T, d, H, KV = 9, 256, 4, 2
    x = rng.standard_normal((T, d)).astype(np.float64)
    w = [rng.standard_normal((d, n)).astype(np.float64) * 0.05 for n in (d, KV * 64, KV * 64, d)]
    cos, sin = om.precompute_rope_table(16, 64, dtype=np.float64)
    out = om.causal_attention(x, *w, H, KV, cos, sin)
    q = om.apply_rope((x @ w[0]).reshape(T, H, 64), cos[:T, None], sin[:T, None])
    k = om.apply_rope((x @ w[1]).reshape(T, KV, 64), cos[:T, None], sin[:T, None])
    v = (x @ w[2]).reshape(T, KV, 64)
    tq = torch.from_numpy(q).permute(1, 0, 2)
    tk = torch.from_numpy(k).permute(1, 0, 2).repeat_interleave(H // KV, 0)
    tv = torch.from_numpy(v).permute(1, 0, 2).repeat_interleave(H // KV, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    ref = ref.permute(1, 0, 2).reshape(T, d).numpy() @ w[3]
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_attend_closed_forms():
    rng = np.random.default_rng(4)
    V = rng.standard_normal((7, 64))
    K = np.zeros((7, 64))
    np.testing.assert_allclose(om._attend(rng.standard_normal(64), K, V, 0.125), V.mean(0), rtol=1e-12)
    K = np.eye(7, 64) * 1e4
    q = np.zeros(64); q[3] = 1.0
    np.testing.assert_allclose(om._attend(q, K, V, 1.0), V[3], rtol=1e-9)
    np.testing.assert_allclose(om._attend(q, K[:1], V[:1], 1.0), V[0])


def _hf_llama(params, config, dtype):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.LlamaConfig(
        vocab_size=config["vocab_size"], hidden_size=config["d_model"],
        intermediate_size=config["d_ff"], num_hidden_layers=config["n_layers"],
        num_attention_heads=config["n_heads"], num_key_value_heads=config["n_kv_heads"],
        head_dim=config["d_head"], max_position_embeddings=config["context_len"],
        rms_norm_eps=1e-5, rope_theta=10000.0, tie_word_embeddings=True,
        attention_bias=False, mlp_bias=False, hidden_act="silu")
    m = transformers.LlamaForCausalLM(cfg).to(dtype).eval()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dtype)
    with torch.no_grad():
        m.model.embed_tokens.weight.copy_(t(params["token_emb"]))
        m.model.norm.weight.copy_(t(params["ln_final.scale"]))
        for i, layer in enumerate(m.model.layers):
            p = f"layer{i}"
            layer.input_layernorm.weight.copy_(t(params[f"{p}.ln1.scale"]))
            layer.post_attention_layernorm.weight.copy_(t(params[f"{p}.ln2.scale"]))
            layer.self_attn.q_proj.weight.copy_(t(params[f"{p}.attn.q"].T))
            layer.self_attn.k_proj.weight.copy_(t(params[f"{p}.attn.k"].T))
            layer.self_attn.v_proj.weight.copy_(t(params[f"{p}.attn.v"].T))
            layer.self_attn.o_proj.weight.copy_(t(params[f"{p}.attn.o"].T))
            layer.mlp.gate_proj.weight.copy_(t(params[f"{p}.ffn.gate"].T))
            layer.mlp.up_proj.weight.copy_(t(params[f"{p}.ffn.up"].T))
            layer.mlp.down_proj.weight.copy_(t(params[f"{p}.ffn.down"].T))
    return m


def test_forward_matches_hf_llama_f64(tiny_params):
    """The oracle forward equals an independent Llama implementation (f64) on the tiny config."""
    cfg = dict(TINY)
    p64 = {k: v.astype(np.float64) for k, v in tiny_params.items()}
    # non-unit norm scales so the scale multiply is exercised
    rng = np.random.default_rng(5)
    for k in p64:
        if k.endswith("scale"):
            p64[k] = 1.0 + 0.1 * rng.standard_normal(p64[k].shape)
    toks = make_prompt(24, cfg["vocab_size"], seed=1)
    ours = om.forward(p64, cfg, toks)
    m = _hf_llama(p64, cfg, torch.float64)
    with torch.no_grad():
        ref = m(torch.from_numpy(toks.astype(np.int64))[None]).logits[0].numpy()
    # Both build the RoPE angles in float32 (model.py:104 as base**(-2i/d), HF as
    # 1/base**(2i/d)); the 1-ulp table difference moves logits by ~1e-7.  A structural
    # mistake (wrong head grouping, rotation pairing, norm, gate/up swap) is >1e-3.
    np.testing.assert_allclose(ours, ref, rtol=0, atol=1e-6)


def test_cached_step_equals_full_forward(tiny_params):
    """A cached decode step with un-rounded KV equals the full re-forward at the last position;
    with the bf16 KV cache it stays within the bf16 tolerance."""
    cfg = dict(TINY)
    p64 = {k: v.astype(np.float64) for k, v in tiny_params.items()}
    toks = make_prompt(12, cfg["vocab_size"], seed=7)
    full = om.forward(p64, cfg, toks)
    kc, vc = om.new_kv_cache(cfg, np.float64)
    import oracle.model as mm
    saved = mm.bf16_round
    try:
        mm.bf16_round = lambda a: a          # un-rounded cache: exact equality expected
        for pos, t in enumerate(toks):
            lg, _ = om.decode_step(p64, cfg, t, pos, kc, vc)
            np.testing.assert_allclose(lg, full[pos], rtol=1e-9, atol=1e-11)
    finally:
        mm.bf16_round = saved
    kc, vc = om.new_kv_cache(cfg, np.float64)
    for pos, t in enumerate(toks):
        lg, _ = om.decode_step(p64, cfg, t, pos, kc, vc)
        np.testing.assert_allclose(lg, full[pos], atol=2e-2, rtol=1e-2)


def test_prefill_kv_and_future_rows_ignored(tiny_params):
    cfg = dict(TINY)
    toks = make_prompt(10, cfg["vocab_size"], seed=3)
    logits, kc, vc = om.prefill_with_kv(tiny_params, cfg, toks)
    np.testing.assert_allclose(logits, om.forward(tiny_params, cfg, toks), rtol=1e-5, atol=1e-5)
    # cache rows equal the per-position K (post-RoPE) / V of the step path, rounded to bf16
    kc2, vc2 = om.new_kv_cache(cfg)
    for p, t in enumerate(toks):
        om.decode_step(tiny_params, cfg, t, p, kc2, vc2)
    assert np.all(kc[0][:, :10] == kc2[0][:, :10]) and np.all(vc[0][:, :10] == vc2[0][:, :10])
    # garbage beyond pos never influences the step
    kc3 = [k.copy() for k in kc]; vc3 = [v.copy() for v in vc]
    for k in kc3 + vc3:
        k[:, 11:, :] = np.nan
    a, _ = om.decode_step(tiny_params, cfg, 5, 10, [k.copy() for k in kc], [v.copy() for v in vc])
    b, _ = om.decode_step(tiny_params, cfg, 5, 10, kc3, vc3)
    np.testing.assert_array_equal(a, b)


def test_act_round_bf16_close_to_f32(tiny_params):
    toks = make_prompt(8, TINY["vocab_size"], seed=9)
    a = om.forward(tiny_params, TINY, toks)
    b = om.forward(tiny_params, TINY, toks, act_round="bf16")
    assert np.max(np.abs(a - b)) < 2e-2
    assert np.max(np.abs(a - b)) > 0


def test_sampling_choice_matches_randomstate():
    rng = np.random.default_rng(11)
    for trial in range(50):
        n = int(rng.integers(1, 300))
        p = rng.random(n).astype(np.float32)
        p /= p.sum()
        keep = rng.permutation(1000)[:n]
        seed = int(rng.integers(0, 2**31))
        ref = np.random.RandomState(seed).choice(keep, p=p)
        u = np.random.RandomState(seed).random_sample()
        assert keep[_choice(p, u)] == ref


def test_sample_token_closed_forms():
    rng = np.random.default_rng(12)
    logits = rng.standard_normal(1000).astype(np.float32)
    assert sample_token(logits, 0.0, 1.0, 1.0, [], 0.3) == int(np.argmax(logits))
    # penalty sign rule: a positive max divided, a negative value multiplied
    lg = np.array([2.0, 1.9, -1.0], np.float32)
    assert sample_token(lg, 0.0, 1.0, 2.0, [0], 0.5) == 1
    lg = np.array([-0.5, -0.6, -3.0], np.float32)
    assert sample_token(lg, 0.0, 1.0, 2.0, [0], 0.5) == 1
    # top_p=1, temp=1: inverse CDF over the full softmax
    p = np.exp(logits - logits.max()); p /= p.sum()
    for u in (0.0, 0.25, 0.999):
        assert sample_token(logits, 1.0, 1.0, 1.0, [], u) == int(np.searchsorted(np.cumsum(p.astype(np.float64)) / p.astype(np.float64).sum(), u, side="right"))
    # tiny top_p keeps only the argmax
    assert sample_token(logits, 0.7, 1e-6, 1.0, [], 0.99) == int(np.argmax(logits))


def test_nucleus_compares_top_p_in_float64():
    # cumsum[0] = float32(0.95) = 0.94999998... < 0.95: numpy's searchsorted compares in
    # float64, so the cutoff moves one further (a float32 comparison would keep one id)
    probs = np.array([0.95, 0.05], np.float32)
    keep, filt = osm.nucleus(probs, 0.95)
    assert list(keep) == [0, 1]
    keep, _ = osm.nucleus(probs, float(np.float32(0.95)))
    assert list(keep) == [0]


def test_nucleus_cutoff_against_exact_sums():
    """Cutoff = one past the first sorted position whose running sum reaches top_p, checked
    with exact rational sums of the float32 probabilities (skipping near-ties)."""
    from fractions import Fraction
    rng = np.random.default_rng(21)
    checked = 0
    for trial in range(300):
        n = int(rng.integers(1, 60))
        p = (rng.random(n) ** 3).astype(np.float32)
        p /= p.sum()
        top_p = float(rng.random())
        order = np.argsort(-p, kind="stable")
        acc, first = Fraction(0), None
        near = False
        for i, j in enumerate(order):
            acc += Fraction(float(p[j]))
            if abs(float(acc) - top_p) < 1e-6:
                near = True
            if first is None and acc >= Fraction(top_p):
                first = i
        if near:
            continue
        keep, filt = osm.nucleus(p, top_p)
        expect = n if first is None else first + 1
        assert len(keep) == expect
        assert list(keep) == list(order[:expect])
        np.testing.assert_allclose(filt.sum(dtype=np.float64), 1.0, atol=1e-6)
        checked += 1
    assert checked > 250


def test_nucleus_equal_probabilities_closed_form():
    n = 1024
    p = np.full(n, 1.0 / n, np.float32)   # exact: sums of powers of two
    for top_p in (0.25, 0.5, 0.75, 0.999):
        keep, filt = osm.nucleus(p, top_p)
        assert list(keep) == list(range(int(np.ceil(top_p * n))))
        assert np.all(filt == np.float32(1.0 / len(keep)))


def test_numpy_exp_versus_rounded_exp():
    """numpy's float32 exp differs from the correctly rounded value by <= 2 ulp; the drawn
    tokens of the two oracle modes agree except where a draw lands within that noise."""
    rng = np.random.default_rng(22)
    same = total = 0
    for trial in range(60):
        lg = (rng.standard_normal(32000) * rng.choice([0.3, 1.0, 4.0])).astype(np.float32)
        a = osm.softmax_probs(lg, 0.7, exp="numpy")
        b = osm.softmax_probs(lg, 0.7, exp="rounded")
        assert np.max(np.abs(a.view(np.int32) - b.view(np.int32))) <= 8   # exp ulps + the sum's
        for u in rng.random(5):
            total += 1
            same += osm.sample_token(lg, 0.7, 0.95, 1.0, [], u, exp="numpy") == \
                osm.sample_token(lg, 0.7, 0.95, 1.0, [], u, exp="rounded")
    assert same >= 0.97 * total, (same, total)


def test_synthetic_generator_is_seeded():
    a = make_params(TINY, seed=0)["layer0.attn.q"]
    b = make_params(TINY, seed=0)["layer0.attn.q"]
    c = make_params(TINY, seed=1)["layer0.attn.q"]
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert np.array_equal(bf16_round_np(a), a)
    assert abs(a.std() - 0.02) < 1e-3


_ROUNDED = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _hf_bf16_inputs(m, skip=None):
    """Forward pre-hooks rounding the input of every projection (and of the tied output
    projection, i.e. the final norm's output) to bf16: float64 -> float32 -> bf16 (RNE), the
    oracle's rounding.  ``skip`` names one projection left unrounded (negative control)."""
    def rnd(mod, args):
        x = args[0]
        return (x.to(torch.float32).to(torch.bfloat16).to(x.dtype),) + tuple(args[1:])
    hooks = []
    for layer in m.model.layers:
        for name in _ROUNDED:
            if name == skip:
                continue
            mod = getattr(layer.self_attn, name, None) or getattr(layer.mlp, name)
            hooks.append(mod.register_forward_pre_hook(rnd))
    if skip != "lm_head":
        hooks.append(m.lm_head.register_forward_pre_hook(rnd))
    return hooks


def _hf_exact_f64(m, cfg):
    """Make the HF model's RMSNorm and RoPE tables float64 end to end (it computes the norm in
    float32 and the RoPE angles' cos/sin in float32 whatever the model dtype); the RoPE tables
    become the oracle's.  Otherwise float32-level differences flip an occasional bf16 rounding
    of a projection input when rounding points are inserted."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    cos, sin = om.precompute_rope_table(cfg["context_len"], cfg["d_head"], dtype=np.float64)
    C = torch.from_numpy(np.concatenate([cos, cos], -1))
    S = torch.from_numpy(np.concatenate([sin, sin], -1))
    m.model.rotary_emb.forward = lambda x, position_ids: (C[position_ids].to(x.dtype), S[position_ids].to(x.dtype))
    for mod in m.modules():
        if isinstance(mod, LlamaRMSNorm):
            mod.forward = (lambda n: lambda h: n.weight * (h / torch.sqrt(h.pow(2).mean(-1, keepdim=True)
                                                                          + n.variance_epsilon)))(mod)


def test_act_round_bf16_matches_hf_llama_with_rounded_projection_inputs(tiny_params):
    """act_round="bf16" (the numerics of the matrix-core prefill and batched decode) equals an
    independent Llama in float64 whose projection inputs are rounded to bf16 by pre-hooks:
    x before q/k/v, the attention output before o, x2 before gate/up, the SwiGLU activation
    before down and the final norm's output before the tied logits
    (kernels/multi_sm_decode.py:143, 229, 268, 289, 320).  Leaving any one of those points
    unrounded moves the logits by far more than the tolerance, so a missing or misplaced
    rounding point in the oracle fails here."""
    cfg = dict(TINY)
    p64 = {k: v.astype(np.float64) for k, v in tiny_params.items()}
    rng = np.random.default_rng(6)
    for k in p64:
        if k.endswith("scale"):
            p64[k] = 1.0 + 0.1 * rng.standard_normal(p64[k].shape)
    toks = make_prompt(24, cfg["vocab_size"], seed=2)
    ours = om.forward(p64, cfg, toks, act_round="bf16")
    m = _hf_llama(p64, cfg, torch.float64)
    _hf_exact_f64(m, cfg)
    ids = torch.from_numpy(toks.astype(np.int64))[None]

    def hf(skip=None):
        hooks = _hf_bf16_inputs(m, skip)
        try:
            with torch.no_grad():
                return m(ids).logits[0].numpy()
        finally:
            for h in hooks:
                h.remove()
    ref = hf()
    err = float(np.max(np.abs(ours - ref)))
    assert err < 1e-6, err
    # the f32 oracle differs from the rounded reference by the bf16 effect itself
    assert float(np.max(np.abs(om.forward(p64, cfg, toks) - ref))) > 1e-4
    # negative controls: each rounding point is needed
    for skip in _ROUNDED + ("lm_head",):
        off = float(np.max(np.abs(ours - hf(skip))))
        assert off > 100 * max(err, 1e-9), (skip, off, err)
