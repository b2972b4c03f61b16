"""The decode step on the reference's other model shapes (GPU).

The reference scales its kernels over d_model 256..1024 with d_ff = 8d/3 rounded up to 128
(model.py:13-20; knowledge/program.md:114-145: d=512/8L, d=768/12L); profile_kernels.py:71
defaults n_kv_heads to n_heads.  Each shape here is decoded greedily token-exact against the
oracle and teacher-forced over random tokens with logits within 2e-2 abs / 1e-2 rel, and the
text command line runs a d=512 checkpoint in the reference's weights.pkl format.
"""
import numpy as np
import pytest

from oracle import model as om
from transformer_amd import checkpoint as ck
from transformer_amd import generate as gen
from transformer_amd.fused_decode_nlayer import prepare_decode_weights_nlayer
from transformer_amd.multi_sm_decode import Decoder
from transformer_amd.synthetic import make_params, make_prompt

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2

D768 = dict(vocab_size=32000, d_model=768, n_heads=12, n_kv_heads=4, n_layers=12, d_head=64, d_ff=2048,
            context_len=512)
D512_MHA = dict(vocab_size=32000, d_model=512, n_heads=8, n_kv_heads=8, n_layers=8, d_head=64, d_ff=1408,
                context_len=256)
D256_REF = dict(vocab_size=32000, d_model=256, n_heads=4, n_kv_heads=2, n_layers=4, d_head=64, d_ff=768,
                context_len=128)


def _greedy(w, cfg, prompt, n):
    dec = Decoder(w, cfg)
    for p, t in enumerate(prompt):
        tok, lg = dec.step(int(t), p)
    toks, logs = [tok], [lg.cpu().numpy().copy()]
    for i in range(n - 1):
        tok, lg = dec.step(toks[-1], len(prompt) + i)
        toks.append(tok)
        logs.append(lg.cpu().numpy().copy())
    return toks, logs


@pytest.mark.parametrize("cfg", [D768, D512_MHA, D256_REF], ids=["d768_12L_gqa3", "d512_8L_mha", "d256_ff768"])
def test_shape_greedy_and_teacher_forced(cfg):
    params = make_params(cfg, seed=3, resid_scaled=True)
    w = prepare_decode_weights_nlayer(params, cfg)
    prompt = make_prompt(24, cfg["vocab_size"], seed=4)
    n = 64
    toks, logs = _greedy(w, cfg, prompt, n)
    rtoks, rlogs = om.greedy_generate(params, cfg, prompt, n, prefill="step", return_logits=True)
    worst = max(float(np.abs(a - b).max()) for a, b in zip(logs, rlogs))
    print(cfg["d_model"], "greedy max |logit diff|", worst)
    assert toks == rtoks
    for a, b in zip(logs, rlogs):
        np.testing.assert_allclose(a, b, atol=ATOL, rtol=RTOL)
    # teacher-forced random tokens over the whole context: every position's logits and argmax
    seq = make_prompt(cfg["context_len"], cfg["vocab_size"], seed=5)
    dec = Decoder(w, cfg)
    kc, vc = om.new_kv_cache(cfg)
    rope = om.precompute_rope_table(cfg["context_len"], 64)
    for p, t in enumerate(seq):
        tok, lg = dec.step(int(t), p)
        if p % 7 == 0 or p == len(seq) - 1:
            ref, rtok = om.decode_step(params, cfg, int(t), p, kc, vc, rope=rope)
            np.testing.assert_allclose(lg.cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
            assert tok == rtok, p
        else:
            om.decode_step(params, cfg, int(t), p, kc, vc, rope=rope)


def test_cli_runs_a_d512_checkpoint(tmp_path):
    from test_checkpoint import _write_tokenizer
    cfg = dict(D512_MHA, n_layers=2)
    params = make_params(cfg, seed=8)
    _write_tokenizer(str(tmp_path))
    ck.save_weights(str(tmp_path / "weights.pkl"), params, cfg)
    prompt = "A wider model through the same command line."
    ids = ck.load_bpe_vocab(str(tmp_path / "data"))["encode_fn"](prompt)
    toks = gen.main(["--prompt", prompt, "--weights", str(tmp_path / "weights.pkl"), "--max-tokens", "16"])
    ref = om.greedy_generate(params, cfg, np.array(ids, np.int32), 16, prefill="full")
    assert toks == ref
