"""Golden regression fixtures of the tiny config (CPU): the seeded weights and the oracle's
greedy tokens/logits must reproduce tests/golden/tiny_greedy.json."""
import json
import os

import numpy as np

from oracle import model as om
from transformer_amd.configs import TINY
from transformer_amd.synthetic import make_params, make_prompt

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_greedy.json")


def _load():
    with open(GOLDEN) as f:
        return json.load(f)


def test_synthetic_weights_match_fixture():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(os.path.dirname(GOLDEN), "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    g = _load()
    assert mg.weights_sha256(make_params(TINY, seed=0)) == g["weights_sha256"]
    assert [int(t) for t in make_prompt(16, TINY["vocab_size"], seed=1)] == g["prompt"]


def test_oracle_reproduces_fixture(tiny_params):
    g = _load()
    prompt = np.array(g["prompt"], dtype=np.int32)
    toks, logs = om.greedy_generate(tiny_params, TINY, prompt, 48, prefill="step", return_logits=True)
    assert toks == g["greedy_tokens_step_prefill"]
    for st, lg in zip(g["steps"], logs):
        np.testing.assert_allclose(lg[:8], st["logits_0_8"], rtol=0, atol=1e-5)
        assert int(np.argmax(lg)) == st["argmax"]
    assert om.greedy_generate(tiny_params, TINY, prompt, 48, prefill="full") == g["greedy_tokens_full_prefill"]
