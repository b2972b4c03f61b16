"""Real-text command line path on the GPU: checkpoint file -> tokenizer -> decode kernels.

Runs ``transformer_amd.generate.main`` (generate.py:133-236) on a tiny checkpoint written
in the reference's ``weights.pkl`` format with a small trained BPE tokenizer, and checks the
generated ids against the oracle's greedy generation from the same prompt ids.
"""
import numpy as np
import pytest

from oracle import model as om
from transformer_amd import checkpoint as ck
from transformer_amd import generate as gen
from transformer_amd.configs import TINY
from test_checkpoint import _write_tokenizer

pytestmark = pytest.mark.gpu


def test_cli_greedy_matches_oracle(tmp_path, tiny_params, capsys):
    _write_tokenizer(str(tmp_path))
    ck.save_weights(str(tmp_path / "weights.pkl"), tiny_params, TINY)
    prompt = "Once upon a time there was a tiny model."
    bpe = ck.load_bpe_vocab(str(tmp_path / "data"))
    ids = bpe["encode_fn"](prompt)
    toks = gen.main(["--prompt", prompt, "--weights", str(tmp_path / "weights.pkl"), "--max-tokens", "24"])
    ref = om.greedy_generate(tiny_params, TINY, np.array(ids, np.int32), 24, prefill="full",
                             prefill_act_round=None)
    out = capsys.readouterr().out
    print("prompt ids", ids, "generated", toks)
    assert toks == ref
    assert out == prompt + "".join(bpe["decode_fn"]([t]) for t in toks) + "\n"
    # all at once: the same ids
    toks2 = gen.main(["--prompt", prompt, "--weights", str(tmp_path / "weights.pkl"), "--max-tokens", "24",
                      "--no-stream"])
    assert toks2 == ref


def test_cli_sampled_is_seeded(tmp_path, tiny_params):
    _write_tokenizer(str(tmp_path))
    ck.save_weights(str(tmp_path / "weights.pkl"), tiny_params, TINY)
    args = ["--prompt", "It decoded tokens", "--weights", str(tmp_path / "weights.pkl"), "--max-tokens", "16",
            "--temp", "0.8", "--top-p", "0.9", "--rep-penalty", "1.2", "--seed", "7"]
    a = gen.main(args)
    b = gen.main(args + ["--no-stream"])
    assert a == b and len(a) == 16
