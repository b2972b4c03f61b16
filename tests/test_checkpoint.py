"""Checkpoint loader, tokenizer and command line plumbing (CPU).

The reference writes ``weights.pkl`` with ``pickle.dump({"params", "config"})``
(train.py:246-248) and ``data/bpe_vocab.pkl`` with the tokenizer path (data.py:46-47); these
tests write files the same way and read them back through the restricted loader.
"""
import os
import pickle

import numpy as np
import pytest

from transformer_amd import checkpoint as ck
from transformer_amd import generate as gen
from transformer_amd.configs import TINY


def _small_params(rng, d=8, ff=16, V=40):
    p = {"token_emb": rng.standard_normal((V, d)).astype(np.float32)}
    p["layer0.ffn.gate"] = rng.standard_normal((d, ff)).astype(np.float32)
    p["ln_final.scale"] = np.ones(d, np.float32)
    return p


@pytest.mark.parametrize("protocol", [2, 4, 5])
def test_weights_round_trip(tmp_path, protocol):
    rng = np.random.default_rng(0)
    params = _small_params(rng)
    params["half"] = rng.standard_normal(5).astype(np.float16)
    params["fortran"] = np.asfortranarray(rng.standard_normal((3, 4)))
    config = {"vocab_size": np.int64(40), "d_model": 8, "n_heads": 1, "n_kv_heads": 1, "n_layers": 1,
              "context_len": 16}
    path = tmp_path / "weights.pkl"
    with open(path, "wb") as f:   # as train.py:246-248 writes it
        pickle.dump({"params": params, "config": config}, f, protocol=protocol)
    got, cfg = ck.load_weights(str(path))
    assert set(got) == set(params)
    for k, v in params.items():
        assert got[k].dtype == np.float32 and got[k].flags.c_contiguous
        np.testing.assert_array_equal(got[k], v.astype(np.float32))
    assert cfg["vocab_size"] == 40 and type(cfg["vocab_size"]) is int
    assert cfg["d_head"] == 8 and cfg["d_ff"] == 16   # filled in from the shapes


def test_save_weights_matches_reference_format(tmp_path, tiny_params):
    path = tmp_path / "w.pkl"
    ck.save_weights(str(path), tiny_params, TINY)
    with open(path, "rb") as f:
        raw = pickle.load(f)   # our own file: the plain loader is fine here
    assert set(raw) == {"params", "config"} and raw["config"] == TINY
    got, cfg = ck.load_weights(str(path))
    assert cfg == TINY
    np.testing.assert_array_equal(got["layer3.ffn.down"], tiny_params["layer3.ffn.down"])


class _Evil:
    def __init__(self, path):
        self.path = path

    def __reduce__(self):
        return (open, (self.path, "w"))


def test_loader_refuses_foreign_globals(tmp_path):
    target = tmp_path / "created_by_pickle"
    blob = pickle.dumps({"params": {"x": _Evil(str(target))}, "config": {}})
    with pytest.raises(pickle.UnpicklingError, match="refusing"):
        ck.safe_loads(blob)
    assert not target.exists()
    path = tmp_path / "weights.pkl"
    path.write_bytes(blob)
    with pytest.raises(pickle.UnpicklingError):
        ck.load_weights(str(path))
    assert not target.exists()
    # os.system through the REDUCE of a module-level function
    blob2 = b"cos\nsystem\n(S'true'\ntR."
    with pytest.raises(pickle.UnpicklingError, match="os.system"):
        ck.safe_loads(blob2)


def test_loader_refuses_object_arrays_and_bad_layout(tmp_path):
    path = tmp_path / "w.pkl"
    with open(path, "wb") as f:
        pickle.dump({"params": {"token_emb": np.array([1, "a"], dtype=object)}, "config": {}}, f)
    with pytest.raises(ValueError, match="dtype"):
        ck.load_weights(str(path))
    with open(path, "wb") as f:
        pickle.dump([1, 2, 3], f)
    with pytest.raises(ValueError, match="params"):
        ck.load_weights(str(path))


def _write_tokenizer(root):
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    tr = trainers.BpeTrainer(vocab_size=300, initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(["Once upon a time there was a tiny model.",
                             "It decoded tokens quickly on a GPU."] * 20, tr)
    os.makedirs(os.path.join(root, "tok"), exist_ok=True)
    os.makedirs(os.path.join(root, "data"), exist_ok=True)
    tok.save(os.path.join(root, "tok", "tokenizer.json"))
    with open(os.path.join(root, "data", "bpe_vocab.pkl"), "wb") as f:   # as data.py:46-47 writes it
        pickle.dump({"tokenizer_path": "tok/tokenizer.json", "vocab_size": tok.get_vocab_size()}, f)
    return tok


def test_bpe_vocab_paths(tmp_path):
    tok = _write_tokenizer(str(tmp_path))
    text = "Once upon a time there was a GPU."
    for src in (str(tmp_path / "data"), str(tmp_path / "data" / "bpe_vocab.pkl"),
                str(tmp_path / "tok" / "tokenizer.json")):
        b = ck.load_bpe_vocab(src)
        assert b["vocab_size"] == tok.get_vocab_size()
        ids = b["encode_fn"](text)
        assert ids == tok.encode(text).ids
        assert b["decode_fn"](np.array(ids)) == text


def test_cli_plumbing(tmp_path, tiny_params, monkeypatch, capsys):
    """Prompt encoding, truncation to ctx-1, the token budget and the printed text."""
    _write_tokenizer(str(tmp_path))
    ck.save_weights(str(tmp_path / "weights.pkl"), tiny_params, TINY)
    calls = []

    def fake_stream(params, config, prompt_ids, max_tokens, temperature, top_p, rep_penalty, seed,
                    device="cuda"):
        calls.append((list(prompt_ids), max_tokens, temperature, top_p, rep_penalty, seed))
        yield from [288, 258, 292][:max_tokens]

    monkeypatch.setattr(gen, "stream_tokens", fake_stream)
    monkeypatch.setattr(gen, "generate_tokens", lambda *a, **k: list(fake_stream(*a, **k)))
    bpe = ck.load_bpe_vocab(str(tmp_path / "data"))
    prompt = "Once upon"
    out = gen.main(["--prompt", prompt, "--weights", str(tmp_path / "weights.pkl"), "--max-tokens", "3"])
    assert out == [288, 258, 292]
    assert calls[-1] == (bpe["encode_fn"](prompt), 3, 0.0, 1.0, 1.0, None)
    text = capsys.readouterr().out
    assert text == prompt + "".join(bpe["decode_fn"]([t]) for t in out) + "\n"
    # a prompt longer than the context keeps ctx-1 tokens and generates one token
    long = "Once upon a time " * 200
    gen.main(["--prompt", long, "--weights", str(tmp_path / "weights.pkl"), "--no-stream",
              "--temp", "0.7", "--top-p", "0.9", "--rep-penalty", "1.2", "--seed", "5",
              "--tokenizer", str(tmp_path / "data" / "bpe_vocab.pkl")])
    ids, n, temp, top_p, pen, seed = calls[-1]
    assert len(ids) == TINY["context_len"] - 1 and ids == bpe["encode_fn"](long)[:TINY["context_len"] - 1]
    assert (n, temp, top_p, pen, seed) == (1, 0.7, 0.9, 1.2, 5)
