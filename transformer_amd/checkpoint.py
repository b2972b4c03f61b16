"""Trained checkpoints and the BPE tokenizer (drop-in for the reference's file formats).

  load_weights(path) -> (params, config)      reads train.py:246-248's ``weights.pkl``
  save_weights(path, params, config)          writes the same format
  load_bpe_vocab(data_dir)                    data.py:55-70 (tokenizer path + vocab size)

``weights.pkl`` is a pickle of ``{"params": {name: numpy array}, "config": dict}``
(train.py:246-248); generate.py:163-168 loads it with ``pickle.load``.  A pickle can name
any importable callable, so this loader never runs ``pickle.load``: its unpickler resolves
only the numpy reconstructors an array needs (ndarray, dtype, ``_reconstruct``,
``_frombuffer``, scalar, and ``_codecs.encode`` for protocol-2 bytes) and refuses every
other global with ``pickle.UnpicklingError`` before anything is called.  Arrays of object dtype are refused as well.  Plain containers,
strings and numbers need no globals.  ``data/bpe_vocab.pkl`` (``{"tokenizer_path",
"vocab_size"}``, data.py:46-47) goes through the same unpickler.
"""
import io
import os
import pickle

import numpy as np

# (module, name) pairs a pickled numpy array may reference (numpy 1.x and 2.x spellings)
_ALLOWED = {
    ("numpy", "ndarray"),
    ("numpy", "dtype"),
    ("numpy.core.multiarray", "_reconstruct"),
    ("numpy._core.multiarray", "_reconstruct"),
    ("numpy.core.multiarray", "scalar"),
    ("numpy._core.multiarray", "scalar"),
    ("numpy.core.numeric", "_frombuffer"),
    ("numpy._core.numeric", "_frombuffer"),
    ("_codecs", "encode"),   # protocol 2 spells bytes as encode(str, "latin1")
}


class SafeUnpickler(pickle.Unpickler):
    """Unpickler that resolves only the numpy array reconstructors (see module doc)."""

    def find_class(self, module, name):
        if (module, name) in _ALLOWED:
            return super().find_class(module, name)
        raise pickle.UnpicklingError(f"refusing to load global {module}.{name}")


def safe_load(f):
    """Unpickle from a binary file object with ``SafeUnpickler``."""
    return SafeUnpickler(f).load()


def safe_loads(data):
    return safe_load(io.BytesIO(data))


def _check_array(name, a):
    if not isinstance(a, np.ndarray):
        raise ValueError(f"parameter {name!r} is not a numpy array ({type(a).__name__})")
    if a.dtype.kind not in "fiu":
        raise ValueError(f"parameter {name!r} has unsupported dtype {a.dtype}")


def _infer_config(params, config):
    """Fill config keys the kernels need but older checkpoints may lack."""
    c = dict(config)
    if "d_head" not in c:
        c["d_head"] = c["d_model"] // c["n_heads"]
    if "d_ff" not in c:
        c["d_ff"] = int(params["layer0.ffn.gate"].shape[1])
    if "vocab_size" not in c:
        c["vocab_size"] = int(params["token_emb"].shape[0])
    return c


def load_weights(path):
    """Load a reference ``weights.pkl``; returns ``(params, config)``.

    ``params`` maps the reference's parameter names (model.py:37-83) to float32 numpy
    arrays in (in, out) orientation; extra entries (for example MTP heads) are kept.
    """
    with open(path, "rb") as f:
        saved = safe_load(f)
    if not isinstance(saved, dict) or "params" not in saved or "config" not in saved:
        raise ValueError(f"{path}: expected a dict with 'params' and 'config'")
    params, config = saved["params"], saved["config"]
    if not isinstance(params, dict) or not isinstance(config, dict):
        raise ValueError(f"{path}: 'params' and 'config' must be dicts")
    out = {}
    for k, v in params.items():
        _check_array(k, v)
        out[str(k)] = np.ascontiguousarray(v, dtype=np.float32)
    config = {str(k): (v.item() if isinstance(v, np.generic) else v) for k, v in config.items()}
    config = _infer_config(out, config)
    for k in ("token_emb", "ln_final.scale"):
        if k not in out:
            raise ValueError(f"{path}: missing parameter {k!r}")
    return out, config


def save_weights(path, params, config):
    """Write ``{"params", "config"}`` the way train.py:246-248 does."""
    with open(path, "wb") as f:
        pickle.dump({"params": {k: np.asarray(v) for k, v in params.items()}, "config": dict(config)}, f)


def load_bpe_vocab(data_dir="data"):
    """Tokenizer of a trained model (data.py:55-70).

    ``data_dir`` holds ``bpe_vocab.pkl``; a relative ``tokenizer_path`` in it is taken
    relative to the directory above ``data_dir`` (the reference's repository root).  A path
    to a ``tokenizer.json`` may be given instead.  Returns a dict with ``tokenizer_path``,
    ``vocab_size``, ``decode_fn`` and ``encode_fn``.
    """
    from tokenizers import Tokenizer

    if os.path.isfile(data_dir) and not data_dir.endswith(".pkl"):
        tok_path, vocab_size = data_dir, None
    else:
        pkl = data_dir if os.path.isfile(data_dir) else os.path.join(data_dir, "bpe_vocab.pkl")
        with open(pkl, "rb") as f:
            saved = safe_load(f)
        if not isinstance(saved, dict) or "tokenizer_path" not in saved:
            raise ValueError(f"{pkl}: expected a dict with 'tokenizer_path'")
        tok_path, vocab_size = str(saved["tokenizer_path"]), saved.get("vocab_size")
        if not os.path.isabs(tok_path):
            tok_path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(pkl))), tok_path)
    tok = Tokenizer.from_file(tok_path)
    if vocab_size is None:
        vocab_size = tok.get_vocab_size()
    return {
        "tokenizer_path": tok_path,
        "vocab_size": int(vocab_size),
        "decode_fn": lambda ids: tok.decode([int(i) for i in ids]),
        "encode_fn": lambda text: tok.encode(text).ids,
    }
