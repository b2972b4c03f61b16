"""Seeded synthetic weights and prompts for the benchmark configurations.

There are no checkpoints or datasets here, so weights are random-init: every
matrix ~ N(0, std) with std 0.02, rounded to bf16 (round-to-nearest-even) and
held in float32 arrays; RMSNorm scales are 1.  With ``resid_scaled=True`` the
residual-branch output projections (``attn.o`` and ``ffn.down``) use
std 0.02/sqrt(2*n_layers).  Matrices are drawn in the order of the reference
initialiser (model.py:49-83: token_emb, then per layer q, k, v, o, gate, up,
down) from one ``numpy.random.Generator(PCG64(seed))`` stream in float32.

The parameter dict uses the reference's names and (in, out) orientation, i.e.
the ``params`` layout ``prepare_decode_weights_nlayer`` consumes
(model.py:37-91, kernels/fused_decode_nlayer.py:250-270).
"""
import numpy as np


def bf16_round_np(a):
    """Round a float32 array to bf16 values (ties to even), returned as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    r = ((u >> 16) & np.uint32(1)) + np.uint32(0x7FFF)
    return ((u + r) & np.uint32(0xFFFF0000)).view(np.float32)


def make_params(config, seed=0, std=0.02, resid_scaled=False):
    rng = np.random.Generator(np.random.PCG64(seed))
    d, V, ff = config["d_model"], config["vocab_size"], config["d_ff"]
    dkv = config["n_kv_heads"] * config["d_head"]
    L = config["n_layers"]
    rstd = std / np.sqrt(2.0 * L) if resid_scaled else std

    def draw(shape, s):
        return bf16_round_np(rng.standard_normal(shape, dtype=np.float32) * np.float32(s))

    params = {"token_emb": draw((V, d), std)}
    for i in range(L):
        p = f"layer{i}"
        params[f"{p}.ln1.scale"] = np.ones(d, np.float32)
        params[f"{p}.attn.q"] = draw((d, d), std)
        params[f"{p}.attn.k"] = draw((d, dkv), std)
        params[f"{p}.attn.v"] = draw((d, dkv), std)
        params[f"{p}.attn.o"] = draw((d, d), rstd)
        params[f"{p}.ln2.scale"] = np.ones(d, np.float32)
        params[f"{p}.ffn.gate"] = draw((d, ff), std)
        params[f"{p}.ffn.up"] = draw((d, ff), std)
        params[f"{p}.ffn.down"] = draw((ff, d), rstd)
    params["ln_final.scale"] = np.ones(d, np.float32)
    return params


def make_prompt(n, vocab_size, seed=1):
    """``n`` token ids uniform in [0, vocab_size) from ``Generator(PCG64(seed))``."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.integers(0, vocab_size, size=n, dtype=np.int64).astype(np.int32)
