"""numpy restatement of the reference model maths and its decode-path semantics.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference files followed (zahlmann/transformer):
  model.py:94-98    rms_norm
  model.py:101-107  precompute_rope_table
  model.py:110-117  apply_rope (rotate-half)
  model.py:122-145  causal_attention (GQA: query head n uses kv head n // (H/KV))
  model.py:150-160  _attn_layer (pre-norm attention + SwiGLU FFN, residuals)
  model.py:163-191  _transformer_trunk / transformer_forward (tied logits)
  model.py:194-231  prefill_with_kv (K post-RoPE and V stored as bf16 caches)
  kernels/multi_sm_decode.py:77-357  one cached decode step: f32 residual,
      new K/V written to the cache as bf16 at ``pos``, the current position's
      K/V used un-rounded (:197, :205), keys beyond ``pos`` masked, logits
      over the vocabulary, argmax resolving ties to the lowest index.

Arithmetic contract ("act_round"):
  * ``None`` — activations stay in the params dtype (f32 by default); this is
    what ``model.py`` computes on f32 parameters and what the HIP decode step
    computes (bf16 weights widened to f32 in registers).
  * ``"bf16"`` — activations are rounded to bf16 right before each matrix
    product (x before Wq/Wk/Wv, the attention output before Wo, x2 before
    gate/up, the SwiGLU activation before down, the final norm before the
    tied logits), as the reference Triton kernel does
    (kernels/multi_sm_decode.py:143, :229, :268, :289, :320) and as an MFMA
    bf16 prefill must.
"""
import numpy as np

from .numerics import bf16_round

F32 = np.float32


def rms_norm(x, scale, eps=1e-5):
    """model.py:94-98: ``scale * (x / sqrt(mean(x^2) + eps))``."""
    x32 = x.astype(F32) if x.dtype != np.float64 else x
    rms = np.sqrt(np.mean(x32 * x32, axis=-1, keepdims=True) + x32.dtype.type(eps)).astype(x.dtype)
    return scale * (x / rms)


def precompute_rope_table(context_len, d_head, base=10000.0, dtype=F32):
    """model.py:101-107: cos/sin of ``pos * base^(-2i/d_head)``, shape (ctx, d_head/2)."""
    half = d_head // 2
    freqs = (np.asarray(base, dtype=F32) ** (-np.arange(0, half, dtype=F32) * F32(2.0) / F32(d_head))).astype(F32)
    positions = np.arange(context_len, dtype=F32)
    angles = positions[:, None] * freqs[None, :]
    if dtype == np.float64:
        angles = angles.astype(np.float64)
    return np.cos(angles).astype(dtype), np.sin(angles).astype(dtype)


def apply_rope(x, cos, sin):
    """model.py:110-117: rotate-half RoPE; x (..., d_head), cos/sin broadcastable to (..., d_head/2)."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * cos - x2 * sin, x1 * sin + x2 * cos], axis=-1)


def silu(x):
    """jax.nn.silu (model.py:159): x * sigmoid(x)."""
    one = x.dtype.type(1.0)
    return x * (one / (one + np.exp(-x)))


def _maybe_round(x, act_round):
    return bf16_round(x) if act_round == "bf16" else x


def _attend(q, K, V, scale):
    """Softmax attention of one query over rows of K/V (all valid). q (dh,), K/V (n, dh)."""
    s = (K @ q) * scale
    s = s - s.max()
    p = np.exp(s)
    p = p / p.sum()
    return p @ V


def causal_attention(x, wq, wk, wv, wo, n_heads, n_kv_heads, cos, sin, act_round=None,
                     return_kv=False):
    """model.py:122-145 on one sequence x (T, d). Returns (T, d) [and post-RoPE K, V]."""
    T, d = x.shape
    dh = d // n_heads
    grp = n_heads // n_kv_heads
    xr = _maybe_round(x, act_round)
    q = (xr @ wq).reshape(T, n_heads, dh)
    k = (xr @ wk).reshape(T, n_kv_heads, dh)
    v = (xr @ wv).reshape(T, n_kv_heads, dh)
    c, s = cos[:T, None, :], sin[:T, None, :]
    q = apply_rope(q, c, s)
    k = apply_rope(k, c, s)
    scale = x.dtype.type(1.0 / np.sqrt(dh))
    out = np.empty((T, n_heads, dh), dtype=x.dtype)
    for n in range(n_heads):
        g = n // grp
        sc = (q[:, n, :] @ k[:, g, :].T) * scale          # (T, T)
        sc = np.where(np.tril(np.ones((T, T), dtype=bool)), sc, -np.inf)
        sc = sc - sc.max(axis=1, keepdims=True)
        p = np.exp(sc)
        p = p / p.sum(axis=1, keepdims=True)
        out[:, n, :] = p @ v[:, g, :]
    o = _maybe_round(out.reshape(T, d), act_round) @ wo
    if return_kv:
        return o, k, v
    return o


def _layer_params(params, i):
    p = f"layer{i}"
    return (params[f"{p}.ln1.scale"], params[f"{p}.attn.q"], params[f"{p}.attn.k"],
            params[f"{p}.attn.v"], params[f"{p}.attn.o"], params[f"{p}.ln2.scale"],
            params[f"{p}.ffn.gate"], params[f"{p}.ffn.up"], params[f"{p}.ffn.down"])


def _ffn(x2, wg, wu, wd, act_round):
    xr = _maybe_round(x2, act_round)
    a = silu(xr @ wg) * (xr @ wu)
    return _maybe_round(a, act_round) @ wd


def forward(params, config, tokens, act_round=None):
    """model.py:188-191 transformer_forward: logits (T, V) for token ids (T,)."""
    emb = params["token_emb"]
    cos, sin = precompute_rope_table(config["context_len"], config["d_head"], dtype=emb.dtype)
    h = emb[np.asarray(tokens)]
    for i in range(config["n_layers"]):
        ln1, wq, wk, wv, wo, ln2, wg, wu, wd = _layer_params(params, i)
        h = h + causal_attention(rms_norm(h, ln1), wq, wk, wv, wo, config["n_heads"],
                                 config["n_kv_heads"], cos, sin, act_round)
        h = h + _ffn(rms_norm(h, ln2), wg, wu, wd, act_round)
    hf = _maybe_round(rms_norm(h, params["ln_final.scale"]), act_round)
    return hf @ emb.T


def new_kv_cache(config, dtype=F32):
    """Per-layer K and V caches of shape (n_kv_heads, context_len, d_head), zero-filled."""
    shp = (config["n_kv_heads"], config["context_len"], config["d_head"])
    return [np.zeros(shp, dtype) for _ in range(config["n_layers"])], \
           [np.zeros(shp, dtype) for _ in range(config["n_layers"])]


def prefill_with_kv(params, config, tokens, act_round=None):
    """model.py:194-231: full forward over ``tokens``; returns (logits (T,V), k_caches, v_caches).

    Caches hold bf16-rounded values (model.py:212-215) stored in the params dtype, of shape
    (n_kv_heads, context_len, d_head); rows >= T stay zero.
    """
    emb = params["token_emb"]
    T = len(tokens)
    cos, sin = precompute_rope_table(config["context_len"], config["d_head"], dtype=emb.dtype)
    kc, vc = new_kv_cache(config, emb.dtype)
    h = emb[np.asarray(tokens)]
    for i in range(config["n_layers"]):
        ln1, wq, wk, wv, wo, ln2, wg, wu, wd = _layer_params(params, i)
        a, k, v = causal_attention(rms_norm(h, ln1), wq, wk, wv, wo, config["n_heads"],
                                   config["n_kv_heads"], cos, sin, act_round, return_kv=True)
        kc[i][:, :T, :] = bf16_round(k.transpose(1, 0, 2))
        vc[i][:, :T, :] = bf16_round(v.transpose(1, 0, 2))
        h = h + a
        h = h + _ffn(rms_norm(h, ln2), wg, wu, wd, act_round)
    hf = _maybe_round(rms_norm(h, params["ln_final.scale"]), act_round)
    return hf @ emb.T, kc, vc


def decode_step(params, config, token, pos, k_caches, v_caches, act_round=None, rope=None):
    """One cached decode step (kernels/multi_sm_decode.py:77-357 semantics).

    Writes bf16(K_new), bf16(V_new) at ``pos`` into the caches (in place), attends over
    cache rows 0..pos-1 plus the un-rounded current K/V, and returns (logits (V,), argmax).
    Cache rows > pos are never read.
    """
    emb = params["token_emb"]
    H, KV, dh = config["n_heads"], config["n_kv_heads"], config["d_head"]
    grp = H // KV
    if rope is None:
        rope = precompute_rope_table(config["context_len"], dh, dtype=emb.dtype)
    cos, sin = rope[0][pos], rope[1][pos]
    scale = emb.dtype.type(1.0 / np.sqrt(dh))
    h = emb[int(token)].copy()
    for i in range(config["n_layers"]):
        ln1, wq, wk, wv, wo, ln2, wg, wu, wd = _layer_params(params, i)
        x = _maybe_round(rms_norm(h, ln1), act_round)
        q = apply_rope((x @ wq).reshape(H, dh), cos, sin)
        k = apply_rope((x @ wk).reshape(KV, dh), cos, sin)
        v = (x @ wv).reshape(KV, dh)
        k_caches[i][:, pos, :] = bf16_round(k)
        v_caches[i][:, pos, :] = bf16_round(v)
        att = np.empty((H, dh), dtype=h.dtype)
        for n in range(H):
            g = n // grp
            Kg = k_caches[i][g, :pos + 1, :].copy()
            Vg = v_caches[i][g, :pos + 1, :].copy()
            Kg[pos] = k[g]
            Vg[pos] = v[g]
            att[n] = _attend(q[n], Kg, Vg, scale)
        h = h + _maybe_round(att.reshape(-1), act_round) @ wo
        h = h + _ffn(rms_norm(h, ln2), wg, wu, wd, act_round)
    hf = _maybe_round(rms_norm(h, params["ln_final.scale"]), act_round)
    logits = emb @ hf
    return logits, int(np.argmax(logits))


def greedy_generate(params, config, prompt, n_new, prefill="step", act_round=None,
                    return_logits=False, prefill_act_round="same"):
    """Greedy generation following generate.py:92-123.

    prefill="full": the prompt goes through ``prefill_with_kv`` (the reference pipeline),
    with ``prefill_act_round`` (default: the same as ``act_round``);
    prefill="step": the prompt is fed through ``decode_step`` at positions 0..P-1.
    The first new token is the argmax at position P-1; step i then runs at pos P+i on
    the previous token.  Returns the list of n_new tokens (and per-token logits).
    """
    P = len(prompt)
    rope = precompute_rope_table(config["context_len"], config["d_head"], dtype=params["token_emb"].dtype)
    if prefill == "full":
        par = act_round if prefill_act_round == "same" else prefill_act_round
        logits_all, kc, vc = prefill_with_kv(params, config, prompt, par)
        last = logits_all[P - 1]
    else:
        kc, vc = new_kv_cache(config, params["token_emb"].dtype)
        for p, t in enumerate(prompt):
            last, _ = decode_step(params, config, t, p, kc, vc, act_round, rope)
    toks, logs = [int(np.argmax(last))], [last]
    for i in range(n_new - 1):
        lg, nt = decode_step(params, config, toks[-1], P + i, kc, vc, act_round, rope)
        toks.append(nt)
        logs.append(lg)
    return (toks, logs) if return_logits else toks
