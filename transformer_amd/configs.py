"""Model configurations (same keys as the reference config dict, model.py:37-47)."""

# Tiny GQA config: d=256, 4 heads, 1 kv head, 4 layers, d_ff=704, ctx 128.
TINY = dict(vocab_size=32000, d_model=256, n_heads=4, n_kv_heads=1, n_layers=4,
            d_head=64, d_ff=704, context_len=128)

# 306M config: d=1024, 16 heads, 4 kv heads, 24 layers, d_ff=2816, ctx 512.
M306 = dict(vocab_size=32000, d_model=1024, n_heads=16, n_kv_heads=4, n_layers=24,
            d_head=64, d_ff=2816, context_len=512)


def check_config(config, need=("decode", "prefill")):
    """Validate a config against the library's paths; returns d_head, raises ValueError.

    The shape relations come first (n_heads * d_head == d_model, GQA grouping); then every path
    named in ``need`` (``"decode"``, ``"prefill"``, ``"verify"``, ``"batched"``, ``"sample"``) must
    accept the config (``msd_config_support``, no device call), so an unsupported checkpoint is
    refused before any weight reaches the device."""
    d, H, KV = config["d_model"], config["n_heads"], config["n_kv_heads"]
    dh = config.get("d_head", d // H)
    if H * dh != d:
        raise ValueError(f"n_heads*d_head ({H}*{dh}) != d_model ({d})")
    if H % KV != 0:
        raise ValueError(f"n_heads ({H}) not a multiple of n_kv_heads ({KV})")
    missing = [p for p in need if p not in supported_paths(config)]
    if missing:
        raise ValueError(f"config (d_model {d}, d_ff {config['d_ff']}, d_head {dh}, context_len "
                         f"{config['context_len']}, vocab {config['vocab_size']}) is not supported by the "
                         f"{', '.join(missing)} path(s): the fused decode step takes d_head 64, (d_model, d_ff) in "
                         f"{DECODE_SHAPES} and context_len <= 2048; prefill takes d_model <= 1024")
    return dh


# (d_model, d_ff) pairs the fused decode step is compiled for: the reference's
# d_ff = 8 d / 3 rounded up to 128 (model.py:13-20) for d_model 256..1024, and d_ff 704 at 256
DECODE_SHAPES = ((256, 704), (256, 768), (512, 1408), (768, 2048), (1024, 2816))


def supported_paths(config, n_workgroups=0):
    """Names of the library paths that accept ``config`` (``msd_config_support``)."""
    import ctypes

    from . import _lib
    c = _lib.MsdConfig.from_dict(config)
    bits = _lib.check(_lib.lib().msd_config_support(ctypes.byref(c), int(n_workgroups)), "msd_config_support")
    return {name for name, b in _lib.PATHS.items() if bits & b}


def bytes_per_token(config, pos):
    """Algorithmic HBM bytes of one decode step at position ``pos`` (bf16 weights and KV).

    weights: 2*[L*(2d + 2d^2 + 2d*d_kv + 3d*d_ff) + V*d + 2d + d_head]: per-layer norm scales
      and projections, the tied output projection, the embedding row, the final norm scale
      and one RoPE cos/sin row (606,703,744 B for the 306M config);
    KV read: L*2*KV*(pos+1)*d_head*2 (24,576*(pos+1) B at 306M);
    KV write: L*2*KV*d_head*2 (24,576 B at 306M).
    """
    d, L, V = config["d_model"], config["n_layers"], config["vocab_size"]
    KV, dh, ff = config["n_kv_heads"], config["d_head"], config["d_ff"]
    dkv = KV * dh
    w = 2 * (L * (2 * d + 2 * d * d + 2 * d * dkv + 3 * d * ff) + V * d + 2 * d + dh)
    kv_row = L * 2 * KV * dh * 2
    return w + kv_row * (pos + 1) + kv_row
