"""Weight and KV packing for the fused decode step (drop-in for the reference module).

Same names, arguments and dict keys as zahlmann/transformer
kernels/fused_decode_nlayer.py:250-321, over torch tensors on the GPU.

Packed weight layout (kernel layout, bf16, per layer, one contiguous block):
    ln1_scale (d) | ln2_scale (d)
    | qkv rows ((H + 2*KV) * 64 rows of d)   row r of head h = column of wq/wk/wv
    | o rows   (d rows of d)                 row j = column j of wo
    | gate/up rows (2*d_ff rows of d)        gate column f, then up column f, interleaved
    | down rows (d rows of d_ff)             row j = column j of down
Every output element of a projection is one contiguous row (the transpose of the
reference's (in, out) matrices, fused_decode_nlayer.py:260-268), so the kernel reads
each output's weights as one run of 128-bit loads.  Within each q and k head the rows
are ordered (0, 32, 1, 33, ..., 31, 63) so a rotate-half RoPE pair (model.py:110-117)
is two adjacent rows.  Within every row the input dimension is permuted by
``kernel_perm`` (blocks of 512; in block b, position 8*l + k holds input 512*b + k*m + l,
m = lanes of the block), so each lane of a wave multiplies its 8 loaded weights with
inputs that consecutive lanes read from consecutive LDS words.

The reference's ``output_proj_padded`` (the transposed, padded embedding,
fused_decode_nlayer.py:312-319) becomes ``output_proj``: the (V, d) embedding with every
row in the kernel row layout (no transpose, no padding).  ``vocab_pad`` is still
reported as the reference computes it.  RoPE tables stay float32 (model.py:101-107) instead of the reference's bf16
copies (fused_decode_nlayer.py:317-318); ``rope`` holds them as one (ctx, d_head) table.
"""
import ctypes

import numpy as np
import torch

from . import _lib


def _dev(device):
    return torch.device(device if device is not None else "cuda")


def _bf16(a, device):
    if isinstance(a, torch.Tensor):
        return a.to(device=device, dtype=torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(device)


def kernel_perm(k):
    """Index array p with packed_row = row[p] for the kernel row layout of a k-long row."""
    assert k % 8 == 0
    p = np.empty(k, dtype=np.int64)
    for b in range(0, k, 512):
        s = min(512, k - b)
        m = s // 8
        lanes = np.arange(m)
        for q in range(8):
            p[b + 8 * lanes + q] = b + q * m + lanes
    return torch.from_numpy(p)


def _rope_perm(dh=64):
    half = dh // 2
    return torch.tensor([i // 2 if i % 2 == 0 else half + i // 2 for i in range(dh)])


def precompute_rope_table(context_len, d_head, base=10000.0):
    """model.py:101-107 in float32: cos, sin of shape (context_len, d_head // 2)."""
    half = d_head // 2
    freqs = (np.float32(base) ** (-np.arange(0, half, dtype=np.float32) * np.float32(2.0)
                                   / np.float32(d_head))).astype(np.float32)
    ang = np.arange(context_len, dtype=np.float32)[:, None] * freqs[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def pack_layer(params, config, i, device=None):
    """Kernel-layout bf16 block of layer ``i`` (see module docstring)."""
    dev = _dev(device)
    d, H, KV = config["d_model"], config["n_heads"], config["n_kv_heads"]
    dh = config.get("d_head", d // H)
    p = f"layer{i}"
    perm = _rope_perm(dh).to(dev)
    kd = kernel_perm(d).to(dev)
    kf = kernel_perm(config["d_ff"]).to(dev)
    wq = _bf16(params[f"{p}.attn.q"], dev).t().reshape(H, dh, d)[:, perm].reshape(H * dh, d)[:, kd]
    wk = _bf16(params[f"{p}.attn.k"], dev).t().reshape(KV, dh, d)[:, perm].reshape(KV * dh, d)[:, kd]
    wv = _bf16(params[f"{p}.attn.v"], dev).t()[:, kd]
    wo = _bf16(params[f"{p}.attn.o"], dev).t()[:, kd]
    g = _bf16(params[f"{p}.ffn.gate"], dev).t()[:, kd]
    u = _bf16(params[f"{p}.ffn.up"], dev).t()[:, kd]
    gu = torch.stack([g, u], dim=1).reshape(-1, d)
    dn = _bf16(params[f"{p}.ffn.down"], dev).t()[:, kf]
    parts = [_bf16(params[f"{p}.ln1.scale"], dev).reshape(-1), _bf16(params[f"{p}.ln2.scale"], dev).reshape(-1),
             wq, wk, wv, wo, gu, dn]
    return torch.cat([t.contiguous().reshape(-1) for t in parts])


def pack_weights(params, config, device=None):
    """Pack all layers into one bf16 buffer (reference: fused_decode_nlayer.py:250-270)."""
    cfg = _lib.MsdConfig.from_dict(config)
    n = _lib.check(_lib.lib().msd_packed_weight_elems(cfg), "msd_packed_weight_elems")
    out = torch.empty(n, dtype=torch.bfloat16, device=_dev(device))
    per = n // config["n_layers"]
    for i in range(config["n_layers"]):
        out[i * per:(i + 1) * per] = pack_layer(params, config, i, device)
    return out


def pack_kv_caches(k_caches, v_caches, device=None):
    """Flat bf16 KV buffer [layer][K, V][kv_head][max_seq][d_head] (fused_decode_nlayer.py:273-283).

    Inputs: per-layer K and V caches of shape (n_kv_heads, max_seq, d_head), K post-RoPE.
    """
    dev = _dev(device)
    parts = []
    for k, v in zip(k_caches, v_caches):
        parts.append(_bf16(k, dev).reshape(-1))
        parts.append(_bf16(v, dev).reshape(-1))
    return torch.cat(parts)


def unpack_kv_caches(packed, n_layers, n_kv_heads, max_seq, d_head):
    """Inverse of pack_kv_caches (fused_decode_nlayer.py:286-296); returns views."""
    layer = 2 * n_kv_heads * max_seq * d_head
    cache = n_kv_heads * max_seq * d_head
    ks, vs = [], []
    for i in range(n_layers):
        b = i * layer
        ks.append(packed[b:b + cache].view(n_kv_heads, max_seq, d_head))
        vs.append(packed[b + cache:b + layer].view(n_kv_heads, max_seq, d_head))
    return ks, vs


def new_kv_packed(config, device=None):
    """Zero-filled packed KV buffer for ``config``."""
    n = config["n_layers"] * 2 * config["n_kv_heads"] * config["context_len"] * config.get(
        "d_head", config["d_model"] // config["n_heads"])
    return torch.zeros(n, dtype=torch.bfloat16, device=_dev(device))


def prepare_decode_weights_nlayer(params, config, kv_splits=1, device=None):
    """Decode weight dict (reference: fused_decode_nlayer.py:299-321).

    Keys: token_emb (V, d) bf16, output_proj (V, d) bf16 in the kernel row layout,
    packed_w (kernel layout), lnf_s (d) bf16, cos/sin (ctx, d_head/2) f32,
    rope (ctx, d_head) f32 = [cos | sin], vocab_pad (reference value).  The multi-row passes add
    ``tiles`` (``weight_tiles``) on first use.
    """
    from .configs import check_config
    dh = check_config(config, need=("decode",))
    dev = _dev(device)
    vocab = config["vocab_size"]
    align = 32 * config["n_heads"] * kv_splits
    vocab_pad = ((vocab + align - 1) // align) * align
    cos, sin = precompute_rope_table(config["context_len"], dh)
    rope = np.concatenate([cos, sin], axis=1)
    emb = _bf16(params["token_emb"], dev).contiguous()
    return {
        "token_emb": emb,
        "output_proj": emb[:, kernel_perm(config["d_model"]).to(dev)].contiguous(),
        "packed_w": pack_weights(params, config, dev),
        "lnf_s": _bf16(params["ln_final.scale"], dev).contiguous(),
        "cos": torch.from_numpy(cos).to(dev),
        "sin": torch.from_numpy(sin).to(dev),
        "rope": torch.from_numpy(np.ascontiguousarray(rope)).to(dev),
        "vocab_pad": vocab_pad,
    }


def weight_tiles(w, config):
    """The tile copy of ``w``'s projection weights (``msd_pack_tiles``: every matrix as 16 x 32
    tiles in matrix-core operand order), built on the device on first use and kept in
    ``w["tiles"]``.  The multi-row passes (prefill, verification, the multi-kernel batched step)
    read their projections from it; it takes as much device memory as ``packed_w``."""
    t = w.get("tiles")
    if t is None:
        cfg = _lib.MsdConfig.from_dict(config)
        L = _lib.lib()
        nbytes = _lib.check(L.msd_tiles_bytes(ctypes.byref(cfg)), "msd_tiles_bytes")
        dev = w["packed_w"].device
        t = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev)
        s = torch.cuda.current_stream(dev)
        _lib.check(L.msd_pack_tiles(ctypes.byref(cfg), w["packed_w"].data_ptr(), t.data_ptr(),
                                    ctypes.c_void_p(s.cuda_stream)), "msd_pack_tiles")
        w["tiles"] = t
    return t
