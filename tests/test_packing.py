"""Packing layout contract (CPU): kernel-layout rows equal the reference matrices' columns."""
import ctypes

import numpy as np
import torch

from transformer_amd import _lib
from transformer_amd.configs import TINY
from transformer_amd.fused_decode_nlayer import (kernel_perm, pack_kv_caches, pack_layer,
                                                 precompute_rope_table, unpack_kv_caches)
from transformer_amd.synthetic import make_params


def test_library_exports_every_declared_symbol():
    """Every function the headers under include/ declare is exported by the library, and the
    binding's list is exactly that set."""
    import glob
    import re
    L = _lib.lib()
    declared = set()
    for h in sorted(glob.glob(_lib.os.path.join(_lib.HERE, "..", "include", "*.h"))):
        declared |= set(re.findall(r"\b(msd_[a-z_]+)\s*\(", open(h).read()))
    assert declared == set(_lib.EXPORTS)
    for name in declared:
        assert getattr(L, name) is not None


def test_packed_layer_layout(tiny_params):
    cfg = TINY
    d, H, KV, ff, dh = cfg["d_model"], cfg["n_heads"], cfg["n_kv_heads"], cfg["d_ff"], 64
    blk = pack_layer(tiny_params, cfg, 1, device="cpu").float().numpy()
    n = _lib.lib().msd_packed_weight_elems(ctypes.byref(_lib.MsdConfig.from_dict(cfg)))
    assert blk.size * cfg["n_layers"] == n
    p = "layer1"
    o = 0
    np.testing.assert_array_equal(blk[o:o + d], tiny_params[f"{p}.ln1.scale"]); o += d
    np.testing.assert_array_equal(blk[o:o + d], tiny_params[f"{p}.ln2.scale"]); o += d
    # undo the in-dimension permutation of the kernel row layout
    inv_d = np.argsort(kernel_perm(d).numpy())
    inv_f = np.argsort(kernel_perm(ff).numpy())
    qkv = blk[o:o + (H + 2 * KV) * dh * d].reshape(-1, d)[:, inv_d]; o += (H + 2 * KV) * dh * d
    for h in range(H):
        for r in range(dh):
            orig = r // 2 if r % 2 == 0 else 32 + r // 2
            np.testing.assert_array_equal(qkv[h * dh + r], tiny_params[f"{p}.attn.q"][:, h * dh + orig])
    for g in range(KV):
        for r in range(dh):
            orig = r // 2 if r % 2 == 0 else 32 + r // 2
            np.testing.assert_array_equal(qkv[(H + g) * dh + r], tiny_params[f"{p}.attn.k"][:, g * dh + orig])
            np.testing.assert_array_equal(qkv[(H + KV + g) * dh + r], tiny_params[f"{p}.attn.v"][:, g * dh + r])
    wo = blk[o:o + d * d].reshape(d, d)[:, inv_d]; o += d * d
    np.testing.assert_array_equal(wo, tiny_params[f"{p}.attn.o"].T)
    gu = blk[o:o + 2 * ff * d].reshape(2 * ff, d)[:, inv_d]; o += 2 * ff * d
    np.testing.assert_array_equal(gu[0::2], tiny_params[f"{p}.ffn.gate"].T)
    np.testing.assert_array_equal(gu[1::2], tiny_params[f"{p}.ffn.up"].T)
    dn = blk[o:o + d * ff].reshape(d, ff)[:, inv_f]; o += d * ff
    np.testing.assert_array_equal(dn, tiny_params[f"{p}.ffn.down"].T)
    assert o == blk.size


def test_kv_pack_roundtrip():
    rng = np.random.default_rng(0)
    ks = [rng.standard_normal((2, 16, 64)).astype(np.float32) for _ in range(3)]
    vs = [rng.standard_normal((2, 16, 64)).astype(np.float32) for _ in range(3)]
    flat = pack_kv_caches(ks, vs, device="cpu")
    assert flat.dtype == torch.bfloat16 and flat.numel() == 3 * 2 * 2 * 16 * 64
    k2, v2 = unpack_kv_caches(flat, 3, 2, 16, 64)
    for a, b in zip(ks + vs, k2 + v2):
        np.testing.assert_array_equal(torch.from_numpy(a).to(torch.bfloat16).float().numpy(), b.float().numpy())
    # layer 1 K starts after layer 0's K and V
    assert torch.equal(flat[2 * 2 * 16 * 64:3 * 2 * 16 * 64].view(2, 16, 64), k2[1])


def test_rope_table_matches_reference_formula():
    c, s = precompute_rope_table(512, 64)
    f = np.float32(10000.0) ** (-np.arange(32, dtype=np.float32) * np.float32(2.0) / np.float32(64))
    ang = np.arange(512, dtype=np.float32)[:, None] * f[None, :]
    np.testing.assert_array_equal(c, np.cos(ang))
    np.testing.assert_array_equal(s, np.sin(ang))


def test_kernel_perm_layout():
    """Block b, lane l, value q of the packed row is input 512*b + q*m + l (m lanes in the block)."""
    for k in (256, 1024, 704, 2816):
        p = kernel_perm(k).numpy()
        assert sorted(p.tolist()) == list(range(k))
        for b in range(0, k, 512):
            m = min(512, k - b) // 8
            for lane in (0, m - 1):
                for q in (0, 7):
                    assert p[b + 8 * lane + q] == b + q * m + lane


def test_config_support_query():
    """msd_config_support (no device call): the benchmark shapes take every path up to a
    2048-position context (the persistent batched step up to 512); beyond it only prefill and the
    sampler; a d_model 2048 checkpoint is refused by check_config and by the weight preparation
    before anything reaches a device."""
    import pytest
    from transformer_amd.configs import M306, TINY, check_config, supported_paths
    from transformer_amd.fused_decode_nlayer import prepare_decode_weights_nlayer
    every = {"decode", "prefill", "verify", "batched", "sample"}
    for cfg in (TINY, M306):
        for ctx in (128, 512, 1024, 2048):
            step = {"batched_step"} if ctx <= 512 else set()
            assert supported_paths(dict(cfg, context_len=ctx)) == every | step
        assert supported_paths(dict(cfg, context_len=4096)) == {"prefill", "sample"}
    big = dict(M306, d_model=2048, n_heads=32, d_ff=5504)
    assert supported_paths(big) == {"sample"}
    with pytest.raises(ValueError, match="decode"):
        check_config(big)
    with pytest.raises(ValueError, match="decode"):
        prepare_decode_weights_nlayer({}, big, device="cpu")
    assert "decode" not in supported_paths(dict(M306, d_ff=2944))   # no instance for this d_ff
    assert supported_paths(dict(TINY, vocab_size=40000)) == (every | {"batched_step"}) - {"sample"}
