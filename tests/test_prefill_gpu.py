"""Parity of the matrix-core prefill (msd_prefill) with the oracle (GPU).

Every projection input enters the matrix cores as two bf16 parts (hi + lo, f32 to about
2^-17), so the oracle is the f32 ``prefill_with_kv`` (model.py:194-231); logits are compared to
2e-2 abs / 1e-2 rel, the bf16 KV cache rows to the same bound.
"""
import numpy as np
import pytest
import torch

from oracle import model as om
from transformer_amd.configs import M306, TINY
from transformer_amd.fused_decode_nlayer import (kernel_perm, new_kv_packed, prepare_decode_weights_nlayer,
                                                 unpack_kv_caches, weight_tiles)
from transformer_amd.multi_sm_decode import Decoder
from transformer_amd.prefill import Prefiller, prefill_with_kv
from transformer_amd.synthetic import make_params, make_prompt

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2
SENTINEL = 7.0


@pytest.fixture(scope="module")
def tiny():
    params = make_params(TINY, seed=0)
    return params, prepare_decode_weights_nlayer(params, TINY)


@pytest.fixture(scope="module")
def m306():
    params = make_params(M306, seed=0, resid_scaled=True)
    return params, prepare_decode_weights_nlayer(params, M306)


def _run(w, cfg, toks, all_logits=True, tiles=True):
    T = len(toks)
    pf = Prefiller(w, cfg, max_tokens=T, tiles=tiles)
    kv = new_kv_packed(cfg).fill_(SENTINEL)
    la = torch.empty((T, cfg["vocab_size"]), dtype=torch.float32, device="cuda") if all_logits else None
    out = pf.launch(toks, kv, logits_all=la)
    torch.cuda.synchronize()
    return (None if la is None else la.cpu().numpy()), pf.logits.cpu().numpy(), out.cpu().numpy(), kv


def _check_kv(kv, cfg, T, kc, vc):
    ks, vs = unpack_kv_caches(kv, cfg["n_layers"], cfg["n_kv_heads"], cfg["context_len"], cfg["d_head"])
    for l in range(cfg["n_layers"]):
        k = ks[l].float().cpu().numpy()
        v = vs[l].float().cpu().numpy()
        np.testing.assert_allclose(k[:, :T], kc[l][:, :T], atol=ATOL, rtol=RTOL)
        np.testing.assert_allclose(v[:, :T], vc[l][:, :T], atol=ATOL, rtol=RTOL)
        assert np.all(k[:, T:] == SENTINEL) and np.all(v[:, T:] == SENTINEL), "rows >= T were written"


@pytest.mark.parametrize("tiles", [True, False], ids=["tiles", "rows"])
@pytest.mark.parametrize("T", [1, 16, 77, 128])
def test_tiny_prefill_matches_oracle(tiny, T, tiles):
    """Both weight layouts: the tile copy (msd_pack_tiles) and the packed rows."""
    params, w = tiny
    toks = make_prompt(T, TINY["vocab_size"], seed=100 + T)
    la, last, out, kv = _run(w, TINY, toks, tiles=tiles)
    ref, kc, vc = om.prefill_with_kv(params, TINY, toks)
    np.testing.assert_allclose(la, ref, atol=ATOL, rtol=RTOL)
    assert np.array_equal(last, la[-1])
    assert out[0] == int(np.argmax(la[-1])) and out[1] == 0
    _check_kv(kv, TINY, T, kc, vc)
    # the last-position-only path computes the same row bitwise
    _, last2, out2, _ = _run(w, TINY, toks, all_logits=False, tiles=tiles)
    assert np.array_equal(last2, last) and out2[0] == out[0]


def test_pack_tiles_layout(tiny):
    """msd_pack_tiles against a numpy re-tiling of every projection matrix of every layer: tile
    (n / 16, k / 32) holds rows 16 (n / 16) .. + 16 x columns 32 (k / 32) .. + 32, lane
    r + 16 q = row r, columns 8 q .. 8 q + 8.  Orders: the O and down rows in packed order (row n
    of the copy = row kernel_perm(d)[n]), so their outputs land in the residual's packed order;
    the gate/up row pairs in the down projection's input order (pair f = pair kernel_perm(d_ff)[f]);
    the O columns in natural order (column k = packed column j with kernel_perm(d)[j] = k); each
    layer ends with its two RMSNorm scales in packed order."""
    params, w = tiny
    cfg = TINY
    d, ff, L = cfg["d_model"], cfg["d_ff"], cfg["n_layers"]
    nqkv = (cfg["n_heads"] + 2 * cfg["n_kv_heads"]) * cfg["d_head"]
    got = weight_tiles(w, cfg).view(torch.int16).cpu().numpy()
    packed = w["packed_w"].view(torch.int16).cpu().numpy()
    perm = kernel_perm(d).cpu().numpy()
    fperm = kernel_perm(ff).cpu().numpy()
    pairs = np.stack([2 * fperm, 2 * fperm + 1], axis=1).reshape(-1)
    natural = np.argsort(perm)
    layer = 2 * d + nqkv * d + d * d + 2 * ff * d + d * ff
    want = []
    for l in range(L):
        base = l * layer
        off = base + 2 * d
        for N, K, rows, cols in ((nqkv, d, None, None), (d, d, perm, natural), (2 * ff, d, pairs, None),
                                 (d, ff, perm, None)):
            W = packed[off:off + N * K].reshape(N, K)
            if rows is not None:
                W = W[rows]
            if cols is not None:
                W = W[:, cols]
            want.append(W.reshape(N // 16, 16, K // 32, 4, 8).transpose(0, 2, 3, 1, 4).reshape(-1))
            off += N * K
        want.append(packed[base:base + d][perm])
        want.append(packed[base + d:base + 2 * d][perm])
    want = np.concatenate(want)
    assert got.shape == want.shape and np.array_equal(got, want)


def test_306m_prefill_128_matches_oracle(m306):
    """The prefill of a 128-token prompt on the 306M configuration."""
    params, w = m306
    toks = make_prompt(128, M306["vocab_size"], seed=3)
    la, last, out, kv = _run(w, M306, toks)
    ref, kc, vc = om.prefill_with_kv(params, M306, toks)
    print("306M prefill max |logit diff| vs f32 model.py:", float(np.max(np.abs(la - ref))))
    np.testing.assert_allclose(la, ref, atol=ATOL, rtol=RTOL)
    _check_kv(kv, M306, 128, kc, vc)
    # the reference kernel's bf16 rounding points move the logits by more than this path does
    b16 = om.prefill_with_kv(params, M306, toks, act_round="bf16")[0]
    assert np.max(np.abs(la - ref)) < 0.25 * np.max(np.abs(b16 - ref))


def test_306m_prefill_odd_row_tiles(m306):
    """A 100-token prompt: 7 row tiles of 16.  The gate/up projection then runs on workgroups of
    two row tiles and six column tiles (7 x 44 one-tile workgroups would exceed the 256 compute
    units), so one workgroup's second row tile lies past the prompt (read, never stored) and the
    last column group is short (352 column tiles = 58 x 6 + 4)."""
    params, w = m306
    toks = make_prompt(100, M306["vocab_size"], seed=5)
    la, last, out, kv = _run(w, M306, toks)
    ref, kc, vc = om.prefill_with_kv(params, M306, toks)
    print("306M 100-token prefill max |logit diff| vs f32 model.py:", float(np.max(np.abs(la - ref))))
    np.testing.assert_allclose(la, ref, atol=ATOL, rtol=RTOL)
    _check_kv(kv, M306, 100, kc, vc)
    np.testing.assert_array_equal(last, la[-1])


def _gpu_greedy_after_prefill(w, cfg, prompt, n):
    dec = Decoder(w, cfg)
    pf = Prefiller(w, cfg, max_tokens=len(prompt))
    out = pf.launch(prompt, dec.kv)
    toks = [int(out[0])]
    for i in range(n - 1):
        t, _ = dec.step(toks[-1], len(prompt) + i)
        toks.append(t)
    return toks


@pytest.mark.parametrize("cfgname", ["tiny", "m306"])
def test_prefill_then_decode_token_exact(cfgname, request):
    """The reference pipeline: prefill the prompt, then decode greedily (generate.py:70-123)."""
    params, w = request.getfixturevalue(cfgname)
    cfg = TINY if cfgname == "tiny" else M306
    prompt = make_prompt(48 if cfgname == "tiny" else 128, cfg["vocab_size"], seed=9)
    n = 48 if cfgname == "tiny" else 128
    got = _gpu_greedy_after_prefill(w, cfg, prompt, n)
    ref = om.greedy_generate(params, cfg, prompt, n, prefill="full")
    assert got == ref


def test_reference_signature_prefill_with_kv(tiny):
    params, w = tiny
    toks = make_prompt(20, TINY["vocab_size"], seed=4)
    logits, ks, vs = prefill_with_kv(params, TINY, toks)
    ref, kc, vc = om.prefill_with_kv(params, TINY, toks)
    assert tuple(logits.shape) == (20, TINY["vocab_size"])
    np.testing.assert_allclose(logits.cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    assert len(ks) == TINY["n_layers"] and tuple(ks[0].shape) == (1, 128, 64)
    np.testing.assert_allclose(ks[2][:, :20].float().cpu().numpy(), kc[2][:, :20], atol=ATOL, rtol=RTOL)


def test_prefill_rejects_bad_input(tiny):
    params, w = tiny
    pf = Prefiller(w, TINY, max_tokens=8)
    kv = new_kv_packed(TINY)
    with pytest.raises(ValueError):
        pf.launch([1, 2, 40000], kv)
    with pytest.raises(ValueError):
        pf.launch(list(range(9)), kv)
    bad = torch.tensor([1, 2, 99999], dtype=torch.int32, device="cuda")   # device ids: reported in the status
    out = pf.launch(bad, kv)
    torch.cuda.synchronize()
    assert int(out[1]) & 2


def test_306m_prefill_full_context(m306):
    """A prompt filling the whole 512-token context (projections large enough to run unsplit)."""
    params, w = m306
    toks = make_prompt(512, M306["vocab_size"], seed=8)
    _, last, out, kv = _run(w, M306, toks, all_logits=False)
    ref, kc, vc = om.prefill_with_kv(params, M306, toks)
    np.testing.assert_allclose(last, ref[-1], atol=ATOL, rtol=RTOL)
    ks, vs = unpack_kv_caches(kv, M306["n_layers"], M306["n_kv_heads"], M306["context_len"], M306["d_head"])
    for l in (0, 11, 23):
        np.testing.assert_allclose(ks[l].float().cpu().numpy(), kc[l], atol=ATOL, rtol=RTOL)
        np.testing.assert_allclose(vs[l].float().cpu().numpy(), vc[l], atol=ATOL, rtol=RTOL)


def _graph_vs_eager(w, cfg, prompts):
    """Each prompt through the same buffers, eager launches then the cached graph's replay, with
    eager torch work and synchronisations between the passes: every replay bitwise equal."""
    from transformer_amd import _lib
    L = _lib.lib()
    T = len(prompts[0])
    pf = Prefiller(w, cfg, max_tokens=T)
    kv = new_kv_packed(cfg)
    la = torch.empty((T, cfg["vocab_size"]), dtype=torch.float32, device="cuda")
    before = L.msd_set_launch_graphs(0)
    try:
        for i, toks in enumerate(prompts):
            got = {}
            for mode in (0, 1, 1):   # eager, then the graph captured by the first pass, replayed
                L.msd_set_launch_graphs(mode)
                kv.fill_(SENTINEL + i)
                la.fill_(-1.0)
                out = pf.launch(toks, kv, logits_all=la)
                torch.cuda.synchronize()
                res = (la.cpu().numpy().copy(), pf.logits.cpu().numpy().copy(), out.cpu().numpy().copy(),
                       kv.view(torch.int16).cpu().numpy().copy())
                if mode == 0:
                    got["eager"] = res
                else:
                    for a, b in zip(res, got["eager"]):
                        assert np.array_equal(a, b), f"prompt {i}: graph replay differs from the eager launches"
            assert int(got["eager"][2][1]) == 0
    finally:
        L.msd_set_launch_graphs(before)


def test_tiny_graph_replays_equal_eager_launches(tiny):
    """Three prompts of one length (one argument set: the same graph replayed over new tokens),
    then a shorter one (a second graph)."""
    _, w = tiny
    rng = np.random.default_rng(11)
    prompts = [rng.integers(0, TINY["vocab_size"], 40).tolist() for _ in range(3)]
    _graph_vs_eager(w, TINY, prompts)
    _graph_vs_eager(w, TINY, [rng.integers(0, TINY["vocab_size"], 23).tolist()])


def test_306m_graph_replays_equal_eager_launches(m306):
    """The 128-token prompt of the 306M model (the timed prefill workload), two prompts."""
    _, w = m306
    rng = np.random.default_rng(13)
    _graph_vs_eager(w, M306, [rng.integers(0, M306["vocab_size"], 128).tolist() for _ in range(2)])
