"""Batched decode over a paged KV cache (GPU), checked against the oracle per sequence.

Workload of the batched-paged configuration: 8 sequences, prompt lengths drawn from
U[16, 256] (seeded), 16-token pages handed out from a shuffled pool, every sequence stepped
in the same call (M = 8).  The oracle runs each sequence alone: prefill_with_kv and
decode_step in f32 (model.py's maths with the bf16 cache; the batched path feeds every projection
its input as two bf16 parts, f32 to about 2^-17), fed the GPU's own tokens (teacher forcing), so
every step's logits are compared.
"""
import numpy as np
import pytest
import torch

from oracle import model as om
from transformer_amd.configs import M306, TINY
from transformer_amd.fused_decode_nlayer import prepare_decode_weights_nlayer
from transformer_amd.paged import PAGE, PagedBatchDecoder, PagePool
from transformer_amd.synthetic import make_params, make_prompt

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _setup(cfg, params, B, lens, steps, pool_pages, seed):
    w = prepare_decode_weights_nlayer(params, cfg)
    pool = PagePool(cfg, pool_pages)
    bd = PagedBatchDecoder(w, cfg, pool, B)
    rng = np.random.default_rng(seed)
    free = list(rng.permutation(pool_pages))
    tables, prompts, first = [], [], []
    for b in range(B):
        need = -(-(lens[b] + steps) // PAGE)
        pages = [int(free.pop()) for _ in range(need)]
        tables.append(pages)
        prompts.append(make_prompt(lens[b], cfg["vocab_size"], seed=50 + b))
        out = bd.prefill(b, prompts[b], pages)
        torch.cuda.synchronize()
        assert int(out[1]) == 0
        first.append(int(out[0]))
    return bd, pool, tables, prompts, first


def _run_and_check(cfg, params, B, lens, steps, pool_pages, seed, check_every=1):
    bd, pool, tables, prompts, first = _setup(cfg, params, B, lens, steps, pool_pages, seed)
    toks = [[t] for t in first]
    rec = []
    for i in range(steps):
        cur = [toks[b][-1] for b in range(B)]
        pos = [lens[b] + i for b in range(B)]
        nxt, logits = bd.step(cur, pos)
        rec.append(logits.cpu().numpy().copy())
        for b in range(B):
            toks[b].append(nxt[b])
    # oracle per sequence, teacher-forced on the GPU's tokens
    rope = om.precompute_rope_table(cfg["context_len"], cfg["d_head"])
    worst, flips = 0.0, 0
    for b in range(B):
        ref0, kc, vc = om.prefill_with_kv(params, cfg, prompts[b])
        assert first[b] == int(np.argmax(ref0[-1])) or np.sort(ref0[-1])[-2] > ref0[-1].max() - 1e-2
        for i in range(steps):
            lg, _ = om.decode_step(params, cfg, toks[b][i], lens[b] + i, kc, vc, rope=rope)
            if i % check_every == 0 or i == steps - 1:
                np.testing.assert_allclose(rec[i][b], lg, atol=ATOL, rtol=RTOL)
                worst = max(worst, float(np.max(np.abs(rec[i][b] - lg))))
            ra = int(np.argmax(lg))
            if toks[b][i + 1] != ra:
                srt = np.sort(lg)
                assert srt[-1] - srt[-2] < 2 * ATOL, (b, i)   # only a near-tie may resolve differently
                flips += 1
        # the pages hold the oracle's cache rows
        n = lens[b] + steps
        for l in (0, cfg["n_layers"] - 1):
            K, V = pool.gather(tables[b], n)[l]
            np.testing.assert_allclose(K.float().cpu().numpy(), kc[l][:, :n], atol=ATOL, rtol=RTOL)
            np.testing.assert_allclose(V.float().cpu().numpy(), vc[l][:, :n], atol=ATOL, rtol=RTOL)
    return toks, worst, flips


def test_tiny_batched_paged_decode():
    params = make_params(TINY, seed=0)
    rng = np.random.default_rng(1)
    lens = [int(x) for x in rng.integers(16, 65, 8)]
    toks, worst, flips = _run_and_check(TINY, params, 8, lens, 48, 96, seed=2)
    print("tiny batched: max |logit diff|", worst, "near-tie flips", flips)
    assert flips <= 1


def test_306m_batched_paged_decode_8x128():
    """8 sequences, prompt lengths U[16, 256], 16-token pages from a shuffled pool, 128 steps."""
    params = make_params(M306, seed=0, resid_scaled=True)
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(16, 257, 8)]
    toks, worst, flips = _run_and_check(M306, params, 8, lens, 128, 256, seed=5, check_every=8)
    print("306M batched: lens", lens, "max |logit diff|", worst, "near-tie flips", flips)
    assert flips <= 1


def test_batched_step_matches_single_sequence_rows():
    """Row b of a batched step equals the same sequence stepped alone (batch 1)."""
    params = make_params(TINY, seed=0)
    lens = [20, 37, 16]
    bd, pool, tables, prompts, first = _setup(TINY, params, 3, lens, 4, 64, seed=3)
    nxt, logits = bd.step(first, lens)
    lb = logits.cpu().numpy().copy()
    w = bd.w
    for b in range(3):
        pool1 = PagePool(TINY, 64)
        pool1.data.copy_(pool.data)
        one = PagedBatchDecoder(w, TINY, pool1, 1)
        one.set_pages(0, tables[b])
        n1, l1 = one.step([first[b]], [lens[b]])
        np.testing.assert_allclose(l1.cpu().numpy()[0], lb[b], atol=1e-5, rtol=1e-5)
        assert n1[0] == nxt[b]


def test_bad_positions_and_pages_are_reported():
    params = make_params(TINY, seed=0)
    bd, pool, tables, prompts, first = _setup(TINY, params, 2, [16, 16], 4, 32, seed=7)
    t = torch.tensor(first, dtype=torch.int32, device="cuda")
    p = torch.tensor([16, TINY["context_len"] + 5], dtype=torch.int32, device="cuda")   # row 1 out of range
    out = bd.launch(t, p).cpu().numpy()
    assert out[3] & 4 and out[1] & 4
    bd.tables[0, 0] = 10 ** 6                      # a page outside the pool
    p = torch.tensor([16, 16], dtype=torch.int32, device="cuda")
    out = bd.launch(t, p).cpu().numpy()
    assert out[1] & 4


def test_persistent_step_matches_multi_kernel_step():
    """Up to 8 sequences step in one persistent launch; 9 take the multi-kernel pass.  The same
    8 sequences through both agree (different summation orders: 1e-4), with the same tokens."""
    params = make_params(TINY, seed=0)
    rng = np.random.default_rng(11)
    lens = [int(x) for x in rng.integers(16, 65, 9)]
    bd9, pool9, tables, prompts, first = _setup(TINY, params, 9, lens, 6, 128, seed=12)
    pool8 = PagePool(TINY, 128)
    pool8.data.copy_(pool9.data)
    bd8 = PagedBatchDecoder(bd9.w, TINY, pool8, 8)
    for b in range(8):
        bd8.set_pages(b, tables[b])
    toks9, toks8 = list(first), list(first[:8])
    for i in range(6):
        n9, l9 = bd9.step(toks9, [lens[b] + i for b in range(9)])
        n8, l8 = bd8.step(toks8, [lens[b] + i for b in range(8)])
        np.testing.assert_allclose(l8.cpu().numpy(), l9.cpu().numpy()[:8], atol=1e-4, rtol=1e-4)
        assert n8 == n9[:8]
        toks9, toks8 = n9, n8


def test_persistent_step_epoch_wrap():
    """The step's epoch (first word of its workspace) wraps from 0xFFFFFFFE to 1: steps across
    the wrap give the same results as on a fresh workspace."""
    params = make_params(TINY, seed=0)
    lens = [18, 40, 25]
    bd, pool, tables, prompts, first = _setup(TINY, params, 3, lens, 4, 64, seed=13)
    pool2 = PagePool(TINY, 64)
    pool2.data.copy_(pool.data)
    bd2 = PagedBatchDecoder(bd.w, TINY, pool2, 3)
    for b in range(3):
        bd2.set_pages(b, tables[b])
    bd2.workspace[:4].copy_(torch.tensor([0xFFFFFFFD], dtype=torch.int64).to(torch.int32).view(torch.uint8))
    ta, tb = list(first), list(first)
    for i in range(4):
        na, la = bd.step(ta, [lens[b] + i for b in range(3)])
        nb, lb = bd2.step(tb, [lens[b] + i for b in range(3)])
        assert np.array_equal(la.cpu().numpy(), lb.cpu().numpy())
        assert na == nb
        ta, tb = na, nb
    assert int(bd2.workspace[:4].view(torch.int32).item()) == 3   # 0xFFFFFFFE, 1, 2, 3 after 0xFFFFFFFD


def _paged_run(params, lens, steps):
    """9 sequences (the multi-kernel step): prefills, then `steps` steps; every output on the host."""
    bd, pool, tables, prompts, first = _setup(TINY, params, 9, lens, steps, 128, seed=12)
    toks, outs = list(first), [list(first)]
    for i in range(steps):
        nxt, lg = bd.step(toks, [lens[b] + i for b in range(9)])
        outs.append((list(nxt), lg.cpu().numpy().copy()))
        toks = nxt
    torch.cuda.synchronize()
    return outs, pool.data.view(torch.int16).cpu().numpy().copy()


def test_launch_graphs_equal_eager_paged_prefill_and_multi_kernel_step():
    """Paged prefills and the multi-kernel batched step replayed from launch graphs (the later
    steps replay the first step's graph over new tokens and positions in the same buffers):
    tokens, logits and the page pool bitwise equal to eager launches."""
    from transformer_amd import _lib
    L = _lib.lib()
    params = make_params(TINY, seed=0)
    lens = [int(x) for x in np.random.default_rng(11).integers(16, 65, 9)]
    before = L.msd_set_launch_graphs(0)
    try:
        eager = _paged_run(params, lens, 4)
        L.msd_set_launch_graphs(1)
        graphed = _paged_run(params, lens, 4)
    finally:
        L.msd_set_launch_graphs(before)
    assert eager[0][0] == graphed[0][0]
    for (ta, la), (tb, lb) in zip(eager[0][1:], graphed[0][1:]):
        assert ta == tb
        assert np.array_equal(la, lb)
    assert np.array_equal(eager[1], graphed[1])
