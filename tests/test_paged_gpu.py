"""Batched decode over a paged KV cache (GPU), checked against the oracle per sequence.

Workload of the batched-paged configuration: 8 sequences, prompt lengths drawn from
U[16, 256] (seeded), 16-token pages handed out from a shuffled pool, every sequence stepped
in the same call (M = 8).  The oracle runs each sequence alone and free-running: its own
prefill_with_kv and its own greedy decode_step chain in f32 (model.py's maths with the bf16
cache).  Every greedy token of every sequence must equal the oracle's (no teacher forcing, no
near-tie allowance), and every step's logits must agree within 2e-2 abs / 1e-2 rel.
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

_ORACLE = {}
_PARAMS = {}


def _params(name):
    if name not in _PARAMS:
        _PARAMS[name] = (make_params(TINY, seed=0) if name.startswith("tiny")
                         else make_params(M306, seed=0, resid_scaled=True))
    return _PARAMS[name]


def _oracle_generation(name, cfg, prompt, steps):
    """The oracle's own greedy chain for one sequence: (tokens (steps + 1), logits (steps, V),
    K caches, V caches).  Token 0 is the prefill's argmax; step i runs at len(prompt) + i on the
    oracle's previous token.  Cached per (config, prompt) so several tests share a chain."""
    key = (name, tuple(int(t) for t in prompt))
    if key not in _ORACLE or len(_ORACLE[key][1]) < steps:
        params = _params(name)
        rope = om.precompute_rope_table(cfg["context_len"], cfg["d_head"])
        lg0, kc, vc = om.prefill_with_kv(params, cfg, prompt)
        toks, logs = [int(np.argmax(lg0[-1]))], []
        for i in range(steps):
            lg, nt = om.decode_step(params, cfg, toks[-1], len(prompt) + i, kc, vc, rope=rope)
            logs.append(lg)
            toks.append(nt)
        _ORACLE[key] = (toks, np.stack(logs), kc, vc)
    toks, logs, kc, vc = _ORACLE[key]
    return toks[:steps + 1], logs[:steps], kc, vc     # cache rows past the chain are not compared


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


def _top2_gap(lg):
    s = np.sort(lg)
    return float(s[-1] - s[-2])


def _run_and_check(name, cfg, B, lens, steps, pool_pages, seed):
    """Free-running batched generation of B sequences; every token equal to the oracle's own
    generation and every step's logits within tolerance.  Returns (max |logit diff|, smallest
    top-2 gap the oracle's chains passed through)."""
    params = _params(name)
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
    worst, min_gap = 0.0, np.inf
    for b in range(B):
        otoks, ologs, kc, vc = _oracle_generation(name, cfg, prompts[b], steps)
        for i in range(steps):
            min_gap = min(min_gap, _top2_gap(ologs[i]))
            np.testing.assert_allclose(rec[i][b], ologs[i], atol=ATOL, rtol=RTOL, err_msg=f"sequence {b} step {i}")
            worst = max(worst, float(np.max(np.abs(rec[i][b] - ologs[i]))))
        bad = [i for i in range(steps + 1) if toks[b][i] != otoks[i]]
        assert not bad, (f"sequence {b}: first token difference at step {bad[0]} "
                         f"(gpu {toks[b][bad[0]]}, oracle {otoks[bad[0]]})")
        # the pages hold the oracle's cache rows
        n = lens[b] + steps
        for l in (0, cfg["n_layers"] - 1):
            K, V = pool.gather(tables[b], n)[l]
            np.testing.assert_allclose(K.float().cpu().numpy(), kc[l][:, :n], atol=ATOL, rtol=RTOL)
            np.testing.assert_allclose(V.float().cpu().numpy(), vc[l][:, :n], atol=ATOL, rtol=RTOL)
    return worst, min_gap


def test_tiny_batched_paged_decode():
    rng = np.random.default_rng(1)
    lens = [int(x) for x in rng.integers(16, 65, 8)]
    worst, gap = _run_and_check("tiny", TINY, 8, lens, 48, 96, seed=2)
    print("tiny batched: max |logit diff|", worst, "smallest oracle top-2 gap", gap)


def test_306m_batched_paged_decode_8x128():
    """8 sequences, prompt lengths U[16, 256], 16-token pages from a shuffled pool, 128 steps:
    all 8 x 128 greedy tokens equal to the oracle's own generations."""
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(16, 257, 8)]
    worst, gap = _run_and_check("306m", M306, 8, lens, 128, 256, seed=5)
    print("306M batched: lens", lens, "max |logit diff|", worst, "smallest oracle top-2 gap", gap)


def test_tiny_multi_kernel_step_9_sequences():
    """Nine sequences take the multi-kernel matrix-core step: all nine rows against the oracle."""
    rng = np.random.default_rng(11)
    lens = [int(x) for x in rng.integers(16, 65, 9)]
    worst, gap = _run_and_check("tiny", TINY, 9, lens, 32, 128, seed=12)
    print("tiny multi-kernel: max |logit diff|", worst, "smallest oracle top-2 gap", gap)


def test_306m_multi_kernel_step_9_sequences():
    """The config-4 prompts plus a ninth sequence through the multi-kernel step at 306M."""
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(16, 257, 8)] + [200]
    worst, gap = _run_and_check("306m", M306, 9, lens, 64, 288, seed=5)
    print("306M multi-kernel: lens", lens, "max |logit diff|", worst, "smallest oracle top-2 gap", gap)


def test_tiny_batched_context_2048():
    """A 2048-position context (beyond the persistent step's reach: the multi-kernel step takes
    it): 3 sequences with prompts of 700-1900 tokens, 8 free-running steps against the oracle."""
    cfg = dict(TINY, context_len=2048)
    worst, gap = _run_and_check("tiny2048", cfg, 3, [1900, 700, 1333], 8, 320, seed=14)
    print("tiny ctx-2048 batched: max |logit diff|", worst, "smallest oracle top-2 gap", gap)


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
    the wrap, on an ordinary zero-filled tensor as the workspace, give the same results as on a
    fresh workspace from the library's uncached pool (the decoder's default)."""
    params = make_params(TINY, seed=0)
    lens = [18, 40, 25]
    bd, pool, tables, prompts, first = _setup(TINY, params, 3, lens, 4, 64, seed=13)
    pool2 = PagePool(TINY, 64)
    pool2.data.copy_(pool.data)
    bd2 = PagedBatchDecoder(bd.w, TINY, pool2, 3, uncached=False)
    assert bd.workspace is None and bd2.workspace is not None
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
