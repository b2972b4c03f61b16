"""Parity of the HIP decode step against the oracle (GPU)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import model as om
import json
import os

from transformer_amd.configs import M306, TINY
from transformer_amd.fused_decode_nlayer import prepare_decode_weights_nlayer, unpack_kv_caches
from transformer_amd.multi_sm_decode import Decoder, multi_sm_decode_nlayer
from transformer_amd.synthetic import make_params, make_prompt

pytestmark = pytest.mark.gpu

# logits tolerance stated by the task: 2e-2 abs / 1e-2 rel against the reference maths
ATOL, RTOL = 2e-2, 1e-2


@pytest.fixture(scope="module")
def tiny():
    params = make_params(TINY, seed=0)
    prompt = make_prompt(16, TINY["vocab_size"], seed=1)
    w = prepare_decode_weights_nlayer(params, TINY)
    return params, prompt, w


def _gpu_generate(w, cfg, prompt, n_new):
    dec = Decoder(w, cfg)
    for p, t in enumerate(prompt):
        tok, lg = dec.step(int(t), p)
    toks, logs = [tok], [lg.cpu().numpy().copy()]
    for i in range(n_new - 1):
        tok, lg = dec.step(toks[-1], len(prompt) + i)
        toks.append(tok)
        logs.append(lg.cpu().numpy().copy())
    return toks, logs, dec


def test_tiny_first_step_logits(tiny):
    params, prompt, w = tiny
    dec = Decoder(w, TINY)
    tok, lg = dec.step(int(prompt[0]), 0)
    kc, vc = om.new_kv_cache(TINY)
    ref, rtok = om.decode_step(params, TINY, int(prompt[0]), 0, kc, vc)
    got = lg.cpu().numpy()
    print("max |diff| at pos 0:", np.abs(got - ref).max())
    np.testing.assert_allclose(got, ref, atol=1e-4, rtol=1e-4)
    assert tok == rtok


def test_tiny_greedy_token_exact(tiny):
    """Config 1: 16-token prompt, 48 greedy tokens; tokens bit-exact, logits within tolerance."""
    params, prompt, w = tiny
    toks, logs, dec = _gpu_generate(w, TINY, prompt, 48)
    rtoks, rlogs = om.greedy_generate(params, TINY, prompt, 48, prefill="step", return_logits=True)
    diffs = [float(np.abs(a - b).max()) for a, b in zip(logs, rlogs)]
    print("max |logit diff| per step:", max(diffs))
    assert toks == rtoks
    for a, b in zip(logs, rlogs):
        np.testing.assert_allclose(a, b, atol=ATOL, rtol=RTOL)
    # KV cache rows 0..P+47-1 match the oracle's bf16 cache (one bf16 ulp of rounding slack)
    kc, vc = unpack_kv_caches(dec.kv, TINY["n_layers"], TINY["n_kv_heads"], TINY["context_len"], 64)
    okc, ovc = om.new_kv_cache(TINY)
    seq = list(prompt) + rtoks[:-1]
    for p, t in enumerate(seq):
        om.decode_step(params, TINY, t, p, okc, ovc)
    n = len(seq)
    for l in range(TINY["n_layers"]):
        np.testing.assert_allclose(kc[l][:, :n].float().cpu().numpy(), okc[l][:, :n], rtol=1e-2, atol=1e-3)
        np.testing.assert_allclose(vc[l][:, :n].float().cpu().numpy(), ovc[l][:, :n], rtol=1e-2, atol=1e-3)


def test_tiny_logits_close_to_full_forward(tiny):
    """Against the literal model.py forward (f32, un-rounded K/V) over the whole sequence."""
    params, prompt, w = tiny
    toks, logs, _ = _gpu_generate(w, TINY, prompt, 16)
    seq = np.array(list(prompt) + toks[:-1])
    full = om.forward(params, TINY, seq)
    for i, lg in enumerate(logs):
        np.testing.assert_allclose(lg, full[len(prompt) - 1 + i], atol=ATOL, rtol=RTOL)


def test_tiny_replay_is_bitwise_deterministic(tiny):
    params, prompt, w = tiny
    a, la, _ = _gpu_generate(w, TINY, prompt, 8)
    b, lb, _ = _gpu_generate(w, TINY, prompt, 8)
    assert a == b
    for x, y in zip(la, lb):
        assert np.array_equal(x, y)


def test_reference_signature_dropin(tiny):
    params, prompt, w = tiny
    from transformer_amd.fused_decode_nlayer import new_kv_packed
    kv = new_kv_packed(TINY)
    for p, t in enumerate(prompt):
        nt, logits, kv2 = multi_sm_decode_nlayer(w, TINY, int(t), p, kv)
        assert kv2 is kv
    kc, vc = om.new_kv_cache(TINY)
    for p, t in enumerate(prompt):
        ref, rt = om.decode_step(params, TINY, int(t), p, kc, vc)
    assert int(nt) == rt and logits.shape == (TINY["vocab_size"],)
    np.testing.assert_allclose(logits.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)


def test_device_token_chaining(tiny):
    """The input token can be the previous step's device output (no host round trip)."""
    params, prompt, w = tiny
    dec = Decoder(w, TINY)
    for p, t in enumerate(prompt):
        dec.launch(int(t), p)
    toks = []
    for i in range(8):
        out = dec.launch(dec.out[0:1], len(prompt) + i)
        toks.append(out[0:1].clone())
    got = [int(t) for t in toks]
    ref = om.greedy_generate(params, TINY, prompt, 9, prefill="step")
    assert got == ref[1:]


def test_tiny_matches_golden_fixture(tiny):
    params, prompt, w = tiny
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_greedy.json")) as f:
        g = json.load(f)
    toks, logs, _ = _gpu_generate(w, TINY, np.array(g["prompt"]), 48)
    assert toks == g["greedy_tokens_step_prefill"]
    for st, lg in zip(g["steps"], logs):
        np.testing.assert_allclose(lg[:8], st["logits_0_8"], atol=1e-4, rtol=1e-4)


def _teacher_forced(params, w, cfg, seq):
    """Feed a fixed token stream; compare every position's logits and argmax with the oracle."""
    dec = Decoder(w, cfg)
    kc, vc = om.new_kv_cache(cfg)
    rope = om.precompute_rope_table(cfg["context_len"], cfg["d_head"])
    worst, flips = 0.0, []
    for p, t in enumerate(seq):
        tok, lg = dec.step(int(t), p)
        ref, rtok = om.decode_step(params, cfg, int(t), p, kc, vc, rope=rope)
        got = lg.cpu().numpy()
        worst = max(worst, float(np.abs(got - ref).max()))
        np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL)
        if tok != rtok:
            top = np.sort(ref)[-2:]
            flips.append((p, tok, rtok, float(top[1] - top[0])))
    return worst, flips


def test_tiny_teacher_forced_all_positions(tiny):
    """Random token stream over the whole 128-token context: argmax exact at every position."""
    params, prompt, w = tiny
    seq = make_prompt(TINY["context_len"], TINY["vocab_size"], seed=5)
    worst, flips = _teacher_forced(params, w, TINY, seq)
    print("tiny teacher-forced max |logit diff|:", worst)
    assert not flips, flips


def test_bad_arguments_are_rejected_or_reported(tiny):
    """Host-side checks (pos, host token) raise before launch; an out-of-range device token is
    reported in the status word (the kernel clamps it for addressing) and the decoder recovers."""
    from transformer_amd import _lib
    params, prompt, w = tiny
    dec = Decoder(w, TINY)
    with pytest.raises(ValueError):
        dec.step(int(prompt[0]), TINY["context_len"])
    with pytest.raises(ValueError):
        dec.step(TINY["vocab_size"], 0)
    bad = torch.tensor([TINY["vocab_size"] + 5], dtype=torch.int32, device="cuda")
    with pytest.raises(_lib.MsdError) as e:
        dec.step(bad, 0)
    assert e.value.code == _lib.MSD_E_ARG
    # the status word was cleared: a valid step works and matches the oracle
    tok, lg = dec.step(int(prompt[0]), 0)
    kc, vc = om.new_kv_cache(TINY)
    ref, rtok = om.decode_step(params, TINY, int(prompt[0]), 0, kc, vc)
    np.testing.assert_allclose(lg.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)
    assert tok == rtok


def _status_word(dec, value=None):
    """Read (or write) the status word at the start of a decoder's workspace."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    torch.cuda.synchronize()
    word = ctypes.c_uint32(0 if value is None else value)
    if value is None:
        assert hip.hipMemcpy(ctypes.addressof(word), dec.workspace_ptr, 4, 2) == 0   # device to host
    else:
        assert hip.hipMemcpy(dec.workspace_ptr, ctypes.addressof(word), 4, 1) == 0   # host to device
    return word.value


def test_workspace_pool_reuses_zeroed_blocks(tiny):
    """A released workspace goes back to the pool; the next acquire of the same size gets
    the same block zero-filled again; a block in use is never handed out twice; a decoder
    whose workspace came from the pool decodes exactly."""
    from transformer_amd import _lib
    L = _lib.lib()
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    dev = torch.cuda.current_device()
    n = 4096 * 3 + 40   # a size no decoder uses, so the pool holds no other free block of it
    p1 = ctypes.c_void_p()
    assert L.msd_workspace_acquire(dev, n, ctypes.byref(p1)) == 0
    junk = (ctypes.c_uint8 * n)(*([0xA5] * n))
    assert hip.hipMemcpy(p1, ctypes.addressof(junk), n, 1) == 0
    p2 = ctypes.c_void_p()
    assert L.msd_workspace_acquire(dev, n, ctypes.byref(p2)) == 0   # p1 in use: a new block
    assert p2.value != p1.value
    assert L.msd_workspace_release(p1) == 0
    assert L.msd_workspace_release(p1) == _lib.MSD_E_ARG   # not in use any more
    p3 = ctypes.c_void_p()
    assert L.msd_workspace_acquire(dev, n, ctypes.byref(p3)) == 0
    assert p3.value == p1.value
    host = (ctypes.c_uint8 * n)()
    assert hip.hipMemcpy(ctypes.addressof(host), p3, n, 2) == 0
    assert not any(host)
    for p in (p2, p3):
        assert L.msd_workspace_release(p) == 0
    assert L.msd_workspace_acquire(dev, 0, ctypes.byref(p3)) == _lib.MSD_E_ARG
    assert L.msd_workspace_release(ctypes.c_void_p(12345)) == _lib.MSD_E_ARG
    params, prompt, w = tiny
    dec = Decoder(w, TINY)
    kc, vc = om.new_kv_cache(TINY)
    for p, t in enumerate(prompt[:3]):
        tok, lg = dec.step(int(t), p)
        ref, rtok = om.decode_step(params, TINY, int(t), p, kc, vc)
        np.testing.assert_allclose(lg.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)
        assert tok == rtok
    dec.close()
    assert dec.workspace_ptr is None


def test_reported_timeout_is_cleared_and_the_decoder_recovers(tiny):
    """A timeout bit left in the status word (as a failed step leaves it) is reported by the
    next step as MSD_E_TIMEOUT (waits that run long see it and stop; the others finish), the
    check clears it, and the decoder then produces the oracle's results again."""
    from transformer_amd import _lib
    params, prompt, w = tiny
    dec = Decoder(w, TINY)
    _status_word(dec, 1)   # status = timeout
    with pytest.raises(_lib.MsdError) as e:
        dec.step(int(prompt[0]), 0)
    assert e.value.code == _lib.MSD_E_TIMEOUT
    assert _status_word(dec) == 0   # cleared by the check
    kc, vc = om.new_kv_cache(TINY)
    for p, t in enumerate(prompt[:4]):   # restart from position 0 (the failed step wrote row 0)
        tok, lg = dec.step(int(t), p)
        ref, rtok = om.decode_step(params, TINY, int(t), p, kc, vc)
        np.testing.assert_allclose(lg.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)
        assert tok == rtok


def test_tiny_long_context_two_splits(tiny):
    """Context 1024: each head's cached positions are split over two attention workgroups, whose
    (max, sum, output) partials the row workgroups merge; every position checked."""
    params, _, _ = tiny
    cfg = dict(TINY, context_len=1024)
    w = prepare_decode_weights_nlayer(params, cfg)
    seq = make_prompt(cfg["context_len"], cfg["vocab_size"], seed=7)
    worst, flips = _teacher_forced(params, w, cfg, seq)
    print("tiny ctx-1024 teacher-forced max |logit diff|:", worst)
    assert not flips, flips


def test_tiny_long_context_four_splits(tiny):
    """Context 2048: each head's cached positions are split over four attention workgroups (the
    row workgroups' merge buffer then shares LDS with vectors that are dead during the merge);
    every position of a random stream over the whole context checked."""
    params, _, _ = tiny
    cfg = dict(TINY, context_len=2048)
    w = prepare_decode_weights_nlayer(params, cfg)
    seq = make_prompt(cfg["context_len"], cfg["vocab_size"], seed=8)
    worst, flips = _teacher_forced(params, w, cfg, seq)
    print("tiny ctx-2048 teacher-forced max |logit diff|:", worst)
    assert not flips, flips


@pytest.fixture(scope="module")
def m306():
    params = make_params(M306, seed=0, resid_scaled=True)
    w = prepare_decode_weights_nlayer(params, M306)
    return params, w


def test_306m_teacher_forced(m306):
    """306M: a random token stream over the whole 512-token context, every position checked."""
    params, w = m306
    seq = make_prompt(M306["context_len"], M306["vocab_size"], seed=6)
    worst, flips = _teacher_forced(params, w, M306, seq)
    print("306M teacher-forced max |logit diff|:", worst)
    assert not flips, flips


def test_306m_greedy_full_generation_token_exact(m306):
    """Config 2: 32-token prompt, 480 greedy tokens (prompt fed step by step, positions 32..510)."""
    params, w = m306
    prompt = make_prompt(32, M306["vocab_size"], seed=1)
    toks, logs, _ = _gpu_generate(w, M306, prompt, 480)
    rtoks, rlogs = om.greedy_generate(params, M306, prompt, 480, prefill="step", return_logits=True)
    diffs = [float(np.abs(a - b).max()) for a, b in zip(logs, rlogs)]
    print("306M greedy: max |logit diff|", max(diffs), "distinct tokens", len(set(toks)))
    assert toks == rtoks
    for a, b in zip(logs[::40], rlogs[::40]):
        np.testing.assert_allclose(a, b, atol=ATOL, rtol=RTOL)


def _poke(ptr, offset, data):
    """Write raw bytes into device memory at ptr + offset (synchronous)."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    torch.cuda.synchronize()
    buf = ctypes.create_string_buffer(bytes(data), len(data))
    assert hip.hipMemcpy(ptr + offset, ctypes.addressof(buf), len(data), 1) == 0


def test_arrival_counter_near_wrap_and_stale_key(tiny):
    """The arrival counter 16 below 2**32 and a garbage argmax key left in the workspace: every
    step still publishes exactly the oracle's token (the counter and key are reset at the start
    of each step), and the logits match."""
    params, prompt, w = tiny
    dec = Decoder(w, TINY)
    _poke(dec.workspace_ptr, 4, (2**32 - 16).to_bytes(4, "little"))
    _poke(dec.workspace_ptr, 8, (0xDEADBEEFCAFEF00D).to_bytes(8, "little"))
    kc, vc = om.new_kv_cache(TINY)
    for p, t in enumerate(prompt[:3]):
        tok, lg = dec.step(int(t), p)
        ref, rtok = om.decode_step(params, TINY, int(t), p, kc, vc)
        np.testing.assert_allclose(lg.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)
        assert tok == rtok


def test_argmax_ties_resolve_to_the_lowest_index(tiny):
    """Planted ties at the maximum (a copy of the argmax's embedding row elsewhere: tied logits
    are bitwise equal): the token is the lower id, whether the two rows belong to different
    workgroups, to neighbouring rows of one workgroup or to one wave (multi_sm_decode.py:348-357,
    np.argmax)."""
    params, prompt, _ = tiny
    kc, vc = om.new_kv_cache(TINY)
    _, a = om.decode_step(params, TINY, int(prompt[0]), 0, kc, vc)
    V = TINY["vocab_size"]
    for off in (7919, 1, 8):
        other = a - off if a - off >= 0 else a + off
        lo, hi = min(a, other), max(a, other)
        p2 = dict(params)
        emb = params["token_emb"].copy()
        emb[other] = emb[a]
        p2["token_emb"] = emb
        assert int(prompt[0]) not in (lo, hi) and hi < V
        w2 = prepare_decode_weights_nlayer(p2, TINY)
        dec = Decoder(w2, TINY)
        tok, lg = dec.step(int(prompt[0]), 0)
        got = lg.cpu().numpy()
        assert got[lo] == got[hi] == got.max(), (off, got[lo], got[hi], got.max())
        assert tok == lo, (off, tok, lo, hi)
        dec.close()


def test_dropin_reports_a_bad_device_token():
    """The reference-signature entry point returns before its step runs; a step whose device
    token is out of range is reported (MsdError) by the next call, the status is cleared, and
    later calls give the oracle's results again."""
    from transformer_amd import _lib
    from transformer_amd import multi_sm_decode as msd
    from transformer_amd.fused_decode_nlayer import new_kv_packed
    params = make_params(TINY, seed=0)
    prompt = make_prompt(4, TINY["vocab_size"], seed=1)
    w = prepare_decode_weights_nlayer(params, TINY)
    kv = new_kv_packed(TINY)
    bad = torch.tensor([TINY["vocab_size"] + 5], dtype=torch.int32, device="cuda")
    msd.multi_sm_decode_nlayer(w, TINY, bad, 0, kv)
    with pytest.raises(_lib.MsdError) as e:
        msd.multi_sm_decode_nlayer(w, TINY, int(prompt[0]), 0, kv)
    assert e.value.code == _lib.MSD_E_ARG
    msd.check_pending()   # nothing left to report
    kc, vc = om.new_kv_cache(TINY)
    for p, t in enumerate(prompt):
        nt, logits, _ = msd.multi_sm_decode_nlayer(w, TINY, int(t), p, kv)
        ref, rt = om.decode_step(params, TINY, int(t), p, kc, vc)
    msd.check_pending()
    assert int(nt) == rt
    np.testing.assert_allclose(logits.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)
    # a bad token at the last call is reported by check_pending()
    msd.multi_sm_decode_nlayer(w, TINY, bad, 4, kv)
    with pytest.raises(_lib.MsdError):
        msd.check_pending()


def test_dropin_cache_is_bounded():
    from transformer_amd import multi_sm_decode as msd
    from transformer_amd.fused_decode_nlayer import new_kv_packed
    params = make_params(TINY, seed=0)
    w = prepare_decode_weights_nlayer(params, TINY)
    for _ in range(msd.MAX_CACHED_DECODERS + 3):
        msd.multi_sm_decode_nlayer(w, TINY, 1, 0, new_kv_packed(TINY))
    msd.check_pending()
    assert len(msd._decoders) <= msd.MAX_CACHED_DECODERS


def test_grid_larger_than_the_device_is_rejected(m306):
    """Every workgroup of a step waits on others, so the grid must be resident at once: a grid of
    twice the compute units is refused with MSD_E_CONFIG before anything is launched."""
    from transformer_amd import _lib
    params, w = m306
    cus = _lib.lib().msd_default_workgroups(torch.cuda.current_device())
    dec = Decoder(w, M306, n_workgroups=2 * cus)
    with pytest.raises(_lib.MsdError) as e:
        dec.launch(1, 0)
    assert e.value.code == _lib.MSD_E_CONFIG
    dec.close()


def test_tiny_steps_in_one_launch_equal_single_steps(tiny):
    """n greedy steps in one launch (the next token fed back inside the kernel) give the oracle's
    tokens, and bit for bit the logits of one launch per step."""
    params, prompt, w = tiny
    P = len(prompt)
    single = Decoder(w, TINY)
    for p, t in enumerate(prompt):
        tok, _ = single.step(int(t), p)
    first = tok
    sl = []
    for i in range(32):
        tok, lg = single.step(tok, P + i)
        sl.append(lg.cpu().numpy().copy())
    multi = Decoder(w, TINY)
    for p, t in enumerate(prompt):
        multi.step(int(t), p)
    toks, logits = multi.generate(first, P, 32, all_logits=True)
    ml = logits.cpu().numpy()
    rtoks = om.greedy_generate(params, TINY, prompt, 33, prefill="step")
    assert toks == rtoks[1:]
    for i in range(32):
        assert np.array_equal(ml[i], sl[i]), i
    # launches of several steps chained with single steps: the tags carry on
    more = multi.generate(toks[-1], P + 32, 8)
    t2, _ = multi.step(more[-1], P + 40)
    ref = om.greedy_generate(params, TINY, prompt, 43, prefill="step")
    assert more == ref[33:41] and t2 == ref[41]


def test_tiny_steps_in_one_launch_two_splits(tiny):
    """Context 1024 (two attention workgroups per head): 24 greedy steps in one launch give the
    logits of one launch per step bit for bit.  Each step's first layer copies its older cached
    rows before the previous step's token is published and the newest row after it; the newest
    row belongs to the last split."""
    params, prompt, _ = tiny
    cfg = dict(TINY, context_len=1024)
    w = prepare_decode_weights_nlayer(params, cfg)
    P = len(prompt)
    single = Decoder(w, cfg)
    for p, t in enumerate(prompt):
        tok, _ = single.step(int(t), p)
    first = tok
    sl, st = [], []
    for i in range(24):
        tok, lg = single.step(tok, P + i)
        st.append(tok)
        sl.append(lg.cpu().numpy().copy())
    multi = Decoder(w, cfg)
    for p, t in enumerate(prompt):
        multi.step(int(t), p)
    toks, logits = multi.generate(first, P, 24, all_logits=True)
    ml = logits.cpu().numpy()
    assert toks == st
    for i in range(24):
        assert np.array_equal(ml[i], sl[i]), i


def test_306m_whole_generation_in_one_launch(m306):
    """Config 2's 479 greedy steps (positions 32..510) in a single launch, token-exact."""
    params, w = m306
    prompt = make_prompt(32, M306["vocab_size"], seed=1)
    dec = Decoder(w, M306)
    for p, t in enumerate(prompt):
        first, _ = dec.step(int(t), p)
    toks, logits = dec.generate(first, 32, 479, all_logits=True)
    rtoks, rlogs = om.greedy_generate(params, M306, prompt, 480, prefill="step", return_logits=True)
    assert [first] + toks == rtoks
    lg = logits.cpu().numpy()
    for i in range(0, 479, 60):
        np.testing.assert_allclose(lg[i], rlogs[i + 1], atol=ATOL, rtol=RTOL)


def _zeros_workspace_run(w, cfg, tokens_in, positions):
    """Steps through msd_decode_step with an ordinary torch.zeros workspace (the integration
    guide's ctypes path): one step per (token, pos), tokens from the host."""
    from transformer_amd import _lib
    from transformer_amd.fused_decode_nlayer import new_kv_packed
    L = _lib.lib()
    cfg_c = _lib.MsdConfig.from_dict(cfg)
    G = _lib.check(L.msd_default_workgroups(torch.cuda.current_device()), "msd_default_workgroups")
    ws = torch.zeros(_lib.check(L.msd_workspace_bytes(ctypes.byref(cfg_c), G), "msd_workspace_bytes"),
                     dtype=torch.uint8, device="cuda")
    kv = new_kv_packed(cfg)
    logits = torch.empty(cfg["vocab_size"], dtype=torch.float32, device="cuda")
    out = torch.zeros(2, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream()
    res = []
    for epoch, (t, p) in enumerate(zip(tokens_in, positions), start=1):
        rc = L.msd_decode_step(ctypes.byref(cfg_c), w["token_emb"].data_ptr(), w["output_proj"].data_ptr(),
                               w["packed_w"].data_ptr(), w["lnf_s"].data_ptr(), w["rope"].data_ptr(), int(t), None,
                               int(p), kv.data_ptr(), ws.data_ptr(), epoch, logits.data_ptr(), out.data_ptr(), G,
                               ctypes.c_void_p(s.cuda_stream))
        assert rc == 0
        o = out.cpu().numpy()
        assert o[1] == 0
        res.append((int(o[0]), logits.cpu().numpy().copy()))
    return res, kv


@pytest.mark.parametrize("shape", ["tiny", "306m"])
def test_ordinary_zeroed_workspace_matches_pool_workspace(shape):
    """The workspace may be any zero-filled device memory: torch.zeros memory gives the pooled
    uncached workspace's tokens, logits and cache bitwise (tiny: the prompt fed step by step,
    then greedy steps; 306M: a prompt of 8 and 12 greedy steps), and the tiny tokens equal the
    oracle's greedy generation."""
    cfg = TINY if shape == "tiny" else M306
    params = make_params(TINY, seed=0) if shape == "tiny" else make_params(M306, seed=0, resid_scaled=True)
    w = prepare_decode_weights_nlayer(params, cfg)
    P, n_new = (16, 24) if shape == "tiny" else (8, 12)
    prompt = make_prompt(P, cfg["vocab_size"], seed=1)
    dec = Decoder(w, cfg)
    toks_pool, logs_pool = [], []
    inputs, positions = [int(t) for t in prompt], list(range(P))
    for t, p in zip(inputs, positions):
        tok, lg = dec.step(t, p)
    toks_pool.append(tok)
    logs_pool.append(lg.cpu().numpy().copy())
    for i in range(n_new - 1):
        tok, lg = dec.step(toks_pool[-1], P + i)
        toks_pool.append(tok)
        logs_pool.append(lg.cpu().numpy().copy())
    # the same inputs through the ordinary workspace
    all_in = inputs + toks_pool[:-1]
    all_pos = positions + [P + i for i in range(n_new - 1)]
    res, kv = _zeros_workspace_run(w, cfg, all_in, all_pos)
    got = res[P - 1:]
    assert [t for t, _ in got] == toks_pool
    for (_, a), b in zip(got, logs_pool):
        assert np.array_equal(a, b)
    assert torch.equal(kv.view(torch.int16), dec.kv.view(torch.int16))
    if shape == "tiny":
        assert toks_pool == om.greedy_generate(params, TINY, prompt, n_new, prefill="step")


def test_306m_context_2048_prefill_then_decode(m306):
    """306M with a 2048-position context: a 1900-token prompt prefilled in one pass (last-row
    logits against the oracle), then 24 decode steps at positions 1900..1923 on a random stream
    (four context splits per head): argmax exact, logits within tolerance."""
    from transformer_amd.fused_decode_nlayer import new_kv_packed
    from transformer_amd.prefill import Prefiller
    params, _ = m306
    cfg = dict(M306, context_len=2048)
    w = prepare_decode_weights_nlayer(params, cfg)
    P = 1900
    prompt = make_prompt(P, cfg["vocab_size"], seed=31)
    dec = Decoder(w, cfg)
    pf = Prefiller(w, cfg, max_tokens=P)
    out = pf.launch(prompt, dec.kv).cpu().numpy()
    assert out[1] == 0
    ref_all, kc, vc = om.prefill_with_kv(params, cfg, prompt)
    assert out[0] == int(np.argmax(ref_all[-1]))
    np.testing.assert_allclose(pf.logits.cpu().numpy(), ref_all[-1], atol=ATOL, rtol=RTOL)
    rope = om.precompute_rope_table(cfg["context_len"], cfg["d_head"])
    seq = make_prompt(24, cfg["vocab_size"], seed=32)
    worst = 0.0
    for i, t in enumerate(seq):
        tok, lg = dec.step(int(t), P + i)
        ref, rtok = om.decode_step(params, cfg, int(t), P + i, kc, vc, rope=rope)
        got = lg.cpu().numpy()
        worst = max(worst, float(np.abs(got - ref).max()))
        np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL)
        assert tok == rtok, (P + i, tok, rtok)
    print("306M ctx-2048 decode max |logit diff|:", worst)
