"""The allocation-free sampler entry point (msd_sample_token_noalloc) against the workspace one.

msd_sample_token_noalloc keeps its scratch in a static device array of the library (sized
for the largest vocabulary, 32768 ids) instead of a caller workspace, for callers that cannot
allocate.  Every call is compared, bit for bit (drawn token, probabilities, kept-set size and
the updated `seen` mask), with msd_sample_token on the same inputs, calls in a row with
shrinking and growing vocabularies so that leftovers of an earlier call in the shared scratch
would show.
"""
import ctypes

import numpy as np
import pytest
import torch

from transformer_amd import _lib

pytestmark = pytest.mark.gpu


def _bind():
    L = _lib.lib()
    P, I32, D = ctypes.c_void_p, ctypes.c_int32, ctypes.c_double
    L.msd_sample_token_noalloc.argtypes = [P, I32, D, D, D, P, P, P, P, P, P]
    L.msd_sample_token_noalloc.restype = I32
    return L


def _inputs(V, seed):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(V, generator=g) * 3.0).float().cuda()
    seen = (torch.rand(V, generator=g) < 0.01).to(torch.uint8).cuda()
    u = torch.tensor([float(torch.rand(1, generator=g))], dtype=torch.float64).cuda()
    return logits, seen, u


def _sample(L, noalloc, logits, seen, u, temp, top_p, pen):
    V = logits.numel()
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    probs = torch.full((V,), -1.0, dtype=torch.float32, device="cuda")
    kept = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    seen = seen.clone()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (logits.data_ptr(), V, temp, top_p, pen, seen.data_ptr(), None if temp == 0 else u.data_ptr(),
            tok.data_ptr(), probs.data_ptr(), kept.data_ptr())
    if noalloc:
        rc = L.msd_sample_token_noalloc(*args, s)
    else:
        ws = torch.empty(L.msd_sample_workspace_bytes(V), dtype=torch.uint8, device="cuda")
        rc = L.msd_sample_token(*args, ws.data_ptr(), s)
    assert rc == 0
    torch.cuda.synchronize()
    return int(tok), probs.cpu().numpy(), int(kept), seen.cpu().numpy()


CASES = [   # (vocab, temperature, top_p, repetition penalty)
    (32000, 0.7, 0.95, 1.2),
    (777, 0.7, 0.95, 1.2),      # smaller right after a larger one
    (32768, 1.0, 1.0, 1.0),     # the largest vocabulary, full-distribution draw
    (5000, 0.9, 0.5, 1.1),
    (5, 0.0, 1.0, 1.3),         # greedy
]


def test_noalloc_sampler_matches_workspace_sampler():
    L = _bind()
    for i, (V, temp, top_p, pen) in enumerate(CASES):
        logits, seen, u = _inputs(V, 100 + i)
        a = _sample(L, False, logits, seen, u, temp, top_p, pen)
        b = _sample(L, True, logits, seen, u, temp, top_p, pen)
        assert a[0] == b[0], (V, a[0], b[0])
        assert np.array_equal(a[1], b[1]), V
        assert a[2] == b[2] and np.array_equal(a[3], b[3]), V
        assert 0 <= b[0] < V


def test_noalloc_sampler_rejects_vocab_beyond_its_scratch():
    L = _bind()
    logits, seen, u = _inputs(16, 7)
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.msd_sample_token_noalloc(logits.data_ptr(), 32769, 0.7, 0.9, 1.0, seen.data_ptr(), u.data_ptr(),
                                    tok.data_ptr(), None, None, s)
    assert rc == _lib.MSD_E_CONFIG
