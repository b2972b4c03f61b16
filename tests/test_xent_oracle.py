"""The fused cross-entropy oracle (CPU): pinned against torch's cross_entropy + autograd in f64
and against closed forms, before it is used to check the HIP kernels."""
import numpy as np
import pytest
import torch

from oracle import xent as ox


def _torch_ref(h, w, t, g=1.0):
    ht = torch.tensor(h, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    loss = torch.nn.functional.cross_entropy(ht @ wt.T, torch.tensor(t, dtype=torch.long))
    gh, gw = torch.autograd.grad(loss * g, (ht, wt))
    return float(loss.detach()), gh.numpy(), gw.numpy()


@pytest.mark.parametrize("chunk", [7, 64, 1000])
def test_oracle_matches_torch_cross_entropy(chunk):
    rng = np.random.default_rng(0)
    N, V, d = 37, 203, 24
    h = rng.standard_normal((N, d)) * 3.0
    w = rng.standard_normal((V, d)) * 0.5
    t = rng.integers(0, V, N)
    t[5] = t[9] = t[11]          # repeated targets: the scatter-add must accumulate
    loss = ox.chunked_ce_fwd(h, w, t, chunk)
    gh, gw = ox.fused_ce_bwd(h, w, t, 0.7, chunk)
    rl, rgh, rgw = _torch_ref(h, w, t, 0.7)
    assert abs(loss - rl) < 1e-12 * max(1.0, abs(rl))
    np.testing.assert_allclose(gh, rgh, rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(gw, rgw, rtol=1e-10, atol=1e-13)


def test_oracle_closed_forms():
    """Zero logits (h = 0): loss = log V, grad_w = 0 except nothing (h is zero), grad_h = mean of
    (uniform softmax - onehot) rows times W; a planted dominant logit gives loss -> 0."""
    rng = np.random.default_rng(1)
    N, V, d = 5, 11, 4
    w = rng.standard_normal((V, d))
    t = rng.integers(0, V, N)
    h = np.zeros((N, d))
    assert abs(ox.chunked_ce_fwd(h, w, t, 3) - np.log(V)) < 1e-14
    gh, gw = ox.fused_ce_bwd(h, w, t, 1.0, 3)
    assert np.all(gw == 0)
    expect = (np.full((N, V), 1.0 / V) - np.eye(V)[t]) @ w / N
    np.testing.assert_allclose(gh, expect, rtol=1e-13, atol=1e-15)
    # the gradient with respect to the logits sums to zero per row: sum_v grad_w[v] . h_n terms
    h = rng.standard_normal((N, d))
    gh, gw = ox.fused_ce_bwd(h, w, t, 1.0, 4)
    # d loss / d logits = G (N x V) with zero row sums; grad_w = G^T h, so 1^T grad_w = (G 1)^T h = 0
    np.testing.assert_allclose(gw.sum(axis=0), 0.0, atol=1e-14)
    # a dominant target logit: h along the target rows of an orthonormal W
    q, _ = np.linalg.qr(rng.standard_normal((d, d)))
    w2 = q[: min(V, d)]
    t2 = np.arange(N) % w2.shape[0]
    h2 = 60.0 * w2[t2]
    assert ox.chunked_ce_fwd(h2, w2, t2, 2) < 1e-20


def test_oracle_chunk_invariance_and_f32_mode():
    rng = np.random.default_rng(2)
    N, V, d = 16, 300, 32
    h = rng.standard_normal((N, d))
    w = rng.standard_normal((V, d)) * 0.1
    t = rng.integers(0, V, N)
    a = ox.fused_ce_bwd(h, w, t, 1.0, 300)
    b = ox.fused_ce_bwd(h, w, t, 1.0, 17)
    np.testing.assert_allclose(a[0], b[0], rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(a[1], b[1], rtol=1e-12, atol=1e-15)
    f = ox.fused_ce_bwd(h, w, t, 1.0, 64, dtype=np.float32)
    assert f[0].dtype == np.float32
    np.testing.assert_allclose(f[0], a[0], rtol=1e-4, atol=1e-6)
