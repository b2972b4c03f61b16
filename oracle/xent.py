"""numpy restatement of the reference's fused cross-entropy -- TEST INFRASTRUCTURE ONLY.

Reference files followed (zahlmann/transformer):
  model.py:281-302  _chunked_ce_fwd: target logits from the gathered target rows, then an online
                    logsumexp over vocabulary chunks (max_logit starts at -1e30, sum_exp at 0,
                    each chunk rescales the running sum by exp(old_max - new_max)); the loss is
                    mean(logsumexp - target_logit)
  model.py:320-361  _fused_ce_bwd: f32 maths, scale = g / N, the logsumexp recomputed by the same
                    chunk loop, then per chunk grad_h += (softmax_chunk @ w_chunk) * scale and
                    grad_weight[chunk] += (softmax_chunk^T @ h) * scale, and finally the target
                    terms grad_h -= weight[targets] * scale, grad_weight[targets] -= h * scale
                    (a scatter-add: repeated targets accumulate)

``dtype`` selects the arithmetic (float64 by default: the yardstick the GPU path is held to;
float32 is the reference's own backward precision).  Pinned against torch's independent
``cross_entropy`` and its autograd gradients in float64, and against closed forms (uniform
logits: loss = log V, gradient rows summing to zero) in ``tests/test_xent_oracle.py``.
"""
import numpy as np


def _lse(h, w, chunk, dtype):
    N = h.shape[0]
    V = w.shape[0]
    max_logit = np.full(N, -1e30, dtype)
    sum_exp = np.zeros(N, dtype)
    for start in range(0, V, chunk):
        end = min(start + chunk, V)
        cl = h @ w[start:end].T
        new_max = np.maximum(max_logit, cl.max(axis=-1))
        sum_exp = sum_exp * np.exp(max_logit - new_max) + np.exp(cl - new_max[:, None]).sum(axis=-1)
        max_logit = new_max
    return max_logit + np.log(sum_exp)


def chunked_ce_fwd(h, weight, targets, chunk_size=4096, dtype=np.float64):
    """model.py:281-302: mean over rows of logsumexp(h W^T) - (h W^T)[target]."""
    h = np.asarray(h, dtype)
    w = np.asarray(weight, dtype)
    t = np.asarray(targets, np.int64)
    target_logits = np.sum(h * w[t], axis=-1)
    return (_lse(h, w, chunk_size, dtype) - target_logits).mean()


def fused_ce_bwd(h, weight, targets, g=1.0, chunk_size=4096, dtype=np.float64):
    """model.py:320-361: (grad_h, grad_weight) of ``chunked_ce_fwd`` times g."""
    h = np.asarray(h, dtype)
    w = np.asarray(weight, dtype)
    t = np.asarray(targets, np.int64)
    N = h.shape[0]
    V = w.shape[0]
    scale = dtype(g) / dtype(N)
    lse = _lse(h, w, chunk_size, dtype)
    grad_h = np.zeros_like(h)
    grad_w = np.zeros_like(w)
    for start in range(0, V, chunk_size):
        end = min(start + chunk_size, V)
        wc = w[start:end]
        sm = np.exp(h @ wc.T - lse[:, None])
        grad_h = grad_h + (sm @ wc) * scale
        grad_w[start:end] += (sm.T @ h) * scale
    grad_h = grad_h - w[t] * scale
    np.add.at(grad_w, t, -h * scale)
    return grad_h, grad_w
