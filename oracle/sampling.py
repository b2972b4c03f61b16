"""numpy restatement of the host sampling tail — TEST INFRASTRUCTURE ONLY.

Follows generate.py:28-65 (``sample_token``) with three changes that make it a
function of its inputs (all stated in the reference analysis):

* the uniform draw ``u`` in [0, 1) is supplied by the caller instead of being
  drawn from numpy's hidden global RNG inside ``np.random.choice``
  (generate.py:63, :65); legacy ``RandomState.choice(a, p=p)`` maps one draw
  ``u`` to ``searchsorted(cdf / cdf[-1], u, side='right')`` with ``cdf`` the
  float64 cumulative sum of ``p`` — restated in ``_choice``;
* the descending sort of the probabilities (generate.py:55) is stable, so
  equal probabilities keep ascending token order (``np.argsort`` default
  quicksort leaves their order unspecified);
* ``exp="rounded"`` evaluates the softmax exponential as the correctly rounded
  float32 value ``float32(exp(float64(x)))``.  numpy's float32 ``exp``
  (generate.py:49, ``exp="numpy"``) is a vectorised approximation that differs
  from the correctly rounded value by 1-2 ulp on about a third of inputs
  (measured), and its result depends on the CPU's SIMD path; the GPU sampler
  computes the correctly rounded value, so parity is stated against
  ``exp="rounded"``.

Everything else follows numpy's arithmetic literally: float32 penalty,
temperature and normalisation (NEP 50 casts the Python floats to float32),
numpy's pairwise float32 ``sum``, the sequential float32 ``cumsum`` of the
sorted probabilities, and ``searchsorted(cumsum, top_p)`` comparing in float64
(the Python float ``top_p`` is not cast down).

The repetition penalty applies once to each distinct previously generated id
(generate.py:33-39): positive logits are divided by the penalty, others
multiplied.  The first generated token sees an empty history.
"""
import numpy as np


def _choice(p, u):
    """RandomState.choice's inverse-CDF step on one uniform draw (float64 cdf)."""
    cdf = np.cumsum(np.asarray(p, dtype=np.float64))
    cdf /= cdf[-1]
    return int(np.searchsorted(cdf, u, side="right"))


def apply_repetition_penalty(logits, rep_penalty, generated_ids):
    """generate.py:33-39."""
    logits = np.array(logits, dtype=np.float32)
    if rep_penalty != 1.0 and generated_ids:
        pen = np.float32(rep_penalty)
        for tid in sorted(set(int(t) for t in generated_ids)):
            if logits[tid] > 0:
                logits[tid] /= pen
            else:
                logits[tid] *= pen
    return logits


def softmax_probs(logits, temperature, exp="rounded"):
    """generate.py:43-51: float32 temperature scaling, max shift, exp, normalise."""
    logits = np.array(logits, dtype=np.float32)
    if temperature != 1.0:
        logits = logits / np.float32(temperature)
    logits -= logits.max()
    if exp == "numpy":
        probs = np.exp(logits)
    elif exp == "rounded":
        probs = np.exp(logits.astype(np.float64)).astype(np.float32)
    else:
        raise ValueError(exp)
    probs /= probs.sum()
    return probs


def nucleus(probs, top_p):
    """generate.py:54-61: (keep_idx, renormalised float32 probabilities of the kept ids)."""
    sorted_idx = np.argsort(-probs, kind="stable")
    sorted_probs = probs[sorted_idx]
    cumsum = np.cumsum(sorted_probs)
    cutoff = int(np.searchsorted(cumsum, top_p)) + 1
    keep_idx = sorted_idx[:cutoff]
    filtered = probs[keep_idx]
    filtered /= filtered.sum()
    return keep_idx, filtered


def sample_token(logits, temperature, top_p, rep_penalty, generated_ids, u, exp="rounded"):
    """generate.py:28-65 with the uniform ``u`` supplied."""
    logits = apply_repetition_penalty(logits, rep_penalty, generated_ids)
    if temperature == 0.0:
        return int(np.argmax(logits))
    probs = softmax_probs(logits, temperature, exp=exp)
    if top_p < 1.0:
        keep_idx, filtered = nucleus(probs, top_p)
        return int(keep_idx[_choice(filtered, u)])
    return _choice(probs, u)
