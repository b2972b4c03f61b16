"""CPU oracle for the fused decode step — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference decode path
(zahlmann/transformer): the JAX model maths in ``model.py``, the KV-cache
semantics of ``prefill_with_kv`` and of the Triton decode kernel, and the
host sampling tail of ``generate.py``.  It exists to check the HIP path.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker: the product path
(``transformer_amd``) never imports, links or calls anything in here, and
fails loudly when its HIP library is missing instead of falling back to it.

Pinning status of each function (what checks it, besides the HIP path):

* ``rms_norm``, ``precompute_rope_table``, ``apply_rope``,
  ``causal_attention``, ``forward`` — pinned against an independent library
  implementation of the same architecture (Hugging Face ``LlamaForCausalLM``
  with RMSNorm eps 1e-5, RoPE base 10000 rotate-half, GQA, SwiGLU, no bias,
  tied embeddings) on the tiny config, and against closed forms (constant
  vectors, pos 0 = identity rotation, rotation invariants, one-hot and
  uniform attention, torch ``scaled_dot_product_attention``).
* ``prefill_with_kv`` / ``decode_step`` — pinned by the invariant that a
  cached step equals the full re-forward at the last position (within the
  bf16-KV rounding), that KV rows beyond ``pos`` never influence the output,
  and that prefill KV equals the per-position projections.
* ``sample_token`` — pinned against ``numpy.random.RandomState.choice``
  (the routine ``generate.py`` calls) on the same uniform draw, plus closed
  forms (temperature 0 = argmax, penalty sign rule).
* ``bf16_round`` — pinned against torch's round-to-nearest-even cast.
* ``xent.chunked_ce_fwd`` / ``xent.fused_ce_bwd`` (the training-side fused
  cross-entropy, model.py:281-361) — pinned against torch's
  ``cross_entropy`` and its autograd gradients in float64, repeated targets
  included, and against closed forms (zero logits: loss = log V and grad_h
  = (uniform - onehot) W / N; the logit gradient's rows sum to zero, so the
  rows of grad_weight sum to zero; a dominant target logit gives loss 0);
  independent of the chunk size.
"""
