/* C ABI of the fused output projection + cross-entropy (libmsdecode.so), training side.
 *
 * Entry points and the reference interface each replaces (zahlmann/transformer):
 *   msd_xent_forward   <- model.py:305-312 fused_cross_entropy(h, weight, targets, chunk_size)
 *                         forward = _chunked_ce_fwd (model.py:281-302): mean over rows of
 *                         logsumexp(h W^T) - (h W^T)[target], without storing the logits
 *   msd_xent_backward  <- model.py:320-361 _fused_ce_bwd (the custom_vjp backward, :364):
 *                         grad_h and grad_weight of that loss times the incoming gradient g
 *   msd_xent_workspace_bytes
 *                      <- the chunk buffers of the reference's loops (model.py:293-301, 344-353)
 *
 * Shapes: h (n_rows, d_model) bf16 row-major, weight (vocab, d_model) bf16 row-major, targets
 * int32 (n_rows).  d_model a multiple of 128, n_rows and vocab >= 1.  Every logit is a bf16 x bf16
 * dot product accumulated in f32 on the matrix cores; the softmax statistics are f32.
 * All calls are asynchronous on `stream` (a hipStream_t) and return MSD_OK or a negative
 * MSD_E_* code (msdecode.h); a target id outside [0, vocab) is replaced by 0 and reported as bit 2
 * (value 4) of *status, which the caller zero-fills and reads after the stream.
 */
#ifndef MSXENT_H
#define MSXENT_H

#include <stdint.h>

#include "msdecode.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of device workspace for both calls with this shape and chunk (the backward's probability
 * blocks are n_rows x chunk, chunk rounded up to a multiple of 256 and capped at the vocabulary;
 * the forward uses a prefix of it).  MSD_E_CONFIG for an unsupported shape. */
int64_t msd_xent_workspace_bytes(int32_t n_rows, int32_t vocab, int32_t d_model, int32_t chunk);

/* Forward.  loss: device f32 scalar, the mean over rows of lse - target logit; lse: device f32
 * (n_rows), each row's logsumexp, kept for the backward (the reference recomputes it,
 * model.py:331-340). */
int32_t msd_xent_forward(const void* h, const void* weight, const int32_t* targets, int32_t n_rows,
                         int32_t vocab, int32_t d_model, void* workspace, float* loss, float* lse,
                         int32_t* status, void* stream);

/* Backward.  lse: the forward's output for the same h, weight; grad_loss: device f32 scalar g
 * (the gradient of the loss).  grad_h (n_rows, d_model) and grad_weight (vocab, d_model) bf16
 * outputs (the reference casts to the input dtypes, model.py:361):
 *   grad_h      = (softmax(h W^T) - onehot(targets)) W * g / n_rows
 *   grad_weight = (softmax(h W^T) - onehot(targets))^T h * g / n_rows
 * computed chunk by chunk over the vocabulary (chunk columns at a time, as the reference's loop),
 * with the softmax block rounded to bf16 before its two products; grad_h is summed over the
 * chunks in f32 in vocabulary order.  Deterministic. */
int32_t msd_xent_backward(const void* h, const void* weight, const int32_t* targets, const float* lse,
                          const float* grad_loss, int32_t n_rows, int32_t vocab, int32_t d_model,
                          int32_t chunk, void* workspace, void* grad_h, void* grad_weight,
                          int32_t* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSXENT_H */
