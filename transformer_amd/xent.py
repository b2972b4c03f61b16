"""Fused output projection + cross-entropy on the matrix cores (training side).

Drop-in for the reference's memory-efficient loss (model.py:279-379):

  fused_cross_entropy(h, weight, targets, chunk_size)      # model.py:305-312 (custom_vjp)
  fused_output_and_loss(h, token_emb, targets, chunk_size)  # model.py:367-379

over torch tensors on the GPU: h (N, d) and weight (V, d) bf16 (train.py:113 runs the loss on
bf16 parameters), targets integer (N,).  The result is the mean cross-entropy as an f32 scalar
tensor with autograd: its backward gives grad_h and grad_weight in the inputs' dtype (bf16), as
the reference's backward casts them (model.py:361).

What runs (``msd_xent_forward`` / ``msd_xent_backward``, ``csrc/xent.hip``): the forward streams
the whole vocabulary through one MFMA GEMM whose epilogue keeps only each row's running
(max, sum of exponentials), so no logits are stored; the per-row logsumexp is kept for the
backward.  The backward runs chunk by chunk over the vocabulary (``chunk_size`` columns, rounded
up to a multiple of 256): the softmax block minus the one-hot targets, scaled by g / N, is
formed in bf16 and multiplied into grad_weight (final per chunk) and grad_h (summed over chunks
in f32).  Differences from the reference: the forward's logits are f32 sums of exact bf16
products (the reference's forward runs in the bf16 params dtype), and the backward's softmax
block is rounded to bf16 before its two products (the reference keeps f32; both end in bf16
gradients).
"""
import ctypes

import torch

from . import _lib

STATUS_BAD_TARGET = 4


class _Workspace:
    """Device workspace per (device, N, V, d, chunk), kept for reuse."""
    cache = {}

    @classmethod
    def get(cls, device, n, V, d, chunk):
        key = (str(device), n, V, d, chunk)
        ws = cls.cache.get(key)
        if ws is None:
            nbytes = _lib.check(_lib.lib().msd_xent_workspace_bytes(n, V, d, chunk), "msd_xent_workspace_bytes")
            if len(cls.cache) >= 4:
                cls.cache.pop(next(iter(cls.cache)))
            ws = cls.cache[key] = torch.empty(nbytes, dtype=torch.uint8, device=device)
        return ws


def _check_inputs(h, weight, targets):
    if h.dim() != 2 or weight.dim() != 2 or h.shape[1] != weight.shape[1]:
        raise ValueError(f"h (N, d) and weight (V, d) expected, got {tuple(h.shape)} and {tuple(weight.shape)}")
    if h.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("h and weight must be bfloat16")
    if not (h.is_cuda and weight.is_cuda and targets.is_cuda) or len({h.device, weight.device, targets.device}) != 1:
        raise ValueError("h, weight and targets must be on one GPU")
    if targets.shape != (h.shape[0],):
        raise ValueError(f"targets must have shape ({h.shape[0]},)")
    if h.shape[1] % 128:
        raise ValueError(f"d_model must be a multiple of 128 (got {h.shape[1]})")


class FusedCrossEntropy(torch.autograd.Function):
    """The custom_vjp pair of model.py:305-364 as a torch autograd function."""

    @staticmethod
    def forward(ctx, h, weight, targets, chunk_size, check_targets):
        _check_inputs(h, weight, targets)
        h, weight = h.contiguous(), weight.contiguous()
        tg = targets.to(torch.int32).contiguous()
        N, d = h.shape
        V = weight.shape[0]
        chunk = int(chunk_size)
        ws = _Workspace.get(h.device, N, V, d, chunk)
        loss = torch.empty((), dtype=torch.float32, device=h.device)
        lse = torch.empty(N, dtype=torch.float32, device=h.device)
        status = torch.zeros(1, dtype=torch.int32, device=h.device)
        s = torch.cuda.current_stream(h.device)
        rc = _lib.lib().msd_xent_forward(h.data_ptr(), weight.data_ptr(), tg.data_ptr(), N, V, d, ws.data_ptr(),
                                         loss.data_ptr(), lse.data_ptr(), status.data_ptr(),
                                         ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_xent_forward")
        if check_targets and int(status.item()) & STATUS_BAD_TARGET:
            raise ValueError(f"a target id outside [0, {V})")
        ctx.save_for_backward(h, weight, tg, lse)
        ctx.chunk = chunk
        return loss

    @staticmethod
    def backward(ctx, g):
        h, weight, tg, lse = ctx.saved_tensors
        N, d = h.shape
        V = weight.shape[0]
        ws = _Workspace.get(h.device, N, V, d, ctx.chunk)
        gl = g.detach().to(torch.float32).reshape(1).contiguous()
        grad_h = torch.empty_like(h)
        grad_w = torch.empty_like(weight)
        status = torch.zeros(1, dtype=torch.int32, device=h.device)
        s = torch.cuda.current_stream(h.device)
        rc = _lib.lib().msd_xent_backward(h.data_ptr(), weight.data_ptr(), tg.data_ptr(), lse.data_ptr(),
                                          gl.data_ptr(), N, V, d, ctx.chunk, ws.data_ptr(), grad_h.data_ptr(),
                                          grad_w.data_ptr(), status.data_ptr(), ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_xent_backward")
        ctx.keep = (gl, status)
        return grad_h, grad_w, None, None, None


def fused_cross_entropy(h, weight, targets, chunk_size=4096, check_targets=True):
    """model.py:305-312: mean cross-entropy of h @ weight.T against targets without storing the
    logits.  h (N, d), weight (V, d) bf16 on the GPU, targets (N,) integers in [0, V).
    ``check_targets`` reads the kernel's status back (one small synchronising copy) and raises
    ValueError for ids outside the vocabulary (they are used as 0 otherwise)."""
    return FusedCrossEntropy.apply(h, weight, targets, chunk_size, check_targets)


def fused_output_and_loss(h, token_emb, targets, chunk_size=4096, check_targets=True):
    """model.py:367-379: h (batch, seq, d), token_emb (V, d), targets (batch, seq)."""
    b, t, d = h.shape
    return fused_cross_entropy(h.reshape(b * t, d), token_emb, targets.reshape(b * t), chunk_size, check_targets)
