"""Fused whole-model decode step (drop-in for the reference's multi_sm_decode module).

``multi_sm_decode_nlayer(w, config, token_id, pos, kv_packed)`` keeps the reference
signature and return triple (kernels/multi_sm_decode.py:369-432); ``Decoder`` is the
stateful form with ``step(token, pos) -> (next_token, logits)`` that owns the workspace.

Differences from the reference call, by design:
  * the KV cache is updated in place at ``pos`` (the returned kv is the same tensor); a
    step writes ``pos`` before reading it and never reads rows > pos, so replaying from
    the same start position (profile_kernels.py:54-63) gives the same results;
  * the workspace is taken once per decoder from the library's pool of zero-filled
    uncached device memory (msd_workspace_acquire: the polled exchange words bypass the L2
    caches) and never re-zeroed while the decoder lives: exchange words are tagged with a
    per-call epoch instead (multi_sm_decode.py:400 zero-fills per call).
  * a step reports failures in its status output; ``Decoder.step`` raises on them at once,
    ``multi_sm_decode_nlayer`` (which returns before the step has run, as the reference's
    asynchronous dispatch does) raises them on its next call or from ``check_pending()``.
"""
import collections
import ctypes

import numpy as np
import torch

from . import _lib


class Decoder:
    """One decode stream: weights dict, packed KV buffer, workspace and output buffers."""

    def __init__(self, w, config, kv_packed=None, device=None, n_workgroups=None):
        from .fused_decode_nlayer import new_kv_packed
        self.w = w
        self.config = dict(config)
        self.device = torch.device(device) if device is not None else w["packed_w"].device
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self._cfg = _lib.MsdConfig.from_dict(self.config)
        L = _lib.lib()
        if n_workgroups is None:
            idx = self.device.index if self.device.index is not None else torch.cuda.current_device()
            n_workgroups = _lib.check(L.msd_default_workgroups(idx), "msd_default_workgroups")
        self.n_workgroups = int(n_workgroups)
        nbytes = _lib.check(L.msd_workspace_bytes(ctypes.byref(self._cfg), self.n_workgroups),
                            "msd_workspace_bytes")
        # zero-filled uncached device memory from the library's pool (never freed; returned to
        # the pool when this decoder goes away)
        ws = ctypes.c_void_p()
        _lib.check(L.msd_workspace_acquire(self._device_index(), nbytes, ctypes.byref(ws)),
                   "msd_workspace_acquire")
        self.workspace_ptr = ws.value
        self.workspace_bytes = nbytes
        self.kv = kv_packed if kv_packed is not None else new_kv_packed(self.config, self.device)
        self.logits = torch.empty(self.config["vocab_size"], dtype=torch.float32, device=self.device)
        self.out = torch.zeros(2, dtype=torch.int32, device=self.device)   # [token, status]
        self._host = torch.zeros(2, dtype=torch.int32).pin_memory()
        self.epoch = 0
        self._check_kv(self.kv)

    def _device_index(self):
        return self.device.index if self.device.index is not None else torch.cuda.current_device()

    def close(self):
        """Return the workspace to the library's pool (the decoder is unusable afterwards)."""
        ptr, self.workspace_ptr = getattr(self, "workspace_ptr", None), None
        if ptr:
            _lib.lib().msd_workspace_release(ptr)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check_kv(self, kv):
        c = self.config
        n = c["n_layers"] * 2 * c["n_kv_heads"] * c["context_len"] * c.get("d_head", c["d_model"] // c["n_heads"])
        if kv.dtype != torch.bfloat16 or kv.numel() != n or not kv.is_contiguous() or kv.device != self.device:
            raise ValueError("kv_packed must be a contiguous bf16 tensor of "
                             f"{n} elements on {self.device}")

    def launch(self, token, pos, stream=None, out=None):
        """Enqueue one step; ``token`` is an int or a device int32 tensor (read on device).

        Returns the device int32[2] output (token, status) without synchronising.
        """
        c = self.config
        pos = int(pos)
        if not 0 <= pos < c["context_len"]:
            raise ValueError(f"pos {pos} outside [0, {c['context_len']})")
        tok_dev = None
        tok = 0
        if isinstance(token, torch.Tensor) and token.is_cuda:
            if token.dtype != torch.int32:
                raise ValueError("device token must be int32")
            tok_dev = token.data_ptr()
        else:
            tok = int(token)
            if not 0 <= tok < c["vocab_size"]:
                raise ValueError(f"token {tok} outside [0, {c['vocab_size']})")
        out = self.out if out is None else out
        epoch = self._next_epochs(1)
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        w = self.w
        rc = _lib.lib().msd_decode_step(
            ctypes.byref(self._cfg), w["token_emb"].data_ptr(), w["output_proj"].data_ptr(),
            w["packed_w"].data_ptr(),
            w["lnf_s"].data_ptr(), w["rope"].data_ptr(), tok, tok_dev, pos, self.kv.data_ptr(),
            self.workspace_ptr, epoch, self.logits.data_ptr(), out.data_ptr(),
            self.n_workgroups, ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_decode_step")
        return out

    def _next_epochs(self, n):
        """Tags for n steps: the next n values after the last one used, restarting at 1 when they
        would pass 0xFFFFFFFE (every step rewrites every exchange word, so old tags never linger)."""
        if self.epoch + n > 0xFFFFFFFE:
            self.epoch = 0
        e = self.epoch + 1
        self.epoch += n
        return e

    def launch_steps(self, token, pos, n_steps, all_logits=False, out=None, logits=None, stream=None):
        """Enqueue ``n_steps`` greedy steps in one launch (step s at pos + s on step s - 1's argmax).

        Returns the device int32 (n_steps, 2) array of (argmax, status) per step; the logits of
        every step land in ``logits`` (n_steps, V) with ``all_logits``, else the last step's in
        ``self.logits``.
        """
        c = self.config
        pos, n_steps = int(pos), int(n_steps)
        if n_steps < 1 or not 0 <= pos or pos + n_steps > c["context_len"]:
            raise ValueError(f"positions {pos}..{pos + n_steps - 1} outside [0, {c['context_len']})")
        tok_dev, tok = None, 0
        if isinstance(token, torch.Tensor) and token.is_cuda:
            if token.dtype != torch.int32:
                raise ValueError("device token must be int32")
            tok_dev = token.data_ptr()
        else:
            tok = int(token)
            if not 0 <= tok < c["vocab_size"]:
                raise ValueError(f"token {tok} outside [0, {c['vocab_size']})")
        if out is None:
            out = torch.empty((n_steps, 2), dtype=torch.int32, device=self.device)
        if all_logits:
            if logits is None:
                logits = torch.empty((n_steps, c["vocab_size"]), dtype=torch.float32, device=self.device)
        else:
            logits = self.logits
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        w = self.w
        rc = _lib.lib().msd_decode_steps(
            ctypes.byref(self._cfg), w["token_emb"].data_ptr(), w["output_proj"].data_ptr(),
            w["packed_w"].data_ptr(), w["lnf_s"].data_ptr(), w["rope"].data_ptr(), tok, tok_dev, pos, n_steps,
            self.kv.data_ptr(), self.workspace_ptr, self._next_epochs(n_steps), logits.data_ptr(),
            1 if all_logits else 0, out.data_ptr(), self.n_workgroups, ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_decode_steps")
        self._keep = (out, logits)
        return out

    def generate(self, token, pos, n_steps, all_logits=False):
        """``n_steps`` greedy tokens after ``token`` at ``pos`` in one launch; returns the host list
        of tokens (and the (n_steps, V) logits when ``all_logits``)."""
        out = self.launch_steps(token, pos, n_steps, all_logits=all_logits)
        logits = self._keep[1]
        host = out.cpu().numpy()
        bad = np.nonzero(host[:, 1])[0]
        if len(bad):
            self.raise_for_status(int(host[bad[0], 1]), f"decode step at pos {int(pos) + int(bad[0])}")
        toks = [int(t) for t in host[:, 0]]
        return (toks, logits) if all_logits else toks

    def raise_for_status(self, status, what):
        """Raise the MsdError for a non-zero step status, after clearing the workspace's
        status word (a timeout bit left set would cut every later step's waits short)."""
        if int(status) == 0:
            return
        _lib.lib().msd_check_status(self.workspace_ptr,
                                    ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream))
        raise _lib.status_error(status, what)

    def step(self, token, pos):
        """Run one step and return (next_token: int, logits: (V,) f32 device tensor).

        The logits tensor is this decoder's buffer and is overwritten by the next step.
        """
        out = self.launch(token, pos)
        self._host.copy_(out, non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        tok, status = int(self._host[0]), int(self._host[1])
        self.raise_for_status(status, f"decode step at pos {pos}")
        return tok, self.logits


# Decoders of the reference-signature entry point, keyed by (weights dict, KV buffer); the
# least recently used one is dropped (its workspace returns to the pool) beyond this many.
MAX_CACHED_DECODERS = 4
_decoders = collections.OrderedDict()


class _Pending:
    """Status of a launched step, copied to pinned host memory behind an event."""

    def __init__(self, dec, out, pos):
        self.dec, self.pos = dec, pos
        self.host = torch.empty(1, dtype=torch.int32).pin_memory()
        self.host.copy_(out[1:2], non_blocking=True)
        self.event = torch.cuda.Event()
        self.event.record(torch.cuda.current_stream(dec.device))

    def check(self):
        self.event.synchronize()
        self.dec.raise_for_status(int(self.host[0]), f"decode step at pos {self.pos}")


_pending = []


def check_pending():
    """Wait for the steps ``multi_sm_decode_nlayer`` launched and not yet checked, and raise
    the MsdError of the first one whose status is set (the later ones are dropped)."""
    global _pending
    todo, _pending = _pending, []
    for p in todo:
        p.check()


def multi_sm_decode_nlayer(w, config, token_id, pos, kv_packed, kv_splits=1):
    """Reference signature (multi_sm_decode.py:369): returns (next_token, logits[:V] f32, kv).

    next_token is a device int32 scalar tensor, logits a fresh (V,) f32 tensor, kv the
    same ``kv_packed`` tensor updated in place.  ``kv_splits`` is accepted for signature
    compatibility; the kernel chooses its own split of the attention work.

    The step runs asynchronously.  Its status is checked when the next call has been
    enqueued (or by ``check_pending()``): a failed step (a cross-workgroup wait that ran out,
    an out-of-range device token) raises ``MsdError`` there.
    """
    key = (id(w), kv_packed.data_ptr())
    dec = _decoders.pop(key, None)
    if dec is None or dec.w is not w or dec.kv is not kv_packed:
        if dec is not None:
            dec.close()
        dec = Decoder(w, config, kv_packed)
    _decoders[key] = dec
    while len(_decoders) > MAX_CACHED_DECODERS:
        _, old = _decoders.popitem(last=False)
        check_pending()
        old.close()
    out = torch.empty(2, dtype=torch.int32, device=dec.device)
    dec.launch(token_id, pos, out=out)
    earlier = _pending[:]
    _pending.append(_Pending(dec, out, int(pos)))
    for p in earlier:   # the previous steps ran before this one: check them now
        _pending.remove(p)
        try:
            p.check()
        except _lib.MsdError:
            _pending.clear()   # later steps ran with the failed state
            raise
    return out[0].clone(), dec.logits.clone(), kv_packed
