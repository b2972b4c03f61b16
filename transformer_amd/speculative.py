"""Speculative decoding: draft tokens verified by the target model in one pass.

The reference describes (knowledge/program.md:147-155; no code of it is in the snapshot) a
parallel verification kernel that runs K draft tokens through the full target model in one
call, a mini-prefill over the existing KV cache, with greedy acceptance.  ``Verifier`` drives
``msd_verify``; ``speculative_generate`` is the greedy loop around it:

  * the target holds the accepted sequence x_0..x_n in its cache up to x_{n-1}; x_n is the last
    accepted token, not yet fed;
  * the draft model proposes d_1..d_K autoregressively from x_n;
  * the target verifies [x_n, d_1, ..., d_K] at positions n..n+K in one call; with a_i the
    argmax of row i, d_1..d_j are accepted while d_i == a_{i-1}, and a_j is appended as the
    target's own next token.

Every emitted token is an argmax of the target (prefill for the first, verification rows for the
rest), so the output is the target's greedy generation under the matrix-core numerics whatever
the draft proposes; the draft only changes how many tokens one verification yields.
"""
import ctypes

import numpy as np
import torch

from . import _lib


class Verifier:
    """``msd_verify`` for up to ``max_tokens`` rows with the prepared target weights ``w``."""

    def __init__(self, w, config, max_tokens=8, device=None, tiles=True):
        from .fused_decode_nlayer import weight_tiles
        self.w = w
        self.tiles = weight_tiles(w, config) if tiles else None
        self.config = dict(config)
        self.device = torch.device(device) if device is not None else w["packed_w"].device
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self._cfg = _lib.MsdConfig.from_dict(self.config)
        self.max_tokens = int(max_tokens)
        nbytes = _lib.check(_lib.lib().msd_verify_workspace_bytes(ctypes.byref(self._cfg), self.max_tokens),
                            "msd_verify_workspace_bytes")
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self.logits = torch.empty((self.max_tokens, self.config["vocab_size"]), dtype=torch.float32,
                                  device=self.device)
        self.argmax = torch.zeros((self.max_tokens, 2), dtype=torch.int32, device=self.device)
        self._tok = torch.zeros(self.max_tokens, dtype=torch.int32, device=self.device)

    def launch(self, tokens, start, kv, stream=None):
        """Enqueue the verification of ``tokens`` at positions start.. into ``kv``; returns the
        (n, V) logits and the (n, 2) device int32 (argmax, status) views."""
        c = self.config
        n = len(tokens)
        if not 1 <= n <= self.max_tokens:
            raise ValueError(f"{n} tokens outside [1, {self.max_tokens}]")
        if not 1 <= start or start + n > c["context_len"]:
            raise ValueError(f"positions {start}..{start + n - 1} outside [1, {c['context_len']})")
        arr = np.asarray(tokens, dtype=np.int64)
        if arr.min() < 0 or arr.max() >= c["vocab_size"]:
            raise ValueError("token id outside the vocabulary")
        self._tok[:n].copy_(torch.from_numpy(arr.astype(np.int32)), non_blocking=False)
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        w = self.w
        rc = _lib.lib().msd_verify(
            ctypes.byref(self._cfg), w["token_emb"].data_ptr(), w["output_proj"].data_ptr(), w["packed_w"].data_ptr(),
            None if self.tiles is None else self.tiles.data_ptr(), w["lnf_s"].data_ptr(), w["rope"].data_ptr(),
            self._tok.data_ptr(), n, int(start), kv.data_ptr(),
            self.workspace.data_ptr(), self.logits.data_ptr(), self.argmax.data_ptr(), ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_verify")
        return self.logits[:n], self.argmax[:n]

    def __call__(self, tokens, start, kv):
        """Verify synchronously; returns the host list of row argmaxes."""
        _, am = self.launch(tokens, start, kv)
        a = am.cpu().numpy()
        bad = np.nonzero(a[:, 1])[0]
        if len(bad):
            raise _lib.status_error(int(a[bad[0], 1]), "verification")
        return [int(x) for x in a[:, 0]]


def speculative_generate(target_w, config, draft_w, draft_config, prompt_ids, max_tokens, k=4, device=None):
    """Greedy speculative generation of ``max_tokens`` tokens after ``prompt_ids``.

    Returns (tokens, stats) with stats = {"verifications": ..., "accepted_draft_tokens": ...}.
    The target prefills the prompt (matrix-core numerics) and verifies k draft tokens per call;
    the draft (any model over the same vocabulary) runs the fused decode step.
    """
    from .fused_decode_nlayer import new_kv_packed
    from .multi_sm_decode import Decoder
    from .prefill import Prefiller

    P = len(prompt_ids)
    if P < 1:
        raise ValueError("empty prompt")
    if P + max_tokens > config["context_len"] or P + max_tokens > draft_config["context_len"]:
        raise ValueError("prompt + tokens exceed a model's context")
    target_kv = new_kv_packed(config, device)
    pf = Prefiller(target_w, config, max_tokens=P, device=device)
    out = pf.launch(prompt_ids, target_kv)
    first = out.cpu().numpy()
    if first[1] != 0:
        raise _lib.status_error(int(first[1]), "prefill")
    draft = Decoder(draft_w, draft_config, device=device)
    dpf = Prefiller(draft_w, draft_config, max_tokens=P, device=device)
    dpf.launch(prompt_ids, draft.kv)
    ver = Verifier(target_w, config, max_tokens=k + 1, device=device)
    toks = [int(first[0])]
    n = P   # position of the last accepted token toks[-1]
    stats = {"verifications": 0, "accepted_draft_tokens": 0}
    while len(toks) < max_tokens:
        kk = min(k, config["context_len"] - 1 - n)
        if kk <= 0:
            break
        d, t = [], toks[-1]
        for i in range(kk):   # the draft feeds x_n, d_1, ..., d_{kk-1} at n..n+kk-1
            t, _ = draft.step(t, n + i)
            d.append(t)
        a = ver([toks[-1]] + d, n, target_kv)
        stats["verifications"] += 1
        j = 0
        while j < kk and d[j] == a[j]:
            j += 1
        stats["accepted_draft_tokens"] += j
        toks.extend(d[:j] + [a[j]])
        if j == kk:   # the draft has not fed d_kk yet
            draft.step(d[kk - 1], n + kk)
        n += j + 1
    return toks[:max_tokens], stats
