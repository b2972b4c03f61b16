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
the draft proposes; the draft only changes how many tokens one verification yields.  The draft's
proposals never leave the device: one multi-step launch writes them, the verification reads them
in place, and one read-back per cycle decides the acceptance.
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
        (n, V) logits and the (n, 2) device int32 (argmax, status) views.

        ``tokens`` is a host sequence of ids (checked here and copied to the device on the launch
        stream) or a device int32 tensor of n ids, read by the kernel where it lies (an id outside
        the vocabulary is then replaced by 0 and reported in that row's status)."""
        c = self.config
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        if isinstance(tokens, torch.Tensor) and tokens.is_cuda:
            if tokens.dtype != torch.int32 or tokens.dim() != 1 or not tokens.is_contiguous():
                raise ValueError("device tokens must be a contiguous 1-D int32 tensor")
            if tokens.device != self.device:
                raise ValueError(f"device tokens on {tokens.device}, verifier on {self.device}")
            tok, n = tokens, tokens.numel()
        else:
            arr = np.asarray(tokens, dtype=np.int64).reshape(-1)
            n = arr.size
            if n and (arr.min() < 0 or arr.max() >= c["vocab_size"]):
                raise ValueError("token id outside the vocabulary")
            tok = None
        if not 1 <= n <= self.max_tokens:
            raise ValueError(f"{n} tokens outside [1, {self.max_tokens}]")
        if not 1 <= start or start + n > c["context_len"]:
            raise ValueError(f"positions {start}..{start + n - 1} outside [1, {c['context_len']})")
        if tok is None:
            tok = self._tok[:n]
            with torch.cuda.stream(s):   # ordered before this launch and after earlier ones on s
                tok.copy_(torch.from_numpy(arr.astype(np.int32)))
        w = self.w
        rc = _lib.lib().msd_verify(
            ctypes.byref(self._cfg), w["token_emb"].data_ptr(), w["output_proj"].data_ptr(), w["packed_w"].data_ptr(),
            None if self.tiles is None else self.tiles.data_ptr(), w["lnf_s"].data_ptr(), w["rope"].data_ptr(),
            tok.data_ptr(), n, int(start), kv.data_ptr(),
            self.workspace.data_ptr(), self.logits.data_ptr(), self.argmax.data_ptr(), ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_verify")
        self._keep = tok
        return self.logits[:n], self.argmax[:n]

    def __call__(self, tokens, start, kv):
        """Verify synchronously; returns the host list of row argmaxes."""
        _, am = self.launch(tokens, start, kv)
        a = am.cpu().numpy()
        bad = np.nonzero(a[:, 1])[0]
        if len(bad):
            raise _lib.status_error(int(a[bad[0], 1]), "verification")
        return [int(x) for x in a[:, 0]]


class DraftProposer:
    """Draft model proposals for ``speculative_generate``: the fused decode step, k + 1 greedy
    steps in one launch (``Decoder.launch_steps``).  ``propose(x, n, k)`` feeds the accepted
    token x at position n and returns the device int32 (k + 2) buffer [x, d_1, ..., d_k + 1]
    together with the (k + 1, 2) device (argmax, status) array; nothing is read back.  The step
    after d_k also feeds d_k at n + k, so the draft's cache holds every row a full acceptance
    keeps (a rejected row is rewritten when the next cycle feeds that position)."""

    def __init__(self, draft_w, draft_config, device=None):
        from .multi_sm_decode import Decoder
        self.config = dict(draft_config)
        self.decoder = Decoder(draft_w, draft_config, device=device)
        self.device = self.decoder.device
        self._buf = torch.empty(draft_config["context_len"] + 1, dtype=torch.int32, device=self.device)

    def prefill(self, prompt_ids):
        """Prompt rows into the draft's cache (prefill pass; its argmax is not used)."""
        from .prefill import Prefiller
        pf = Prefiller(self.decoder.w, self.config, max_tokens=len(prompt_ids), device=self.device)
        out = pf.launch(prompt_ids, self.decoder.kv)
        self._pf = pf
        return out

    def propose(self, x, n, k):
        out = self.decoder.launch_steps(int(x), n, k + 1)
        buf = self._buf[:k + 2]
        buf[0].fill_(int(x))
        buf[1:].copy_(out[:, 0])
        return buf, out


def speculative_generate(target_w, config, draft_w, draft_config, prompt_ids, max_tokens, k=4, device=None,
                         proposer=None):
    """Greedy speculative generation of ``max_tokens`` tokens after ``prompt_ids``.

    Returns (tokens, stats) with stats = {"verifications", "accepted_draft_tokens",
    "accepted_per_verification"}.  The target prefills the prompt (matrix-core numerics) and
    verifies k draft tokens per call; the draft proposals stay on the device (``DraftProposer``:
    the draft model's fused decode step, k + 1 greedy steps per launch, any model over the same
    vocabulary; ``proposer`` replaces it).  One host read-back per cycle decides the acceptance.
    """
    from .fused_decode_nlayer import new_kv_packed
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
    prop = proposer if proposer is not None else DraftProposer(draft_w, draft_config, device=device)
    prop.prefill(prompt_ids)
    ver = Verifier(target_w, config, max_tokens=k + 1, device=device)
    toks = [int(first[0])]
    n = P   # position of the last accepted token toks[-1]
    stats = {"verifications": 0, "accepted_draft_tokens": 0, "accepted_per_verification": []}
    limit = min(config["context_len"], draft_config["context_len"]) - 1
    while len(toks) < max_tokens:
        kk = min(k, limit - n)
        if kk <= 0:
            break
        buf, dstat = prop.propose(toks[-1], n, kk)          # [x_n, d_1, ..., d_kk, (d_kk+1)] on device
        _, am = ver.launch(buf[:kk + 1], n, target_kv)    # rows n..n+kk
        a_host = am.cpu().numpy()
        d_host = dstat.cpu().numpy()
        if d_host[:, 1].any():
            raise _lib.status_error(int(d_host[np.nonzero(d_host[:, 1])[0][0], 1]), "draft steps")
        if a_host[:, 1].any():
            raise _lib.status_error(int(a_host[np.nonzero(a_host[:, 1])[0][0], 1]), "verification")
        d, a = [int(t) for t in d_host[:kk, 0]], [int(t) for t in a_host[:, 0]]
        stats["verifications"] += 1
        j = 0
        while j < kk and d[j] == a[j]:
            j += 1
        stats["accepted_draft_tokens"] += j
        stats["accepted_per_verification"].append(j)
        toks.extend(d[:j] + [a[j]])
        n += j + 1
    return toks[:max_tokens], stats
