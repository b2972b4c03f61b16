"""Multi-token prefill on the GPU (drop-in for the reference's model.prefill_with_kv).

``prefill_with_kv(params, config, x)`` keeps the reference signature and returns
``(logits (T, V), k_caches, v_caches)`` (model.py:194-231); ``Prefiller`` is the form the
generation loop uses: it fills a packed KV buffer in place and returns the last position's
logits and argmax without leaving the device.

The projections run on the matrix cores (``msd_prefill``) with every input activation split
into two bf16 parts (hi + lo, f32 to about 2^-17) against the bf16 weights, accumulated in f32,
so the numerics are those of the f32 reference maths (model.py:194-231).
"""
import ctypes

import numpy as np
import torch

from . import _lib


class Prefiller:
    """Prefill of prompts up to ``max_tokens`` long with the prepared decode weights ``w``.
    With ``tiles`` (default) the projections read the tile copy of the weights
    (``weight_tiles``, one more copy of ``packed_w`` on the device); without, the packed rows."""

    def __init__(self, w, config, max_tokens=None, device=None, tiles=True):
        from .fused_decode_nlayer import weight_tiles
        self.w = w
        self.tiles = weight_tiles(w, config) if tiles else None
        self.config = dict(config)
        self.device = torch.device(device) if device is not None else w["packed_w"].device
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self._cfg = _lib.MsdConfig.from_dict(self.config)
        self.max_tokens = int(max_tokens or self.config["context_len"])
        nbytes = _lib.check(_lib.lib().msd_prefill_workspace_bytes(ctypes.byref(self._cfg), self.max_tokens),
                            "msd_prefill_workspace_bytes")
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self.logits = torch.empty(self.config["vocab_size"], dtype=torch.float32, device=self.device)
        self.out = torch.zeros(2, dtype=torch.int32, device=self.device)   # [argmax, status]
        # host prompts are copied here, so repeated passes keep their argument set (and replay
        # the library's cached launch graph when launch graphs are on)
        self._tok = torch.empty(self.max_tokens, dtype=torch.int32, device=self.device)

    def launch(self, tokens, kv, logits_all=None, out=None, stream=None):
        """Enqueue the prefill of ``tokens`` (host sequence or device int32 tensor) into ``kv``.

        Returns the device int32[2] (argmax of the last position, status); the last
        position's logits are in ``self.logits``.
        """
        c = self.config
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        if isinstance(tokens, torch.Tensor) and tokens.is_cuda:
            tok = tokens.to(torch.int32).contiguous()
            T = tok.numel()
        else:
            arr = np.asarray(tokens, dtype=np.int64).reshape(-1)
            if arr.size and (arr.min() < 0 or arr.max() >= c["vocab_size"]):
                raise ValueError("token id outside the vocabulary")
            T = arr.size
        if not 1 <= T <= self.max_tokens:
            raise ValueError(f"prompt length {T} outside [1, {self.max_tokens}]")
        if not (isinstance(tokens, torch.Tensor) and tokens.is_cuda):
            tok = self._tok[:T]
            with torch.cuda.stream(s):
                tok.copy_(torch.from_numpy(arr.astype(np.int32)))
        if logits_all is not None and (logits_all.dtype != torch.float32 or logits_all.numel() != T * c["vocab_size"]):
            raise ValueError("logits_all must be a (T, V) f32 tensor")
        out = self.out if out is None else out
        w = self.w
        rc = _lib.lib().msd_prefill(
            ctypes.byref(self._cfg), w["token_emb"].data_ptr(), w["output_proj"].data_ptr(),
            w["packed_w"].data_ptr(), None if self.tiles is None else self.tiles.data_ptr(), w["lnf_s"].data_ptr(),
            w["rope"].data_ptr(), tok.data_ptr(), T,
            kv.data_ptr(), self.workspace.data_ptr(), self.logits.data_ptr(),
            None if logits_all is None else logits_all.data_ptr(), out.data_ptr(), ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_prefill")
        self._keep = tok   # alive until the stream has used it
        return out


def prefill_with_kv(params, config, x, device="cuda"):
    """Reference signature (model.py:194): (logits (T, V) f32, k_caches, v_caches).

    ``params`` is the reference parameter dict (or an already prepared decode weight dict);
    caches are per-layer (n_kv_heads, context_len, d_head) bf16 views of one packed buffer,
    rows >= T zero.
    """
    from .fused_decode_nlayer import new_kv_packed, prepare_decode_weights_nlayer, unpack_kv_caches
    w = params if "packed_w" in params else prepare_decode_weights_nlayer(params, config, device=device)
    toks = np.asarray(x).reshape(-1)
    pf = Prefiller(w, config, max_tokens=len(toks))
    kv = new_kv_packed(config, pf.device)
    logits = torch.empty((len(toks), config["vocab_size"]), dtype=torch.float32, device=pf.device)
    out = pf.launch(toks, kv, logits_all=logits)
    if int(out[1]) != 0:
        raise _lib.MsdError(_lib.MSD_E_ARG, "prefill (token id out of range)")
    ks, vs = unpack_kv_caches(kv, config["n_layers"], config["n_kv_heads"], config["context_len"],
                              config.get("d_head", config["d_model"] // config["n_heads"]))
    return logits, ks, vs
