"""Batched decode of independent sequences over a paged KV cache (GPU).

The reference describes this path without shipping it (a PagePool with in-kernel page
tables and batched decode kernels, knowledge/program.md:214-216, 245-250); here it is built
on the matrix-core passes of ``msd_prefill_paged`` / ``msd_batch_decode_step``:

  pool = PagePool(config, n_pages)                 # [layer][K, V][kv_head][pages * 16][d_head] bf16
  bd = PagedBatchDecoder(w, config, pool, batch=8)
  first = bd.prefill(b, prompt, pages)             # one sequence's prompt into its pages
  toks, logits = bd.step(tokens, positions)        # one token of every sequence per call

Page tables are int32 (batch, max_pages); sequence b's position p lives in page
``tables[b, p // 16]``, slot ``p % 16``.  Up to 8 sequences step in ONE persistent kernel
launch (grid-wide barriers between the phases of a layer); larger batches use the
multi-kernel matrix-core pass.  Projection inputs enter the matrix cores as hi/lo bf16 parts
(f32 to about 2^-17), accumulated in f32; the current position attends with its un-rounded
K/V.
"""
import ctypes

import numpy as np
import torch

from . import _lib

PAGE = 16
STEP_MAX_BATCH = 8   # sequences one persistent launch of msd_batch_decode_step takes


class PagePool:
    """KV pages for every layer: bf16 [layer][K, V][kv_head][n_pages * 16][d_head]."""

    def __init__(self, config, n_pages, device=None):
        self.config = dict(config)
        self.n_pages = int(n_pages)
        dh = config.get("d_head", config["d_model"] // config["n_heads"])
        n = config["n_layers"] * 2 * config["n_kv_heads"] * self.n_pages * PAGE * dh
        self.data = torch.zeros(n, dtype=torch.bfloat16, device=device if device is not None else "cuda")

    def view(self):
        """(layers, 2, kv_heads, pool positions, d_head) view of the pages."""
        c = self.config
        return self.data.view(c["n_layers"], 2, c["n_kv_heads"], self.n_pages * PAGE, c["d_head"])

    def gather(self, table, n_pos):
        """Per-layer (K, V) of one sequence, (kv_heads, n_pos, d_head) each, read through ``table``."""
        t = torch.as_tensor(np.asarray(table), dtype=torch.long, device=self.data.device)
        p = torch.arange(n_pos, device=self.data.device)
        rows = t[p // PAGE] * PAGE + p % PAGE
        v = self.view()
        return [(v[l, 0][:, rows], v[l, 1][:, rows]) for l in range(self.config["n_layers"])]


class PagedBatchDecoder:
    """Batched decode of ``batch`` sequences over ``pool``.  With ``tiles`` (default) the prompt
    prefill and the multi-kernel step read the tile copy of the weights (``weight_tiles``).
    ``uncached`` places the step's workspace in the library's pool of uncached device memory
    (default: when the step runs as one persistent launch, whose barrier polls are cheaper
    there); otherwise it is an ordinary zero-filled tensor, ``self.workspace``."""

    def __init__(self, w, config, pool, batch, max_pages=None, device=None, tiles=True, uncached=None):
        from .fused_decode_nlayer import weight_tiles
        self.w = w
        self.tiles = weight_tiles(w, config) if tiles else None
        self.config = dict(config)
        self.pool = pool
        self.batch = int(batch)
        self.device = pool.data.device
        self.max_pages = int(max_pages or -(-config["context_len"] // PAGE))
        self._cfg = _lib.MsdConfig.from_dict(self.config)
        L = _lib.lib()
        nb = _lib.check(L.msd_batch_workspace_bytes(ctypes.byref(self._cfg), self.batch), "msd_batch_workspace_bytes")
        npf = _lib.check(L.msd_prefill_workspace_bytes(ctypes.byref(self._cfg), config["context_len"]),
                         "msd_prefill_workspace_bytes")
        # the step's workspace holds its barrier flags and epoch: zero-filled once, used by no
        # other call (the prompt prefill has its own)
        if uncached is None:
            from .configs import supported_paths
            uncached = self.batch <= STEP_MAX_BATCH and "batched_step" in supported_paths(self.config)
        self.workspace = None
        self._pooled = None
        if uncached:   # zero-filled on acquire, returned to the pool by close()
            ws = ctypes.c_void_p()
            dev = self.device.index if self.device.index is not None else torch.cuda.current_device()
            _lib.check(L.msd_workspace_acquire(dev, nb, ctypes.byref(ws)), "msd_workspace_acquire")
            self._pooled = ws.value
            self.workspace_ptr = ws.value
        else:
            self.workspace = torch.zeros(nb, dtype=torch.uint8, device=self.device)
            self.workspace_ptr = self.workspace.data_ptr()
        self.pf_workspace = torch.empty(npf, dtype=torch.uint8, device=self.device)
        self.tables = torch.zeros((self.batch, self.max_pages), dtype=torch.int32, device=self.device)
        self.logits = torch.empty((self.batch, config["vocab_size"]), dtype=torch.float32, device=self.device)
        self.out = torch.zeros(2 * self.batch, dtype=torch.int32, device=self.device)
        self.last = torch.empty(config["vocab_size"], dtype=torch.float32, device=self.device)
        self.pf_out = torch.zeros(2, dtype=torch.int32, device=self.device)
        # host prompts, tokens and positions are copied into these, so repeated calls keep their
        # argument set (and replay the library's cached launch graph when launch graphs are on)
        self._prompt = torch.empty(config["context_len"], dtype=torch.int32, device=self.device)
        self._step_in = torch.empty((2, self.batch), dtype=torch.int32, device=self.device)

    def _w(self):
        w = self.w
        return (w["token_emb"].data_ptr(), w["output_proj"].data_ptr(), w["packed_w"].data_ptr(),
                None if self.tiles is None else self.tiles.data_ptr(), w["lnf_s"].data_ptr(), w["rope"].data_ptr())

    def set_pages(self, b, pages):
        pages = np.asarray(pages, dtype=np.int32)
        if pages.size > self.max_pages or (pages.size and (pages.min() < 0 or pages.max() >= self.pool.n_pages)):
            raise ValueError("page table entries outside the pool or too many pages")
        row = np.zeros(self.max_pages, np.int32)
        row[:pages.size] = pages
        self.tables[b].copy_(torch.from_numpy(row))

    def prefill(self, b, prompt, pages=None, stream=None):
        """Prefill sequence b's prompt into its pages; returns the device int32[2] (argmax, status)."""
        if pages is not None:
            self.set_pages(b, pages)
        arr = np.asarray(prompt, dtype=np.int32).reshape(-1)
        if not 1 <= arr.size <= self._prompt.numel():
            raise ValueError(f"prompt length {arr.size} outside [1, {self._prompt.numel()}]")
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        toks = self._prompt[:arr.size]
        with torch.cuda.stream(s):
            toks.copy_(torch.from_numpy(arr))
        rc = _lib.lib().msd_prefill_paged(
            ctypes.byref(self._cfg), *self._w(), toks.data_ptr(), toks.numel(), self.tables[b].data_ptr(),
            self.max_pages, self.pool.data.data_ptr(), self.pool.n_pages, self.pf_workspace.data_ptr(),
            self.last.data_ptr(), self.pf_out.data_ptr(), ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_prefill_paged")
        self._keep = toks
        return self.pf_out

    def launch(self, tokens, positions, out=None, stream=None):
        """Enqueue one step of all sequences (device int32 tensors of ``batch``); returns out."""
        out = self.out if out is None else out
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        rc = _lib.lib().msd_batch_decode_step(
            ctypes.byref(self._cfg), *self._w(), tokens.data_ptr(), positions.data_ptr(), self.batch,
            self.tables.data_ptr(), self.max_pages, self.pool.data.data_ptr(), self.pool.n_pages,
            self.workspace_ptr, self.logits.data_ptr(), out.data_ptr(), ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_batch_decode_step")
        return out

    def close(self):
        """Return a pooled workspace to the library (the decoder is unusable afterwards)."""
        ptr, self._pooled = getattr(self, "_pooled", None), None
        if ptr:
            self.workspace_ptr = None
            _lib.lib().msd_workspace_release(ptr)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def step(self, tokens, positions):
        """One step from host lists; returns (next tokens (batch,) list, logits (batch, V) tensor)."""
        self._step_in.copy_(torch.from_numpy(np.stack([np.asarray(tokens, dtype=np.int32).reshape(self.batch),
                                                        np.asarray(positions, dtype=np.int32).reshape(self.batch)])))
        out = self.launch(self._step_in[0], self._step_in[1]).cpu().numpy()
        st = int(np.bitwise_or.reduce(out[1::2]))
        if st:
            raise _lib.status_error(st, "batched decode step")
        return [int(x) for x in out[0::2]], self.logits
