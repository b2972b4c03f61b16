"""Token generation on the GPU (drop-in for the reference's generate.py loop).

  sample_token(logits, temperature, top_p, rep_penalty, generated_ids)   generate.py:28-65
  stream_tokens(params, config, prompt_ids, max_tokens, temperature,
                top_p, rep_penalty, seed)                                 generate.py:92-123
  generate_tokens(...)                                                    generate.py:126-130
  main()  (python -m transformer_amd.generate)                           generate.py:133-236

Sampling runs on the device (``msd_sample_token``): the logits never leave the GPU and the
drawn token feeds the next decode step on the device.  The uniform draw of each sampled
token comes from numpy's global RandomState, one ``random_sample()`` per sampled token, which
is the draw ``np.random.choice`` makes in the reference (generate.py:63,65), so a seeded run
consumes the same uniform sequence.

The prompt goes through the matrix-core prefill (``Prefiller``, model.py:194-231 as called
by generate.py:75-82): it writes the KV rows 0..P-1 and its last-position logits are the
reference's ``first_logits``.  The reference pads the prompt to the context length first
(generate.py:75); rows >= P are never read before a decode step writes them, so only the P
prompt tokens are processed.  ``prefill="step"`` feeds the prompt through the decode step
one token at a time instead.
"""
import ctypes

import numpy as np
import torch

from . import _lib


class Sampler:
    """Device state of one sequence's sampler: generated-id flags and the workspace."""

    def __init__(self, vocab, device=None):
        self.vocab = int(vocab)
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        L = _lib.lib()
        nbytes = _lib.check(L.msd_sample_workspace_bytes(self.vocab), "msd_sample_workspace_bytes")
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self.seen = torch.zeros(self.vocab, dtype=torch.uint8, device=self.device)
        self.token = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.kept = torch.zeros(1, dtype=torch.int32, device=self.device)

    def reset(self, generated_ids=()):
        """Forget the history; mark ``generated_ids`` as generated."""
        self.seen.zero_()
        ids = sorted(set(int(t) for t in generated_ids))
        if ids:
            if ids[0] < 0 or ids[-1] >= self.vocab:
                raise ValueError("generated id outside the vocabulary")
            self.seen[torch.tensor(ids, dtype=torch.long, device=self.device)] = 1

    def launch(self, logits, temperature, top_p, rep_penalty, u=None, out=None, probs_out=None,
               kept_out=None, stream=None):
        """Enqueue one draw; returns the device int32 token slot (``out`` or own buffer).

        ``u`` is a device float64 tensor whose first element is the uniform (unused when
        temperature == 0).  ``logits`` is a device f32 tensor of ``vocab`` entries.
        """
        if logits.dtype != torch.float32 or logits.numel() != self.vocab or not logits.is_contiguous():
            raise ValueError(f"logits must be a contiguous f32 device tensor of {self.vocab} entries")
        if temperature != 0.0 and (u is None or u.dtype != torch.float64):
            raise ValueError("a float64 device uniform is required when temperature != 0")
        out = self.token if out is None else out
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        rc = _lib.lib().msd_sample_token(
            logits.data_ptr(), self.vocab, float(temperature), float(top_p), float(rep_penalty),
            self.seen.data_ptr(), None if u is None else u.data_ptr(), out.data_ptr(),
            None if probs_out is None else probs_out.data_ptr(),
            None if kept_out is None else kept_out.data_ptr(),
            self.workspace.data_ptr(), ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "msd_sample_token")
        return out


_samplers = {}


def _sampler_for(vocab, device):
    key = (int(vocab), str(device))
    if key not in _samplers:
        _samplers[key] = Sampler(vocab, device)
    return _samplers[key]


def sample_token(logits, temperature, top_p, rep_penalty, generated_ids, u=None):
    """Reference signature (generate.py:28): one token from ``logits`` on the GPU.

    ``logits`` is a (V,) tensor or array; ``generated_ids`` the ids generated so far.  When
    temperature != 0 the draw is ``u`` if given, else numpy's global ``random_sample()``.
    """
    if isinstance(logits, torch.Tensor) and logits.is_cuda:
        lg = logits.detach().to(torch.float32).contiguous()
    else:
        lg = torch.as_tensor(np.asarray(logits, dtype=np.float32)).cuda()
    smp = _sampler_for(lg.numel(), lg.device)
    smp.reset(generated_ids)
    ud = None
    if temperature != 0.0:
        if u is None:
            u = np.random.random_sample()
        ud = torch.tensor([float(u)], dtype=torch.float64, device=lg.device)
    tok = smp.launch(lg, temperature, top_p, rep_penalty, u=ud)
    return int(tok.item())


def _prepare(params, config, device):
    from .fused_decode_nlayer import prepare_decode_weights_nlayer
    from .multi_sm_decode import Decoder
    w = prepare_decode_weights_nlayer(params, config, device=device)
    return Decoder(w, config, device=device)


def _check_status(dec, st, what):
    """Raise for the first non-zero status in ``st`` (clearing the decoder's status word)."""
    bad = np.nonzero(st)[0]
    if len(bad):
        dec.raise_for_status(int(st[bad[0]]), what)


def run_generation(dec, prompt_ids, max_tokens, temperature=0.0, top_p=1.0, rep_penalty=1.0,
                   uniforms=None, sampler=None, record_logits=None, sync_each=False, prefill="kernel",
                   prefiller=None):
    """Generate ``max_tokens`` tokens after ``prompt_ids`` with decoder ``dec``.

    Yields token ids.  With ``sync_each`` every token is read back as soon as it is drawn
    (streaming); otherwise all steps are enqueued back to back, each step reading the previous
    token on the device, and the tokens are read once at the end.  ``uniforms`` holds one
    draw per token (needed unless temperature == 0).  ``record_logits``, if given, is a
    (max_tokens, V) f32 device tensor that receives the logits each token was drawn from.
    """
    c = dec.config
    P = len(prompt_ids)
    if P < 1:
        raise ValueError("empty prompt")
    if max_tokens < 1:
        return
    if P + max_tokens - 1 > c["context_len"]:
        raise ValueError(f"prompt {P} + {max_tokens} tokens exceeds context {c['context_len']}")
    greedy = temperature == 0.0 and rep_penalty == 1.0
    dev = dec.device
    if not greedy:
        if sampler is None:
            sampler = Sampler(c["vocab_size"], dev)
        sampler.reset()
        if temperature != 0.0:
            if uniforms is None or len(uniforms) < max_tokens:
                raise ValueError("one uniform per token is required when temperature != 0")
            u_dev = torch.as_tensor(np.asarray(uniforms[:max_tokens], dtype=np.float64)).to(dev)
    dec_out = torch.zeros((max_tokens, 2), dtype=torch.int32, device=dev)   # decode (argmax, status)
    toks = dec_out[:, 0] if greedy else torch.zeros(max_tokens, dtype=torch.int32, device=dev)
    host = torch.zeros(2, dtype=torch.int32).pin_memory()
    pre = torch.zeros(2, dtype=torch.int32, device=dev)
    if prefill == "kernel":
        from .prefill import Prefiller
        pf = prefiller if prefiller is not None else Prefiller(dec.w, c, max_tokens=P, device=dev)
    elif prefill == "step":
        for p, t in enumerate(prompt_ids[:-1]):
            dec.launch(int(t), p, out=pre)
    else:
        raise ValueError(prefill)
    for i in range(max_tokens):
        if i == 0 and prefill == "kernel":
            pf.launch(prompt_ids, dec.kv, out=dec_out[0])
            logits = pf.logits
        elif i == 0:
            dec.launch(int(prompt_ids[-1]), P - 1, out=dec_out[0])
            logits = dec.logits
        else:
            dec.launch(toks[i - 1:i], P - 1 + i, out=dec_out[i])
            logits = dec.logits
        if record_logits is not None:
            record_logits[i].copy_(logits)
        if not greedy:
            sampler.launch(logits, temperature, top_p, rep_penalty,
                           u=None if temperature == 0.0 else u_dev[i:i + 1], out=toks[i:i + 1])
        if sync_each:
            host[0:1].copy_(toks[i:i + 1], non_blocking=True)
            host[1:2].copy_(dec_out[i, 1:2], non_blocking=True)
            torch.cuda.current_stream(dev).synchronize()
            _check_status(dec, np.array([int(host[1])]), f"decode step at pos {P - 1 + i}")
            yield int(host[0])
    if not sync_each:
        out = torch.stack([toks, dec_out[:, 1]], 1).cpu().numpy()
        st = np.concatenate([out[:, 1], pre.cpu().numpy()[1:]])
        _check_status(dec, st, "decode step")
        for t in out[:, 0]:
            yield int(t)


def _uniforms(n, temperature, seed):
    if seed is not None:
        np.random.seed(seed)
    if temperature == 0.0:
        return None
    return np.random.random_sample(n)


def stream_tokens(params, config, prompt_ids, max_tokens=128, temperature=0.0, top_p=1.0,
                  rep_penalty=1.0, seed=None, device="cuda"):
    """Reference signature (generate.py:68): yield token ids one at a time."""
    dec = _prepare(params, config, device)
    us = _uniforms(max_tokens, temperature, seed)
    yield from run_generation(dec, [int(t) for t in prompt_ids], max_tokens, temperature, top_p,
                              rep_penalty, uniforms=us, sync_each=True)


def generate_tokens(params, config, prompt_ids, n_tokens=128, temperature=0.0, top_p=1.0,
                    rep_penalty=1.0, seed=None, device="cuda"):
    """Reference signature (generate.py:126): all tokens at once (one read-back at the end)."""
    dec = _prepare(params, config, device)
    us = _uniforms(n_tokens, temperature, seed)
    return list(run_generation(dec, [int(t) for t in prompt_ids], n_tokens, temperature, top_p,
                               rep_penalty, uniforms=us, sync_each=False))


def main(argv=None):
    """Command line text generation from a trained checkpoint (generate.py:133-236).

    ``python -m transformer_amd.generate --prompt TEXT --weights weights.pkl`` with the
    reference's options (--max-tokens, --no-stream, --temp, --top-p, --rep-penalty,
    --seed).  Relative ``--weights`` paths are taken from the working directory; the
    tokenizer comes from ``--tokenizer`` (a data directory holding ``bpe_vocab.pkl``, that
    file itself, or a ``tokenizer.json``), by default the ``data`` directory beside the
    weights file, the reference's layout.  Generated text goes to stdout, the model summary
    and timing to stderr, as in the reference.
    """
    import argparse
    import os
    import sys
    import time

    from .checkpoint import load_bpe_vocab, load_weights

    parser = argparse.ArgumentParser(description="Generate text with the MI355X decode kernels")
    parser.add_argument("--prompt", type=str, default="Once upon a time", help="Text prompt to continue")
    parser.add_argument("--max-tokens", type=int, default=256, help="Maximum tokens to generate")
    parser.add_argument("--weights", type=str, default="weights.pkl", help="Path to weights file")
    parser.add_argument("--tokenizer", type=str, default=None,
                        help="data directory with bpe_vocab.pkl, that file, or a tokenizer.json")
    parser.add_argument("--no-stream", action="store_true", help="Generate all tokens at once (no streaming)")
    parser.add_argument("--temp", type=float, default=0.0, help="Sampling temperature (0 = greedy)")
    parser.add_argument("--top-p", type=float, default=1.0, help="Nucleus sampling threshold")
    parser.add_argument("--rep-penalty", type=float, default=1.0, help="Repetition penalty (1.0 = off)")
    parser.add_argument("--seed", type=int, default=None, help="Random seed for reproducible sampling")
    parser.add_argument("--device", type=str, default="cuda", help="torch device of the GPU")
    args = parser.parse_args(argv)

    params, config = load_weights(args.weights)
    from .configs import check_config
    check_config(config, need=("decode", "prefill", "sample"))   # before any weight reaches the device
    tok_src = args.tokenizer or os.path.join(os.path.dirname(os.path.abspath(args.weights)), "data")
    bpe = load_bpe_vocab(tok_src)
    decode_fn, encode_fn = bpe["decode_fn"], bpe["encode_fn"]
    ctx_len = config["context_len"]

    print(f"Model: d={config['d_model']} h={config['n_heads']} l={config['n_layers']} ctx={ctx_len}",
          file=sys.stderr)
    print(f"Params: {sum(p.size for p in params.values()):,}", file=sys.stderr)
    if args.temp > 0:
        print(f"Sampling: temp={args.temp} top_p={args.top_p} rep_penalty={args.rep_penalty}", file=sys.stderr)
    else:
        print("Decoding: greedy (argmax)", file=sys.stderr)
    print(file=sys.stderr)

    prompt_ids = list(encode_fn(args.prompt))
    if len(prompt_ids) >= ctx_len:
        prompt_ids = prompt_ids[:ctx_len - 1]
    if not prompt_ids:
        raise SystemExit("the prompt encodes to no tokens")
    max_gen = min(args.max_tokens, ctx_len - len(prompt_ids))

    print(f"Prompt ({len(prompt_ids)} tokens): {args.prompt}", file=sys.stderr)
    print(f"Generating {max_gen} tokens...", file=sys.stderr)
    print(file=sys.stderr)
    sys.stdout.write(args.prompt)
    sys.stdout.flush()

    t0 = time.perf_counter()
    if args.no_stream:
        tokens = generate_tokens(params, config, prompt_ids, max_gen, args.temp, args.top_p,
                                 args.rep_penalty, args.seed, device=args.device)
        elapsed = time.perf_counter() - t0
        sys.stdout.write(decode_fn(tokens))
        sys.stdout.write("\n")
        sys.stdout.flush()
        print(f"\n[{max_gen} tokens in {elapsed * 1000:.0f}ms = {max_gen / elapsed:.0f} tok/s"
              f" (includes weight packing)]", file=sys.stderr)
        return tokens
    tokens, t_first = [], None
    for token_id in stream_tokens(params, config, prompt_ids, max_gen, args.temp, args.top_p,
                                  args.rep_penalty, args.seed, device=args.device):
        if t_first is None:
            t_first = time.perf_counter()
        tokens.append(token_id)
        new_text = decode_fn([token_id])
        if new_text:
            sys.stdout.write(new_text)
            sys.stdout.flush()
    elapsed = time.perf_counter() - t0
    sys.stdout.write("\n")
    sys.stdout.flush()
    ttft = (t_first - t0) * 1000 if t_first else 0
    decode_time = elapsed - (t_first - t0) if t_first else elapsed
    decode_tok_s = (max_gen - 1) / decode_time if decode_time > 0 else 0
    print(f"\n[{max_gen} tokens, TTFT={ttft:.0f}ms (includes weight packing), decode={decode_tok_s:.0f} tok/s]",
          file=sys.stderr)
    return tokens


if __name__ == "__main__":
    main()
