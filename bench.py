"""Benchmark: batch-1 greedy decode of the 306M config on one MI355X.

Workload (one "step" = one fused decode step = one token): 306M GQA decoder (d 1024,
16 heads, 4 KV heads, 24 layers, d_ff 2816, vocab 32000, ctx 512), random-init bf16
weights (N(0, 0.02), residual projections 0.02/sqrt(48), seed 0), a 32-token uniform
random prompt (seed 1) fed step by step, then one untimed greedy pass over positions
32..510 that fills the KV cache.  The timed region runs K steps at positions spread evenly
over 32..510 (all of them when K = 479), so its average position is that of the whole
generation whatever K is; each step reads the previous step's token on the device, so no
host round trip sits between steps.  The KV cache is updated in place, so the warmup and
timed passes replay the same positions with the same inputs.

Prints one JSON line.  value = decoded tokens per second; roofline.achieved = algorithmic
bytes per step (weights + KV rows read + KV row written, averaged over the timed
positions) / measured average step time; cpu_baseline = the numpy oracle's cached decode
step on the host (a bounded sample of positions).

Secondary figures on the same weights (not the headline value):
  prefill_128     matrix-core prefill of a 128-token prompt (ms, median of runs), then 128
                  greedy decode steps after it (tok/s)
  sampled_decode  64-token prompt, then 256 tokens with temperature 0.7, top-p 0.95 and
                  repetition penalty 1.2 drawn on the device (decode + sampler chained, tok/s),
                  and the sampler alone per token (us)
  decode_one_launch, batched_paged_decode
                  the headline generation in one launch; 8 sequences over a paged cache
  fused_cross_entropy
                  the training-side fused output projection + cross-entropy (forward and
                  backward) on 4096 rows of the 306M output layer, with its matrix-core roofline
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s @batch1 306M on 1 MI355X; % of HBM roofline"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_step_306m_hbm_traffic.json")


def measured_traffic():
    """HBM bytes per decode step from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return float(t["fetch_bytes"]) + float(t["write_bytes"])
    except (OSError, KeyError, ValueError):
        return None
PEAK_HBM_GBS = 8000.0


def positions(start, stop, k):
    """k positions spread evenly over start..stop (inclusive), ascending."""
    span = stop - start + 1
    return [start + (i * span) // k for i in range(k)]


def _events_ms(fn, reps):
    import torch
    s = torch.cuda.current_stream()
    times = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(s)
        fn()
        e1.record(s)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    times.sort()
    return times[len(times) // 2]


def secondary(w, cfg, dec, first_token):
    """Prefill (128 tokens) and sampled-decode figures, on the decoder's weights and KV."""
    import numpy as np
    import torch

    from transformer_amd.generate import Sampler
    from transformer_amd.prefill import Prefiller
    from transformer_amd.synthetic import make_prompt

    out = {}
    # prefill of a 128-token prompt, then 128 greedy steps chained on the device
    prompt = make_prompt(128, cfg["vocab_size"], seed=2)
    pf = Prefiller(w, cfg, max_tokens=128)
    tok_dev = torch.as_tensor(np.asarray(prompt, dtype=np.int32)).cuda()
    ring = torch.zeros((129, 2), dtype=torch.int32, device="cuda")
    pf.launch(tok_dev, dec.kv, out=ring[0])
    ms = _events_ms(lambda: pf.launch(tok_dev, dec.kv, out=ring[0]), 7)

    def steps():
        for i in range(128):
            dec.launch(ring[i, 0:1], 128 + i, out=ring[i + 1])
    steps()
    dms = _events_ms(steps, 3)
    if bool((ring[:, 1] != 0).any()):
        raise RuntimeError("decode status set after prefill")
    out["prefill_128"] = {"prefill_ms": round(ms, 4), "prefill_tok_s": round(128 / (ms / 1e3), 1),
                          "decode_after_tok_s": round(128 / (dms / 1e3), 1),
                          "workload": "306M, 128-token prompt prefilled in one call, then 128 greedy steps"}
    # sampled decode: 64-token prompt, 256 tokens, temperature 0.7 / top-p 0.95 / penalty 1.2
    prompt = make_prompt(64, cfg["vocab_size"], seed=1)
    pf64 = Prefiller(w, cfg, max_tokens=64)
    smp = Sampler(cfg["vocab_size"])
    u = torch.as_tensor(np.random.RandomState(11).random_sample(256)).cuda()
    toks = torch.zeros(256, dtype=torch.int32, device="cuda")
    st = torch.zeros((256, 2), dtype=torch.int32, device="cuda")
    tok_dev = torch.as_tensor(np.asarray(prompt, dtype=np.int32)).cuda()

    def sampled():
        smp.reset()
        pf64.launch(tok_dev, dec.kv, out=st[0])
        smp.launch(pf64.logits, 0.7, 0.95, 1.2, u=u[0:1], out=toks[0:1])
        for i in range(1, 256):
            dec.launch(toks[i - 1:i], 63 + i, out=st[i])
            smp.launch(dec.logits, 0.7, 0.95, 1.2, u=u[i:i + 1], out=toks[i:i + 1])
    sampled()
    sms = _events_ms(sampled, 3)
    if bool((st[:, 1] != 0).any()):
        raise RuntimeError("decode status set in the sampled run")
    one = _events_ms(lambda: [smp.launch(dec.logits, 0.7, 0.95, 1.2, u=u[0:1], out=toks[0:1]) for _ in range(50)], 3)
    out["sampled_decode"] = {"tok_s": round(256 / (sms / 1e3), 1), "sampler_us_per_token": round(one / 50 * 1e3, 2),
                             "workload": "306M, 64-token prompt, 256 tokens, temp 0.7 top-p 0.95 rep-penalty 1.2"}
    # batched paged decode: 8 sequences, prompts U[16, 256], 16-token pages from a shuffled pool
    from transformer_amd.paged import PAGE, PagedBatchDecoder, PagePool
    B, steps = 8, 128
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(16, 257, B)]
    pool = PagePool(cfg, 256)
    bd = PagedBatchDecoder(w, cfg, pool, B)
    free = list(rng.permutation(256))
    first = []
    for b in range(B):
        pages = [int(free.pop()) for _ in range(-(-(lens[b] + steps) // PAGE))]
        first.append(int(bd.prefill(b, make_prompt(lens[b], cfg["vocab_size"], seed=50 + b), pages)[0]))
    ring = torch.zeros((steps + 1, 2 * B), dtype=torch.int32, device="cuda")
    ring[0, 0::2] = torch.tensor(first, dtype=torch.int32, device="cuda")
    posr = torch.tensor([[lens[b] + i for b in range(B)] for i in range(steps)], dtype=torch.int32, device="cuda")
    toks = torch.zeros((steps + 1, B), dtype=torch.int32, device="cuda")

    def batched():
        toks[0] = ring[0, 0::2]
        for i in range(steps):
            bd.launch(toks[i], posr[i], out=ring[i + 1])
            toks[i + 1] = ring[i + 1, 0::2]
    batched()
    bms = _events_ms(batched, 3)
    if bool((ring[1:, 1::2] != 0).any()):
        raise RuntimeError("status set in the batched run")
    # the whole generation of the headline workload in one launch (tokens fed back on the device)
    pos_end = cfg["context_len"] - 1
    tok0 = torch.tensor([int(first_token)], dtype=torch.int32, device="cuda")
    nsteps = pos_end - 32
    one_out = torch.zeros((nsteps, 2), dtype=torch.int32, device="cuda")
    one = lambda: dec.launch_steps(tok0, 32, nsteps, out=one_out)
    one()
    lms = _events_ms(one, 3)
    if bool((one_out[:, 1] != 0).any()):
        raise RuntimeError("status set in the one-launch generation")
    out["decode_one_launch"] = {"tok_s": round(nsteps / (lms / 1e3), 1), "us_per_token": round(lms / nsteps * 1e3, 2),
                                "workload": f"306M, {nsteps} greedy steps at positions 32..{pos_end - 1} in one "
                                            "launch (each step's argmax fed to the next inside the kernel)"}
    out["batched_paged_decode"] = {"tok_s": round(B * steps / (bms / 1e3), 1), "ms_per_step": round(bms / steps, 4),
                                   "workload": "306M, 8 sequences (prompts U[16,256]) x 128 steps, 16-token "
                                               "pages from a shuffled pool, all 8 stepped per call"}
    out["fused_cross_entropy"] = cross_entropy_figure(cfg)
    return out


PEAK_BF16_TFLOPS = 2500.0


def cross_entropy_figure(cfg, n_rows=4096, chunk=4096):
    """The training-side fused output projection + cross-entropy on the 306M output layer:
    4096 token rows, the tied 32000 x 1024 embedding, chunk 4096.  Algorithmic work: the forward
    is one (N x d) . (d x V) product, the backward three (logits again, grad_h, grad_weight)."""
    import torch

    from transformer_amd.xent import fused_cross_entropy
    V, d = cfg["vocab_size"], cfg["d_model"]
    g = torch.Generator().manual_seed(0)
    h = torch.randn(n_rows, d, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    wt = (torch.randn(V, d, generator=g) * 0.02).to(torch.bfloat16).cuda().requires_grad_()
    t = torch.randint(0, V, (n_rows,), generator=g).cuda()
    loss = fused_cross_entropy(h, wt, t, chunk)          # checks the targets once
    loss.backward()
    fwd = lambda: fused_cross_entropy(h, wt, t, chunk, check_targets=False)
    fms = _events_ms(fwd, 7)
    saved = fwd()
    bms = _events_ms(lambda: torch.autograd.grad(saved, (h, wt), retain_graph=True), 7)
    flop = 2.0 * n_rows * V * d
    f_tf, b_tf = flop / (fms * 1e9), 3 * flop / (bms * 1e9)
    return {"forward_ms": round(fms, 4), "backward_ms": round(bms, 4), "forward_tflops": round(f_tf, 1),
            "backward_tflops": round(b_tf, 1),
            "roofline": {"bound": "mfma", "achieved": round(4 * flop / ((fms + bms) * 1e9), 1),
                         "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(4 * flop / ((fms + bms) * 1e9) / PEAK_BF16_TFLOPS, 4)},
            "workload": f"306M output layer: {n_rows} rows, vocab {V}, d {d}, chunk {chunk}; bf16 operands, "
                        "f32 accumulation; forward + backward (4 products of 2 N V d flops)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=479)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--cpu-sample", type=int, default=479,
                    help="oracle decode steps timed for cpu_baseline, from position 32 (0 = skip)")
    ap.add_argument("--synced-steps", type=int, default=128, help="host-synced steps for the secondary figure")
    ap.add_argument("--secondary", type=int, default=1, help="also time the prefill and sampled-decode workloads")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="run one device-to-device copy of this many MiB before decoding (reference "
                         "kernel for scaling HBM byte counters; not timed)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported "
              "(the decode step runs on a single MI355X; see DESIGN.md for how it would shard)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from transformer_amd.configs import M306, bytes_per_token
    from transformer_amd.fused_decode_nlayer import prepare_decode_weights_nlayer
    from transformer_amd.multi_sm_decode import Decoder
    from transformer_amd.synthetic import make_params, make_prompt

    cfg = dict(M306)
    prompt_len = 32
    t0 = time.time()
    params = make_params(cfg, seed=0, resid_scaled=True)
    prompt = make_prompt(prompt_len, cfg["vocab_size"], seed=1)
    w = prepare_decode_weights_nlayer(params, cfg, device="cuda")
    dec = Decoder(w, cfg)
    print(f"[bench] weights ready in {time.time() - t0:.1f}s; workgroups={dec.n_workgroups}",
          file=sys.stderr, flush=True)

    if args.copy_calibration_mb > 0:
        n = args.copy_calibration_mb << 20
        src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # prompt ingest (not timed): one step per prompt token
    for p, t in enumerate(prompt):
        first, _ = dec.step(int(t), p)
    stream = torch.cuda.current_stream()
    start, stop = prompt_len, cfg["context_len"] - 2   # positions 32..510 (inclusive): 479 steps

    def run(ps):
        # ring[i] = (token, status) written by step i-1; step i reads ring[i][0] on device
        ring = torch.zeros((len(ps) + 1, 2), dtype=torch.int32, device="cuda")
        ring[0, 0] = first
        for i, p in enumerate(ps):
            dec.launch(ring[i, 0:1], p, out=ring[i + 1])
        return ring

    run(list(range(start, stop + 1)))   # fills the KV cache rows the timed steps attend over
    warm = positions(start, stop, args.warmup)
    if warm:
        run(warm)
    torch.cuda.synchronize()
    ps = positions(start, stop, args.steps)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    ring = run(ps)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    bad = torch.nonzero(ring[1:, 1]).flatten()
    status = int(ring[1 + int(bad[0]), 1]) & 0xFFFFFFFF if len(bad) else 0
    if status != 0:
        raise RuntimeError(f"decode status {status:#x} during the timed run")
    ms_per_step = ms / args.steps
    tok_s = args.steps / (ms / 1e3)
    avg_bytes = float(np.mean([bytes_per_token(cfg, p) for p in ps]))
    achieved = avg_bytes / (ms_per_step * 1e-3) / 1e9
    print(f"[bench] timed {args.steps} steps: {ms_per_step * 1e3:.1f} us/step, {tok_s:.0f} tok/s, "
          f"{achieved:.0f} GB/s", file=sys.stderr, flush=True)

    # secondary: host-synchronised loop (token read back after every step, as generate.py does)
    synced = None
    if args.synced_steps > 0:
        sp = list(range(start, start + args.synced_steps))
        tok = first
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for p in sp:
            tok, _ = dec.step(tok, p)
        synced = len(sp) / (time.perf_counter() - t1)

    # CPU baseline: the oracle's cached decode step on the host, bounded sample
    cpu = None
    if args.cpu_sample > 0:
        from oracle import model as om
        try:
            from threadpoolctl import threadpool_info
            cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
        except Exception:
            cores = os.cpu_count()
        kc, vc = om.new_kv_cache(cfg)
        rope = om.precompute_rope_table(cfg["context_len"], cfg["d_head"])
        n = args.cpu_sample
        # cache rows come from the GPU run (bf16 values), so the sample attends over a full prompt
        from transformer_amd.fused_decode_nlayer import unpack_kv_caches
        gk, gv = unpack_kv_caches(dec.kv, cfg["n_layers"], cfg["n_kv_heads"], cfg["context_len"], cfg["d_head"])
        for l in range(cfg["n_layers"]):
            kc[l][:, :start] = gk[l][:, :start].float().cpu().numpy()
            vc[l][:, :start] = gv[l][:, :start].float().cpu().numpy()
        om.decode_step(params, cfg, int(first), start, kc, vc, rope=rope)   # warm
        tc = time.perf_counter()
        tk = int(first)
        for p in positions(start, stop, n):
            _, tk = om.decode_step(params, cfg, tk, p, kc, vc, rope=rope)
        cpu_s = time.perf_counter() - tc
        cpu = {"value": round(n / cpu_s, 3), "unit": "tok/s", "cores": int(cores), "kind": "port",
               "sample": f"{n} greedy cached decode steps of the numpy oracle (f32 on bf16-valued 306M "
                         f"weights) from position {start}, {cpu_s:.1f}s"}

    extra = {}
    if args.secondary:
        extra = secondary(w, cfg, dec, first)

    line = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights N(0,0.02), seeded uniform prompt)",
        "config": {"workload": f"306M batch-1 greedy decode, 32-token prompt; {args.steps} timed steps at "
                               f"positions spread evenly over {start}..{stop} (first {ps[0]}, last {ps[-1]})",
                   "d_model": cfg["d_model"], "n_layers": cfg["n_layers"], "n_heads": cfg["n_heads"],
                   "n_kv_heads": cfg["n_kv_heads"], "d_ff": cfg["d_ff"], "vocab": cfg["vocab_size"],
                   "context_len": cfg["context_len"], "batch": 1},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": measured_traffic(),
                     "bytes_per_step": round(avg_bytes)},
        "cpu_baseline": cpu,
        "host_synced_tok_s": None if synced is None else round(synced, 1),
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
