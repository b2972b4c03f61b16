"""Phase timeline of the fused decode step from its built-in trace (profiling build).

``python -m transformer_amd.trace --build`` compiles ``libmsdecode_trace.so`` (the decode
library with ``-DMSD_TRACE``: lane 0 of every wave stamps ``s_memrealtime``, a 100 MHz clock,
at each phase boundary of every layer).  ``python -m transformer_amd.trace --pos 300 --layers
0,10,23`` runs the 306M configuration (synthetic weights, seed 0; a 32-token prompt, then
greedy steps up to position ``pos``) on that library and prints, for each listed layer, when
each phase boundary was reached across the workgroups (min / median / max, us from the
layer's first QKV start), the five exchange hops (last producer's post to the consumers'
gathered vector), and every layer's length.

Row-workgroup slots: 16 QKV rows ready, 11 normed, 14 dots done, 17 QKV outputs posted,
3 attention vector gathered, 1 attention vector ready, 18 O rows ready, 19 O outputs posted,
2 O vector gathered, 20 gate/up rows ready, 8 normed, 9 dots done, 10 stored, 21 posted,
5 activation gathered, 22 down rows ready, 15 dots done, 23 posted, 6 down vector gathered;
loader slots 28-31 the QKV / O / gate-up / down rows of the layer landed in LDS.
Attention-workgroup slots: 28 cached K/V rows landed, 24 q gathered, 25 rows ready,
29 scores done, 30 P.V done, 26 blocks merged, 27 head output published.
Tail (layer index n_layers): 1 worker wave 0's logit rows streamed, 12 logits and argmax of the
workgroup done.
"""
import argparse
import ctypes
import os
import subprocess
import sys

import numpy as np

from . import build as _build

HERE = os.path.dirname(os.path.abspath(__file__))
TRACE_LIB = os.path.join(HERE, "libmsdecode_trace.so")
LAYERS, WGS, SLOTS = 64, 512, 32

ROW = [(16, "QKV rows ready"), (11, "QKV normed"), (14, "QKV dots done"), (17, "QKV posted"),
       (3, "attention gathered"), (1, "attention ready"), (18, "O rows ready"), (19, "O posted"),
       (2, "O gathered"), (20, "gate/up rows ready"), (8, "gate/up normed"), (9, "gate/up dots done"),
       (21, "gate/up posted"), (5, "activation gathered"), (22, "down rows ready"), (15, "down dots done"),
       (23, "down posted"), (6, "down gathered")]
LOADER = [(28, "loader: QKV rows landed"), (29, "loader: O rows landed"), (30, "loader: gate/up rows landed"),
          (31, "loader: down rows landed")]
ATT = [(28, "cached K/V landed"), (24, "q gathered"), (25, "K/V rows ready"), (29, "scores done"),
       (30, "P.V done"), (26, "blocks merged"), (27, "head output published")]
# (name, producer slot and workgroup kind, consumer slot and kind)
HOPS = [("QKV -> attention", (17, "row"), (24, "att")),
        ("attention -> rows", (27, "att"), (3, "row")),
        ("O -> rows", (19, "row"), (2, "row")),
        ("gate/up -> rows", (21, "row"), (5, "row")),
        ("down -> rows", (23, "row"), (6, "row"))]


def build_trace(verbose=False):
    cmd = [_build.hipcc(), *_build.HIPCC_FLAGS, "-DMSD_TRACE", "-o", TRACE_LIB,
           *[os.path.join(HERE, s) for s in _build.LIBS["libmsdecode.so"]]]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return TRACE_LIB


def _stats(v):
    return f"min {v.min():7.2f}  med {np.median(v):7.2f}  max {v.max():7.2f}"


def run(pos, layers, n_prompt=32, trace_layer=10):
    from . import _lib
    _lib.LIB_PATH = TRACE_LIB
    import torch
    from .configs import M306
    from .fused_decode_nlayer import prepare_decode_weights_nlayer
    from .multi_sm_decode import Decoder
    from .synthetic import make_params, make_prompt

    cfg = dict(M306)
    params = make_params(cfg, seed=0, resid_scaled=True)
    w = prepare_decode_weights_nlayer(params, cfg)
    dec = Decoder(w, cfg)
    L = _lib.lib()
    L.msd_trace_copy.argtypes = [ctypes.c_void_p]
    L.msd_trace_waves_copy.argtypes = [ctypes.c_void_p]
    tok = 0
    for p, t in enumerate(make_prompt(n_prompt, cfg["vocab_size"], seed=1)):
        tok, _ = dec.step(int(t), p)
    for p in range(n_prompt, pos + 1):
        tok, _ = dec.step(tok, p)
    torch.cuda.synchronize()
    buf = np.zeros(LAYERS * WGS * SLOTS, dtype=np.uint64)
    assert L.msd_trace_copy(buf.ctypes.data) == 0
    tr = buf.reshape(LAYERS, WGS, SLOTS).astype(np.int64)
    G = dec.n_workgroups
    NA = cfg["n_heads"]   # one attention workgroup per head at this context
    GR = G - NA
    nl = cfg["n_layers"]
    print(f"306M decode step at position {pos}: {G} workgroups ({GR} row, {NA} attention); "
          f"times in us (s_memrealtime, 100 MHz)")
    starts = np.array([tr[l, :GR, 16].min() for l in range(nl)])
    t_begin = starts[0]
    t_logits = tr[nl, :GR, 12]
    lens = np.diff(np.append(starts, t_logits.max())) / 100.0
    print("layer lengths (QKV start to next QKV start; last: to the last workgroup's logits):")
    print("  " + " ".join(f"{x:.2f}" for x in lens))
    print(f"  sum {lens.sum():.2f}; last down vector gathered -> logits done: "
          f"{_stats((t_logits - tr[nl - 1, :GR, 6].max()) / 100.0)}")
    print(f"  step span from the first QKV start: {(t_logits.max() - t_begin) / 100.0:.2f}")
    t_dn = tr[nl - 1, :GR, 6].max()
    print("  tail, us from the last down vector gathered (slowest workgroup):")
    for slot, name in ((1, "logit rows streamed"), (12, "logits and argmax done")):
        col = tr[nl, :GR, slot]
        col = col[col > 0]
        if len(col):
            print(f"    {name:24s} {_stats((col - t_dn) / 100.0)}")
    for l in layers:
        t0 = starts[l]
        print(f"\n=== layer {l} (us from its first QKV start)")
        for slot, name in ROW:
            col = tr[l, :GR, slot]
            col = col[col > 0]
            if len(col):
                print(f"  row  {name:28s} {_stats((col - t0) / 100.0)}")
        for slot, name in LOADER:
            col = tr[l, :GR, slot]
            col = col[col > 0]
            if len(col):
                print(f"  row  {name:28s} {_stats((col - t0) / 100.0)}")
        for slot, name in ATT:
            col = tr[l, GR:G, slot]
            col = col[col > 0]
            if len(col):
                print(f"  att  {name:28s} {_stats((col - t0) / 100.0)}")
        if l == trace_layer:
            wv = np.zeros(4096 * 16 * 8, dtype=np.uint64)
            assert L.msd_trace_waves_copy(wv.ctypes.data) == 0
            wv = wv.reshape(4096, 16, 8).astype(np.int64)
            print("  row worker waves, gate/up phase (median over workgroups, us from the rows ready):")
            names = ["normed", "dots done", "stored", "after the barrier"]
            for k in range(8):
                base = wv[:GR, k, 0]
                cells = "  ".join(f"{n} {np.median((wv[:GR, k, j + 1] - base) / 100.0):5.2f}"
                                  for j, n in enumerate(names))
                print(f"    wave {k}: {cells}")
            print("  attention waves (median over workgroups, us from q gathered):")
            names = ["rows ready", "scores", "P.V", "k/v polled", "waves met", "published"]
            for k in range(8):
                base = wv[GR:G, k, 0]
                cells = "  ".join(f"{n} {np.median((wv[GR:G, k, j + 1] - base) / 100.0):5.2f}"
                                  for j, n in enumerate(names))
                print(f"    wave {k}: {cells}")
        print("  hops (last producer's post -> each consumer's gathered vector):")
        for name, (ps, pk), (cs, ck) in HOPS:
            prod = tr[l, :GR, ps] if pk == "row" else tr[l, GR:G, ps]
            cons = tr[l, :GR, cs] if ck == "row" else tr[l, GR:G, cs]
            d = (cons - prod.max()) / 100.0
            print(f"    {name:20s} {_stats(d)}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--build", action="store_true", help="compile libmsdecode_trace.so and exit")
    ap.add_argument("--pos", type=int, default=300)
    ap.add_argument("--layers", default="0,10,23")
    args = ap.parse_args()
    if args.build:
        print("built", build_trace(verbose=True))
        return
    if not os.path.exists(TRACE_LIB):
        sys.exit(f"{TRACE_LIB} is missing: run python -m transformer_amd.trace --build")
    run(args.pos, [int(x) for x in args.layers.split(",")])


if __name__ == "__main__":
    main()
