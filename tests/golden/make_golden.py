"""Write the tiny-config regression fixtures (tests/golden/tiny_greedy.json).

The reference implementation cannot run here (jax, jaxlib and jax-triton are not installed),
so these vectors come from the numpy oracle (oracle/model.py), which is itself pinned by
tests/test_oracle.py.  They freeze: the seeded synthetic weights (SHA-256 of the bf16 bytes),
the prompt, the greedy tokens of the cached-step pipeline and of the prefill pipeline, and a
few logits per step with their top-2 margin.

    python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import model as om  # noqa: E402
from transformer_amd.configs import TINY  # noqa: E402
from transformer_amd.synthetic import make_params, make_prompt  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tiny_greedy.json")


def weights_sha256(params):
    h = hashlib.sha256()
    for k in sorted(params):
        a = np.ascontiguousarray(params[k], dtype=np.float32)
        h.update(k.encode())
        h.update((a.view(np.uint32) >> 16).astype(np.uint16).tobytes())
    return h.hexdigest()


def main():
    params = make_params(TINY, seed=0)
    prompt = make_prompt(16, TINY["vocab_size"], seed=1)
    toks, logs = om.greedy_generate(params, TINY, prompt, 48, prefill="step", return_logits=True)
    toks_full = om.greedy_generate(params, TINY, prompt, 48, prefill="full")
    steps = []
    for i, lg in enumerate(logs):
        top = np.argsort(-lg, kind="stable")[:2]
        steps.append({"step": i, "argmax": int(top[0]), "top2_margin": float(lg[top[0]] - lg[top[1]]),
                      "logits_0_8": [float(v) for v in lg[:8]], "logit_max": float(lg[top[0]])})
    out = {
        "config": TINY, "weights": "make_params(TINY, seed=0)", "weights_sha256": weights_sha256(params),
        "prompt": [int(t) for t in prompt], "greedy_tokens_step_prefill": toks,
        "greedy_tokens_full_prefill": toks_full, "steps": steps,
        "source": "numpy oracle (oracle/model.py), f32 maths on bf16-valued weights, bf16 KV cache",
    }
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
