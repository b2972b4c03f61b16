"""bf16 helpers for the oracle — TEST INFRASTRUCTURE ONLY.

bf16 values are kept in float32 (or float64) arrays; ``bf16_round`` applies
round-to-nearest-even on the float32 bit pattern, which is what
``astype(bfloat16)`` does in the reference (model.py:212-215,
kernels/fused_decode_nlayer.py:270).
"""
import numpy as np


def bf16_round(x):
    """Round to the nearest bf16 (ties to even); returns the input dtype."""
    dt = x.dtype
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u >> 16) & 1) + 0x7FFF
    out = (((u + r) >> 16) << 16).astype(np.uint32).view(np.float32)
    return out.astype(dt).reshape(x.shape)
