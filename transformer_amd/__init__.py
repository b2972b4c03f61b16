"""MI355X-native fused whole-model decode step for the zahlmann/transformer GQA decoder.

Python surface (drop-in for the reference's decode path):
  * ``transformer_amd.fused_decode_nlayer`` — ``prepare_decode_weights_nlayer``,
    ``pack_weights``, ``pack_kv_caches``, ``unpack_kv_caches``
    (reference kernels/fused_decode_nlayer.py:250-321);
  * ``transformer_amd.multi_sm_decode`` — ``multi_sm_decode_nlayer`` and the
    ``Decoder.step(token, pos)`` object (reference kernels/multi_sm_decode.py:369-432);
  * ``transformer_amd.generate`` — ``sample_token``, ``stream_tokens``,
    ``generate_tokens`` (reference generate.py:28-130).

All compute runs in hand-written HIP kernels for gfx950 behind the C-ABI library
``libmsdecode.so`` (declared in ``include/msdecode.h``).
"""
from .configs import TINY, M306  # noqa: F401
