"""ctypes binding of libmsdecode.so (C ABI in include/msdecode.h).

torch is imported first so that the library's HIP runtime dependency resolves to the
runtime torch already loaded (one runtime per process, shared device pointers/streams).
There is no fallback: a missing library raises.
"""
import ctypes
import os

import torch  # noqa: F401  (load torch's HIP runtime before the library)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmsdecode.so")

MSD_OK = 0
MSD_E_CONFIG = -1
MSD_E_ARG = -2
MSD_E_HIP = -3
MSD_E_TIMEOUT = -4
_ERRNAMES = {MSD_E_CONFIG: "unsupported config", MSD_E_ARG: "invalid argument",
             MSD_E_HIP: "HIP runtime error", MSD_E_TIMEOUT: "cross-workgroup wait timed out"}

EXPORTS = ("msd_packed_weight_elems", "msd_workspace_bytes", "msd_default_workgroups",
           "msd_decode_step", "msd_check_status", "msd_sample_workspace_bytes", "msd_sample_token",
           "msd_prefill_workspace_bytes", "msd_prefill", "msd_prefill_paged", "msd_batch_workspace_bytes",
           "msd_batch_decode_step", "msd_workspace_acquire", "msd_workspace_release",
           "msd_sample_token_noalloc", "msd_verify_workspace_bytes", "msd_verify",
           "msd_decode_steps", "msd_tiles_bytes", "msd_pack_tiles", "msd_set_launch_graphs",
           "msd_config_support", "msd_xent_workspace_bytes", "msd_xent_forward", "msd_xent_backward")

# Paths of the library (bits of msd_config_support)
PATHS = {"decode": 1, "prefill": 2, "verify": 4, "batched": 8, "sample": 16, "batched_step": 32}


class MsdConfig(ctypes.Structure):
    _fields_ = [(k, ctypes.c_int32) for k in ("vocab_size", "d_model", "n_heads", "n_kv_heads",
                                              "n_layers", "d_head", "d_ff", "context_len")]

    @classmethod
    def from_dict(cls, c):
        return cls(c["vocab_size"], c["d_model"], c["n_heads"], c["n_kv_heads"], c["n_layers"],
                   c.get("d_head", c["d_model"] // c["n_heads"]), c["d_ff"], c["context_len"])


class MsdError(RuntimeError):
    def __init__(self, code, what):
        super().__init__(f"{what}: {_ERRNAMES.get(code, 'error')} ({code})")
        self.code = code


# Bits of a step's status output (next_token[1]): a cross-workgroup wait ran out, a device
# token was out of range, or the step never completed its arrivals (the value it starts with).
STATUS_TIMEOUT = 0x1
STATUS_BAD_TOKEN = 0x2
STATUS_UNFINISHED = 0x80000000


def status_error(status, what):
    """The MsdError for a non-zero step status word (timeouts and unfinished steps first)."""
    status = int(status) & 0xFFFFFFFF
    code = MSD_E_TIMEOUT if status & (STATUS_TIMEOUT | STATUS_UNFINISHED) else MSD_E_ARG
    return MsdError(code, f"{what} (status {status:#x})")


_lib = None


def lib():
    """Load libmsdecode.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m transformer_amd.build` "
                           "(or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    P, I32, I64, U32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
    CP = ctypes.POINTER(MsdConfig)
    L.msd_packed_weight_elems.argtypes = [CP]
    L.msd_packed_weight_elems.restype = I64
    L.msd_workspace_bytes.argtypes = [CP, I32]
    L.msd_workspace_bytes.restype = I64
    L.msd_default_workgroups.argtypes = [I32]
    L.msd_default_workgroups.restype = I32
    L.msd_decode_step.argtypes = [CP, P, P, P, P, P, I32, P, I32, P, P, U32, P, P, I32, P]
    L.msd_decode_step.restype = I32
    L.msd_decode_steps.argtypes = [CP, P, P, P, P, P, I32, P, I32, I32, P, P, U32, P, I32, P, I32, P]
    L.msd_decode_steps.restype = I32
    L.msd_check_status.argtypes = [P, P]
    L.msd_check_status.restype = I32
    L.msd_workspace_acquire.argtypes = [I32, I64, ctypes.POINTER(ctypes.c_void_p)]
    L.msd_workspace_acquire.restype = I32
    L.msd_workspace_release.argtypes = [P]
    L.msd_workspace_release.restype = I32
    D = ctypes.c_double
    L.msd_sample_workspace_bytes.argtypes = [I32]
    L.msd_sample_workspace_bytes.restype = I64
    L.msd_sample_token.argtypes = [P, I32, D, D, D, P, P, P, P, P, P, P]
    L.msd_sample_token.restype = I32
    L.msd_sample_token_noalloc.argtypes = [P, I32, D, D, D, P, P, P, P, P, P]
    L.msd_sample_token_noalloc.restype = I32
    L.msd_prefill_workspace_bytes.argtypes = [CP, I32]
    L.msd_prefill_workspace_bytes.restype = I64
    L.msd_tiles_bytes.argtypes = [CP]
    L.msd_tiles_bytes.restype = I64
    L.msd_pack_tiles.argtypes = [CP, P, P, P]
    L.msd_pack_tiles.restype = I32
    L.msd_prefill.argtypes = [CP, P, P, P, P, P, P, P, I32, P, P, P, P, P, P]
    L.msd_prefill.restype = I32
    L.msd_prefill_paged.argtypes = [CP, P, P, P, P, P, P, P, I32, P, I32, P, I32, P, P, P, P]
    L.msd_prefill_paged.restype = I32
    L.msd_batch_workspace_bytes.argtypes = [CP, I32]
    L.msd_batch_workspace_bytes.restype = I64
    L.msd_batch_decode_step.argtypes = [CP, P, P, P, P, P, P, P, P, I32, P, I32, P, I32, P, P, P, P]
    L.msd_batch_decode_step.restype = I32
    L.msd_set_launch_graphs.argtypes = [I32]
    L.msd_set_launch_graphs.restype = I32
    L.msd_verify_workspace_bytes.argtypes = [CP, I32]
    L.msd_verify_workspace_bytes.restype = I64
    L.msd_verify.argtypes = [CP, P, P, P, P, P, P, P, I32, I32, P, P, P, P, P]
    L.msd_verify.restype = I32
    L.msd_config_support.argtypes = [CP, I32]
    L.msd_config_support.restype = I32
    L.msd_xent_workspace_bytes.argtypes = [I32, I32, I32, I32]
    L.msd_xent_workspace_bytes.restype = I64
    L.msd_xent_forward.argtypes = [P, P, P, I32, I32, I32, P, P, P, P, P]
    L.msd_xent_forward.restype = I32
    L.msd_xent_backward.argtypes = [P, P, P, P, P, I32, I32, I32, I32, P, P, P, P, P]
    L.msd_xent_backward.restype = I32
    _lib = L
    return L


def check(code, what):
    if code < 0:
        raise MsdError(code, what)
    return code
