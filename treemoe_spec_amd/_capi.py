"""ctypes binding of libtreemoe_amd.so (declared in include/treemoe_amd.h).

The library is loaded once per process.  A missing library is an error: the
product path has no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

_LIB_PATH = Path(os.environ.get(
    "TREEMOE_AMD_LIB", Path(__file__).resolve().parent / "libtreemoe_amd.so"))

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float

# name -> argtypes; every entry point returns int (0 = ok)
SIGNATURES: dict[str, list] = {
    "tm_op1_router_gates": [P, P, I64, I64, I64, P, I32, P],
    "tm_op1_route_bucket": [P, P, I64, I64, I64, F32, I32, I64, I64, I64] + [P] * 10 + [P],
    "tm_op1_route": [P, P, P, I64, I64, I64, I64, F32, I32, I64, I64, I64] + [P] * 11 + [I32, P],
    "tm_op1_gemm1": [P, P, P, P, P, P, I64, I64, I64, I64, I64, I32, P],
    "tm_op1_gemm2": [P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I32, P],
    "tm_op1_combine": [P, P, P, I64, I64, I64, I32, P],
    "tm_op1_prefill_gemm1": [P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I32, P],
    "tm_op1_prefill_gemm2": [P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I32, P],
    "tm_op1_prefill_gemm1_routed": [P] * 6 + [I64] * 5 + [F32, I32, I64, I64, I64] + [P] * 10
                                   + [I32, P],
    "tm_op4_argmax_walk": [P, I32, I64, I64, I64, P, P, P, P, I64, I64, I32, P, P, P, P, P, P],
    "tm_op4_kv_commit": [P, P, I64, I64, I64, I64, I64, I64, I64, P, P, P, I64, P, I64, I64,
                         I64, P, P],
    "tm_host_device_pointer": [P, P],
    "tm_op4_argmax_walk_noalloc": [P, I32, I64, I64, I64, P, P, P, P, I64, I64, I32, P, P, P,
                                   P, P],
    "tm_op4_rep_penalty": [P, I32, I64, I64, I64, P, I64, F32, P, I64, P],
    "tm_op4_sample_walk": [P, I32, I64, I64, I64, P, I64, P, P, P, P, I64, P, P, F32, P, P, P,
                           P, P],
    "tm_tree_attention": [P, I64, P, P, I64, P, P, I64, I64, I64, P, I64, I64, P, I64, I32, P,
                          I64, I64, I64, I64, F32, P, I64, I64, P, I64, P],
    "tm_tree_attention_plan": [I64, I64, I64, I64, I64, I64, I64, P, P],
    "tm_tree_mask_pack": [P, I64, I64, P, P],
}

TM_OBJECTIVE = {"mass": 0, "critical_path": 1}
TM_DTYPE_F32 = 0
TM_DTYPE_BF16 = 1
TM_DTYPE_F16 = 2
TM_GEMM_TILE_M = 64
TM_OP4_MAX_PARTS = 64
TM_OP4_NOALLOC_MAX_NODES = 2048

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"treemoe_spec_amd: native library {_LIB_PATH} is missing; build it with "
                "`python -m treemoe_spec_amd._build` (there is no CPU fallback)")
        handle = ctypes.CDLL(str(_LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        handle.tm_version.argtypes = []
        handle.tm_version.restype = ctypes.c_int
        handle.tm_status_string.argtypes = [ctypes.c_int]
        handle.tm_status_string.restype = ctypes.c_char_p
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().tm_status_string(rc).decode()
        raise RuntimeError(f"{what} failed with status {rc}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def ptr(t) -> int:
    """Device address of a torch tensor (None -> NULL)."""
    return 0 if t is None else t.data_ptr()


def stream_of(device) -> int:
    """Raw handle of torch's current stream on ``device`` (a torch.device,
    'cuda[:N]' or an index)."""
    import torch

    if isinstance(device, int):
        idx = device
    else:
        idx = (device if isinstance(device, torch.device) else torch.device(device)).index
    if idx is None:
        idx = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)
