"""ctypes binding of libgranite_switch_amd.so (the C ABI in include/granite_switch_amd.h).

The library is loaded after torch, so it binds to the HIP runtime torch
already mapped (same soname) and every launch can go on torch's current
stream.  There is no fallback: if the library is missing, every entry point
raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  -- must be imported before the HIP library is loaded

from .build import LIB_PATH

c_void_p = ctypes.c_void_p
c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64

GS_OK = 0
GS_ERR_INVALID = 1
GS_ERR_HIP = 2
GS_ERR_WORKSPACE = 3
GS_DTYPE_BF16 = 0
GS_DTYPE_FP32 = 1
GS_MAX_ADAPTERS = 256
GS_MAX_SLICES = 8
GS_MAX_RANK = 512
GS_RANK_CLASS_SPLIT = 64
GS_NOALLOC_SCRATCH_BYTES = 64 << 20

# name -> (restype, argtypes); mirrors include/granite_switch_amd.h
SIGNATURES = {
    "gs_version": (c_i32, []),
    "gs_last_error": (ctypes.c_char_p, []),
    "gs_build_segments_workspace_bytes": (c_i64, [c_i64, c_i32]),
    "gs_build_segments": (c_i32, [c_void_p, c_void_p, c_void_p, c_void_p, c_i64, c_i32, c_i32, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_i64, c_void_p]),
    "gs_route_latest_wins": (c_i32, [c_void_p, c_void_p, c_i64, c_i32, c_void_p, c_i32, c_i32, c_void_p, c_void_p,
                                     c_void_p]),
    "gs_shrink_workspace_bytes": (c_i64, [c_i64, c_i32, c_i32, c_i32, c_i32, c_void_p]),
    "gs_shrink_ksplits": (c_i32, [c_i32, c_i64, c_i32, c_i32, c_i32, c_i32, c_void_p, c_void_p]),
    "gs_switched_lora_pair": (c_i32, [c_i32, c_i64, c_i32, c_i32, c_void_p, c_i32, c_i32, c_i32, c_void_p]),
    "gs_check_segment_addresses": (c_i64, [c_i32, c_i64, c_i32, c_i64, c_i32, c_i64, c_void_p, c_i32, c_void_p, c_i64,
                                           c_void_p, c_i64, c_void_p, c_i32, c_i32, c_void_p, c_void_p, c_void_p,
                                           c_i64, ctypes.c_char_p, c_i64, c_void_p]),
    "gs_check_gemm_addresses": (c_i64, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_char_p, c_i64, c_void_p]),
    "gs_check_token_addresses": (c_i64, [c_i64, c_i32, c_void_p, c_i32, c_void_p, c_i32, c_i32, c_i32, c_i32,
                                         ctypes.c_char_p, c_i64, c_void_p]),
    "gs_check_build_addresses": (c_i64, [c_i64, c_i32, c_i32, c_void_p, c_void_p, c_void_p, c_void_p, c_i32,
                                         ctypes.c_char_p, c_i64, c_void_p]),
    "gs_check_small_addresses": (c_i64, [c_i32, c_i64, c_i32, c_i64, c_i32, c_i64, c_void_p, c_i32, c_void_p, c_i64,
                                         c_void_p, c_i64, c_void_p, c_i32, c_i32, c_void_p, c_i32, c_i32, c_i32,
                                         ctypes.c_char_p, c_i64, c_void_p]),
    "gs_check_xext_addresses": (c_i64, [c_i32, c_i64, c_i64, c_i64, c_void_p, c_i32, c_void_p, c_i64, c_i64, c_i64,
                                        c_void_p, c_i64, c_void_p, c_void_p, c_i32, c_i32, c_i32, c_i32, c_i64, c_i32,
                                        ctypes.c_char_p, c_i64, c_void_p]),
    "gs_shrink": (c_i32, [c_i32, c_void_p, c_i64, c_i64, c_i32, c_void_p, c_void_p, c_void_p, c_i32, c_i32, c_i32,
                          c_void_p, c_void_p, c_void_p, c_void_p, c_i64, c_void_p, c_i64, c_void_p]),
    "gs_expand_add": (c_i32, [c_i32, c_void_p, c_i64, c_i64, c_i32, c_void_p, c_i32, c_void_p, c_i64, c_i32, c_void_p,
                              c_void_p, c_void_p, c_void_p, c_i32, c_i32, c_void_p, c_void_p, c_void_p, c_void_p]),
    "gs_switched_lora": (c_i32, [c_i32, c_void_p, c_i64, c_void_p, c_i64, c_i64, c_i32, c_i32, c_void_p, c_i32,
                                 c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_i32, c_i32, c_void_p, c_void_p,
                                 c_void_p, c_void_p, c_void_p, c_i64, c_void_p]),
    "gs_switched_lora_noalloc": (c_i32, [c_i32, c_void_p, c_i64, c_void_p, c_i64, c_i64, c_i32, c_i32, c_void_p,
                                         c_i32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_i32, c_i32,
                                         c_void_p, c_void_p, c_void_p, c_void_p]),
    "gs_small_eligible": (c_i32, [c_i64, c_i32, c_i32, c_void_p, c_i32, c_i32]),
    "gs_small_workspace_bytes": (c_i64, [c_i32, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_void_p]),
    "gs_small_sync_bytes": (c_i64, []),
    "gs_small_set_wait_limit": (c_i64, [c_i64]),
    "gs_small_workgroups": (c_i64, [c_i32, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_void_p, c_i32]),
    "gs_switched_lora_small": (c_i32, [c_i32, c_void_p, c_void_p, c_void_p, c_void_p, c_i32, c_void_p, c_void_p,
                                       c_i64, c_void_p, c_i64, c_i64, c_i32, c_i32, c_void_p, c_i32, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_i32, c_i32, c_void_p, c_i64,
                                       c_void_p, c_i64, c_i32, c_i32, c_void_p]),
    "gs_compute_bitmasks": (c_i32, [c_void_p, c_i32, c_i64, c_void_p, c_i32, c_i32, c_i32, c_void_p, c_void_p,
                                    c_void_p]),
    "gs_switch_lora_expand": (c_i32, [c_void_p, c_i64, c_i64, c_i64, c_void_p, c_i32, c_void_p, c_i64, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_i32, c_i32, c_i32, c_void_p]),
    "gs_switch_lora_expand_swiglu": (c_i32, [c_void_p, c_i64, c_i64, c_void_p, c_i64, c_i64, c_i64, c_void_p, c_i32,
                                             c_void_p, c_i64, c_void_p, c_void_p, c_void_p, c_i32, c_i32, c_i32, c_i32,
                                             c_void_p]),
    "gs_split_adapter_indices": (c_i32, [c_void_p, c_i32, c_void_p, c_i32, c_i64, c_void_p, c_void_p, c_void_p]),
    "gs_switch_lora_shrink_expand": (c_i32, [c_void_p, c_i32, c_i64, c_i64, c_void_p, c_i64, c_i64, c_i64, c_void_p,
                                             c_i32, c_void_p, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, c_i32,
                                             c_i32, c_i32, c_void_p]),
    "gs_gemm_bf16_tn": (c_i32, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_i64, c_i64, c_i64, c_void_p]),
}


class GraniteSwitchError(RuntimeError):
    """A library entry point returned a non-OK status."""

    def __init__(self, func: str, status: int, message: str):
        super().__init__(f"{func} failed (status {status}): {message}")
        self.func = func
        self.status = status


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() or "
                "python granite-switch_amd/build.py (there is no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().gs_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> int:
    """Call an entry point; raise GraniteSwitchError on a non-OK status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != GS_OK:
        msg = lib.gs_last_error()
        raise GraniteSwitchError(name, rc, msg.decode() if msg else "")
    return rc


def stream_ptr(device: torch.device | None = None) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
