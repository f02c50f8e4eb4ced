"""ctypes binding of libember_ops.so (the C ABI declared in include/ember_ops.h).

The library is loaded once, on first use. A missing or stale library is an error, never a
silent fallback: every GPU op of this package goes through it.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libember_ops.so"
ABI_VERSION = 16

F32, F16, BF16 = 0, 1, 2
ERR_EMBED_ID = 1
ERR_ROPE_POS = 2
ERR_KV_SLOT = 4
ERR_DECODE_CTX = 8
ERR_BLOCK_ID = 16
ERR_ROW_INDEX = 32
ERR_SYNC = 64
ERR_EXPERT_ID = 128
DECODE_FP32 = 1

_DTYPE_TAG = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes, in the order of include/ember_ops.h
SIGNATURES: dict[str, list] = {
    "ember_rmsnorm": [_p, _i64, _p, _i32, _p, _i64, _i64, _i64, _f32, _i32, _p],
    "ember_fused_add_rmsnorm": [_p, _i64, _p, _i64, _p, _i32, _p, _i64, _p, _i64, _i64, _i64, _f32, _i32, _p],
    "ember_rope": [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _i64, _i32, _p],
    "ember_silu_and_mul": [_p, _i64, _p, _i64, _i64, _i64, _i32, _p],
    "ember_embedding": [_p, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _p],
    "ember_gather_rows": [_p, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64, _p],
    "ember_stream_copy": [_p, _p, _i64, _p],
    "ember_scatter_rows2": [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64, _p],
    "ember_qk_norm_rope": [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p, _p, _i32, _f32,
                           _p, _p, _i64, _i64, _p, _i64, _i32, _p],
    "ember_mla_latent_rope": [_p, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i32, _f32,
                              _p, _p, _i64, _i64, _p, _i64, _p, _i64, _i32, _p],
    "ember_kv_cache_write": [_p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _i64, _i64, _i64,
                             _i64, _p],
    "ember_latent_cache_write": [_p, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64, _p],
    "ember_rope_kv_cache": [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _p, _i32, _f32,
                            _p, _p, _i64, _i64, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _i32, _p],
    "ember_mla_latent_rope_cache": [_p, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i32, _f32,
                                    _p, _p, _i64, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _i64, _i32, _p],
    "ember_paged_decode_workspace_bytes": [_i64, _i64, _i64, _i64],
    "ember_paged_decode": [_p, _i64, _i64, _i32, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                           _i64, _i32, _p, _i64, _i64, _p, _i64, _i64, _f32, _i64, _i32, _p, _i64, _p, _i64,
                           _i64, _p],
    "ember_paged_decode_noalloc_max_bytes": [],
    "ember_paged_decode_noalloc": [_p, _i64, _i64, _i32, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                   _i64, _i64, _i32, _p, _i64, _i64, _p, _i64, _i64, _f32, _i64, _i32, _p, _i64,
                                   _i64, _p],
    "ember_mla_decode_workspace_bytes": [_i64, _i64, _i64, _i64],
    "ember_mla_decode": [_p, _i64, _i64, _p, _i64, _i64, _i32, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
                         _p, _i64, _i64, _p, _i64, _i64, _f32, _i64, _p, _i64, _p, _i64, _i64, _p],
    "ember_gate_up_silu_workspace_bytes": [_i64, _i64, _i64, _i64],
    "ember_gate_up_silu": [_p, _i64, _p, _i64, _i32, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p],
    "ember_gate_up_silu_pack_weight": [_p, _i64, _i32, _i64, _i64, _i64, _p, _p],
    "ember_gate_up_silu_gemm": [_p, _i64, _p, _i64, _i32, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "ember_moe_gate_up_silu_gemm": [_p, _i64, _i64, _p, _i64, _i64, _i32, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64,
                                    _i64, _i64, _p, _i64, _p],
    "ember_gate_up_silu_packed": [_p, _i64, _p, _i32, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _p],
    "ember_gate_up_silu_gemm_packed": [_p, _i64, _p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "ember_moe_gate_up_silu_gemm_packed": [_p, _i64, _i64, _p, _i32, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64,
                                           _i64, _p, _i64, _p],
    "ember_moe_gate_up_silu": [_p, _i64, _i64, _p, _i64, _i64, _i32, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64,
                               _i64, _p, _i64, _p, _i64, _p],
    "ember_moe_gate_up_silu_workspace_bytes": [_i64, _i64, _i64, _i64],
    "ember_moe_gate_up_silu_pack_weight": [_p, _i64, _i64, _i32, _i64, _i64, _i64, _p, _p],
    "ember_moe_gate_up_silu_direct": [_p, _i64, _i64, _p, _i32, _i64, _i64, _i64, _p, _i32, _i64, _i64, _i64, _p, _i64,
                                      _p],
    "ember_moe_gate_up_silu_packed": [_p, _i64, _i64, _p, _i32, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                      _p, _i64, _p, _i64, _p],
    "ember_moe_align_padded_size": [_i64, _i64, _i64],
    "ember_moe_align_workspace_bytes": [_i64, _i64],
    "ember_moe_align": [_p, _i32, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p],
    "ember_read_errors": [ctypes.POINTER(ctypes.c_uint32), _i32],
    "ember_abi_version": [],
    "ember_status_string": [_i32],
}

_RESTYPE = {"ember_status_string": ctypes.c_char_p, "ember_paged_decode_workspace_bytes": ctypes.c_int64,
            "ember_mla_decode_workspace_bytes": ctypes.c_int64,
            "ember_gate_up_silu_workspace_bytes": ctypes.c_int64,
            "ember_moe_gate_up_silu_workspace_bytes": ctypes.c_int64,
            "ember_moe_align_padded_size": ctypes.c_int64,
            "ember_moe_align_workspace_bytes": ctypes.c_int64,
            "ember_paged_decode_noalloc_max_bytes": ctypes.c_int64}


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Returns the loaded library, loading it on first call. Raises RuntimeError when it
    is missing or was built for another ABI version."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"emberserve_amd: {p} is not built; run `python -m emberserve_amd.build` "
                "(or __graft_entry__.build()) first")
        lib = ctypes.CDLL(str(p))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPE.get(name, ctypes.c_int)
        got = lib.ember_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"emberserve_amd: {p} has ABI version {got}, expected {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


def dtype_tag(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_TAG[dtype]
    except KeyError:
        raise TypeError(f"emberserve_amd: unsupported dtype {dtype} (float32, float16, bfloat16)") from None


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (the capture stream while a
    torch.cuda.graph is being recorded)."""
    return torch.cuda.current_stream(device).cuda_stream


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().ember_status_string(status).decode()
        raise RuntimeError(f"emberserve_amd: {what} failed: {msg} (status {status})")


def read_errors(clear: bool = True) -> int:
    """The current device's index-error word (EMBER_ERR_* bits). Synchronises."""
    flags = ctypes.c_uint32(0)
    check(load().ember_read_errors(ctypes.byref(flags), 1 if clear else 0), "ember_read_errors")
    return flags.value
