"""ctypes binding of libmkv.so, the C ABI declared in include/mkv.h.

The library is loaded lazily on first use from mkv/libmkv.so, or from the
path in the MKV_LIBRARY environment variable.  Loading never falls back to
anything: if the shared object is missing or has the wrong ABI version, every
operator raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmkv.so"
ABI_VERSION = 5

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_FP8E4M3 = 3
DTYPE_I8 = 4
SCALE_PER_TENSOR = 0
SCALE_PER_TOKEN_HEAD = 1
APPEND_CALIBRATE_SENTINEL = 1
NOALLOC_SCRATCH_BYTES = 32 << 20  # MKV_NOALLOC_SCRATCH_BYTES
INDEX_I32 = 0
INDEX_I64 = 1
DECODE_WORKGROUP = -1  # MKV_DECODE_WORKGROUP: split_tokens value of the workgroup route
DECODE_STREAM = -2  # MKV_DECODE_STREAM: split_tokens value of the stream-K route
# mkv_paged_decode_route results
ROUTE_STREAM = 0
ROUTE_SPLIT = 1
ROUTE_WORKGROUP = 2

# name -> (restype, argtypes); mirrors include/mkv.h one to one.
SIGNATURES: dict[str, tuple] = {
    "mkv_abi_version": (c_int, []),
    "mkv_status_string": (ctypes.c_char_p, [c_int]),
    "mkv_kv_append": (c_int, [
        c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64,
        c_int, c_int, c_int, c_int64, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p]),
    "mkv_kv_append_per_token_head": (c_int, [
        c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
        c_int64, c_int, c_int, c_int, c_int64, c_int, c_int, c_void_p]),
    "mkv_fp8_calibrate_workspace_size": (c_size_t, []),
    "mkv_fp8_calibrate_per_tensor": (c_int, [
        c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int, c_int, c_void_p, c_void_p,
        c_void_p, c_void_p]),
    "mkv_paged_decode_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "mkv_paged_decode_split_tokens": (c_int, [c_int, c_int, c_int, c_int, c_int]),
    "mkv_paged_decode_route": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "mkv_paged_decode": (c_int, [
        c_void_p, c_int64, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_int, c_int64,
        c_void_p, c_void_p, c_int, c_void_p, c_int64, c_int, c_void_p, c_int, c_int, c_int, c_int,
        c_int, c_int, c_float, c_int, c_void_p, c_size_t, c_void_p]),
    "mkv_paged_decode_noalloc": (c_int, [
        c_void_p, c_int64, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_int, c_int64,
        c_void_p, c_void_p, c_int, c_void_p, c_int64, c_int, c_void_p, c_int, c_int, c_int, c_int,
        c_int, c_int, c_float, c_int, c_void_p]),
    "mkv_paged_prefill_workspace_size": (c_size_t, [c_int, c_int64, c_int, c_int]),
    "mkv_paged_prefill": (c_int, [
        c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p, c_int,
        c_void_p, c_int64, c_int, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int64,
        c_int, c_int, c_int, c_int, c_float, c_void_p, c_size_t, c_void_p]),
    "mkv_flash_prefill_workspace_size": (c_size_t, [c_int, c_int64, c_int, c_int]),
    "mkv_flash_prefill": (c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int64, c_int, c_int,
        c_int, c_float, c_void_p, c_size_t, c_void_p]),
    "mkv_qkv_norm_rope_append": (c_int, [
        c_void_p, c_int64, c_int, c_int64, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_float,
        c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int,
        c_int, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int, c_void_p]),
    "mkv_qkv_norm_rope_append_decode": (c_int, [
        c_void_p, c_int64, c_int, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_int, c_float,
        c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_void_p,
        c_void_p, c_int, c_void_p, c_int, c_void_p, c_int64, c_int, c_void_p, c_int, c_int,
        c_int, c_int, c_int, c_int, c_float, c_void_p]),
    "mkv_decode_metadata": (c_int, [
        c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int64, c_int, c_int, c_int,
        c_void_p]),
    "mkv_rmsnorm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_float, c_int,
                            c_void_p]),
    "mkv_silu_mul": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_void_p]),
    "mkv_gather_kv": (c_int, [
        c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64, c_int, c_void_p, c_int, c_int,
        c_int, c_int, c_int, c_int, c_void_p]),
    "mkv_stream_read_probe_sink_words": (c_size_t, [c_int]),
    "mkv_stream_read_probe": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_void_p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class MkvError(RuntimeError):
    """A libmkv entry point returned a non-zero status."""

    def __init__(self, func: str, status: int, message: str):
        super().__init__(f"{func} failed with status {status}: {message}")
        self.func = func
        self.status = status


def load(path: str | Path | None = None) -> ctypes.CDLL:
    """Load libmkv.so once, bind every entry point and check the ABI version."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else Path(os.environ.get("MKV_LIBRARY", LIB_PATH))
        if not p.exists():
            raise RuntimeError(
                f"libmkv.so not found at {p}; build it first (python -m mkv.build or "
                "__graft_entry__.build()). There is no fallback implementation.")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        got = lib.mkv_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"libmkv ABI version {got} != expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Invoke an int-returning entry point and raise MkvError on failure."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.mkv_status_string(status).decode()
        raise MkvError(name, status, msg)


def query(name: str, *args):
    """Invoke a size/info entry point and return its value."""
    return getattr(load(), name)(*args)
