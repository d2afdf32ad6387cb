"""ctypes binding of libaicas_decode.so (the C ABI declared in include/aicas_decode.h).

torch is imported before the library is loaded: torch ships its own HIP runtime with the soname
``libamdhip64.so.7``, and the dynamic linker then resolves the library's HIP dependency to that same
runtime, so torch's streams and device pointers are valid in every call.

There is no fallback: if the library is missing or fails to load, :func:`lib` raises :class:`AicasError`.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the library load, see above)

LIB_NAME = "libaicas_decode.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

ABI_VERSION = 7

DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP8_E4M3 = 2

OK = 0
ERR_INVALID = 1
ERR_UNSUPPORTED = 2
ERR_WORKSPACE = 3
ERR_LAUNCH = 4

STATUS_LEN_CLAMPED = 1
STATUS_BLOCK_OUT_OF_RANGE = 2
STATUS_APPEND_OVERFLOW = 4
STATUS_OUT_OF_BLOCKS = 8
STATUS_NONFINITE_ROW = 16

# Entry points declared in include/aicas_decode.h, in declaration order.
EXPORTED_SYMBOLS = (
    "aicas_kv_append",
    "aicas_kv_gather",
    "aicas_decode_plan",
    "aicas_decode_attention",
    "aicas_decode_attention_append",
    "aicas_decode_attention_append_noalloc",
    "aicas_decode_attention_append_qk",
    "aicas_block_pool_init",
    "aicas_block_alloc",
    "aicas_block_free",
    "aicas_last_error",
    "aicas_abi_version",
)


class AicasError(RuntimeError):
    """A C-ABI call returned a nonzero status; the message is the library's aicas_last_error()."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[aicas {code}] {message}")
        self.code = code


class KVCacheDesc(ctypes.Structure):
    """Mirror of ``aicas_kv_cache_t``."""

    _fields_ = [
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p),
        ("block_table_stride", ctypes.c_int64),
        ("num_blocks", ctypes.c_int64),
        ("stride_blk", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_t", ctypes.c_int64),
        ("scale_stride_blk", ctypes.c_int64),
        ("scale_stride_h", ctypes.c_int64),
        ("page_size", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
    ]


class BlockPoolDesc(ctypes.Structure):
    """aicas_block_pool_t (include/aicas_decode.h)."""

    _fields_ = [("free_blocks", ctypes.c_void_p), ("free_count", ctypes.c_void_p), ("num_blocks", ctypes.c_int32)]


class QKPrologueDesc(ctypes.Structure):
    """Mirror of ``aicas_qk_prologue_t`` (include/aicas_decode.h)."""

    _fields_ = [
        ("q_norm_weight", ctypes.c_void_p),
        ("k_norm_weight", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("cos_stride_b", ctypes.c_int64),
        ("sin_stride_b", ctypes.c_int64),
        ("q_out", ctypes.c_void_p),
        ("q_out_stride_b", ctypes.c_int64),
        ("q_out_stride_h", ctypes.c_int64),
    ]


_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_P = ctypes.c_void_p
_SIZE = ctypes.c_size_t

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def _bind(handle: ctypes.CDLL) -> ctypes.CDLL:
    handle.aicas_last_error.restype = ctypes.c_char_p
    handle.aicas_last_error.argtypes = []
    handle.aicas_abi_version.restype = _I32
    handle.aicas_abi_version.argtypes = []
    handle.aicas_kv_append.restype = ctypes.c_int
    handle.aicas_kv_append.argtypes = [
        ctypes.POINTER(KVCacheDesc), _I32,
        _P, _I64, _I64, _I64,
        _P, _I64, _I64, _I64,
        _P, _P, _P,
        _I32, _I32, _I32, _I32,
        _P,
    ]
    handle.aicas_kv_gather.restype = ctypes.c_int
    handle.aicas_kv_gather.argtypes = [
        ctypes.POINTER(KVCacheDesc), _P, _I32, _I32, _I32, _I32,
        _P, _P, _I64, _I64, _I64, _I32, _P,
        _P,
    ]
    handle.aicas_decode_plan.restype = ctypes.c_int
    handle.aicas_decode_plan.argtypes = [
        _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
        ctypes.POINTER(_I32), ctypes.POINTER(_I32), ctypes.POINTER(_SIZE),
    ]
    handle.aicas_decode_attention.restype = ctypes.c_int
    handle.aicas_decode_attention.argtypes = [
        ctypes.POINTER(KVCacheDesc), _I32, _P, _I64, _I64,
        _P, _I64, _I64,
        _P, _I32, _I32, _I32, _I32,
        _I32, _I32, _I32, ctypes.c_float,
        _I32, _P, _SIZE, _P,
        _P,
    ]
    handle.aicas_decode_attention_append.restype = ctypes.c_int
    handle.aicas_decode_attention_append.argtypes = [
        ctypes.POINTER(KVCacheDesc), _I32, _P, _I64, _I64,
        _P, _I64, _I64, _P, _I64, _I64,
        _P, _I64, _I64,
        _P, _P, _I32, _I32,
        _I32, _I32, _I32, _I32, ctypes.c_float,
        _I32, _P, _SIZE, _P,
        _P,
    ]
    handle.aicas_decode_attention_append_noalloc.restype = ctypes.c_int
    # aicas_decode_attention_append's arguments without (workspace, workspace_bytes)
    handle.aicas_decode_attention_append_noalloc.argtypes = \
        handle.aicas_decode_attention_append.argtypes[:-4] + handle.aicas_decode_attention_append.argtypes[-2:]
    handle.aicas_decode_attention_append_qk.restype = ctypes.c_int
    handle.aicas_decode_attention_append_qk.argtypes = [ctypes.POINTER(KVCacheDesc), ctypes.POINTER(QKPrologueDesc)] + \
        handle.aicas_decode_attention_append.argtypes[1:]
    handle.aicas_block_pool_init.restype = ctypes.c_int
    handle.aicas_block_pool_init.argtypes = [ctypes.POINTER(BlockPoolDesc), _P]
    handle.aicas_block_alloc.restype = ctypes.c_int
    handle.aicas_block_alloc.argtypes = [ctypes.POINTER(BlockPoolDesc), _P, _I64, _I32, _P, _I32, _I32, _I32, _P, _P]
    handle.aicas_block_free.restype = ctypes.c_int
    handle.aicas_block_free.argtypes = [ctypes.POINTER(BlockPoolDesc), _P, _I64, _I32, _P, _P, _I32, _P, _P]
    return handle


def lib() -> ctypes.CDLL:
    """Load (once) and return the bound library; raise AicasError if it is not built or does not load."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise AicasError(
                    ERR_INVALID,
                    f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `python -m aicas_amd.build` first",
                )
            try:
                handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
            except OSError as exc:
                raise AicasError(ERR_INVALID, f"failed to load {LIB_PATH}: {exc}") from exc
            _bind(handle)
            version = handle.aicas_abi_version()
            if version != ABI_VERSION:
                raise AicasError(ERR_INVALID, f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}")
            _lib = handle
    return _lib


def check(code: int) -> None:
    """Raise AicasError carrying aicas_last_error() if a C-ABI call failed."""
    if code != OK:
        msg = lib().aicas_last_error().decode("utf-8", "replace")
        raise AicasError(code, msg)
