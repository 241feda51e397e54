"""ctypes binding of ``libasrattn.so``, the C ABI declared in ``include/asrattn.h``.

The library is loaded after ``import torch`` on purpose: PyTorch-ROCm ships its
own HIP runtime (SONAME ``libamdhip64.so.7``), and the dynamic loader resolves
the library's dependency to that already-loaded copy, so kernels launch on the
very streams torch hands out.  Loading the library first would map a second
HIP runtime into the process.

There is no fallback: when the library is missing or fails to load, every
call raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the library; see above)

LIBRARY = Path(__file__).resolve().with_name("libasrattn.so")
ABI_VERSION = 11

# enum asrattn_status / asrattn_dtype / asrattn_causal
OK = 0
ERR_INVALID = 1
ERR_UNSUPPORTED = 2
ERR_HIP = 3
ERR_WORKSPACE = 4
F32 = 0
BF16 = 1
CAUSAL_NONE = 0
CAUSAL_TOP_LEFT = 1
CAUSAL_BOTTOM_RIGHT = 2
FWD_FORCE_VALU = 1
FWD_ZERO_PADDED_ROWS = 2

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_ptr = ctypes.c_void_p


class FwdParams(ctypes.Structure):
    """``asrattn_fwd_params``."""

    _fields_ = [
        ("q", _ptr),
        ("k", _ptr),
        ("v", _ptr),
        ("out", _ptr),
        ("q_batch_stride", _i64),
        ("q_token_stride", _i64),
        ("q_head_stride", _i64),
        ("k_batch_stride", _i64),
        ("k_token_stride", _i64),
        ("k_head_stride", _i64),
        ("v_batch_stride", _i64),
        ("v_token_stride", _i64),
        ("v_head_stride", _i64),
        ("o_batch_stride", _i64),
        ("o_token_stride", _i64),
        ("o_head_stride", _i64),
        ("cu_seqlens_q", _ptr),
        ("cu_seqlens_k", _ptr),
        ("seqused_k", _ptr),
        ("batch", _i32),
        ("heads_q", _i32),
        ("heads_kv", _i32),
        ("head_dim", _i32),
        ("max_len_q", _i32),
        ("max_len_k", _i32),
        ("causal", _i32),
        ("dtype", _i32),
        ("scale", ctypes.c_float),
        ("flags", _i32),
        ("window", _i32),
    ]


class DecodeParams(ctypes.Structure):
    """``asrattn_decode_params``."""

    _fields_ = [
        ("q", _ptr),
        ("k", _ptr),
        ("v", _ptr),
        ("out", _ptr),
        ("q_batch_stride", _i64),
        ("q_head_stride", _i64),
        ("k_batch_stride", _i64),
        ("k_token_stride", _i64),
        ("k_head_stride", _i64),
        ("v_batch_stride", _i64),
        ("v_token_stride", _i64),
        ("v_head_stride", _i64),
        ("o_batch_stride", _i64),
        ("o_head_stride", _i64),
        ("seqused_k", _ptr),
        ("positions", _ptr),
        ("batch", _i32),
        ("heads_q", _i32),
        ("heads_kv", _i32),
        ("head_dim", _i32),
        ("max_len_k", _i32),
        ("num_splits", _i32),
        ("dtype", _i32),
        ("scale", ctypes.c_float),
        ("window", _i32),
    ]


class AppendParams(ctypes.Structure):
    """``asrattn_append_params``."""

    _fields_ = [
        ("k_new", _ptr),
        ("v_new", _ptr),
        ("kn_batch_stride", _i64),
        ("kn_head_stride", _i64),
        ("vn_batch_stride", _i64),
        ("vn_head_stride", _i64),
        ("q_norm", _ptr),
        ("k_norm", _ptr),
        ("eps", ctypes.c_float),
        ("cos", _ptr),
        ("sin", _ptr),
        ("rope_batch_stride", _i64),
        ("v_norm", _i32),
    ]


class FsmnParams(ctypes.Structure):
    """``asrattn_fsmn_params``."""

    _fields_ = [
        ("weight", _ptr),
        ("bias", _ptr),
        ("memory", _ptr),
        ("m_batch_stride", _i64),
        ("m_token_stride", _i64),
        ("kernel_size", _i32),
    ]


class PagedKV(ctypes.Structure):
    """``asrattn_paged_kv``."""

    _fields_ = [
        ("block_table", _ptr),
        ("bt_stride", _i64),
        ("page_size", _i32),
        ("num_pages", _i32),
        ("k_page_stride", _i64),
        ("v_page_stride", _i64),
    ]


class LocalParams(ctypes.Structure):
    """``asrattn_local_params``."""

    _fields_ = [
        ("q", _ptr),
        ("k", _ptr),
        ("v", _ptr),
        ("rel", _ptr),
        ("out", _ptr),
        *[(f"{t}_{axis}_stride", _i64) for t in ("q", "k", "v", "o") for axis in ("batch", "token", "head")],
        ("rel_position_stride", _i64),
        ("rel_head_stride", _i64),
        ("lengths", _ptr),
        ("batch", _i32),
        ("tokens", _i32),
        ("heads", _i32),
        ("head_dim", _i32),
        ("chunk", _i32),
        ("past", _i32),
        ("future", _i32),
        ("rel_positions", _i32),
        ("softcap", ctypes.c_float),
        ("invalid", ctypes.c_float),
    ]


# Every symbol include/asrattn.h declares, with (restype, argtypes).
SIGNATURES = {
    "asrattn_fwd": (ctypes.c_int, [ctypes.POINTER(FwdParams), _ptr]),
    "asrattn_fwd_fsmn": (ctypes.c_int, [ctypes.POINTER(FwdParams), ctypes.POINTER(FsmnParams), _ptr]),
    "asrattn_decode": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeParams), _ptr, ctypes.c_size_t, _ptr],
    ),
    "asrattn_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(DecodeParams), _ptr]),
    "asrattn_decode_append": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeParams), ctypes.POINTER(AppendParams), _ptr, ctypes.c_size_t, _ptr],
    ),
    "asrattn_decode_paged": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeParams), ctypes.POINTER(AppendParams), ctypes.POINTER(PagedKV), _ptr,
         ctypes.c_size_t, _ptr],
    ),
    "asrattn_local": (ctypes.c_int, [ctypes.POINTER(LocalParams), _ptr]),
    "asrattn_choose": (
        ctypes.c_int,
        [_ptr, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _ptr, _ptr, _ptr, _ptr, ctypes.c_size_t, _ptr],
    ),
    "asrattn_choose_workspace_size": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64]),
    "asrattn_decode_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(DecodeParams)]),
    "asrattn_decode_num_splits": (ctypes.c_int, [ctypes.POINTER(DecodeParams)]),
    "asrattn_last_error": (ctypes.c_char_p, []),
    "asrattn_abi_version": (ctypes.c_int, []),
}


class AttentionError(RuntimeError):
    """A nonzero status from the C ABI; ``status`` is the ``asrattn_status`` code."""

    def __init__(self, status: int, message: str) -> None:
        super().__init__(message)
        self.status = status


_lock = threading.Lock()
_handle: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The loaded library (loaded once per process)."""
    global _handle
    if _handle is not None:
        return _handle
    with _lock:
        if _handle is None:
            if not LIBRARY.is_file():
                raise RuntimeError(
                    f"{LIBRARY} is not built; run `python -m asrback_amd.build` "
                    "(there is no fallback path for the attention kernels)"
                )
            handle = ctypes.CDLL(str(LIBRARY))
            for name, (restype, argtypes) in SIGNATURES.items():
                function = getattr(handle, name)
                function.restype = restype
                function.argtypes = argtypes
            version = handle.asrattn_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(
                    f"{LIBRARY} has ABI version {version}, expected {ABI_VERSION}; rebuild it"
                )
            _handle = handle
    return _handle


def check(status: int, what: str) -> None:
    """Raise :class:`AttentionError` for a nonzero ``status``."""
    if status != OK:
        message = load().asrattn_last_error().decode("utf-8", "replace")
        raise AttentionError(status, f"{what} failed (status {status}): {message}")
