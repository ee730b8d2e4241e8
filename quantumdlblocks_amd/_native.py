"""ctypes binding of libqdl_flash_born.so (C ABI in include/qdl_flash_born.h).

The library links ``libamdhip64.so.7``; torch is imported before the library
is opened so that the dynamic linker binds it to the HIP runtime torch already
loaded (one runtime per process, so torch's streams and allocations are valid
in the library).
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_NAME = "libqdl_flash_born.so"
LIB_PATH = Path(__file__).resolve().parent / "lib" / LIB_NAME

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

# Size of the fixed device array qdl_flash_born_bwd_noalloc uses
# (QDL_BORN_BWD_SCRATCH_BYTES in the header).
BWD_SCRATCH_BYTES = 16 * 1024 * 1024

# Every symbol the header declares (checked by tests/test_native_abi.py).
EXPORTED_SYMBOLS = (
    "qdl_flash_born_version",
    "qdl_flash_born_strerror",
    "qdl_flash_born_supported",
    "qdl_flash_born_fwd",
    "qdl_flash_born_bwd_workspace_size",
    "qdl_flash_born_bwd",
    "qdl_flash_born_bwd_noalloc",
    "qdl_flash_purified_born_fwd",
    "qdl_flash_purified_born_bwd_workspace_size",
    "qdl_flash_purified_born_bwd",
    "qdl_flash_born_qk_prologue_fwd",
    "qdl_flash_born_qk_prologue_bwd",
    "qdl_flash_born_fwd_qk_prologue",
)


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, failed to load, or returned an error."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_dbl = ctypes.c_double


def _bind(lib: ctypes.CDLL) -> None:
    lib.qdl_flash_born_version.restype = ctypes.c_char_p
    lib.qdl_flash_born_version.argtypes = []
    lib.qdl_flash_born_strerror.restype = ctypes.c_char_p
    lib.qdl_flash_born_strerror.argtypes = [_int]
    lib.qdl_flash_born_supported.restype = _int
    lib.qdl_flash_born_supported.argtypes = [_int, _i64]
    lib.qdl_flash_born_fwd.restype = _int
    lib.qdl_flash_born_fwd.argtypes = [
        _int, _i64, _i64, _i64, _i64,      # dtype, B, H, T, D
        _ptr, _ptr, _ptr, _ptr, _ptr,      # q, k, v, out, z
        _ptr, _i64, _ptr,                  # scale, n_scale, doc_ids
        _int, _i64, _dbl, _ptr,            # is_causal, window_size, eps, stream
    ]
    lib.qdl_flash_born_bwd_workspace_size.restype = _i64
    lib.qdl_flash_born_bwd_workspace_size.argtypes = [_int, _i64, _i64, _i64, _i64, _i64]
    lib.qdl_flash_born_bwd.restype = _int
    lib.qdl_flash_born_bwd.argtypes = [
        _int, _i64, _i64, _i64, _i64,      # dtype, B, H, T, D
        _ptr, _ptr, _ptr, _ptr, _ptr,      # q, k, v, out, dout
        _ptr, _ptr, _i64, _ptr,            # z, scale, n_scale, doc_ids
        _int, _i64, _dbl,                  # is_causal, window_size, eps
        _ptr, _ptr, _ptr, _ptr,            # dq, dk, dv, dscale
        _ptr, _i64, _ptr,                  # workspace, workspace_bytes, stream
    ]
    lib.qdl_flash_born_bwd_noalloc.restype = _int
    lib.qdl_flash_born_bwd_noalloc.argtypes = [
        _int, _i64, _i64, _i64, _i64,      # dtype, B, H, T, D
        _ptr, _ptr, _ptr, _ptr, _ptr,      # q, k, v, out, dout
        _ptr, _ptr, _i64, _ptr,            # z, scale, n_scale, doc_ids
        _int, _i64, _dbl,                  # is_causal, window_size, eps
        _ptr, _ptr, _ptr, _ptr, _ptr,      # dq, dk, dv, dscale, stream
    ]
    lib.qdl_flash_purified_born_fwd.restype = _int
    lib.qdl_flash_purified_born_fwd.argtypes = [
        _int, _i64, _i64, _i64, _i64,      # dtype, B, H, T, D
        _ptr, _ptr, _ptr, _ptr, _ptr,      # q, k, v, out (fp32), z
        _ptr, _i64, _ptr, _i64, _dbl,      # scale, n_scale, tau, n_tau, eps_base
        _ptr, _int, _i64, _dbl, _ptr,      # doc_ids, is_causal, window_size, eps, stream
    ]
    lib.qdl_flash_purified_born_bwd_workspace_size.restype = _i64
    lib.qdl_flash_purified_born_bwd_workspace_size.argtypes = [_int, _i64, _i64, _i64, _i64]
    lib.qdl_flash_purified_born_bwd.restype = _int
    lib.qdl_flash_purified_born_bwd.argtypes = [
        _int, _i64, _i64, _i64, _i64,      # dtype, B, H, T, D
        _ptr, _ptr, _ptr, _ptr, _ptr,      # q, k, v, out (fp32), dout
        _ptr, _ptr, _i64, _ptr, _i64,      # z, scale, n_scale, tau, n_tau
        _dbl, _ptr, _int, _i64,            # eps_base, doc_ids, is_causal, window_size
        _ptr, _ptr, _ptr, _ptr, _ptr,      # dq, dk, dv, dscale, dtau
        _ptr, _i64, _ptr,                  # workspace, workspace_bytes, stream
    ]
    lib.qdl_flash_born_qk_prologue_fwd.restype = _int
    lib.qdl_flash_born_qk_prologue_fwd.argtypes = [
        _int, _i64, _i64, _i64, _i64,      # dtype, B, H, T, D
        _ptr, _ptr, _ptr, _ptr,            # q, q_strides, k, k_strides
        _ptr, _ptr, _i64, _i64, _dbl,      # cos, sin, n_freq, table_ld, eps
        _ptr, _ptr, _ptr, _ptr, _ptr,      # q_out, k_out, q_rinv, k_rinv, stream
    ]
    lib.qdl_flash_born_fwd_qk_prologue.restype = _int
    lib.qdl_flash_born_fwd_qk_prologue.argtypes = [
        _int, _i64, _i64, _i64, _i64,      # dtype, B, H, T, D
        _ptr, _ptr, _ptr, _ptr, _ptr,      # q, q_strides, k, k_strides, v
        _ptr, _ptr, _i64, _i64, _dbl,      # cos, sin, n_freq, table_ld, norm_eps
        _ptr, _i64, _ptr, _int, _i64, _dbl,  # scale, n_scale, doc_ids, is_causal, window_size, eps
        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,  # out, z, q_out, k_out, q_rinv, k_rinv
        _ptr,                              # stream
    ]
    lib.qdl_flash_born_qk_prologue_bwd.restype = _int
    lib.qdl_flash_born_qk_prologue_bwd.argtypes = [
        _int, _i64, _i64, _i64, _i64,      # dtype, B, H, T, D
        _ptr, _ptr, _ptr, _ptr, _ptr, _ptr,  # dq_out, dk_out, q_out, k_out, q_rinv, k_rinv
        _ptr, _ptr, _i64, _i64,            # cos, sin, n_freq, table_ld
        _ptr, _ptr, _ptr, _ptr, _ptr,      # dq, dq_strides, dk, dk_strides, stream
    ]


def load() -> ctypes.CDLL:
    """Open (once) and return the library; raise NativeLibraryError otherwise."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (bind to torch's HIP runtime, see module doc)

        path = Path(os.environ.get("QDL_FLASH_BORN_LIB", LIB_PATH))
        if not path.exists():
            _load_error = (
                f"{path} not found; build it with `python -m quantumdlblocks_amd.build`"
            )
            raise NativeLibraryError(_load_error)
        try:
            lib = ctypes.CDLL(str(path))
            _bind(lib)
        except (OSError, AttributeError) as exc:
            _load_error = f"failed to load {path}: {exc}"
            raise NativeLibraryError(_load_error) from exc
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except NativeLibraryError:
        return False


def library_path() -> Path | None:
    return Path(os.environ.get("QDL_FLASH_BORN_LIB", LIB_PATH)) if _lib is not None else None


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().qdl_flash_born_strerror(int(rc)).decode()
        raise NativeLibraryError(f"{what} failed (code {rc}): {msg}")
