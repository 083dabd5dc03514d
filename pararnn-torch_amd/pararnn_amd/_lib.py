"""ctypes binding of ``libpararnn_amd.so`` (the C ABI in include/pararnn_amd.h).

The library is loaded lazily, after torch, so it shares torch's HIP runtime
(both resolve the SONAME ``libamdhip64.so.7``).  There is no fallback: when
the library is missing every fused entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

from pararnn_amd._build import LIB_PATH

PRNN_F32 = 0
PRNN_BF16 = 1
PRNN_F16 = 2
PRNN_OK = 0
PRNN_ERR_VALUE = 1
PRNN_ERR_TYPE = 2
PRNN_ERR_RUNTIME = 3
ABI_VERSION = 10

# name -> (restype, argtypes); mirrors include/pararnn_amd.h
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.c_size_t
SIGNATURES: dict[str, tuple] = {
    "prnn_abi_version": (_I, []),
    "prnn_last_error": (ctypes.c_char_p, []),
    "prnn_set_deterministic": (None, [_I]),
    "prnn_deterministic": (_I, []),
    "prnn_set_kernel_timing": (None, [_I]),
    "prnn_set_spin_limit": (None, [_I]),
    "prnn_slstm_lookback_status": (_I, [_P, ctypes.POINTER(ctypes.c_int), _P]),
    "prnn_last_kernel_ms": (ctypes.c_float, []),
    "prnn_slstm_init_workspace_size": (_S, [_I, _I, _I, _I, _I]),
    "prnn_slstm_init": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _P, _S, _P]),
    "prnn_slstm_newton_workspace_size": (_S, [_I, _I, _I, _I, _I]),
    "prnn_slstm_newton": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _F, _I, _P, _S, _P]),
    "prnn_gru_head_newton_workspace_size": (_S, [_I, _I, _I, _I, _I, _I]),
    "prnn_gru_head_newton": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _P, _S, _P],
    ),
    "prnn_slstm_backward_workspace_size": (_S, [_I, _I, _I, _I]),
    "prnn_slstm_backward": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _I, _P, _S, _P],
    ),
    "prnn_slstm_init_ex": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _P, _S, _I, _P]),
    "prnn_slstm_newton_ex": (
        _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _F, _I, _P, _S, _I, _P]),
    "prnn_slstm_backward_ex": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _I, _P, _S, _I, _P],
    ),
    "prnn_gru_head_backward_workspace_size": (_S, [_I, _I, _I, _I, _I]),
    "prnn_gru_head_backward": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _S, _P],
    ),
    "prnn_slstm_newton_noalloc_max_bytes": (_S, []),
    "prnn_slstm_newton_noalloc": (
        _I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _F, _I, _P]),
    "prnn_slstm_newton_step": (
        _I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _F, _F, _I, _P, _S, _I, _P]),
    "prnn_slstm_newton_eager": (
        _I, [_P, _P, _P, _P, _P, _I, _I, _I, _F, _F, _I, _P, _S, _I, _P]),
    "prnn_slstm_newton_eager_packed": (
        _I, [_P, _P, _P, _P, _P, _I, _I, _F, _F, _I, _P, _I, _P, _P, _S, _I, _P]),
    "prnn_slstm_init_packed_workspace_size": (_S, [_I, _I, _I, _I]),
    "prnn_slstm_init_packed": (
        _I, [_P, _P, _P, _P, _I, _I, _I, _F, _I, _P, _I, _P, _P, _S, _I, _P]),
    "prnn_slstm_newton_packed_workspace_size": (_S, [_I, _I, _I, _I]),
    "prnn_slstm_newton_packed": (
        _I, [_P, _P, _P, _P, _P, _I, _I, _I, _F, _F, _I, _P, _I, _P, _P, _S, _I, _P]),
    "prnn_slstm_newton_step_packed": (
        _I, [_P, _P, _P, _P, _I, _P, _I, _I, _F, _F, _I, _P, _I, _P, _P, _S, _I, _P]),
    "prnn_slstm_backward_packed": (
        _I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _I, _P, _I, _P, _S, _I, _P]),
    "prnn_gru_head_newton_packed_workspace_size": (_S, [_I, _I, _I, _I, _I]),
    "prnn_gru_head_newton_packed": (
        _I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _P, _I, _P, _P, _S, _P]),
    "prnn_gru_head_backward_packed_workspace_size": (_S, [_I, _I, _I, _I]),
    "prnn_gru_head_backward_packed": (
        _I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _S, _P]),
    "prnn_gru_wide_walk": (
        _I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _P, _I, _P]),
    "prnn_gru_wide_reverse": (
        _I, [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _P]),
    "prnn_gru_wide_gates": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "prnn_gru_wide_newton_workspace_size": (_S, [_I, _I, _I, _I, _I]),
    "prnn_gru_wide_newton": (
        _I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _P, _I, _P, _S, _I, _P]),
    "prnn_slstm_decode": (_I, [_P, _P, _P, _P, _P, _I, _I, _F, _F, _I, _I, _P]),
    "prnn_gru_decode": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _I, _I, _P]),
}

_lock = threading.Lock()
_handle: ctypes.CDLL | None = None


def lib_path() -> str:
    return os.environ.get("PARARNN_AMD_LIB", LIB_PATH)


def load() -> ctypes.CDLL:
    """Load (once) and type the C ABI.  Raises RuntimeError if it is missing."""
    global _handle
    if _handle is not None:
        return _handle
    with _lock:
        if _handle is not None:
            return _handle
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"pararnn_amd HIP library not found at {path}; build it with "
                "`python -m pararnn_amd._build` (or __graft_entry__.build()). "
                "The fused Newton path has no CPU fallback."
            )
        import torch  # noqa: F401  -- load torch's HIP runtime first

        handle = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.prnn_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{path}: ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        _handle = handle
        return handle


def sync_deterministic(handle: ctypes.CDLL) -> None:
    """Mirror ``torch.are_deterministic_algorithms_enabled()`` into the
    library's deterministic look-back switch (the reference keys its own
    determinism checks on the same torch flag, pararnn/determinism.py:41-45)."""
    import torch

    on = int(bool(torch.are_deterministic_algorithms_enabled()))
    if handle.prnn_deterministic() != on:
        handle.prnn_set_deterministic(on)


def check(rc: int, what: str) -> None:
    """Map a C return code to the reference's exception types."""
    if rc == PRNN_OK:
        return
    msg = f"{what}: {load().prnn_last_error().decode(errors='replace')}"
    if rc == PRNN_ERR_VALUE:
        raise ValueError(msg)
    if rc == PRNN_ERR_TYPE:
        raise TypeError(msg)
    raise RuntimeError(msg)
