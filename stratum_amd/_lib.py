"""ctypes binding of libstratum_nf4.so (the C ABI declared in include/stratum_nf4.h).

torch is imported first on purpose: torch ships its own HIP runtime with the
same SONAME (libamdhip64.so.7), so loading the library after torch binds it to
that runtime and torch's streams and device pointers are valid handles for it.
There is no fallback: if the library is missing every call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded before the HIP library, see above)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libstratum_nf4.so")

STM_OK = 0
STM_ERR_INVALID = -1
STM_ERR_UNSUPPORTED = -2
STM_ERR_HIP = -3

STM_F16, STM_BF16, STM_F32 = 0, 1, 2
STM_NF4_ARGMIN, STM_NF4_THRESHOLD = 0, 1

ABI_VERSION = 5

# (name, argtypes) of every entry point of include/stratum_nf4.h
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
SIGNATURES = {
    "stm_nf4_abi_version": ([], _I),
    "stm_last_error": ([], ctypes.c_char_p),
    "stm_nf4_quantize": ([_P, _I, _I64, _I, _I, _P, _P, _P], _I),
    "stm_nf4_dequantize": ([_P, _P, _I64, _I, _P, _I, _P], _I),
    "stm_nf4_gemm_fwd": ([_P, _P, _P, _P, _P, _P, _I, _P, _I64, _I64, _I64, _I, _I, _P, _I64, _P], _I),
    "stm_nf4_gemm_bwd_dx": ([_P, _P, _P, _P, _P, _I, _P, _I64, _I64, _I64, _I, _I, _P, _I64, _P], _I),
    "stm_nf4_gemm_workspace_bytes": ([_I64, _I64, _I64, _I], _I64),
    "stm_nf4_gemm_fwd_noalloc": ([_P, _P, _P, _P, _P, _P, _I, _P, _I64, _I64, _I64, _I, _I, _P], _I),
    "stm_nf4_gemm_set_tile": ([_I], _I),
    "stm_nf4_grouped_gemm_fwd": ([_P, _P, _P, _P, _P, _I, _I64, _P, _I64, _I64, _I, _I, _P], _I),
    "stm_nf4_grouped_tile_rows": ([_P, _I], _I),
    "stm_nf4_quantize_many": ([_I, _P, _P, _I, _I, _I, _P, _P, _P], _I),
    "stm_nf4_dequantize_many": ([_I, _P, _P, _P, _I, _P, _I, _P], _I),
    "stm_nf4_grouped_gemm_bwd_dx": ([_P, _P, _P, _P, _P, _I, _I64, _P, _I64, _I64, _I, _I, _P], _I),
    "stm_swiglu_fwd": ([_P, _P, _I64, _I64, _I, _P], _I),
    "stm_swiglu_bwd": ([_P, _P, _P, _I64, _I64, _I, _P], _I),
    "stm_lora_workspace_bytes": ([_I64, _I64, _I, _I], _I64),
    "stm_lora_down": ([_P, _P, _P, _I64, _I64, _I, ctypes.c_float, _I, _P, _I64, _P], _I),
    "stm_lora_dy": ([_P, _P, _P, _P, _P, _I64, _I64, _I, ctypes.c_float, _I, _P, _I64, _P], _I),
    "stm_lora_da": ([_P, _P, _P, _I64, _I64, _I, _I, _P, _I64, _P], _I),
    "stm_nf4_decision_boundaries": ([_I, _P], _I),
    "stm_nf4_cell_table": ([_I, _P, _P], _I),
}


class NF4LibraryError(RuntimeError):
    """The HIP library is missing or failed to load."""


class NF4KernelError(RuntimeError):
    """A library entry point returned a non-zero status."""

    def __init__(self, what: str, code: int, reason: str):
        super().__init__(f"{what} failed (status {code}): {reason}")
        self.code = code
        self.reason = reason


_lib = None
_lock = threading.Lock()


def lib():
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NF4LibraryError(
                    f"{LIB_PATH} is not built; build it with `python -m stratum_amd._build` "
                    "(or __graft_entry__.build())")
            try:
                L = ctypes.CDLL(LIB_PATH)
            except OSError as exc:
                raise NF4LibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = res
            if L.stm_nf4_abi_version() != ABI_VERSION:
                raise NF4LibraryError(f"ABI version {L.stm_nf4_abi_version()} != {ABI_VERSION}")
            _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != STM_OK:
        reason = (lib().stm_last_error() or b"").decode(errors="replace")
        if rc in (STM_ERR_INVALID, STM_ERR_UNSUPPORTED):
            raise ValueError(f"{what}: {reason} (status {rc})")
        raise NF4KernelError(what, rc, reason)


def dtype_tag(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return STM_F16
    if dtype == torch.bfloat16:
        return STM_BF16
    if dtype == torch.float32:
        return STM_F32
    raise ValueError(f"unsupported dtype {dtype} (expected float16, bfloat16 or float32)")


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on *device*."""
    return torch.cuda.current_stream(device).cuda_stream
