"""ctypes binding of ``libresihp_hip.so`` (the C ABI declared in include/resihp_hip.h).

Only plumbing lives here: loading the library, declaring argument types, turning
a nonzero status into a Python exception, and handing out device pointers and
the current HIP stream.  There is no fallback: if the library or a GPU is
missing, every call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("RESIHP_HIP_LIB", Path(__file__).with_name("libresihp_hip.so")))

RH_OK = 0
RH_ERR_INVALID = 1
RH_ERR_HIP = 2
RH_ERR_UNSUPPORTED = 3

RH_DTYPE_F32 = 0
RH_DTYPE_BF16 = 1

RH_GEMM_NT = 0
RH_GEMM_NN = 1
RH_GEMM_TN = 2

RH_EPI_NONE = 0
RH_EPI_GELU = 1
RH_EPI_GELU_GRAD = 2
RH_EPI_GELU_DERIV = 3
RH_EPI_MUL_AUX = 4

RH_GEMM_STAGE_MAIN = 1
RH_GEMM_STAGE_REDUCE = 2

RH_MAX_SEG = 4

c_i64 = ctypes.c_int64
c_ptr = ctypes.c_void_p
c_int = ctypes.c_int
c_float = ctypes.c_float


class rh_gemm_desc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("epilogue", ctypes.c_int32),
        ("b_nseg", ctypes.c_int32),
        ("d_nseg", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("M", c_i64),
        ("N", c_i64),
        ("K", c_i64),
        ("A", c_ptr),
        ("lda", c_i64),
        ("B", c_ptr * RH_MAX_SEG),
        ("ldb", c_i64),
        ("b_seg_rows", c_i64),
        ("alpha", c_float),
        ("beta", c_float),
        ("C", c_ptr),
        ("ldc", c_i64),
        ("D", c_ptr * RH_MAX_SEG),
        ("ldd", c_i64),
        ("d_seg_rows", c_i64),
        ("aux", c_ptr),
        ("aux_out", c_ptr),
        ("ldaux", c_i64),
    ]


class rh_copy2d(ctypes.Structure):
    _fields_ = [
        ("src", c_ptr),
        ("dst", c_ptr),
        ("src_ld_bytes", c_i64),
        ("dst_ld_bytes", c_i64),
        ("rows", c_i64),
        ("row_bytes", c_i64),
    ]


class rh_adamw_tensor(ctypes.Structure):
    _fields_ = [
        ("param", c_ptr),
        ("grad", c_ptr),
        ("exp_avg", c_ptr),
        ("exp_avg_sq", c_ptr),
        ("step", c_ptr),
        ("numel", c_i64),
    ]


# name -> argtypes (every function returns int, except rh_last_error)
_SIGNATURES = {
    "rh_version": [],
    "rh_gemm_workspace_bytes": [ctypes.POINTER(rh_gemm_desc), ctypes.POINTER(c_i64)],
    "rh_gemm": [ctypes.POINTER(rh_gemm_desc), c_ptr, c_i64, c_ptr],
    "rh_gemm_stage": [ctypes.POINTER(rh_gemm_desc), c_ptr, c_i64, c_int, c_ptr],
    "rh_gemm_kernel_name": [ctypes.POINTER(rh_gemm_desc), ctypes.c_char_p, c_i64],
    "rh_gemm_grouped_workspace_bytes": [ctypes.POINTER(rh_gemm_desc), c_int, ctypes.POINTER(c_i64)],
    "rh_gemm_grouped": [ctypes.POINTER(rh_gemm_desc), c_int, c_ptr, c_i64, c_ptr],
    "rh_gemm_grouped_plan": [ctypes.POINTER(rh_gemm_desc), c_int, ctypes.POINTER(c_int)],
    "rh_gemm_grouped_kernel_name": [ctypes.POINTER(rh_gemm_desc), c_int, ctypes.c_char_p, c_i64],
    "rh_attn_fwd": [c_int, c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_i64, c_ptr,
                    c_float, c_int, c_ptr],
    "rh_attn_bwd_workspace_bytes": [c_i64, c_i64, c_i64, ctypes.POINTER(c_i64)],
    "rh_attn_bwd": [c_int, c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_i64, c_ptr, c_i64,
                    c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_float, c_int, c_ptr, c_i64, c_ptr],
    "rh_attn_bwd_noalloc": [c_int, c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_i64, c_ptr,
                            c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_float, c_int, c_ptr],
    "rh_layernorm_fwd": [c_int, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_float, c_ptr, c_ptr, c_ptr, c_ptr],
    "rh_layernorm_bwd_workspace_bytes": [c_i64, c_i64, ctypes.POINTER(c_i64)],
    "rh_layernorm_bwd": [c_int, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_int,
                         c_ptr, c_i64, c_ptr],
    "rh_gelu_fwd": [c_int, c_i64, c_ptr, c_ptr, c_ptr],
    "rh_gelu_bwd": [c_int, c_i64, c_ptr, c_ptr, c_ptr, c_ptr],
    "rh_add": [c_int, c_i64, c_ptr, c_ptr, c_ptr, c_ptr],
    "rh_scale_by": [c_int, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr],
    "rh_sgd_step": [c_int, c_i64, c_ptr, c_ptr, c_float, c_float, c_ptr],
    "rh_adamw_step": [c_int, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_float, c_float, c_float, c_float, c_float, c_float,
                      c_float, c_ptr],
    "rh_adamw_multi": [c_int, c_int, ctypes.POINTER(rh_adamw_tensor), ctypes.c_double, ctypes.c_double,
                       ctypes.c_double, ctypes.c_double, ctypes.c_double, c_ptr],
    "rh_xent_workspace_bytes": [c_i64, c_i64, ctypes.POINTER(c_i64)],
    "rh_xent_fwd": [c_int, c_i64, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_i64,
                    c_ptr],
    "rh_xent_bwd": [c_int, c_i64, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr],
    "rh_lmhead_xent_workspace_bytes": [c_i64, c_i64, c_i64, c_i64, ctypes.POINTER(c_i64), ctypes.POINTER(c_i64)],
    "rh_lmhead_xent_fwd": [c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr],
    "rh_lmhead_xent_bwd": [c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_int, c_ptr,
                           c_i64, c_ptr],
    "rh_embedding_fwd": [c_int, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_ptr],
    "rh_embedding_bwd_workspace_bytes": [c_i64, c_i64, c_i64, ctypes.POINTER(c_i64)],
    "rh_embedding_bwd": [c_int, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_i64, c_ptr, c_ptr, c_int, c_ptr, c_i64,
                         c_ptr],
    "rh_copy2d_batch": [ctypes.POINTER(rh_copy2d), c_int, c_ptr],
    "rh_reshard_pack": [ctypes.POINTER(c_ptr), ctypes.POINTER(c_i64), c_int, c_i64, c_i64, c_int, c_i64, c_ptr,
                        c_ptr],
    "rh_reshard_unpack": [c_ptr, c_i64, c_i64, c_int, c_i64, c_int, ctypes.POINTER(c_ptr), ctypes.POINTER(c_i64),
                          c_ptr],
}

EXPORTED = tuple(_SIGNATURES) + ("rh_last_error",)

_lib = None


class HipLibraryError(RuntimeError):
    """The native library could not be loaded (not built, or no HIP runtime)."""


def load() -> ctypes.CDLL:
    """Load the library once and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise HipLibraryError(
            f"{LIB_PATH} is missing: build it with `python resihp-reproduction_amd/build.py` "
            "(or __graft_entry__.build()); resihp has no CPU fallback"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.rh_last_error.argtypes = []
    lib.rh_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Invoke ``name`` and raise on a nonzero status with the library's message."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != RH_OK:
        msg = lib.rh_last_error().decode(errors="replace")
        if rc == RH_ERR_INVALID:
            raise ValueError(msg)
        if rc == RH_ERR_UNSUPPORTED:
            raise NotImplementedError(msg)
        raise RuntimeError(msg)


def query(name: str, *args) -> int:
    """Call a ``*_workspace_bytes`` style function and return its int64 result."""
    out = c_i64(0)
    call(name, *args, ctypes.byref(out))
    return int(out.value)


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return RH_DTYPE_F32
    if t.dtype == torch.bfloat16:
        return RH_DTYPE_BF16
    raise TypeError(f"resihp kernels support float32 and bfloat16, got {t.dtype}")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one HIP device; raise (no CPU fallback) otherwise."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"resihp runs on the GPU through its HIP kernels; got a tensor on {t.device} "
                "(move the model and inputs with .to('cuda'))"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no tensor given")
    load()
    return dev


def workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)
