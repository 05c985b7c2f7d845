"""ctypes binding of ``libsfl.so`` (the C ABI in ``include/sfl.h``).

The library is loaded from the package's ``lib/`` directory, where
``systems_for_llms_amd.build`` writes it. There is no fallback: if the library
is missing every GPU entry point raises, naming the build command.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_long, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libsfl.so"

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
DTYPE_BF16X2 = 3  # split-bf16 values in the decode GEMVs' activation layout
DTYPE_F32X = 4    # fp32 values in the decode GEMVs' activation layout
DTYPE_F16X2 = 5   # split-fp16 values in the decode GEMVs' activation layout

P = c_void_p
SIGNATURES: dict[str, list] = {
    "sfl_decode_attention": [P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int,
                             c_float, c_int, c_int, c_int, P],
    "sfl_decode_attention_static": [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int,
                                    c_int, c_int, P],
    "sfl_decode_attention_static_scratch_bytes": [],
    "sfl_decode_attention_out_proj": [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_float, c_int, P],
    "sfl_packed_gemv_elems": [c_int, c_int],
    "sfl_pack_gemv_weights": [P, P, c_int, c_int, c_int, P],
    "sfl_rmsnorm_qkv_rope_append": [P, P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P],
    "sfl_linear_residual": [P, P, P, c_int, c_int, c_int, c_int, c_int, P],
    "sfl_rmsnorm_swiglu": [P, P, P, P, P, c_int, c_int, c_int, c_int, P],
    "sfl_rmsnorm_lm_head": [P, P, P, P, c_long, P, c_long, P, P, c_int, c_int, c_int, c_int, c_int, P],
    "sfl_lm_head_tiles": [c_int],
    "sfl_embedding_gather": [P, c_long, P, P, P, c_int, c_int, c_int, P],
    "sfl_next_token": [P, P, c_int, c_int, P, P, c_long, P, P, P, P, P, c_int, c_int, c_int, c_int, P],
    "sfl_masked_attention": [P, P, P, P, P, c_int, c_int, c_int, c_int, POINTER(c_long), POINTER(c_long),
                             POINTER(c_long), POINTER(c_long), c_float, c_int, c_int, c_int, c_int, P,
                             c_int, P, P, P, c_int, c_int, P],
    "sfl_masked_attention_block": [],
    "sfl_masked_attention_kernel_info": [c_int, c_int, c_int, c_long, c_long, c_int, c_int, c_int, c_int, P],
    "sfl_gemm": [P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, P],
    "sfl_gemm_qkv_rope": [P, P, c_int, c_int, c_int, c_int, P, P, P, P, P, c_int, c_int, P],
    "sfl_gemm_swiglu": [P, P, P, c_int, c_int, c_int, c_int, P],
    "sfl_embed_rows": [P, P, P, c_int, c_int, c_int, P],
    "sfl_rmsnorm_rows": [P, P, P, c_int, c_int, c_int, c_int, P],
    "sfl_rmsnorm_rows_scaled": [P, P, P, P, c_int, c_int, c_int, P],
    "sfl_gemm_residual_norm": [P, P, P, c_int, c_int, c_int, P, P, P, c_int, P],
    "sfl_norm_scale": [P, c_int, c_int, c_int, P, P],
    "sfl_gemm_qkv_rope_scaled": [P, P, P, c_int, c_int, c_int, c_int, P, P, P, P, P, c_int, c_int, P],
    "sfl_gemm_swiglu_scaled": [P, P, P, P, c_int, c_int, c_int, c_int, P],
    "sfl_causal_attention_f32": [P, P, P, P, c_int, c_int, c_int, c_int, POINTER(c_long), POINTER(c_long),
                                 POINTER(c_long), POINTER(c_long), c_float, P],
}

_LIB = None


class KernelInfo(ctypes.Structure):
    """``sfl_kernel_info`` of ``include/sfl.h``."""

    _fields_ = [("name", ctypes.c_char * 96), ("registers", c_int), ("private_bytes", c_int),
                ("shared_bytes", c_int), ("max_threads", c_int), ("threads", c_int),
                ("queries_per_workgroup", c_int)]


class LibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise LibraryMissing(
                f"{LIB_PATH} is not built; run `python -m systems_for_llms_amd.build` "
                "(or __graft_entry__.build()) before using the GPU path")
        handle = ctypes.CDLL(str(LIB_PATH))
        handle.sfl_version.restype = c_char_p
        handle.sfl_version.argtypes = []
        handle.sfl_last_error.restype = c_char_p
        handle.sfl_last_error.argtypes = []
        for name, args in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = c_int
        handle.sfl_packed_gemv_elems.restype = c_long
        handle.sfl_decode_attention_static_scratch_bytes.restype = c_long
        _LIB = handle
    return _LIB


def call(name: str, *args) -> None:
    """Invoke an entry point; a nonzero status becomes RuntimeError with the library's message."""
    handle = lib()
    status = getattr(handle, name)(*args)
    if status != 0:
        message = handle.sfl_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({status}): {message}")


def pack_gemv(w: torch.Tensor) -> torch.Tensor:
    """A decode-GEMV copy of a [N, K] weight in the packed tile layout (``sfl.h``)."""
    n, k = w.shape
    w = w.contiguous()
    packed = torch.empty(lib().sfl_packed_gemv_elems(n, k), device=w.device, dtype=w.dtype)
    call("sfl_pack_gemv_weights", w.data_ptr(), packed.data_ptr(), n, k, dtype_code(w.dtype),
         stream_handle(w.device))
    return packed


def masked_kernel_info(head_dim: int, dtype: torch.dtype, n: int, k_row_stride: int,
                       v_row_stride: int, causal: bool = True, window_left: int = -1, window_right: int = -1,
                       global_prefix: int = 0) -> KernelInfo:
    """Resource data of the kernel ``sfl_masked_attention`` launches for these shapes and mask
    (windows < 0: unbounded)."""
    info = KernelInfo()
    call("sfl_masked_attention_kernel_info", head_dim, dtype_code(dtype), n, k_row_stride, v_row_stride,
         int(causal), window_left, window_right, global_prefix, ctypes.addressof(info))
    return info


_LIB_SHA256 = None


def library_sha256() -> str:
    """SHA-256 of the loaded ``libsfl.so`` (identifies the compiled kernels)."""
    global _LIB_SHA256
    if _LIB_SHA256 is None:
        import hashlib

        _LIB_SHA256 = hashlib.sha256(LIB_PATH.read_bytes()).hexdigest()
    return _LIB_SHA256


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16") from None
