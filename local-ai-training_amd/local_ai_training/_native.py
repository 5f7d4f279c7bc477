"""ctypes binding of libratchet_hip.so (the C ABI declared in include/ratchet_hip.h).

The training path reaches the library through the ``torch.ops.ratchet`` operators
(``ops.py``); this binding serves the KV-cached decode step, whose kernels write into
fixed buffers that a captured HIP graph replays, and callers that want the raw C ABI.
The shared library is the only compute path of this package: if it is missing or
fails to load, every GPU entry point raises. Tensors are passed as raw device
pointers plus element strides; the stream is the caller's current torch stream.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_NAME = "libratchet_hip.so"
LIB_PATH = Path(os.environ.get("RATCHET_HIP_LIB", Path(__file__).with_name(LIB_NAME)))

RK_F32 = 0
RK_BF16 = 1
RK_I8 = 2
RK_F32_AS_BF16 = 3

RK_UPDATE_SRC_SPLITS = 2  # rk_ratchet_update_multi: the gradient as float32 split partials

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_u64 = ctypes.c_uint64
_f32 = ctypes.c_float
_p = ctypes.c_void_p


class UpdateLayer(ctypes.Structure):
    """One entry of rk_ratchet_update_multi's layer table (rk_update_layer, 160 bytes):
    device addresses as integers (0 = absent), strides and sizes in elements."""

    _fields_ = [
        ("packed", _u64), ("g", _u64), ("counts", _u64), ("row_rms", _u64),
        ("rms_ema", _u64), ("grad_scale", _u64), ("nonfinite", _u64), ("reserved0", _u64),
        ("ldp", _i64), ("ldg", _i64), ("rows", _i64), ("K", _i64), ("row_begin", _i64),
        ("reserved1", _i64),
        ("max_code", ctypes.c_int32), ("threshold", ctypes.c_int32), ("nsplit", ctypes.c_int32),
        ("reserved2", ctypes.c_int32),
        ("low", _f32), ("high", _f32), ("eps", _f32), ("beta1", _f32), ("beta2", _f32),
        ("reserved3", _f32 * 3),
    ]


# name -> argument types (all return int status, except where noted)
SIGNATURES: dict[str, list] = {
    "rk_quantize_rows": [_p, _i32, _i64, _i64, _i64, _i64, _p, _i32, _u64, _i64, _p, _i64, _p,
                         _p, _i64, _p],
    "rk_quantize_rows_devseed": [_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _i64, _p,
                                 _p, _i64, _p],
    "rk_philox_word0": [_u64, ctypes.c_uint32, _i64, _p, _p],
    "rk_int8_gemm_nt": [_p, _i64, _p, _i64, _p, _p, _p, _i32, _i64, _i64, _i64, _i64, _p],
    "rk_int8_gemm_packed": [_p, _i64, _p, _i64, _i32, _p, _p, _p, _i32, _i64, _i64, _i64, _i64,
                            _p],
    "rk_int8_gemm_packed_t": [_p, _i64, _p, _i64, _i32, _p, _p, _p, _i32, _i64, _i64, _i64,
                              _i64, _p],
    "rk_int8_gemm_packed_residual": [_p, _i64, _p, _i64, _i32, _p, _p, _p, _i64, _p, _i64,
                                     _i64, _i64, _i64, _p],
    "rk_unpack_transpose": [_p, _i64, _i32, _p, _i64, _i64, _i64, _p],
    "rk_unpack": [_p, _i64, _i32, _p, _p, _p],
    "rk_effective_bf16": [_p, _i64, _i32, _p, _p, _i64, _i64, _i64, _p],
    "rk_grad_input_bf16": [_p, _i64, _p, _i64, _i32, _p, _p, _i32, _i64, _i64, _i64, _i64, _p,
                           _i64, _p],
    "rk_grad_input_bf16_workspace": [_i64, _i64],
    "rk_dequant_bf16": [_p, _i64, _p, _p, _i64, _i64, _i64, _p],
    "rk_transpose_bf16": [_p, _i32, _i64, _p, _i64, _i64, _i64, _p],
    "rk_dequant_transpose_bf16": [_p, _i64, _p, _p, _i64, _i64, _i64, _p],
    "rk_grad_weight_bf16": [_p, _i32, _i64, _p, _i64, _p, _i64, _i64, _i64, _p, _i32, _p,
                            _i64, _p],
    "rk_grad_weight_update": [_p, _i32, _i64, _p, _i32, _i64, _p, _i64, _i64, _i64, _p, _i32,
                              _p, _p, _i64, _i32, _i32, _f32, _f32, _f32, _p, _f32, _f32, _p,
                              _p, _p, _p, _p, _i64, _p],
    "rk_grad_weight_update_counters": [_i64, _i64],
    "rk_grad_weight_bf16_noalloc": [_p, _i32, _i64, _p, _i64, _p, _i64, _i64, _i64, _i32,
                                    _p, _i64, _p],
    "rk_grad_weight_bf16_x": [_p, _i32, _i64, _p, _i32, _i64, _i64, _i64, _i64, _p, _i32, _p,
                              _i64, _p],
    "rk_grad_weight_splits": [_i64, _i64, _i64],
    "rk_ratchet_update": [_p, _i64, _p, _i64, _i64, _i64, _i32, _i32, _f32, _f32, _p, _p],
    "rk_ratchet_update_grad": [_p, _i64, _p, _i32, _i64, _i64, _i64, _i32, _i32, _f32, _f32,
                               _f32, _p, _f32, _f32, _p, _p, _p, _p, _p, _p],
    "rk_ratchet_update_partials": [_p, _i64, _p, _i32, _i64, _i64, _i32, _i32, _f32, _f32,
                                   _f32, _p, _f32, _f32, _p, _p, _p, _p, _p, _p, _i64, _p],
    "rk_ratchet_update_multi": [_p, _p, _i32, _i32, _p],
    "rk_normalize_rows": [_p, _i32, _i64, _i64, _i64, _f32, _p, _f32, _f32, _p, _i64, _p, _p],
    "rk_pressure_leak": [_p, _i64, _i32, _p],
    "rk_validate_state": [_p, _i64, _i32, _p, _i64, _p, _p],
    "rk_rmsnorm_quantize": [_p, _i32, _i64, _p, _f32, _p, _i64, _p, _i64, _i64, _p],
    "rk_gelu_quantize": [_p, _i32, _i64, _p, _i64, _p, _i64, _i64, _p],
    "rk_transpose_quantize": [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p,
                              _i64, _p, _p],
    "rk_rmsnorm_backward": [_p, _i32, _i64, _p, _i32, _i64, _p, _f32, _i64, _i64, _p, _i64, _p,
                            _p, _i64, _p],
    "rk_rmsnorm_backward_parts": [_i64],
    "rk_rmsnorm_backward_residual": [_p, _i32, _i64, _p, _i64, _p, _f32, _i64, _i64, _p, _i64, _p,
                                     _i64, _p, _p, _i64, _p],
    "rk_quantize_rows_parts": [_p, _p, _p, _i32, _i64, _i32, _i64, _i64, _p, _i32, _u64, _p,
                               _i64, _p, _i64, _p, _p],
    "rk_grad_weight_bf16_parts": [_p, _p, _p, _i32, _i64, _i32, _i64, _p, _i32, _i64, _p, _i64,
                                  _i64, _i64, _p, _i32, _p, _i64, _p],
    "rk_gelu_backward": [_p, _i32, _i64, _p, _i32, _i64, _i64, _i64, _p, _i64, _p],
    "rk_decode_gemv": [_p, _i64, _p, _i64, _p, _i32, _p, _f32, _p, _i64, _i32, _p, _p, _i32,
                       _i64, _i32, _i64, _i64, _i64, _p],
    "rk_decode_attention_splits": [_i64, _i64, _i64],
    "rk_decode_attention": [_p, _i32, _i64, _p, _p, _i32, _i64, _i64, _i64, _p, _i64, _i64,
                            _i64, _i64, _f32, _p, _i64, _p, _i64, _p],
    "rk_decode_embed": [_p, _i64, _p, _i64, _i64, _p, _i64, _p, _p, _i64, _p],
    "rk_decode_greedy": [_p, _i64, _i64, _i64, _p, _i64, _p, _p],
    "rk_hbm_stream": [_p, _p, _i64, _i32, _i32, _i32, _p],
    "rk_embedding_backward_workspace": [_i64, _i64, _i64],
    "rk_embedding_backward": [_p, _i32, _i64, _p, _i32, _i64, _i64, _i64, _p, _i64, _p, _i64,
                              _p],
    "rk_cross_entropy_forward": [_p, _i32, _i64, _p, _i64, _i64, _i64, _p, _p, _p, _p],
    "rk_cross_entropy_backward": [_p, _i32, _i64, _p, _i64, _i64, _i64, _p, _p, _p, _p, _i32,
                                  _i64, _p],
    "rk_row_rms_means": [_p, _i64, _p, _i64, _p, _p],
    "rk_attention_forward": [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64,
                             _i64, _i64, _i64, _i64, _i64, _f32, _p, _i64, _i64, _i64, _p, _p],
    "rk_version": [],
    "rk_last_error": [],
}

# return types other than int (the status, or an int count)
RESTYPES = {
    "rk_last_error": ctypes.c_char_p,
    "rk_decode_attention_splits": ctypes.c_int64,
    "rk_grad_weight_update_counters": ctypes.c_int64,
    "rk_embedding_backward_workspace": ctypes.c_int64,
    "rk_grad_input_bf16_workspace": ctypes.c_int64,
}

_lib: ctypes.CDLL | None = None


def load_library() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises RuntimeError if unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.is_file():
        raise RuntimeError(
            f"{LIB_NAME} not found at {LIB_PATH}; build it with "
            "`python local-ai-training_amd/build.py` (the ratchet int8 path has no fallback)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


class NativeError(RuntimeError):
    """A libratchet_hip.so entry point returned a non-zero status."""


def call(name: str, *args) -> None:
    lib = load_library()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.rk_last_error().decode(errors="replace")
        raise NativeError(f"{name} failed (status {status}): {message}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """Raw handle of the caller's current stream on ``device`` (a capture stream inside
    CUDA-graph capture, so launches through the library are captured too)."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return RK_F32
    if dtype == torch.bfloat16:
        return RK_BF16
    raise TypeError(f"unsupported dtype {dtype}; expected float32 or bfloat16")
