"""The ``torch.ops.ratchet`` operators: registration and fake (meta) kernels.

The operators themselves live in ``libratchet_torch.so`` (``csrc/ratchet_torch_ops.cpp``):
each one reads its tensors and calls one entry point of the gfx950 kernel library
``libratchet_hip.so`` on torch's current stream. This module loads that library once and
registers, for every operator, a fake kernel that gives the shapes, dtypes and strides of
its results without running anything, so the operators work with meta tensors,
``FakeTensorMode``, ``torch.library.opcheck`` and tracing.

Mutating operators (``update_from_*``, ``grad_weight_partials*``, ``packed_mm_accumulate``,
``pressure_leak``) declare what they write in their schema and return nothing.
"""

from __future__ import annotations

import os
from pathlib import Path

import torch

LIB_NAME = "libratchet_torch.so"
LIB_PATH = Path(os.environ.get("RATCHET_TORCH_LIB", Path(__file__).with_name(LIB_NAME)))

_loaded = False


def load() -> None:
    """Load the operator library (once) and register the fake kernels; raises RuntimeError
    if it has not been built (the ratchet int8 path has no fallback)."""
    global _loaded
    if _loaded:
        return
    if not LIB_PATH.is_file():
        raise RuntimeError(
            f"{LIB_NAME} not found at {LIB_PATH}; build it with "
            "`python local-ai-training_amd/build.py` (the ratchet int8 path has no fallback)"
        )
    torch.ops.load_library(str(LIB_PATH))
    _register_fakes()
    _loaded = True


def ratchet():
    """The ``torch.ops.ratchet`` namespace, loading the library on first use."""
    load()
    return torch.ops.ratchet


def _register_fakes() -> None:
    fake = torch.library.register_fake

    def rows(x, dtype):
        return x.new_empty((x.shape[0], x.shape[1]), dtype=dtype)

    @fake("ratchet::quantize_rows")
    def _quantize_rows(x, col_scale=None, stochastic=False, seed=0, seed_slot=None,
                       row_offset=0, x_bf16=None, round_bf16=False):
        return rows(x, torch.int8), x.new_empty((x.shape[0],), dtype=torch.float32)

    @fake("ratchet::int8_mm_nt")
    def _int8_mm_nt(a, b, a_scale, b_scale, out_dtype):
        return a.new_empty((a.shape[0], b.shape[0]), dtype=out_dtype)

    @fake("ratchet::packed_mm")
    def _packed_mm(a, packed, max_code, a_scale, row_scale, out_dtype):
        return a.new_empty((a.shape[0], packed.shape[0]), dtype=out_dtype)

    @fake("ratchet::packed_mm_residual")
    def _packed_mm_residual(a, packed, max_code, a_scale, row_scale, residual):
        return a.new_empty((a.shape[0], packed.shape[0]), dtype=torch.float32)

    @fake("ratchet::packed_mm_accumulate")
    def _packed_mm_accumulate(a, packed, max_code, a_scale, row_scale, acc):
        return None

    @fake("ratchet::packed_mm_t")
    def _packed_mm_t(a, packed, max_code, a_scale, row_scale, out_dtype):
        return a.new_empty((a.shape[0], packed.shape[1]), dtype=out_dtype)

    @fake("ratchet::unpack_transpose")
    def _unpack_transpose(packed, max_code):
        return packed.new_empty((packed.shape[1], packed.shape[0]), dtype=torch.int8)

    @fake("ratchet::unpack")
    def _unpack(packed, max_code):
        return (packed.new_empty(packed.shape, dtype=torch.int8),
                packed.new_empty(packed.shape, dtype=torch.int8))

    @fake("ratchet::effective_bf16")
    def _effective_bf16(packed, max_code, scale):
        return rows(packed, torch.bfloat16)

    @fake("ratchet::grad_input_bf16")
    def _grad_input_bf16(g, packed, max_code, scale, out_dtype=torch.bfloat16):
        return g.new_empty((g.shape[0], packed.shape[1]), dtype=out_dtype)

    @fake("ratchet::dequant_bf16")
    def _dequant_bf16(q, s):
        return rows(q, torch.bfloat16)

    @fake("ratchet::transpose_bf16")
    def _transpose_bf16(x):
        return x.new_empty((x.shape[1], x.shape[0]), dtype=torch.bfloat16)

    @fake("ratchet::dequant_transpose_bf16")
    def _dequant_transpose_bf16(q, s):
        return q.new_empty((q.shape[1], q.shape[0]), dtype=torch.bfloat16)

    @fake("ratchet::grad_weight")
    def _grad_weight(g, q, s, nsplit=0):
        return g.new_empty((g.shape[1], q.shape[1]), dtype=torch.bfloat16)

    @fake("ratchet::grad_weight_x")
    def _grad_weight_x(g, x, nsplit=0):
        return g.new_empty((g.shape[1], x.shape[1]), dtype=torch.bfloat16)

    for name in ("grad_weight_partials", "grad_weight_partials_x", "update_from_z",
                 "update_from_grad", "update_from_partials", "update_multi", "pressure_leak"):
        fake(f"ratchet::{name}")(lambda *args, **kwargs: None)

    @fake("ratchet::normalize_rows")
    def _normalize_rows(g, eps, rms_ema, beta):
        return rows(g, torch.float32)

    @fake("ratchet::validate_state")
    def _validate_state(packed, max_code, scale):
        return packed.new_empty((3,), dtype=torch.int32)

    @fake("ratchet::rmsnorm_quantize")
    def _rmsnorm_quantize(x, w, eps):
        return rows(x, torch.int8), x.new_empty((x.shape[0],), dtype=torch.float32)

    @fake("ratchet::gelu_quantize")
    def _gelu_quantize(x):
        return rows(x, torch.int8), x.new_empty((x.shape[0],), dtype=torch.float32)

    @fake("ratchet::transpose_quantize")
    def _transpose_quantize(x):
        b, h, s, d = x.shape
        return (x.new_empty((b * s, h * d), dtype=torch.int8),
                x.new_empty((b * s,), dtype=torch.float32))

    def float_dtype(x):
        return x.dtype if x.dtype in (torch.float32, torch.bfloat16) else torch.float32

    @fake("ratchet::rmsnorm_backward")
    def _rmsnorm_backward(grad_y, x, w, eps, residual_grad=None):
        return (x.new_empty((x.shape[0], x.shape[1]), dtype=float_dtype(x)),
                x.new_empty((x.shape[1],), dtype=torch.float32))

    @fake("ratchet::gelu_backward")
    def _gelu_backward(grad_y, x):
        return x.new_empty((x.shape[0], x.shape[1]), dtype=float_dtype(x))

    @fake("ratchet::quantize_rows_parts")
    def _quantize_rows_parts(parts, col_scale=None, stochastic=False, seed=0, seed_slot=None,
                             row_offset=0):
        m, k = parts[0].shape[0], parts[0].shape[1] * len(parts)
        return (parts[0].new_empty((m, k), dtype=torch.int8),
                parts[0].new_empty((m,), dtype=torch.float32))

    @fake("ratchet::grad_weight_partials_parts")
    def _grad_weight_partials_parts(parts, x, s, work):
        return None

    @fake("ratchet::embedding_backward")
    def _embedding_backward(grad, ids, num_weights):
        return grad.new_empty((num_weights, grad.shape[-1]), dtype=torch.float32)

    @fake("ratchet::attention_forward")
    def _attention_forward(q, k, v, scale):
        b, h, sl, d = q.shape
        o = q.new_empty((b, sl, h, d)).permute(0, 2, 1, 3)
        return o, q.new_empty((b, h, sl), dtype=torch.float32)

    @fake("ratchet::row_rms_means")
    def _row_rms_means(row_rms, offsets):
        return row_rms.new_empty((offsets.shape[0] - 1,))

    @fake("ratchet::cross_entropy_forward")
    def _cross_entropy_forward(logits, targets, ignore_index=-100):
        f32 = torch.float32
        return (logits.new_empty((), dtype=f32), logits.new_empty((3, logits.shape[0]), dtype=f32),
                logits.new_empty((), dtype=f32))

    @fake("ratchet::cross_entropy_backward")
    def _cross_entropy_backward(grad_loss, logits, targets, stats, count, ignore_index=-100):
        return logits.new_empty((logits.shape[0], logits.shape[1]))


# every operator the library defines (the opcheck tests walk this list)
OPERATORS = (
    "quantize_rows", "int8_mm_nt", "packed_mm", "packed_mm_residual", "packed_mm_accumulate",
    "packed_mm_t", "unpack_transpose", "unpack", "effective_bf16", "grad_input_bf16",
    "dequant_bf16",
    "transpose_bf16", "dequant_transpose_bf16", "grad_weight_splits", "grad_weight",
    "grad_weight_x", "grad_weight_partials", "grad_weight_partials_x", "update_from_z",
    "update_from_grad", "update_from_partials", "update_multi", "normalize_rows",
    "pressure_leak",
    "validate_state", "rmsnorm_quantize", "gelu_quantize", "transpose_quantize",
    "rmsnorm_backward", "gelu_backward", "embedding_backward", "quantize_rows_parts",
    "grad_weight_partials_parts", "cross_entropy_forward",
    "cross_entropy_backward", "row_rms_means", "attention_forward",
)
