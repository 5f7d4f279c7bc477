"""Master-weight-free discrete linear layers on MI355X (drop-in for ``ratchet.py``).

Public surface kept from the reference (``ratchet.py:18-831``): ``DiscreteRatchetLinear``
(same constructor arguments, buffers ``packed`` uint8 + ``_scale`` fp32 or parameter
``log_scale``, ``code`` / ``pressure`` / ``scale`` properties, ``forward(x, *, inputs_int8,
inputs_scale)``, ``apply_weight_gradient``, ``apply_normalized_gradient``,
``ratchet_update``, ``discard_pending_gradient``), ``RatchetEmbedding``,
``RatchetUpdateStats``, ``pack_code_pressure`` / ``unpack_code_pressure``,
``bucket_pressure``, ``audit_no_master_weights`` and ``compare_persistent_footprint``.

What changed underneath (behaviour is identical unless noted):

* The int8 forward reads the packed state directly (nibble decode in the GEMM's tile
  staging); no unpacked or transposed code copy is made (``ratchet.py:52``).
* The int8 backward runs SR quantization, the int8 grad_input GEMM, the BF16
  grad_weight GEMM and ONE fused normalize+update launch over all output rows. The
  reference loops over 256-row tiles (``ratchet.py:150-169``); rows are independent,
  so ``tile_size`` no longer changes any result.
* Non-finite weight gradients in the fused path are detected on the device: the rows
  holding them are left unchanged (which is what the reference's arithmetic does to
  them too) and FloatingPointError is raised by the next validating
  ``ratchet_update()`` instead of by a per-tile host sync (``ratchet.py:501``).
* Every tensor computation of the ratchet path runs in libratchet_hip.so; CPU tensors
  raise RuntimeError for the update and int8 paths.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from .int8_matmul import (
    dequant_bf16,
    dequant_transpose_bf16,
    effective_bf16,
    grad_input_bf16,
    grad_input_bf16_supported,
    grad_weight_bf16,
    grad_weight_bf16_parts,
    grad_weight_bf16_x,
    grad_weight_parts_supported,
    grad_weight_splits,
    int8_mm_nt,
    packed_int8_mm,
    packed_int8_mm_residual,
    packed_int8_mm_t,
    packed_t_supported,
    quantize_rows_sr,
    quantize_rows_sr_parts,
    residual_supported,
    transpose_bf16,
    unpack_transpose,
)
from . import _native
from .ops import ratchet as _ops


def _require_gpu(*tensors: Tensor | None, what: str) -> None:
    """The int8 ratchet path runs only on a ROCm GPU (torch device type 'cuda')."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{what} requires CUDA (a ROCm GPU); the int8 path is GPU-only")


# ---------------------------------------------------------------------------
# Packed state helpers
# ---------------------------------------------------------------------------
def pack_code_pressure(code: Tensor, pressure: Tensor, max_code: int) -> Tensor:
    """Pack signed code (low nibble) and pressure (high nibble) into one uint8.

    Lossless for code in [-max_code, max_code] and pressure in [-7, 7]
    (``ratchet.py:185-192``). Used at construction and by tests; the training path
    writes the bytes inside the update kernel.
    """
    low = (code.to(torch.int16) + max_code) & 0x0F
    high = (pressure.to(torch.int16) + 7) & 0x0F
    return (low | (high << 4)).to(torch.uint8)


def unpack_code_pressure(packed: Tensor, max_code: int) -> tuple[Tensor, Tensor]:
    """(code, pressure) int8 tensors from the packed bytes (``ratchet.py:195-199``)."""
    if packed.is_cuda:
        return _ops().unpack(packed, max_code)
    value = packed.to(torch.int16)
    return ((value & 0x0F) - max_code).to(torch.int8), ((value >> 4) - 7).to(torch.int8)


def bucket_pressure(z: Tensor, *, low: float = 0.5, high: float = 1.5) -> Tensor:
    """Normalized gradient -> integer pressure increment in the descent direction.

    Semantics of ``ratchet.py:248-262``; the training path computes this inside the
    update kernel, this function serves inspection and tests.
    """
    if not 0 <= low < high:
        raise ValueError("pressure bucket thresholds must satisfy 0 <= low < high")
    magnitude = z.abs()
    bucket = (magnitude >= high).to(torch.int16) + (magnitude >= low).to(torch.int16)
    return -torch.sign(z).nan_to_num(0.0).to(torch.int16) * bucket


@dataclass(frozen=True)
class RatchetUpdateStats:
    total_weights: int
    positive_moves: int
    negative_moves: int
    blocked_positive_moves: int
    blocked_negative_moves: int
    gradient_rms_mean: float

    @property
    def code_moves(self) -> int:
        return self.positive_moves + self.negative_moves

    @property
    def blocked_moves(self) -> int:
        return self.blocked_positive_moves + self.blocked_negative_moves

    def materialize(self) -> RatchetUpdateStats:
        """Copy with every field as a Python scalar (the one host sync of the stats)."""
        values = [self.total_weights, self.positive_moves, self.negative_moves,
                  self.blocked_positive_moves, self.blocked_negative_moves,
                  self.gradient_rms_mean]
        tensors = [v for v in values if isinstance(v, Tensor)]
        if tensors:
            host = torch.stack([t.detach().double().reshape(()) for t in tensors]).cpu().tolist()
            it = iter(host)
            values = [next(it) if isinstance(v, Tensor) else v for v in values]
        return RatchetUpdateStats(
            total_weights=int(values[0]),
            positive_moves=int(values[1]),
            negative_moves=int(values[2]),
            blocked_positive_moves=int(values[3]),
            blocked_negative_moves=int(values[4]),
            gradient_rms_mean=float(values[5]),
        )


@dataclass(frozen=True)
class RatchetAuditReport:
    ratchet_layers: int
    ratchet_weights: int
    ratchet_state_bytes: int
    support_parameter_bytes: int
    violations: tuple[str, ...]


def _grad_weight_supported(g: Tensor, x: Tensor) -> bool:
    """Shapes the direct grad_weight kernels take (rk_grad_weight_bf16 on int8
    activations, rk_grad_weight_bf16_x on float32 / bfloat16 ones)."""
    n, k = g.shape[1], x.shape[1]
    return (n % 8 == 0 and k % 16 == 0 and g.stride(-1) == 1 and x.stride(-1) == 1
            and (g.stride(0) * g.element_size()) % 16 == 0
            and (x.stride(0) * x.element_size()) % 16 == 0
            and g.data_ptr() % 16 == 0 and x.data_ptr() % 16 == 0)


# ---------------------------------------------------------------------------
# Autograd function
# ---------------------------------------------------------------------------
def _split_residual_grad(ctx, grad_output: Tensor, defer_bf16: bool = False
                         ) -> tuple[Tensor, Tensor | None, bool]:
    """For output = residual + y: y's gradient and the residual's, each cast to its operand's
    dtype as autograd casts the gradients of an add of mixed dtypes (a bf16 y gets the
    bf16-rounded gradient). ``defer_bf16``: a float32 gradient due for that bf16 rounding is
    returned as it is, with True as the third result, for consumers that round it themselves
    (the SR quant's bf16 source mode and the grad_weight GEMM's bf16 staging)."""
    if ctx.residual_dtype is None:
        return grad_output, None, False
    grad_residual = None
    if ctx.needs_input_grad[7]:
        # a residual broadcast against the output gets the gradient summed to its shape
        grad_residual = grad_output.sum_to_size(ctx.residual_shape).to(ctx.residual_dtype)
    if defer_bf16 and ctx.y_dtype == torch.bfloat16 and grad_output.dtype == torch.float32:
        return grad_output, grad_residual, True
    return grad_output.to(ctx.y_dtype), grad_residual, False


def _fusable_residual(residual: Tensor | None, q: Tensor, packed: Tensor,
                      out_dtype: torch.dtype | None,
                      out_shape: tuple[int, ...]) -> Tensor | None:
    """The residual as a float32 [M, N] view when the forward GEMM can add it in its
    epilogue, else None. The kernel's float32 output is the bf16-rounded product widened,
    so residual + product matches the separate add for a bfloat16 or float32 product. Only
    a residual of exactly the output's shape is fused: any other shape (one that would
    broadcast, or an [M, N] residual beside a [B, T, N] output) takes the separate add,
    which broadcasts or raises as the unfused expression does."""
    if residual is None or out_dtype not in (torch.float32, torch.bfloat16):
        return None
    if residual.dtype != torch.float32 or tuple(residual.shape) != tuple(out_shape):
        return None
    flat = residual.reshape(-1, residual.shape[-1])
    return flat if residual_supported(q, packed, flat) else None


class _RatchetMatmul(torch.autograd.Function):
    """Ratchet matmul whose backward feeds the effective-weight gradient to the update.

    Inputs: (inputs, inputs_int8, inputs_scale, packed, scale, layer, out_dtype). The packed
    state is read in place (never unpacked); ``layer`` carries the mode switches and owns the
    update (``ratchet.py:18-182``). ``out_dtype`` (int8 mode, None = the input dtype) lets a
    caller that casts the output anyway take the GEMM's bf16 result directly: the values are
    the same either way (the float32 output is the bf16 result widened).
    """

    @staticmethod
    def forward(ctx, inputs, inputs_int8, inputs_scale, packed, scale, layer, out_dtype=None,
                residual=None, split=1):
        ctx.split = split
        input_shape = inputs.shape
        flat_inputs = inputs.flatten(0, -2)
        mode = layer.matmul_mode
        ctx.layer = layer
        ctx.input_shape = input_shape
        ctx.input_dtype = inputs.dtype
        ctx.generation = layer._generation
        out_features = packed.shape[0]
        requested = out_dtype if mode not in ("fp32", "bf16") else None
        out_dtype = requested or (inputs.dtype if inputs.dtype in (torch.float32, torch.bfloat16)
                                  else None)

        if mode == "int8" and inputs_int8 is not None and inputs_scale is not None:
            _require_gpu(inputs_int8, packed, what="int8 ratchet matmul")
            q = inputs_int8.flatten(0, -2)
            s = inputs_scale.flatten(0, -1).float()
            if q.stride(-1) != 1:
                q = q.contiguous()
            ctx.save_for_backward(q, s, scale)
            ctx.used_fused_int8 = True
            output = None
        else:
            ctx.save_for_backward(flat_inputs, scale)
            ctx.used_fused_int8 = False
            if mode == "fp32":
                effective = layer._effective_weight_f32(scale)
                output = flat_inputs.to(torch.float32) @ effective.t()
            elif mode == "bf16":
                effective = effective_bf16(packed, layer.max_code, scale.detach())
                output = flat_inputs.to(torch.bfloat16) @ effective.t().contiguous()
            else:
                _require_gpu(flat_inputs, packed, what="int8 ratchet matmul")
                x = flat_inputs
                if x.dtype not in (torch.float32, torch.bfloat16):
                    x = x.float()
                q, s = _ops().quantize_rows(x)
                output = None
        # the dtype of the product itself (residual + product is the function's output)
        ctx.y_dtype = requested or inputs.dtype
        ctx.residual_dtype = residual.dtype if residual is not None else None
        ctx.residual_shape = residual.shape if residual is not None else None
        if output is None:
            flat_res = _fusable_residual(residual, q, packed, out_dtype,
                                         (*input_shape[:-1], out_features))
            if flat_res is not None:
                output = packed_int8_mm_residual(q, packed, layer.max_code, s,
                                                 scale.detach().float(), flat_res)
                return output.reshape(*input_shape[:-1], out_features)
            output = packed_int8_mm(q, packed, layer.max_code, s, scale.detach().float(),
                                    out_dtype or torch.bfloat16)
        output = output.reshape(*input_shape[:-1], out_features)
        if requested is None and output.dtype != inputs.dtype:
            output = output.to(inputs.dtype)
        output = output if residual is None else residual + output
        # split > 1: the output's equal column chunks (views), whose gradients reach backward
        # separately and are read there in place instead of being concatenated first
        return tuple(output.chunk(split, dim=-1)) if split > 1 else output

    @staticmethod
    def backward(ctx, *grad_outputs: Tensor):
        layer = ctx.layer
        if layer._generation != ctx.generation:
            raise RuntimeError(
                "ratchet state changed between this layer's forward and backward "
                "(the layer was applied twice before backward; weight sharing is unsupported "
                "with the fused update)"
            )
        if ctx.split > 1:
            parts = _gradient_parts(ctx, layer, grad_outputs)
            if parts is not None:
                return _RatchetMatmul._backward_parts(ctx, layer, parts)
            grad_output = torch.cat(grad_outputs, dim=-1)
        else:
            grad_output = grad_outputs[0]
        packed = layer.packed
        mode = layer.matmul_mode
        if ctx.used_fused_int8:
            q, s, scale = ctx.saved_tensors  # the saved int8 activations and their scales
            inputs_bf16 = None
            if not layer.fuse_backward_update:
                inputs_bf16 = dequant_bf16(q, s)
            inputs_fp32 = None
        else:
            flat_inputs, scale = ctx.saved_tensors
            inputs_bf16 = None  # bf16(inputs), made only where a path needs the copy
            inputs_fp32 = flat_inputs.to(torch.float32) if mode == "fp32" else None
        # grad_weight on a side stream next to the SR quant and grad_input (below)
        overlap = (mode != "fp32" and layer.overlap_weight_gradient and grad_output.is_cuda
                   and torch.cuda.is_current_stream_capturing())
        # Without the side stream, the int8-backward path consumes the gradient only through
        # the SR quant, which takes float32 values as bf16 itself and writes the bf16 copy
        # grad_weight reads: a gradient due for bf16 rounding skips the separate cast. (With
        # it, grad_weight would read the float32 values, which measured slower than the
        # cast.)
        sr_path = (layer.fuse_backward_update and mode == "int8" and layer.int8_backward
                   and ctx.used_fused_int8)
        grad_output, grad_residual, round_bf16 = _split_residual_grad(
            ctx, grad_output, defer_bf16=sr_path and not overlap)
        flat_gradient = grad_output.flatten(0, -2)
        scale_d = scale.detach()
        needs_scale = ctx.needs_input_grad[4]

        if not layer.fuse_backward_update:
            if mode == "fp32":
                gradient_fp32 = flat_gradient.to(torch.float32)
                effective = layer._effective_weight_f32(scale_d)
                grad_input = gradient_fp32 @ effective
                grad_weight_fp32 = gradient_fp32.t() @ inputs_fp32
            else:
                if inputs_bf16 is None:
                    inputs_bf16 = flat_inputs.to(torch.bfloat16)
                gradient_bf16 = flat_gradient.to(torch.bfloat16)
                grad_input = _bf16_grad_input(gradient_bf16, packed, layer.max_code, scale_d,
                                              ctx.input_dtype)
                grad_weight_fp32 = (gradient_bf16.t() @ inputs_bf16).float()
            layer._capture_weight_gradient(grad_weight_fp32)
            grad_scale = None
            if needs_scale:
                grad_scale = (grad_weight_fp32 * layer.code.float()).sum(dim=1)
            return grad_input.reshape(ctx.input_shape).to(ctx.input_dtype), None, None, None, \
                grad_scale, None, None, grad_residual, None

        m, n = flat_gradient.shape
        gradient_bf16 = None
        partials = None  # grad_weight split partials, reduced inside the update

        def split_weight_gradient(g: Tensor) -> Tensor | None:
            """grad_weight's split partials straight from the saved activations (int8 q, s
            or the inputs themselves, bf16 cast while staging), or None where the split
            kernel does not apply. The partials go to the layer's persistent workspace."""
            if ctx.used_fused_int8:
                if not _grad_weight_supported(g, q):
                    return None
                return grad_weight_bf16(g, q, s, reduce=False,
                                        work=layer._split_workspace(m, g.device))
            x_direct = flat_inputs if flat_inputs.dtype in (torch.float32, torch.bfloat16) \
                else flat_inputs.to(torch.bfloat16)
            if not _grad_weight_supported(g, x_direct):
                return None
            return grad_weight_bf16_x(g, x_direct, reduce=False,
                                      work=layer._split_workspace(m, g.device))

        # grad_weight (bf16 MFMA) reads only the upstream gradient and the saved
        # activations: on a side stream it runs concurrently with the SR quant (VALU, Philox)
        # and the grad_input GEMM; the update joins both (it must follow grad_input, which
        # reads the pre-update codes). Done while a HIP graph is being captured, where the
        # fork and join are graph edges; eagerly, a cross-stream wait costs more than the
        # overlap gains at these kernel sizes (measured).
        side = None
        if overlap:
            g_w = flat_gradient if flat_gradient.dtype in (torch.float32, torch.bfloat16) \
                else flat_gradient.float()
            if g_w.stride(-1) != 1:
                g_w = g_w.contiguous()
            main = torch.cuda.current_stream(g_w.device)
            side = _side_stream(g_w.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                partials = split_weight_gradient(g_w)
                if partials is not None and layer._pending_counts is None:
                    # the update's zeroed move counters, made here behind grad_weight rather
                    # than on the main stream after the join (the update's critical path)
                    layer._counts().record_stream(main)
            if partials is None:
                main.wait_stream(side)
                side = None
            else:
                for t in (g_w, *ctx.saved_tensors):
                    t.record_stream(side)

        if mode == "fp32":
            gradient_fp32 = flat_gradient.to(torch.float32)
            grad_input = gradient_fp32 @ layer._effective_weight_f32(scale_d)
        elif layer.int8_backward and ctx.used_fused_int8:
            # int8 grad_input: fold the per-row weight scale into the gradient, SR-quantize
            # (Philox bits), GEMM against the pre-update codes (ratchet.py:125-134).
            g = flat_gradient
            if g.dtype not in (torch.float32, torch.bfloat16):
                g = g.float()
            if partials is None and g.dtype == torch.float32 \
                    and _grad_weight_supported(g, ctx.saved_tensors[0]):
                # The same pass writes bf16(g), the grad_weight GEMM's gradient operand
                # (grad_out_tile.to(bf16), ratchet.py:162), so that GEMM reads 2-byte
                # values instead of converting float32 ones.
                gradient_bf16 = torch.empty((m, n), device=g.device, dtype=torch.bfloat16)
            # one seed per call from the CPU generator (a device slot under graph capture)
            col_scale = scale_d.float().contiguous()
            out_dtype = ctx.input_dtype if ctx.input_dtype in (torch.float32, torch.bfloat16) \
                else torch.bfloat16
            grad_q, grad_s, layer.last_sr_seed = quantize_rows_sr(
                g, col_scale, bf16_out=gradient_bf16, round_bf16=round_bf16)
            if packed_t_supported(grad_q, packed):
                # contraction over the packed rows, read in place (no unpacked copy)
                grad_input = packed_int8_mm_t(grad_q, packed, layer.max_code, grad_s, None,
                                              out_dtype)
            else:
                code_t = unpack_transpose(packed, layer.max_code)
                grad_input = int8_mm_nt(grad_q, code_t, grad_s, None, out_dtype)
        else:
            gradient_bf16 = flat_gradient.to(torch.bfloat16)
            grad_input = _bf16_grad_input(gradient_bf16, packed, layer.max_code, scale_d,
                                          ctx.input_dtype)

        if mode == "fp32":
            grad_weight = gradient_fp32.t() @ inputs_fp32
        elif partials is None:
            # BF16 grad_weight [N, K] = bf16(g)^T @ bf16(x) (ratchet.py:159-163).
            g = flat_gradient if flat_gradient.dtype in (torch.float32, torch.bfloat16) \
                else flat_gradient.float()
            if gradient_bf16 is not None:
                g = gradient_bf16  # the bf16 copy this backward already made
            # the update reduces the split partials itself (the bf16 gradient is never
            # written)
            partials = split_weight_gradient(g)
            if partials is None:
                # NT GEMM on transposed bf16 copies (both operands contiguous along tokens)
                grad_t = transpose_bf16(g)
                if ctx.used_fused_int8:
                    inputs_t = dequant_transpose_bf16(q, s)
                else:
                    x_direct = flat_inputs if flat_inputs.dtype in (torch.float32,
                                                                    torch.bfloat16) \
                        else flat_inputs.to(torch.bfloat16)
                    inputs_t = transpose_bf16(x_direct)
                grad_weight = grad_t @ inputs_t.t()
        if side is not None:
            # joined here even when the update is queued: left to run ahead, grad_weight's
            # backlog on the side stream slows the next layers' backward (1B step measured
            # 0.6 ms slower)
            torch.cuda.current_stream(partials.device).wait_stream(side)
            partials.record_stream(torch.cuda.current_stream(partials.device))
        if partials is not None:
            grad_scale = layer._fused_update(partials, want_grad_scale=needs_scale,
                                             from_partials=True)
        else:
            grad_scale = layer._fused_update(grad_weight, want_grad_scale=needs_scale)
        return grad_input.reshape(ctx.input_shape).to(ctx.input_dtype), None, None, None, \
            grad_scale, None, None, grad_residual, None

    @staticmethod
    def _backward_parts(ctx, layer, parts: list[Tensor]):
        """The int8-backward path for a gradient that arrives as the output's column chunks
        (``split``): the SR quant and grad_weight read the chunks in place, as one row, with
        the results of the concatenated gradient (same seed draw, codes, scales and
        partials)."""
        q, s, scale = ctx.saved_tensors
        packed = layer.packed
        m = parts[0].shape[0]
        scale_d = scale.detach()
        needs_scale = ctx.needs_input_grad[4]
        partials = None
        side = None
        if layer.overlap_weight_gradient and torch.cuda.is_current_stream_capturing():
            # grad_weight on the side stream, as in the single-gradient path
            main = torch.cuda.current_stream(q.device)
            side = _side_stream(q.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                partials = grad_weight_bf16_parts(parts, q, s,
                                                  work=layer._split_workspace(m, q.device))
            for t in (*parts, *ctx.saved_tensors):
                t.record_stream(side)
        col_scale = scale_d.float().contiguous()
        out_dtype = ctx.input_dtype if ctx.input_dtype in (torch.float32, torch.bfloat16) \
            else torch.bfloat16
        grad_q, grad_s, layer.last_sr_seed = quantize_rows_sr_parts(parts, col_scale)
        if packed_t_supported(grad_q, packed):
            grad_input = packed_int8_mm_t(grad_q, packed, layer.max_code, grad_s, None,
                                          out_dtype)
        else:
            code_t = unpack_transpose(packed, layer.max_code)
            grad_input = int8_mm_nt(grad_q, code_t, grad_s, None, out_dtype)
        if partials is None:
            partials = grad_weight_bf16_parts(parts, q, s,
                                              work=layer._split_workspace(m, q.device))
        if side is not None:
            torch.cuda.current_stream(partials.device).wait_stream(side)
            partials.record_stream(torch.cuda.current_stream(partials.device))
        grad_scale = layer._fused_update(partials, want_grad_scale=needs_scale,
                                         from_partials=True)
        return grad_input.reshape(ctx.input_shape).to(ctx.input_dtype), None, None, None, \
            grad_scale, None, None, None, None


def _bf16_grad_input(gradient_bf16: Tensor, packed: Tensor, max_code: int, scale: Tensor,
                     input_dtype: torch.dtype) -> Tensor:
    """gradient_bf16 @ (code.bf16 * scale.bf16[:, None]) (ratchet.py:136-141): one HIP kernel
    that forms the effective weight while staging, written in the input's dtype when that is
    float32 (the bf16 result widened: the cast the caller makes); torch's GEMM on the
    materialized effective weight for shapes the kernel does not take."""
    if gradient_bf16.is_cuda and grad_input_bf16_supported(gradient_bf16, packed):
        out_dtype = torch.float32 if input_dtype == torch.float32 else torch.bfloat16
        return grad_input_bf16(gradient_bf16, packed, max_code, scale, out_dtype)
    return gradient_bf16 @ effective_bf16(packed, max_code, scale)


def _gradient_parts(ctx, layer, grads) -> list[Tensor] | None:
    """The chunk gradients as [M, C] row views for the in-place parts path, or None when
    it does not apply (then they are concatenated): the fused int8-backward layer path, no
    residual, every chunk's gradient present with one dtype and one row layout, and shapes
    the parts kernels take."""
    if not (layer.fuse_backward_update and layer.matmul_mode == "int8" and layer.int8_backward
            and ctx.used_fused_int8 and ctx.residual_dtype is None):
        return None
    if any(g is None for g in grads):
        return None
    dtype = grads[0].dtype
    if dtype not in (torch.float32, torch.bfloat16) or any(g.dtype != dtype for g in grads):
        return None
    parts = []
    for g in grads:
        flat = g.reshape(-1, g.shape[-1])  # a view when the chunk gradient has row layout
        if flat.stride(-1) != 1 or (flat.shape[0] > 1 and flat.data_ptr() != g.data_ptr()):
            return None
        parts.append(flat)
    if len({(p.shape, p.stride()) for p in parts}) != 1 or parts[0].shape[1] % 8 != 0:
        return None
    if not grad_weight_parts_supported(parts, ctx.saved_tensors[0]):
        return None
    return parts


class UpdateQueue:
    """Fused updates that backward queued instead of launching one per layer, run together
    by ``flush``: the queued layers of one gradient source (a bf16 or float32 gradient, or
    float32 split partials) and row-length class go to one ``rk_ratchet_update_multi``
    launch, which runs each row through the per-layer update's code (bit-identical states,
    counts, row rms, EMA and non-finite flags). The layer tables live on the device and are
    kept while the layers' buffers stay where they are, so a replayed graph reuses them with
    no host work; a table that would have to be built during graph capture is not (the
    group's layers are then updated one launch each)."""

    def __init__(self) -> None:
        self._entries: list[tuple] = []
        self._tables: dict[tuple, tuple[Tensor, Tensor]] = {}

    def __len__(self) -> int:
        return len(self._entries)

    def push(self, layer: "DiscreteRatchetLinear", gradient: Tensor, from_partials: bool,
             counts: Tensor, row_rms: Tensor, nonfinite: Tensor) -> None:
        layer._queued = True
        self._entries.append((layer, gradient, from_partials, counts, row_rms, nonfinite))

    @staticmethod
    def _source(gradient: Tensor, from_partials: bool) -> tuple[int, Tensor, int]:
        """(source code, the [rows, K] gradient or [nsplit, rows, K] partials, nsplit)."""
        if from_partials and gradient.dtype == torch.bfloat16:
            return _native.RK_BF16, gradient[0], 1  # one split, written as the gradient
        if from_partials:
            return _native.RK_UPDATE_SRC_SPLITS, gradient, gradient.shape[0]
        if gradient.dtype == torch.bfloat16:
            return _native.RK_BF16, gradient, 1
        return _native.RK_F32, gradient, 1

    @staticmethod
    def _chunk_class(src: int, k: int) -> int:
        """The update kernel's register-resident chunk count for rows of k elements."""
        if src == _native.RK_F32:
            chunks = (k + 255) // 256
            return 2 if chunks <= 2 else (8 if chunks <= 8 else 0)
        chunks = (k + 511) // 512
        return 1 if chunks <= 1 else (4 if chunks <= 4 else (12 if chunks <= 12 else 0))

    def flush(self) -> None:
        if not self._entries:
            return
        entries, self._entries = self._entries, []
        device = entries[0][1].device
        main = torch.cuda.current_stream(device)
        index = device.index if device.index is not None else torch.cuda.current_device()
        side = _SIDE_STREAMS.get(index)
        if side is not None:
            # grad_weight may still be running on the side stream: its workspaces are
            # complete only after this join (backward left it to the queue)
            main.wait_stream(side)
        groups: dict[tuple, list] = {}
        for entry in entries:
            layer, gradient, from_partials = entry[0], entry[1], entry[2]
            src, g, nsplit = self._source(gradient, from_partials)
            if g.dtype == torch.float32 and src != _native.RK_UPDATE_SRC_SPLITS:
                g = g.contiguous()
            key = (src, self._chunk_class(src, layer.in_features), nsplit == 1)
            groups.setdefault(key, []).append((layer, g, nsplit) + tuple(entry[3:]))
        for (src, _, _), group in groups.items():
            self._launch(src, group, device)
        for entry in entries:
            entry[0]._queued = False

    def _launch(self, src: int, group: list, device: torch.device) -> None:
        key = tuple((layer.packed.data_ptr(), g.data_ptr(), tuple(g.shape), tuple(g.stride()),
                     counts.data_ptr(), row_rms.data_ptr(), nonfinite.data_ptr(),
                     layer._ema_ptr(), layer._rule_key())
                    for layer, g, nsplit, counts, row_rms, nonfinite in group) + (src,)
        tables = self._tables.get(key)
        if tables is None:
            if torch.cuda.is_current_stream_capturing():
                # building a table here would record a host-to-device copy: update the
                # group's layers one launch each instead
                for layer, g, nsplit, counts, row_rms, nonfinite in group:
                    layer._launch_update(g, counts, row_rms, None, nonfinite,
                                         from_partials=src == _native.RK_UPDATE_SRC_SPLITS,
                                         defer_mean=True, count_generation=False)
                return
            tables = self._build(src, group, device)
            self._tables[key] = tables
        written = []
        for layer, g, nsplit, counts, row_rms, nonfinite in group:
            written += [layer.packed, counts, row_rms, nonfinite]
            if layer._ema_ptr():
                written.append(layer.rms_ema)
        _ops().update_multi(tables[0], tables[1], src, written)

    @staticmethod
    def _build(src: int, group: list, device: torch.device) -> tuple[Tensor, Tensor]:
        import ctypes

        entries = (_native.UpdateLayer * len(group))()
        row = 0
        for d, (layer, g, nsplit, counts, row_rms, nonfinite) in zip(entries, group):
            rows, k = layer.out_features, layer.in_features
            d.packed = layer.packed.data_ptr()
            d.g = g.data_ptr()
            d.counts = counts.data_ptr()
            d.row_rms = row_rms.data_ptr()
            d.rms_ema = layer._ema_ptr()
            d.grad_scale = 0
            d.nonfinite = nonfinite.data_ptr()
            d.ldp = layer.packed.stride(0)
            d.ldg = g.stride(-2)
            d.rows, d.K, d.row_begin = rows, k, row
            d.max_code, d.threshold, d.nsplit = layer.max_code, layer.pressure_threshold, nsplit
            beta = layer.rms_ema_beta
            d.low, d.high, d.eps = layer.bucket_low, layer.bucket_high, layer.eps
            # beta2 = 1 - beta in float32, as the per-layer operator computes it
            d.beta1 = beta
            d.beta2 = float(torch.tensor(1.0, dtype=torch.float32)
                            - torch.tensor(beta, dtype=torch.float32))
            row += rows
        host = torch.frombuffer(bytearray(ctypes.string_at(ctypes.addressof(entries),
                                                           ctypes.sizeof(entries))),
                                dtype=torch.uint8)
        return host, host.to(device)


_SIDE_STREAMS: dict[int, torch.cuda.Stream] = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """The per-device stream the fused backward runs grad_weight on (default priority)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _SIDE_STREAMS:
        _SIDE_STREAMS[index] = torch.cuda.Stream(device=index)
    return _SIDE_STREAMS[index]


# ---------------------------------------------------------------------------
# Layer
# ---------------------------------------------------------------------------
class DiscreteRatchetLinear(nn.Module):
    """Linear layer with integer codes and pressure, but no master weight parameter."""

    # fused backward under HIP-graph capture: grad_weight on a side stream, concurrent with
    # grad_input (False: one stream, e.g. to compare the two)
    overlap_weight_gradient: bool = True

    def __init__(
        self,
        in_features: int,
        out_features: int,
        *,
        max_code: int,
        pressure_threshold: int = 8,
        bucket_low: float = 0.5,
        bucket_high: float = 1.5,
        eps: float = 1e-8,
        rms_ema_beta: float = 0.0,
        pressure_leak_period: int = 0,
        trainable_scale: bool = False,
        compile_update: bool = False,
        matmul_mode: str = "fp32",
        initial_weight: Tensor | None = None,
        fuse_backward_update: bool = False,
        int8_backward: bool = False,
        tile_size: int = 256,
    ) -> None:
        super().__init__()
        if in_features <= 0 or out_features <= 0:
            raise ValueError("in_features and out_features must be positive")
        if max_code not in (1, 2, 3, 4, 5, 6, 7):
            raise ValueError(
                "max_code must be in 1..7 (3..15 states); 7 is the 4-bit packing cap"
            )
        if pressure_threshold <= 0 or pressure_threshold > 127:
            raise ValueError("pressure_threshold must be in [1, 127]")
        if not 0 <= bucket_low < bucket_high:
            raise ValueError("bucket thresholds must satisfy 0 <= low < high")
        if eps <= 0:
            raise ValueError("eps must be positive")
        if not 0.0 <= rms_ema_beta < 1.0:
            raise ValueError("rms_ema_beta must be in [0, 1)")
        if pressure_leak_period < 0:
            raise ValueError("pressure_leak_period must be a non-negative integer")
        if matmul_mode not in ("fp32", "bf16", "int8"):
            raise ValueError("matmul_mode must be fp32, bf16, or int8")

        self.in_features = in_features
        self.out_features = out_features
        self.max_code = max_code
        self.pressure_threshold = pressure_threshold
        self.bucket_low = bucket_low
        self.bucket_high = bucket_high
        self.eps = eps
        self.rms_ema_beta = rms_ema_beta
        self.pressure_leak_period = pressure_leak_period
        # The fused HIP update replaces both the eager and the torch.compile'd update
        # (ratchet.py:328-330); the flag is kept for configuration compatibility.
        self.compile_update = compile_update
        self._update_count = 0
        if rms_ema_beta > 0.0:
            self.register_buffer("rms_ema", torch.zeros(out_features))
        self.trainable_scale = trainable_scale
        self.matmul_mode = matmul_mode
        self.fuse_backward_update = fuse_backward_update
        # keep the bf16 weight gradient each fused update consumed (last_weight_gradient),
        # e.g. to check it; off by default, since the fused update never writes it
        self.keep_weight_gradient = False
        self.last_weight_gradient: Tensor | None = None
        self._gw_workspace: Tensor | None = None
        # the stochastic-rounding seed of the last int8 backward (the host draw, or the
        # device slot it reads under graph capture)
        self.last_sr_seed: int | Tensor | None = None
        self.int8_backward = int8_backward
        self.tile_size = tile_size

        if initial_weight is None:
            reference = torch.empty(out_features, in_features, dtype=torch.float32)
            nn.init.kaiming_uniform_(reference, a=5**0.5)
        else:
            if initial_weight.shape != (out_features, in_features):
                raise ValueError(
                    f"initial_weight must have shape {(out_features, in_features)}, "
                    f"got {tuple(initial_weight.shape)}"
                )
            reference = initial_weight.detach().to(dtype=torch.float32)
        # Codes from a float matrix: per-row absmax scale, round, clamp
        # (ratchet.py:380-386).
        row_max = reference.abs().amax(dim=1)
        scale = (row_max / max_code).clamp_min(torch.finfo(torch.float32).eps)
        code = torch.round(reference / scale[:, None]).clamp(-max_code, max_code)
        zero_pressure = torch.zeros_like(code, dtype=torch.int8)
        self.register_buffer(
            "packed", pack_code_pressure(code.to(torch.int8), zero_pressure, max_code)
        )
        if trainable_scale:
            self.log_scale = nn.Parameter(scale.log())
        else:
            self.register_buffer("_scale", scale)

        self._effective_weight: Tensor | None = None
        self._pending_weight_gradient: Tensor | None = None
        self._generation = 0
        # a model may hand the layer a [4] view of one counts buffer for all its layers
        # (summed and cleared once per step by the model); `_slot_dirty`: the slot still
        # holds counts a layer-level ratchet_update consumed
        self._counts_slot: Tensor | None = None
        self._slot_dirty = False
        # the model's copy of every slot, taken once for all its layers before their
        # ratchet_update: this layer's stats then own a row of it instead of a clone each
        self._counts_snapshot: Tensor | None = None
        # likewise an [out_features] view of one row-rms buffer for all its layers, with
        # this layer's [2] int64 segment bounds [0, out_features): the first fused update of
        # a step writes its row rms there and leaves the mean to one launch for the whole
        # model (``row_rms_means``) instead of one per layer
        self._rms_slot: Tensor | None = None
        self._rms_slot_bounds: Tensor | None = None
        # a model that batches its layers' fused updates hands every layer one UpdateQueue:
        # backward then queues this layer's update there, and the queue runs it together
        # with the others (before the layer's next forward or statistics at the latest)
        self._update_queue: UpdateQueue | None = None
        self._queued = False
        self._reset_pending_stats()

    # -- state ----------------------------------------------------------------
    def _reset_pending_stats(self) -> None:
        self._pending_stats_total_weights = 0
        self._pending_counts: Tensor | None = None
        # per launch: mean row rms over all out_features rows (a device scalar), or None for
        # the launch whose row rms sits in the row-rms slot (its mean taken later)
        self._pending_rms_means: list[Tensor | None] = []
        self._nonfinite: Tensor | None = None
        # the slot's mean, when the model computed every layer's in one launch
        self._rms_slot_mean: Tensor | None = None

    @classmethod
    def from_reference(cls, reference: Tensor, *, max_code: int, pressure_threshold: int = 8,
                       bucket_low: float = 0.5, bucket_high: float = 1.5,
                       eps: float = 1e-8) -> DiscreteRatchetLinear:
        if reference.ndim != 2:
            raise ValueError("reference weight must be a matrix")
        return cls(reference.shape[1], reference.shape[0], max_code=max_code,
                   pressure_threshold=pressure_threshold, bucket_low=bucket_low,
                   bucket_high=bucket_high, eps=eps, initial_weight=reference)

    @property
    def has_pending_gradient(self) -> bool:
        eager_pending = (
            self._effective_weight is not None and self._effective_weight.grad is not None
        )
        return eager_pending or self._pending_weight_gradient is not None

    @property
    def persistent_state_bytes(self) -> int:
        return (self.packed.numel() * self.packed.element_size()
                + self.scale.numel() * self.scale.element_size())

    def _apply_queued_update(self) -> None:
        """Runs the update queue if it holds this layer's update from the last backward, so
        a read of the state sees it applied (the reference updates inside backward)."""
        if self._queued:
            self._update_queue.flush()

    @property
    def code(self) -> Tensor:
        self._apply_queued_update()
        return unpack_code_pressure(self.packed, self.max_code)[0]

    @property
    def pressure(self) -> Tensor:
        self._apply_queued_update()
        return unpack_code_pressure(self.packed, self.max_code)[1]

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        self._apply_queued_update()
        super()._save_to_state_dict(destination, prefix, keep_vars)

    @property
    def scale(self) -> Tensor:
        return self.log_scale.exp() if self.trainable_scale else self._scale

    def effective_weight(self) -> Tensor:
        return self.code.to(dtype=self.scale.dtype) * self.scale[:, None]

    def _effective_weight_f32(self, scale: Tensor) -> Tensor:
        return self.code.to(torch.float32) * scale.to(torch.float32)[:, None]

    def _counts(self) -> Tensor:
        if self._pending_counts is None:
            slot = self._counts_slot
            if slot is not None and slot.device == self.packed.device:
                if self._slot_dirty:
                    slot.zero_()
                    self._slot_dirty = False
                self._pending_counts = slot
            else:
                self._pending_counts = torch.zeros(4, dtype=torch.int64,
                                                   device=self.packed.device)
        return self._pending_counts

    def _nonfinite_flag(self) -> Tensor:
        if self._nonfinite is None:
            self._nonfinite = torch.zeros(1, dtype=torch.int32, device=self.packed.device)
        return self._nonfinite

    # -- forward --------------------------------------------------------------
    def forward(self, inputs: Tensor, *, inputs_int8: Tensor | None = None,
                inputs_scale: Tensor | None = None,
                out_dtype: torch.dtype | None = None,
                residual: Tensor | None = None, split: int = 1):
        """``out_dtype`` (int8 mode only): the output dtype in place of the input's, for a
        caller that would cast the result anyway (same values).
        ``residual``: return ``residual + output`` (added in the GEMM's epilogue where the
        shapes allow, the same float32 add). ``split`` > 1: return
        ``output.chunk(split, dim=-1)``; on the fused int8-backward path the chunks'
        gradients are then read in place rather than concatenated (the same results)."""
        if self._queued:
            self._update_queue.flush()  # this forward reads the updated state
        if self.matmul_mode != "fp32" or self.fuse_backward_update:
            return _RatchetMatmul.apply(inputs, inputs_int8, inputs_scale, self.packed,
                                        self.scale, self, out_dtype, residual, split)
        effective = self.effective_weight().to(dtype=inputs.dtype)
        if self.training and torch.is_grad_enabled():
            if self.trainable_scale:
                effective.retain_grad()
            else:
                effective = effective.detach().requires_grad_(True)
            self._effective_weight = effective
        output = F.linear(inputs, effective)
        output = output if residual is None else residual + output
        return output.chunk(split, dim=-1) if split > 1 else output

    # -- gradient capture and the fused update --------------------------------
    def _capture_weight_gradient(self, gradient: Tensor) -> None:
        """Non-fused modes: hold the effective-weight gradient until ratchet_update()."""
        if self._pending_weight_gradient is not None:
            raise RuntimeError(
                "ratchet layer has multiple pending effective-weight gradients "
                "(missing ratchet_update or unsupported weight sharing)"
            )
        self._pending_weight_gradient = gradient

    def _split_workspace(self, tokens: int, device: torch.device) -> Tensor:
        """The grad_weight GEMM's output for the update, kept across steps (reused in stream
        order: each backward's GEMM follows the previous update that read it): float32
        [nsplit, out, in] split partials, or with one split a bfloat16 [1, out, in] tensor
        that receives the gradient itself (2 bytes per weight written and read instead of
        4; the values the update forms from one split)."""
        nsplit = grad_weight_splits(tokens, self.out_features, self.in_features)
        shape = (nsplit, self.out_features, self.in_features)
        dtype = torch.bfloat16 if nsplit == 1 else torch.float32
        work = self._gw_workspace
        if (work is None or work.shape != shape or work.device != device
                or work.dtype != dtype):
            work = torch.empty(shape, device=device, dtype=dtype)
            self._gw_workspace = work
        return work

    def _launch_update(self, gradient: Tensor, counts: Tensor, row_rms: Tensor | None,
                       grad_scale: Tensor | None, nonfinite: Tensor | None, *,
                       from_partials: bool = False, defer_mean: bool = False,
                       count_generation: bool = True) -> None:
        """One update launch from a weight gradient [N, K], or (``from_partials``) from the
        grad_weight GEMM's float32 split partials [nsplit, N, K], reduced inside the update
        with the same arithmetic. With ``keep_weight_gradient`` set, the bf16 gradient the
        update consumed is kept in ``last_weight_gradient``."""
        _require_gpu(gradient, self.packed, what="the ratchet update")
        ema = getattr(self, "rms_ema", None) if self.rms_ema_beta > 0.0 else None
        beta = self.rms_ema_beta
        # the launch also writes the mean of row_rms (the stats' gradient_rms_mean), unless
        # that mean is taken later from the row-rms slot
        rms_mean = (torch.empty((), device=self.packed.device, dtype=torch.float32)
                    if row_rms is not None and not defer_mean else None)
        rule = (self.max_code, self.pressure_threshold, self.bucket_low, self.bucket_high,
                self.eps, ema, beta, counts, row_rms, grad_scale, nonfinite, rms_mean)
        if from_partials and gradient.dtype == torch.bfloat16:
            # one split, written as the bf16 gradient by the GEMM: the update from the
            # gradient itself gives what the update from one split's partials gives
            gradient = gradient[0]
            _ops().update_from_grad(self.packed, gradient, *rule)
            self.last_weight_gradient = gradient.clone() if self.keep_weight_gradient else None
        elif from_partials:
            kept = None
            if self.keep_weight_gradient:
                kept = torch.empty(gradient.shape[1:], device=gradient.device,
                                   dtype=torch.bfloat16)
            _ops().update_from_partials(self.packed, gradient, *rule, kept)
            self.last_weight_gradient = kept
        else:
            if gradient.dtype not in (torch.float32, torch.bfloat16):
                gradient = gradient.float()
            _ops().update_from_grad(self.packed, gradient, *rule)
            self.last_weight_gradient = gradient if self.keep_weight_gradient else None
        self._last_rms_mean = rms_mean
        if count_generation:
            self._generation += 1

    def _ema_ptr(self) -> int:
        """Device address of the per-row rms EMA, 0 without one."""
        ema = getattr(self, "rms_ema", None) if self.rms_ema_beta > 0.0 else None
        return 0 if ema is None else ema.data_ptr()

    def _rule_key(self) -> tuple:
        return (self.max_code, self.pressure_threshold, self.bucket_low, self.bucket_high,
                self.eps, self.rms_ema_beta)

    def _will_queue(self, want_grad_scale: bool, device: torch.device) -> bool:
        """Whether the fused update of this backward goes to the model's queue: a queue is
        attached, no trainable-scale gradient is wanted (backward must return it), no copy
        of the gradient is kept, and the row rms go to the model's buffer."""
        slot = self._rms_slot
        return (self._update_queue is not None and not want_grad_scale
                and not self.keep_weight_gradient and device.type == "cuda"
                and slot is not None and slot.device == device
                and None not in self._pending_rms_means)

    def _fused_update(self, grad_weight: Tensor, *, want_grad_scale: bool,
                      from_partials: bool = False) -> Tensor | None:
        """Normalize + update every output row in one launch (fused backward path);
        ``grad_weight`` is the gradient, or its split partials with ``from_partials``."""
        if grad_weight.shape[-2:] != (self.out_features, self.in_features):
            raise ValueError("fused gradient shape mismatch")
        if self._will_queue(want_grad_scale, grad_weight.device):
            self._update_queue.push(self, grad_weight, from_partials, self._counts(),
                                    self._rms_slot, self._nonfinite_flag())
            self._pending_stats_total_weights += self.out_features * self.in_features
            self._pending_rms_means.append(None)
            self._last_rms_mean = None
            self.last_weight_gradient = None
            self._generation += 1
            return None
        slot = self._rms_slot
        defer = (slot is not None and slot.device == grad_weight.device
                 and None not in self._pending_rms_means)
        row_rms = slot if defer else torch.empty(self.out_features, device=grad_weight.device,
                                                 dtype=torch.float32)
        grad_scale = (torch.empty(self.out_features, device=grad_weight.device,
                                  dtype=torch.float32) if want_grad_scale else None)
        self._launch_update(grad_weight, self._counts(), row_rms, grad_scale,
                            self._nonfinite_flag(), from_partials=from_partials,
                            defer_mean=defer)
        self._pending_stats_total_weights += self.out_features * self.in_features
        self._pending_rms_means.append(None if defer else self._last_rms_mean)
        return grad_scale

    def _pending_rms_mean(self) -> Tensor | float:
        means = [self._slot_rms_mean() if m is None else m for m in self._pending_rms_means]
        if not means:
            return 0.0
        return means[0] if len(means) == 1 else torch.stack(means).sum()

    def _slot_rms_mean(self) -> Tensor:
        """Mean of the row rms in this layer's slot: the one the model computed for all its
        layers, else one launch for this layer (the same summation order either way)."""
        if self._rms_slot_mean is not None:
            return self._rms_slot_mean
        return _ops().row_rms_means(self._rms_slot, self._rms_slot_bounds)[0]

    @torch.no_grad()
    def _normalize(self, gradient: Tensor, row_start: int, row_end: int) -> Tensor:
        """z = g / (row rms + eps) (or the per-row EMA rms), ``ratchet.py:539-556``."""
        _require_gpu(gradient, what="ratchet normalization")
        ema = self.rms_ema[row_start:row_end] if self.rms_ema_beta > 0.0 else None
        return _ops().normalize_rows(gradient, self.eps, ema, self.rms_ema_beta)

    @torch.no_grad()
    def apply_weight_gradient(self, gradient: Tensor, *,
                              validate: bool = True) -> RatchetUpdateStats:
        if gradient.shape != (self.out_features, self.in_features):
            raise ValueError(
                f"gradient must have shape {(self.out_features, self.in_features)}, "
                f"got {tuple(gradient.shape)}"
            )
        if validate and not torch.isfinite(gradient).all():
            raise FloatingPointError("ratchet gradient contains NaN or Inf")
        counts = torch.zeros(4, dtype=torch.int64, device=self.packed.device)
        row_rms = torch.empty(self.out_features, device=self.packed.device, dtype=torch.float32)
        self._launch_update(gradient.to(self.packed.device), counts, row_rms, None, None)
        if validate:
            self._validate_state()
        return RatchetUpdateStats(
            total_weights=self.packed.numel(),
            positive_moves=counts[0],
            negative_moves=counts[1],
            blocked_positive_moves=counts[2],
            blocked_negative_moves=counts[3],
            gradient_rms_mean=self._last_rms_mean,
        )

    @torch.no_grad()
    def apply_normalized_gradient(self, normalized: Tensor, *,
                                  validate: bool = True) -> RatchetUpdateStats:
        if normalized.shape != (self.out_features, self.in_features):
            raise ValueError(
                f"normalized gradient must have shape {(self.out_features, self.in_features)}, "
                f"got {tuple(normalized.shape)}"
            )
        z = normalized.to(device=self.packed.device, dtype=torch.float32).contiguous()
        _require_gpu(z, self.packed, what="the ratchet update")
        counts = torch.zeros(4, dtype=torch.int64, device=self.packed.device)
        _ops().update_from_z(self.packed, z, self.max_code, self.pressure_threshold,
                             self.bucket_low, self.bucket_high, counts)
        self._generation += 1
        if validate:
            self._validate_state()
        return RatchetUpdateStats(
            total_weights=self.packed.numel(),
            positive_moves=counts[0],
            negative_moves=counts[1],
            blocked_positive_moves=counts[2],
            blocked_negative_moves=counts[3],
            gradient_rms_mean=0.0,
        )

    @torch.no_grad()
    def _maybe_leak_pressure(self) -> None:
        if self.pressure_leak_period <= 0:
            return
        self._update_count += 1
        if self._update_count % self.pressure_leak_period != 0:
            return
        _require_gpu(self.packed, what="the pressure leak")
        _ops().pressure_leak(self.packed, self.max_code)

    def check_finite_gradients(self) -> None:
        """Raise FloatingPointError if a fused update saw a NaN/Inf gradient (host sync)."""
        if self._nonfinite is not None and int(self._nonfinite.item()):
            self._nonfinite.zero_()
            raise FloatingPointError("ratchet gradient contains NaN or Inf")

    def ratchet_update(self, *, validate: bool = True) -> RatchetUpdateStats:
        if self._queued:
            self._update_queue.flush()
        if self.fuse_backward_update:
            if validate:
                self.check_finite_gradients()
                self._validate_state()
            counts = self._pending_counts
            if counts is None:
                pos = neg = bpos = bneg = 0
            else:
                # the model's shared count slot is cleared by its sum and reused next step:
                # the stats own a copy (32 bytes), as the reference's per-layer stats own
                # their tensors - a row of the model's one copy of all slots when it made one
                if counts is self._counts_slot:
                    snap = self._counts_snapshot
                    own = snap if snap is not None else counts.clone()
                else:
                    own = counts
                pos, neg, bpos, bneg = own[0], own[1], own[2], own[3]
            stats = RatchetUpdateStats(
                total_weights=self._pending_stats_total_weights,
                positive_moves=pos,
                negative_moves=neg,
                blocked_positive_moves=bpos,
                blocked_negative_moves=bneg,
                # sum over launches of sum(row_rms) / out_features; each launch covers all
                # out_features rows, so that is the sum of the launches' mean row rms
                gradient_rms_mean=self._pending_rms_mean(),
            )
            nonfinite = self._nonfinite
            if counts is not None and counts is self._counts_slot:
                self._slot_dirty = True  # cleared by the model's sum, or before next use
            self._counts_snapshot = None
            self._reset_pending_stats()
            self._nonfinite = nonfinite
        elif self.matmul_mode != "fp32":
            if self._pending_weight_gradient is None:
                raise RuntimeError("ratchet layer has no pending effective-weight gradient")
            try:
                stats = self.apply_weight_gradient(self._pending_weight_gradient,
                                                   validate=validate)
            finally:
                self._pending_weight_gradient = None
        else:
            if self._effective_weight is None or self._effective_weight.grad is None:
                raise RuntimeError("ratchet layer has no pending effective-weight gradient")
            try:
                stats = self.apply_weight_gradient(self._effective_weight.grad,
                                                   validate=validate)
            finally:
                self._effective_weight = None
        self._maybe_leak_pressure()
        return stats.materialize() if validate else stats

    def discard_pending_gradient(self) -> None:
        if self._queued:
            # a queued fused update is applied, as the reference applied it inside backward
            self._update_queue.flush()
        self._pending_weight_gradient = None
        self._effective_weight = None

    def _validate_state(self) -> None:
        _require_gpu(self.packed, what="ratchet state validation")
        flags = _ops().validate_state(self.packed, self.max_code, self.scale.detach())
        bad_code, bad_pressure, bad_scale = flags.tolist()
        if bad_code:
            raise RuntimeError("ratchet code escaped its allowed range")
        if bad_pressure:
            raise RuntimeError("ratchet pressure escaped the packed nibble range")
        if bad_scale:
            raise RuntimeError("ratchet row scales must remain positive and finite")

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, "
            f"states={2 * self.max_code + 1}, threshold={self.pressure_threshold}, bias=False"
        )


class RatchetEmbedding(DiscreteRatchetLinear):
    """Master-weight-free token embedding (``ratchet.py:688-749``): a ratchet layer whose
    forward is an embedding lookup; it joins every update/audit sweep."""

    def __init__(self, num_embeddings: int, embedding_dim: int, *, max_code: int,
                 pressure_threshold: int = 8, bucket_low: float = 0.5,
                 bucket_high: float = 1.5, eps: float = 1e-8, rms_ema_beta: float = 0.0,
                 pressure_leak_period: int = 0, trainable_scale: bool = False,
                 compile_update: bool = False, initial_weight: Tensor | None = None) -> None:
        if initial_weight is None:
            initial_weight = torch.randn(num_embeddings, embedding_dim)
        super().__init__(
            embedding_dim, num_embeddings, max_code=max_code,
            pressure_threshold=pressure_threshold, bucket_low=bucket_low,
            bucket_high=bucket_high, eps=eps, rms_ema_beta=rms_ema_beta,
            pressure_leak_period=pressure_leak_period, trainable_scale=trainable_scale,
            compile_update=compile_update, matmul_mode="fp32", initial_weight=initial_weight,
        )
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim

    def forward(self, token_ids: Tensor) -> Tensor:  # type: ignore[override]
        effective = self.effective_weight()
        if self.training and torch.is_grad_enabled():
            effective = effective.detach().requires_grad_(True)
            self._effective_weight = effective
        return F.embedding(token_ids, effective)

    def extra_repr(self) -> str:
        return (
            f"num_embeddings={self.num_embeddings}, embedding_dim={self.embedding_dim}, "
            f"states={2 * self.max_code + 1}, threshold={self.pressure_threshold}"
        )


@dataclass(frozen=True)
class PersistentFootprint:
    """Persistent bytes of the trainable matrices: ratchet vs FP32 + AdamW."""

    ratchet_weights: int
    ratchet_matrix_bytes: int
    fp32_master_bytes: int
    fp32_optimizer_bytes: int

    @property
    def fp32_matrix_bytes(self) -> int:
        return self.fp32_master_bytes + self.fp32_optimizer_bytes

    @property
    def reduction_ratio(self) -> float:
        return self.fp32_matrix_bytes / max(self.ratchet_matrix_bytes, 1)


def compare_persistent_footprint(model: nn.Module) -> PersistentFootprint:
    weights = 0
    ratchet_bytes = 0
    for module in model.modules():
        if isinstance(module, DiscreteRatchetLinear):
            weights += module.packed.numel()
            ratchet_bytes += module.persistent_state_bytes
    return PersistentFootprint(ratchet_weights=weights, ratchet_matrix_bytes=ratchet_bytes,
                               fp32_master_bytes=weights * 4, fp32_optimizer_bytes=weights * 8)


def audit_no_master_weights(model: nn.Module, *,
                            raise_on_violation: bool = False) -> RatchetAuditReport:
    violations: list[str] = []
    layers = weights = state_bytes = 0
    for module_name, module in model.named_modules():
        if not isinstance(module, DiscreteRatchetLinear):
            continue
        layers += 1
        weights += module.packed.numel()
        state_bytes += module.persistent_state_bytes
        prefix = module_name or "<root>"
        for parameter_name, parameter in module.named_parameters(recurse=False):
            if parameter.is_floating_point() and parameter.ndim >= 2:
                violations.append(f"{prefix}.{parameter_name}: floating matrix parameter")
        if module.packed.dtype != torch.uint8:
            violations.append(f"{prefix}.packed: expected uint8, got {module.packed.dtype}")
        if module.scale.ndim != 1 or module.scale.shape[0] != module.out_features:
            violations.append(f"{prefix}.scale: expected one scale per output row")
    support_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    report = RatchetAuditReport(ratchet_layers=layers, ratchet_weights=weights,
                                ratchet_state_bytes=state_bytes,
                                support_parameter_bytes=support_bytes,
                                violations=tuple(violations))
    if raise_on_violation and violations:
        raise RuntimeError("ratchet master-weight audit failed: " + "; ".join(violations))
    return report


def ratchet_layers(model: nn.Module) -> list[DiscreteRatchetLinear]:
    return [m for m in model.modules() if isinstance(m, DiscreteRatchetLinear)]


def persistent_bytes(model: nn.Module) -> int:
    return sum(layer.persistent_state_bytes for layer in ratchet_layers(model))


__all__ = [
    "DiscreteRatchetLinear", "RatchetEmbedding", "RatchetUpdateStats", "RatchetAuditReport",
    "PersistentFootprint", "pack_code_pressure", "unpack_code_pressure", "bucket_pressure",
    "audit_no_master_weights", "compare_persistent_footprint", "ratchet_layers",
    "persistent_bytes",
]
