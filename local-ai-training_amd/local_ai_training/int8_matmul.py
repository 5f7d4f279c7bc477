"""int8 GEMM and per-token quantizers on gfx950, dispatched through ``torch.ops.ratchet``.

Drop-in for the reference module ``int8_matmul.py``: the public functions keep their
names, argument meaning, return dtypes and exception types
(``int8_matmul.py:251-343``). Each call runs one ``torch.ops.ratchet`` operator
(``ops.py``), which calls one entry point of the gfx950 kernel library; CPU tensors are
rejected with RuntimeError exactly where the reference rejects them.

The ratchet layer uses the lower-level functions below (``packed_int8_mm``,
``int8_mm_nt``, ``quantize_rows_sr``) which skip the host-synchronizing scale checks of the
public ``scaled_int8_mm`` (``int8_matmul.py:305-309``).

Stochastic-rounding seeds: the reference draws one seed per stochastic call from the CPU
generator (``int8_matmul.py:200``), and so does every eager call here. Inside a HIP graph
capture a seed drawn on the host would be frozen into the graph, so a capture must run under
``CapturedSeeds.recording()``: each stochastic call then reads its seed from a device slot,
and ``CapturedSeeds.refill()`` draws the slots' seeds from the CPU generator, in call order,
before every replay.
"""

from __future__ import annotations

import contextlib

import torch
from torch import Tensor

from .ops import ratchet as _ops


def _sr_seed() -> int:
    # Host-side RNG, one draw per stochastic call, as int8_matmul.py:200 draws it: the
    # CPU generator's stream stays identical to the reference's.
    return int(torch.randint(0, 2**31 - 1, (1,)).item())


class CapturedSeeds:
    """Device-resident stochastic-rounding seeds for HIP-graph capture.

    While ``recording()`` is active, every stochastic quantization that is being captured
    takes the next int64 slot of ``slots`` (in call order) and its kernel reads the seed
    from there when it runs. ``refill()`` draws one seed per used slot from the CPU
    generator in slot order, exactly the draws an eager step makes in the same order, and
    stores them; call it before each replay.
    """

    def __init__(self, device: torch.device | str, capacity: int = 512) -> None:
        self.slots = torch.zeros(capacity, dtype=torch.int64, device=device)
        self.used = 0
        self.last_drawn: list[int] = []
        # two pinned staging buffers, so a refill never waits for the replay before it and
        # never overwrites staging memory whose copy is still queued
        self._staging = [torch.empty(capacity, dtype=torch.int64, pin_memory=True)
                         for _ in range(2)]
        self._copied: list[torch.cuda.Event | None] = [None, None]
        self._turn = 0

    def take(self) -> Tensor:
        if self.used >= self.slots.numel():
            raise RuntimeError("CapturedSeeds: more stochastic calls than slots")
        slot = self.slots[self.used:self.used + 1]
        self.used += 1
        return slot

    @contextlib.contextmanager
    def recording(self):
        global _ACTIVE_SEEDS
        previous, _ACTIVE_SEEDS = _ACTIVE_SEEDS, self
        self.used = 0
        try:
            yield self
        finally:
            _ACTIVE_SEEDS = previous

    def refill(self) -> list[int]:
        """Draw this replay's seeds (host RNG, reference order) and queue their copy into
        the device slots on the current stream, ahead of the replay that reads them."""
        drawn = [_sr_seed() for _ in range(self.used)]
        if drawn:
            turn = self._turn
            if self._copied[turn] is not None:
                self._copied[turn].synchronize()
            staging = self._staging[turn]
            staging[:self.used] = torch.tensor(drawn, dtype=torch.int64)
            self.slots[:self.used].copy_(staging[:self.used], non_blocking=True)
            event = torch.cuda.Event()
            event.record()
            self._copied[turn] = event
            self._turn = 1 - turn
        self.last_drawn = drawn
        return drawn


_ACTIVE_SEEDS: CapturedSeeds | None = None


def sr_seed_args(device: torch.device) -> tuple[int, Tensor | None]:
    """(seed, device slot) for one stochastic call: a host draw in eager mode, a slot of the
    active CapturedSeeds under graph capture. Capturing without one raises, since the graph
    would replay the capture-time seed forever."""
    if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
        if _ACTIVE_SEEDS is None:
            raise RuntimeError(
                "stochastic rounding inside a HIP graph capture needs a seed source: "
                "capture under CapturedSeeds.recording() and call refill() before replays"
            )
        return 0, _ACTIVE_SEEDS.take()
    return _sr_seed(), None


def quantize_rows_sr(values: Tensor, col_scale: Tensor | None = None, *,
                     bf16_out: Tensor | None = None, row_offset: int = 0,
                     round_bf16: bool = False) -> tuple[Tensor, Tensor, int | Tensor]:
    """Stochastically rounded row quantization of values * col_scale (one Philox draw per
    element); returns (q, scale, seed) where seed is the host seed drawn for this call or,
    under graph capture, the device slot it reads. ``bf16_out`` receives bf16(values).
    ``round_bf16``: float32 values are quantized as values.to(bfloat16), the same result as
    casting first."""
    seed, slot = sr_seed_args(values.device)
    q, s = _ops().quantize_rows(values, col_scale, True, seed, slot, row_offset, bf16_out,
                                round_bf16)
    return q, s, (slot if slot is not None else seed)


def quantize_rows_sr_parts(parts: list[Tensor], col_scale: Tensor | None = None
                           ) -> tuple[Tensor, Tensor, int | Tensor]:
    """quantize_rows_sr of the row concatenation of ``parts`` (each [M, C], unit column
    stride, one shared row stride) without building it: the same seed draw, codes and
    scales as quantizing ``torch.cat(parts, dim=-1)``."""
    seed, slot = sr_seed_args(parts[0].device)
    q, s = _ops().quantize_rows_parts(list(parts), col_scale, True, seed, slot, 0)
    return q, s, (slot if slot is not None else seed)


def _quantize_rows_fused(values: Tensor, col_scale: Tensor | None = None, *,
                         stochastic: bool = False) -> tuple[Tensor, Tensor]:
    """HIP row quantization; bit-exact with the reference's torch formula
    (``int8_matmul.py:225-239``), with Philox stochastic rounding when requested."""
    if values.ndim != 2:
        raise ValueError("row quantization requires a 2D tensor")
    if values.dtype not in (torch.float32, torch.bfloat16):
        values = values.float()
    if stochastic:
        q, s, _ = quantize_rows_sr(values, col_scale)
        return q, s
    return _ops().quantize_rows(values, col_scale)


def _quantize_columns_fused(values: Tensor) -> tuple[Tensor, Tensor]:
    """Per-column quantization = row quantization of the transposed view (no copy)."""
    if values.ndim != 2:
        raise ValueError("column quantization requires a 2D tensor")
    q_t, scale = _quantize_rows_fused(values.t())
    return q_t.t().contiguous(), scale


def quantize_rows(values: Tensor) -> tuple[Tensor, Tensor]:
    """Symmetrically quantize each row; returns int8 values plus float32 scales."""
    if not values.is_cuda:
        raise RuntimeError("quantize_rows requires CUDA (a ROCm GPU); the int8 path is GPU-only")
    return _quantize_rows_fused(values)


def quantize_rows_colscaled(values: Tensor, col_scale: Tensor, *,
                            stochastic: bool = False) -> tuple[Tensor, Tensor]:
    """Row-quantize values * col_scale[None, :] in one pass (no M x N float temp)."""
    if not values.is_cuda:
        raise RuntimeError(
            "quantize_rows_colscaled requires CUDA (a ROCm GPU); the int8 path is GPU-only"
        )
    if col_scale.ndim != 1 or values.ndim != 2 or col_scale.shape[0] != values.shape[1]:
        raise ValueError("col_scale must be 1-D with length values.shape[1]")
    if col_scale.dtype != torch.float32:
        raise TypeError("col_scale must be float32")
    return _quantize_rows_fused(values, col_scale.contiguous(), stochastic=stochastic)


def quantize_columns(values: Tensor) -> tuple[Tensor, Tensor]:
    if not values.is_cuda:
        raise RuntimeError(
            "quantize_columns requires CUDA (a ROCm GPU); the int8 path is GPU-only"
        )
    return _quantize_columns_fused(values)


def int8_mm_nt(a: Tensor, b_nk: Tensor, a_scale: Tensor, b_scale: Tensor | None,
               out_dtype: torch.dtype = torch.bfloat16) -> Tensor:
    """C = bf16((A @ B^T) * a_scale[:, None] * b_scale[None, :]); A [M,K], B [N,K] int8.

    ``out_dtype`` float32 stores the bf16-rounded value widened (a fused `.float()`).
    No host synchronization.
    """
    return _ops().int8_mm_nt(a, b_nk, a_scale, b_scale, out_dtype)


def packed_int8_mm(a: Tensor, packed: Tensor, max_code: int, a_scale: Tensor,
                   row_scale: Tensor | None, out_dtype: torch.dtype = torch.bfloat16) -> Tensor:
    """C = bf16((A @ code^T) * a_scale * row_scale) with code decoded from packed [N, K]."""
    return _ops().packed_mm(a, packed, max_code, a_scale, row_scale, out_dtype)


def residual_supported(a: Tensor, packed: Tensor, residual: Tensor) -> bool:
    """Whether packed_int8_mm_residual can run on these operands: the 32x32x32 kernel's
    shapes (more than 16 rows, K % 64 == 0, N % 8 == 0, 16-byte aligned rows) and a float32
    residual [M, N] with unit column stride."""
    m, k = a.shape
    n = packed.shape[0]
    return (m > 16 and k % 64 == 0 and n % 8 == 0 and residual.dtype == torch.float32
            and residual.shape == (m, n) and residual.stride(-1) == 1
            and a.stride(-1) == 1 and packed.stride(-1) == 1 and _ld(a) % 16 == 0
            and _ld(packed) % 16 == 0 and _ld(residual) % 4 == 0
            and a.data_ptr() % 16 == 0 and packed.data_ptr() % 16 == 0
            and residual.data_ptr() % 16 == 0)


def packed_int8_mm_residual(a: Tensor, packed: Tensor, max_code: int, a_scale: Tensor,
                            row_scale: Tensor | None, residual: Tensor,
                            out: Tensor | None = None) -> Tensor:
    """C = residual + float32(bf16((A @ code^T) * a_scale * row_scale)) in one launch: the
    forward GEMM's float32 output with the residual add fused into its epilogue (the same
    float32 add as adding afterwards). ``out`` may be ``residual`` itself (accumulate in
    place); the library rejects any other overlap of the two."""
    if out is None:
        return _ops().packed_mm_residual(a, packed, max_code, a_scale, row_scale, residual)
    if out is not residual:
        out.copy_(residual)
    _ops().packed_mm_accumulate(a, packed, max_code, a_scale, row_scale, out)
    return out


def packed_t_supported(a: Tensor, packed: Tensor) -> bool:
    """Whether packed_int8_mm_t can run on these operands (aligned shapes)."""
    k, n = packed.shape
    return (k % 64 == 0 and n % 8 == 0 and a.stride(-1) == 1 and packed.stride(-1) == 1
            and _ld(a) % 16 == 0 and _ld(packed) % 16 == 0 and a.data_ptr() % 16 == 0
            and packed.data_ptr() % 16 == 0)


def packed_int8_mm_t(a: Tensor, packed: Tensor, max_code: int, a_scale: Tensor,
                     row_scale: Tensor | None, out_dtype: torch.dtype = torch.bfloat16
                     ) -> Tensor:
    """C = bf16((A @ code) * a_scale * row_scale) with code = decode(packed) as the [K, N]
    operand (A [M, K] int8, packed [K, N]): the grad_input GEMM against the packed state,
    without an unpacked or transposed copy of the codes."""
    return _ops().packed_mm_t(a, packed, max_code, a_scale, row_scale, out_dtype)


def scaled_int8_mm(lhs: Tensor, rhs: Tensor, lhs_scale: Tensor, rhs_scale: Tensor) -> Tensor:
    """Multiply int8 matrices [M,K] @ [K,N] and fuse row/column scales into a BF16 output."""
    if not lhs.is_cuda or not rhs.is_cuda:
        raise RuntimeError("scaled_int8_mm requires CUDA operands (a ROCm GPU)")
    if lhs.ndim != 2 or rhs.ndim != 2:
        raise ValueError("scaled_int8_mm operands must be 2D")
    if lhs.dtype != torch.int8 or rhs.dtype != torch.int8:
        raise TypeError("scaled_int8_mm operands must be int8")
    if lhs.shape[1] != rhs.shape[0]:
        raise ValueError("scaled_int8_mm inner dimensions must match")
    if lhs.device != rhs.device:
        raise ValueError("scaled_int8_mm operands must share a device")
    m, k = lhs.shape
    _, n = rhs.shape
    if lhs_scale.shape != (m,) or rhs_scale.shape != (n,):
        raise ValueError("scaled_int8_mm scales must match output rows and columns")
    for name, scale in (("lhs", lhs_scale), ("rhs", rhs_scale)):
        if scale.device != lhs.device or scale.dtype != torch.float32:
            raise TypeError(f"{name} scale must be FP32 on the operand device")
        if not torch.isfinite(scale).all() or torch.any(scale <= 0):
            raise ValueError(f"{name} scale must be finite and positive")
    # B as its [N, K] transposed view: a strided [K, N] operand needs no copy when its
    # columns are contiguous; the operator copies otherwise
    return int8_mm_nt(lhs, rhs.t(), lhs_scale.contiguous(), rhs_scale.contiguous())


def _ld(t: Tensor) -> int:
    """Row stride of a 2-D operand with unit column stride."""
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


def unpack_transpose(packed: Tensor, max_code: int) -> Tensor:
    """codeT[k, n] = code[n, k] as a contiguous int8 [K, N] tensor."""
    return _ops().unpack_transpose(packed, max_code)


def effective_bf16(packed: Tensor, max_code: int, scale: Tensor) -> Tensor:
    """bf16(code) * bf16(scale)[:, None] rounded to bf16, as ratchet.py:140 computes it."""
    return _ops().effective_bf16(packed, max_code, scale.float())


def grad_input_bf16_supported(g: Tensor, packed: Tensor) -> bool:
    """Whether grad_input_bf16 takes these operands: a bf16 gradient [M, N] with unit column
    stride, N a positive multiple of 8, K % 8 == 0, 16-byte aligned rows."""
    n, k = packed.shape
    return (g.dtype == torch.bfloat16 and g.dim() == 2 and g.shape[1] == n and n > 0
            and n % 8 == 0 and k % 8 == 0 and g.stride(-1) == 1 and _ld(g) % 8 == 0
            and g.data_ptr() % 16 == 0 and packed.stride(-1) == 1 and _ld(packed) % 16 == 0
            and packed.data_ptr() % 16 == 0)


def grad_input_bf16(g: Tensor, packed: Tensor, max_code: int, scale: Tensor,
                    out_dtype: torch.dtype = torch.bfloat16) -> Tensor:
    """bf16(g @ (bf16(code) * bf16(scale)[:, None])): the bf16 grad_input of ratchet.py:136-141,
    the effective weight decoded once into a workspace in the GEMM's operand order."""
    return _ops().grad_input_bf16(g, packed, max_code, scale.float(), out_dtype)


def dequant_bf16(q: Tensor, s: Tensor) -> Tensor:
    """bf16(q) * bf16(s)[:, None] rounded to bf16, as ratchet.py:73-75 computes it."""
    return _ops().dequant_bf16(q, s)


def transpose_bf16(x: Tensor) -> Tensor:
    """bf16 transposed copy of a 2-D float32/bfloat16 tensor."""
    return _ops().transpose_bf16(x)


def dequant_transpose_bf16(q: Tensor, s: Tensor) -> Tensor:
    """(bf16(q) * bf16(s)[:, None])^T as a contiguous bf16 [K, M] tensor."""
    return _ops().dequant_transpose_bf16(q, s)


def grad_weight_splits(m: int, n: int, k: int) -> int:
    """Token-range split count the grad_weight kernels use by default."""
    return int(_ops().grad_weight_splits(m, n, k))


def grad_weight_bf16(grad: Tensor, q: Tensor, s: Tensor, nsplit: int | None = None, *,
                     work: Tensor | None = None, reduce: bool = True) -> Tensor:
    """Gw = bf16(bf16(grad)^T @ bf16(bf16(q) * bf16(s)[:, None])) as [N, K] bf16.

    The BF16 weight gradient of ratchet.py:148-163 computed straight from the saved int8
    activations (q [M, K], s [M]) and the upstream gradient grad [M, N] (float32 or
    bfloat16), with no transposed copies. ``reduce=False`` stops at the float32 split
    partials [nsplit, N, K], written to ``work`` (allocated when not given) and returned, for
    the update that reduces them itself; a bfloat16 [1, N, K] ``work`` receives the gradient
    itself (one split, written by the GEMM's epilogue).
    """
    if reduce:
        return _ops().grad_weight(grad, q, s, nsplit or 0)
    work = _partials_workspace(grad, q.shape[1], nsplit, work)
    _ops().grad_weight_partials(grad, q, s, work)
    return work


def grad_weight_bf16_x(grad: Tensor, x: Tensor, nsplit: int | None = None, *,
                       work: Tensor | None = None, reduce: bool = True) -> Tensor:
    """Gw = bf16(bf16(grad)^T @ bf16(x)) as [N, K] bf16, for activations x [M, K] given
    directly (float32 or bfloat16): the non-fused BF16 grad_weight of ratchet.py:159-163
    (``grad_out_tile.to(bf16) @ flat_inputs.to(bf16)``), or the fused one on a
    dequantized copy (dequant_bf16). ``work`` / ``reduce`` as in grad_weight_bf16."""
    if reduce:
        return _ops().grad_weight_x(grad, x, nsplit or 0)
    work = _partials_workspace(grad, x.shape[1], nsplit, work)
    _ops().grad_weight_partials_x(grad, x, work)
    return work


def grad_weight_parts_supported(parts: list[Tensor], q: Tensor) -> bool:
    """Shapes rk_grad_weight_bf16_parts takes: every part's columns a multiple of the output
    tile the kernel picks for [N, K] (256 where the large tiles apply, else 128)."""
    c, k = parts[0].shape[1], q.shape[1]
    n = c * len(parts)
    big = n >= 256 and k >= 256 and ((n + 255) // 256) * ((k + 255) // 256) >= 64
    feat = 256 if big else 128
    ld = parts[0].stride(0)
    return (c % feat == 0 and k % 16 == 0 and q.stride(-1) == 1
            and all(p.stride(-1) == 1 and p.stride(0) == ld and p.data_ptr() % 16 == 0
                    for p in parts)
            and (ld * parts[0].element_size()) % 16 == 0
            and (q.stride(0) * q.element_size()) % 16 == 0 and q.data_ptr() % 16 == 0)


def grad_weight_bf16_parts(parts: list[Tensor], x: Tensor, s: Tensor | None, *,
                           work: Tensor) -> Tensor:
    """grad_weight's float32 split partials for the gradient ``torch.cat(parts, dim=-1)``,
    read from the parts in place (the same partials as from the concatenation). x: the int8
    activations with their row scale s, or bf16 / float32 activations (s None)."""
    _ops().grad_weight_partials_parts(list(parts), x, s, work)
    return work


def _partials_workspace(grad: Tensor, k: int, nsplit: int | None,
                        work: Tensor | None) -> Tensor:
    if work is not None:
        return work
    m, n = grad.shape
    splits = nsplit or grad_weight_splits(m, n, k)
    return torch.empty((splits, n, k), device=grad.device, dtype=torch.float32)
