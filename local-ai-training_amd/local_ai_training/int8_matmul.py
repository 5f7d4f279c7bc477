"""int8 GEMM and per-token quantizers on gfx950, backed by libratchet_hip.so.

Drop-in for the reference module ``int8_matmul.py``: the public functions keep their
names, argument meaning, return dtypes and exception types
(``int8_matmul.py:251-343``). Compute runs only in the HIP library; CPU tensors are
rejected with RuntimeError exactly where the reference rejects them.

The ratchet layer uses the lower-level entry points below (``packed_int8_mm``,
``int8_mm_nt``, ``quantize_rows_into``) which skip the host-synchronizing scale
checks of the public ``scaled_int8_mm`` (``int8_matmul.py:305-309``).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _native as nat

_TINY = torch.finfo(torch.float32).tiny


def _ld(t: Tensor) -> int:
    """Row stride of a 2-D operand with unit column stride."""
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


def _sr_seed() -> int:
    # Host-side RNG, one draw per stochastic call, as int8_matmul.py:200 draws it: the
    # CPU generator's stream stays identical to the reference's.
    return int(torch.randint(0, 2**31 - 1, (1,)).item())


def quantize_rows_into(values: Tensor, out: Tensor, scale: Tensor, *,
                       col_scale: Tensor | None = None, stochastic: bool = False,
                       seed: int = 0, row_offset: int = 0,
                       bf16_out: Tensor | None = None) -> None:
    """Row-quantize a 2-D float32/bfloat16 tensor (any strides) into preallocated outputs."""
    m, k = values.shape
    nat.call(
        "rk_quantize_rows", values.data_ptr(), nat.dtype_code(values.dtype), m, k,
        values.stride(0), values.stride(1), nat.ptr(col_scale), int(stochastic), seed,
        row_offset, out.data_ptr(), _ld(out), scale.data_ptr(), nat.ptr(bf16_out),
        _ld(bf16_out) if bf16_out is not None else 0, nat.stream_handle(values.device),
    )


def _quantize_rows_fused(values: Tensor, col_scale: Tensor | None = None, *,
                         stochastic: bool = False) -> tuple[Tensor, Tensor]:
    """HIP row quantization; bit-exact with the reference's torch formula
    (``int8_matmul.py:225-239``), with Philox stochastic rounding when requested."""
    if values.ndim != 2:
        raise ValueError("row quantization requires a 2D tensor")
    nat.require_rocm(values, what="row quantization")
    if values.dtype not in (torch.float32, torch.bfloat16):
        values = values.float()
    m, k = values.shape
    out = torch.empty((m, k), device=values.device, dtype=torch.int8)
    scale = torch.empty((m,), device=values.device, dtype=torch.float32)
    seed = _sr_seed() if stochastic else 0
    if m and k:
        quantize_rows_into(values, out, scale, col_scale=col_scale, stochastic=stochastic,
                           seed=seed)
    return out, scale


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
               out_dtype: torch.dtype = torch.bfloat16, out: Tensor | None = None) -> Tensor:
    """C = bf16((A @ B^T) * a_scale[:, None] * b_scale[None, :]); A [M,K], B [N,K] int8.

    ``out_dtype`` float32 stores the bf16-rounded value widened (a fused `.float()`).
    No host synchronization.
    """
    m, k = a.shape
    n = b_nk.shape[0]
    if out is None:
        out = torch.empty((m, n), device=a.device, dtype=out_dtype)
    nat.call(
        "rk_int8_gemm_nt", a.data_ptr(), _ld(a), b_nk.data_ptr(), _ld(b_nk), a_scale.data_ptr(),
        nat.ptr(b_scale), out.data_ptr(), nat.dtype_code(out.dtype), _ld(out), m, n, k,
        nat.stream_handle(a.device),
    )
    return out


def packed_int8_mm(a: Tensor, packed: Tensor, max_code: int, a_scale: Tensor,
                   row_scale: Tensor | None, out_dtype: torch.dtype = torch.bfloat16,
                   out: Tensor | None = None) -> Tensor:
    """C = bf16((A @ code^T) * a_scale * row_scale) with code decoded from packed [N, K]."""
    m, k = a.shape
    n = packed.shape[0]
    if out is None:
        out = torch.empty((m, n), device=a.device, dtype=out_dtype)
    nat.call(
        "rk_int8_gemm_packed", a.data_ptr(), _ld(a), packed.data_ptr(), _ld(packed), max_code,
        a_scale.data_ptr(), nat.ptr(row_scale), out.data_ptr(), nat.dtype_code(out.dtype),
        _ld(out), m, n, k, nat.stream_handle(a.device),
    )
    return out


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
    float32 add as adding afterwards)."""
    m, k = a.shape
    n = packed.shape[0]
    if out is None:
        out = torch.empty((m, n), device=a.device, dtype=torch.float32)
    nat.call(
        "rk_int8_gemm_packed_residual", a.data_ptr(), _ld(a), packed.data_ptr(), _ld(packed),
        max_code, a_scale.data_ptr(), nat.ptr(row_scale), residual.data_ptr(), _ld(residual),
        out.data_ptr(), _ld(out), m, n, k, nat.stream_handle(a.device),
    )
    return out


def packed_t_supported(a: Tensor, packed: Tensor) -> bool:
    """Whether packed_int8_mm_t can run on these operands (aligned shapes)."""
    k, n = packed.shape
    return (k % 64 == 0 and n % 8 == 0 and a.stride(-1) == 1 and packed.stride(-1) == 1
            and _ld(a) % 16 == 0 and _ld(packed) % 16 == 0 and a.data_ptr() % 16 == 0
            and packed.data_ptr() % 16 == 0)


def packed_int8_mm_t(a: Tensor, packed: Tensor, max_code: int, a_scale: Tensor,
                     row_scale: Tensor | None, out_dtype: torch.dtype = torch.bfloat16,
                     out: Tensor | None = None) -> Tensor:
    """C = bf16((A @ code) * a_scale * row_scale) with code = decode(packed) as the [K, N]
    operand (A [M, K] int8, packed [K, N]): the grad_input GEMM against the packed state,
    without an unpacked or transposed copy of the codes."""
    m, k = a.shape
    n = packed.shape[1]
    if out is None:
        out = torch.empty((m, n), device=a.device, dtype=out_dtype)
    nat.call(
        "rk_int8_gemm_packed_t", a.data_ptr(), _ld(a), packed.data_ptr(), _ld(packed),
        max_code, a_scale.data_ptr(), nat.ptr(row_scale), out.data_ptr(),
        nat.dtype_code(out.dtype), _ld(out), m, n, k, nat.stream_handle(a.device),
    )
    return out


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
    a = lhs if lhs.stride(1) == 1 or k <= 1 else lhs.contiguous()
    b_nk = rhs.t()
    if b_nk.stride(1) != 1 and k > 1:
        b_nk = b_nk.contiguous()
    return int8_mm_nt(a, b_nk, lhs_scale.contiguous(), rhs_scale.contiguous())


def unpack_transpose(packed: Tensor, max_code: int) -> Tensor:
    """codeT[k, n] = code[n, k] as a contiguous int8 [K, N] tensor."""
    n, k = packed.shape
    out = torch.empty((k, n), device=packed.device, dtype=torch.int8)
    nat.call("rk_unpack_transpose", packed.data_ptr(), _ld(packed), max_code, out.data_ptr(),
             _ld(out), n, k, nat.stream_handle(packed.device))
    return out


def effective_bf16(packed: Tensor, max_code: int, scale: Tensor) -> Tensor:
    """bf16(code) * bf16(scale)[:, None] rounded to bf16, as ratchet.py:140 computes it."""
    n, k = packed.shape
    out = torch.empty((n, k), device=packed.device, dtype=torch.bfloat16)
    nat.call("rk_effective_bf16", packed.data_ptr(), _ld(packed), max_code,
             scale.float().contiguous().data_ptr(), out.data_ptr(), _ld(out), n, k,
             nat.stream_handle(packed.device))
    return out


def dequant_bf16(q: Tensor, s: Tensor) -> Tensor:
    """bf16(q) * bf16(s)[:, None] rounded to bf16, as ratchet.py:73-75 computes it."""
    m, k = q.shape
    out = torch.empty((m, k), device=q.device, dtype=torch.bfloat16)
    nat.call("rk_dequant_bf16", q.data_ptr(), _ld(q), s.data_ptr(), out.data_ptr(), _ld(out),
             m, k, nat.stream_handle(q.device))
    return out


def transpose_bf16(x: Tensor) -> Tensor:
    """bf16 transposed copy of a 2-D float32/bfloat16 tensor (unit column stride)."""
    if x.stride(-1) != 1:
        x = x.contiguous()
    m, n = x.shape
    out = torch.empty((n, m), device=x.device, dtype=torch.bfloat16)
    nat.call("rk_transpose_bf16", x.data_ptr(), nat.dtype_code(x.dtype), _ld(x), out.data_ptr(),
             _ld(out), m, n, nat.stream_handle(x.device))
    return out


def dequant_transpose_bf16(q: Tensor, s: Tensor) -> Tensor:
    """(bf16(q) * bf16(s)[:, None])^T as a contiguous bf16 [K, M] tensor."""
    m, k = q.shape
    out = torch.empty((k, m), device=q.device, dtype=torch.bfloat16)
    nat.call("rk_dequant_transpose_bf16", q.data_ptr(), _ld(q), s.data_ptr(), out.data_ptr(),
             _ld(out), m, k, nat.stream_handle(q.device))
    return out


def grad_weight_splits(m: int, n: int, k: int) -> int:
    """Token-range split count rk_grad_weight_bf16 uses by default."""
    return int(nat.load_library().rk_grad_weight_splits(m, n, k))


def grad_weight_bf16(grad: Tensor, q: Tensor, s: Tensor, nsplit: int | None = None, *,
                     out: Tensor | None = None, work: Tensor | None = None,
                     reduce: bool = True) -> Tensor:
    """Gw = bf16(bf16(grad)^T @ bf16(bf16(q) * bf16(s)[:, None])) as [N, K] bf16.

    The BF16 weight gradient of ratchet.py:148-163 computed straight from the saved int8
    activations (q [M, K], s [M]) and the upstream gradient grad [M, N] (float32 or
    bfloat16), with no transposed copies. ``work`` (float32 [nsplit, N, K]) and ``out``
    may be passed preallocated. ``reduce=False`` stops at the split partials and returns
    ``work`` (for rk_ratchet_update_partials, which reduces them inside the update).
    """
    m, n = grad.shape
    k = q.shape[1]
    if grad.stride(-1) != 1:
        grad = grad.contiguous()
    if q.stride(-1) != 1:
        q = q.contiguous()
    splits = nsplit or (work.shape[0] if work is not None else grad_weight_splits(m, n, k))
    if work is None:
        work = torch.empty((splits, n, k), device=grad.device, dtype=torch.float32)
    if out is None and reduce:
        out = torch.empty((n, k), device=grad.device, dtype=torch.bfloat16)
    nat.call("rk_grad_weight_bf16", grad.data_ptr(), nat.dtype_code(grad.dtype), _ld(grad),
             q.data_ptr(), _ld(q), s.contiguous().data_ptr(), m, n, k, work.data_ptr(), splits,
             nat.ptr(out) if reduce else None, _ld(out) if reduce else k,
             nat.stream_handle(grad.device))
    return out if reduce else work


def grad_weight_bf16_x(grad: Tensor, x: Tensor, nsplit: int | None = None, *,
                       out: Tensor | None = None, work: Tensor | None = None,
                       reduce: bool = True) -> Tensor:
    """Gw = bf16(bf16(grad)^T @ bf16(x)) as [N, K] bf16, for activations x [M, K] given
    directly (float32 or bfloat16): the non-fused BF16 grad_weight of ratchet.py:159-163
    (``grad_out_tile.to(bf16) @ flat_inputs.to(bf16)``), or the fused one on a
    dequantized copy (dequant_bf16). ``work`` / ``out`` / ``reduce`` as in
    grad_weight_bf16."""
    m, n = grad.shape
    k = x.shape[1]
    if grad.stride(-1) != 1:
        grad = grad.contiguous()
    if x.stride(-1) != 1:
        x = x.contiguous()
    splits = nsplit or (work.shape[0] if work is not None else grad_weight_splits(m, n, k))
    if work is None:
        work = torch.empty((splits, n, k), device=grad.device, dtype=torch.float32)
    if out is None and reduce:
        out = torch.empty((n, k), device=grad.device, dtype=torch.bfloat16)
    nat.call("rk_grad_weight_bf16_x", grad.data_ptr(), nat.dtype_code(grad.dtype), _ld(grad),
             x.data_ptr(), nat.dtype_code(x.dtype), _ld(x), m, n, k, work.data_ptr(), splits,
             nat.ptr(out) if reduce else None, _ld(out) if reduce else k,
             nat.stream_handle(grad.device))
    return out if reduce else work
