// ratchet_torch_ops.cpp — the torch.ops.ratchet.* operators of the ratchet-linear path.
//
// A thin registration layer: every operator reads its tensors' pointers, sizes and strides,
// picks torch's current HIP stream for the tensors' device, and calls one entry point of
// libratchet_hip.so (include/ratchet_hip.h). No arithmetic happens here; this library links
// against torch, the kernel library does not.
//
// Conventions:
//   - Functional operators allocate their results with torch's caching allocator
//     (at::empty on the operands' device), so they are legal under HIP-graph capture.
//   - Mutating operators declare every argument they write as Tensor(x!) and return
//     nothing; they never alias an input to an output.
//   - A failing entry point raises RuntimeError with the library's message, so callers see
//     the reference's exception type (RuntimeError) for a rejected launch.
//
// The Python side (local_ai_training/ops.py) registers the fake (meta) kernels and keeps
// the reference's function names on top (int8_matmul.py, int8_fused.py, int8_backward.py,
// ratchet.py).

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <optional>
#include <utility>
#include <vector>

#include "ratchet_hip.h"

namespace {

using at::Tensor;
using OptTensor = std::optional<Tensor>;

void check_status(int status, const char* entry) {
  TORCH_CHECK(status == RK_OK, entry, " failed (status ", status, "): ", rk_last_error());
}

void* stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void require_gpu(const Tensor& t, const char* what) {
  TORCH_CHECK(t.is_cuda(), what, " requires CUDA (a ROCm GPU); the int8 path is GPU-only");
}

void same_device(const Tensor& a, const Tensor& b, const char* what) {
  TORCH_CHECK(a.device() == b.device(), what, ": operands must share a device");
}

// Row stride of a 2-D operand whose columns are contiguous.
int64_t ld(const Tensor& t) { return t.size(0) > 1 ? t.stride(0) : t.size(1); }

Tensor unit_columns(const Tensor& t) {
  return (t.dim() == 2 && (t.stride(1) == 1 || t.size(1) <= 1)) ? t : t.contiguous();
}

int dtype_code(const Tensor& t, const char* what) {
  if (t.scalar_type() == at::kFloat) return RK_F32;
  if (t.scalar_type() == at::kBFloat16) return RK_BF16;
  TORCH_CHECK(false, what, ": expected float32 or bfloat16, got ", t.scalar_type());
}

int dtype_code(at::ScalarType s) {
  TORCH_CHECK(s == at::kFloat || s == at::kBFloat16,
              "output dtype must be float32 or bfloat16, got ", s);
  return s == at::kFloat ? RK_F32 : RK_BF16;
}

template <typename T>
T* ptr(const OptTensor& t) {
  return t.has_value() ? static_cast<T*>(t->data_ptr()) : nullptr;
}

Tensor f32_vector(const Tensor& v, int64_t n, const char* what) {
  TORCH_CHECK(v.dim() == 1 && v.size(0) == n, what, " must be 1-D with ", n, " entries");
  TORCH_CHECK(v.scalar_type() == at::kFloat, what, " must be float32");
  return v.contiguous();
}

OptTensor f32_vector(const OptTensor& v, int64_t n, const char* what) {
  if (!v.has_value()) return std::nullopt;
  return f32_vector(*v, n, what);
}

void int8_matrix(const Tensor& t, const char* what) {
  TORCH_CHECK(t.dim() == 2 && t.scalar_type() == at::kChar, what, " must be a 2-D int8 matrix");
}

void packed_matrix(const Tensor& t) {
  TORCH_CHECK(t.dim() == 2 && t.scalar_type() == at::kByte,
              "packed ratchet state must be a 2-D uint8 matrix");
  TORCH_CHECK(t.stride(1) == 1 || t.size(1) <= 1, "packed state must have unit column stride");
}

// ---------------------------------------------------------------------------------------
// Row quantization (int8_matmul.py:106-150, 181-207, 251-277)
// ---------------------------------------------------------------------------------------
std::tuple<Tensor, Tensor> quantize_rows(const Tensor& x, const OptTensor& col_scale,
                                         bool stochastic, int64_t seed,
                                         const OptTensor& seed_slot, int64_t row_offset,
                                         const OptTensor& x_bf16, bool round_bf16) {
  require_gpu(x, "row quantization");
  TORCH_CHECK(x.dim() == 2, "row quantization requires a 2D tensor");
  int code = dtype_code(x, "row quantization input");
  // round_bf16: a float32 input is quantized as x.to(bfloat16) (no effect on bf16 inputs)
  if (round_bf16 && code == RK_F32) code = RK_F32_AS_BF16;
  const c10::DeviceGuard guard(x.device());
  const int64_t m = x.size(0), k = x.size(1);
  Tensor q = at::empty({m, k}, x.options().dtype(at::kChar));
  Tensor scale = at::empty({m}, x.options().dtype(at::kFloat));
  const OptTensor cs = f32_vector(col_scale, k, "col_scale");
  uint16_t* xb = nullptr;
  int64_t ld_xb = 0;
  if (x_bf16.has_value()) {
    TORCH_CHECK(x_bf16->scalar_type() == at::kBFloat16 && x_bf16->dim() == 2 &&
                    x_bf16->size(0) == m && x_bf16->size(1) == k &&
                    (x_bf16->stride(1) == 1 || k <= 1),
                "x_bf16 must be a bfloat16 [M, K] matrix with unit column stride");
    xb = static_cast<uint16_t*>(x_bf16->data_ptr());
    ld_xb = ld(*x_bf16);
  }
  if (m == 0 || k == 0) return {q, scale};
  if (seed_slot.has_value()) {
    TORCH_CHECK(stochastic, "a device seed applies to stochastic rounding only");
    TORCH_CHECK(seed_slot->scalar_type() == at::kLong && seed_slot->numel() == 1 &&
                    seed_slot->device() == x.device(),
                "seed_slot must be one int64 on the input's device");
    check_status(rk_quantize_rows_devseed(x.data_ptr(), code, m, k, x.stride(0), x.stride(1),
                                          ptr<const float>(cs),
                                          static_cast<const int64_t*>(seed_slot->data_ptr()),
                                          row_offset, q.data_ptr<int8_t>(), k,
                                          scale.data_ptr<float>(), xb, ld_xb, stream_of(x)),
                 "rk_quantize_rows_devseed");
  } else {
    check_status(rk_quantize_rows(x.data_ptr(), code, m, k, x.stride(0), x.stride(1),
                                  ptr<const float>(cs), stochastic ? 1 : 0,
                                  static_cast<uint64_t>(seed), row_offset, q.data_ptr<int8_t>(),
                                  k, scale.data_ptr<float>(), xb, ld_xb, stream_of(x)),
                 "rk_quantize_rows");
  }
  return {q, scale};
}

// ---------------------------------------------------------------------------------------
// int8 GEMMs (int8_matmul.py:26-79, 289-343; ratchet.py:46-67, 133-134)
// ---------------------------------------------------------------------------------------
struct GemmOperands {
  Tensor a, b, ls;
  OptTensor rs;
};

GemmOperands gemm_operands(const Tensor& a, const Tensor& b, const Tensor& a_scale,
                           const OptTensor& rs, int64_t n) {
  require_gpu(a, "int8 ratchet matmul");
  int8_matrix(a, "A");
  same_device(a, b, "int8 ratchet matmul");
  GemmOperands g{unit_columns(a), b, f32_vector(a_scale, a.size(0), "row scale of A"),
                 f32_vector(rs, n, "column scale")};
  return g;
}

Tensor int8_mm_nt(const Tensor& a, const Tensor& b_nk, const Tensor& a_scale,
                  const OptTensor& b_scale, at::ScalarType out_dtype) {
  int8_matrix(b_nk, "B");
  TORCH_CHECK(a.size(1) == b_nk.size(1), "int8_mm_nt inner dimensions must match");
  const int64_t m = a.size(0), k = a.size(1), n = b_nk.size(0);
  GemmOperands g = gemm_operands(a, b_nk, a_scale, b_scale, n);
  g.b = unit_columns(b_nk);
  const c10::DeviceGuard guard(a.device());
  Tensor out = at::empty({m, n}, a.options().dtype(out_dtype));
  if (m == 0 || n == 0) return out;
  check_status(rk_int8_gemm_nt(g.a.data_ptr<int8_t>(), ld(g.a), g.b.data_ptr<int8_t>(), ld(g.b),
                               g.ls.data_ptr<float>(), ptr<const float>(g.rs), out.data_ptr(),
                               dtype_code(out_dtype), n, m, n, k, stream_of(a)),
               "rk_int8_gemm_nt");
  return out;
}

Tensor packed_mm(const Tensor& a, const Tensor& packed, int64_t max_code, const Tensor& a_scale,
                 const OptTensor& row_scale, at::ScalarType out_dtype) {
  packed_matrix(packed);
  TORCH_CHECK(a.size(1) == packed.size(1), "packed_mm: A has ", a.size(1),
              " columns, the packed state ", packed.size(1));
  const int64_t m = a.size(0), k = a.size(1), n = packed.size(0);
  GemmOperands g = gemm_operands(a, packed, a_scale, row_scale, n);
  const c10::DeviceGuard guard(a.device());
  Tensor out = at::empty({m, n}, a.options().dtype(out_dtype));
  if (m == 0 || n == 0) return out;
  check_status(rk_int8_gemm_packed(g.a.data_ptr<int8_t>(), ld(g.a), packed.data_ptr<uint8_t>(),
                                   ld(packed), static_cast<int>(max_code),
                                   g.ls.data_ptr<float>(), ptr<const float>(g.rs),
                                   out.data_ptr(), dtype_code(out_dtype), n, m, n, k,
                                   stream_of(a)),
               "rk_int8_gemm_packed");
  return out;
}

void residual_launch(const GemmOperands& g, const Tensor& packed, int64_t max_code,
                     const Tensor& residual, const Tensor& out) {
  const int64_t m = g.a.size(0), k = g.a.size(1), n = packed.size(0);
  if (m == 0 || n == 0) return;
  check_status(rk_int8_gemm_packed_residual(
                   g.a.data_ptr<int8_t>(), ld(g.a), packed.data_ptr<uint8_t>(), ld(packed),
                   static_cast<int>(max_code), g.ls.data_ptr<float>(), ptr<const float>(g.rs),
                   residual.data_ptr<float>(), ld(residual), out.data_ptr<float>(), ld(out), m,
                   n, k, stream_of(g.a)),
               "rk_int8_gemm_packed_residual");
}

void check_residual(const Tensor& r, int64_t m, int64_t n) {
  TORCH_CHECK(r.scalar_type() == at::kFloat && r.dim() == 2 && r.size(0) == m &&
                  r.size(1) == n && (r.stride(1) == 1 || n <= 1),
              "residual must be a float32 [M, N] matrix with unit column stride");
}

Tensor packed_mm_residual(const Tensor& a, const Tensor& packed, int64_t max_code,
                          const Tensor& a_scale, const OptTensor& row_scale,
                          const Tensor& residual) {
  packed_matrix(packed);
  TORCH_CHECK(a.size(1) == packed.size(1), "packed_mm_residual inner dimensions must match");
  const int64_t m = a.size(0), n = packed.size(0);
  check_residual(residual, m, n);
  GemmOperands g = gemm_operands(a, packed, a_scale, row_scale, n);
  const c10::DeviceGuard guard(a.device());
  Tensor out = at::empty({m, n}, a.options().dtype(at::kFloat));
  residual_launch(g, packed, max_code, residual, out);
  return out;
}

void packed_mm_accumulate(const Tensor& a, const Tensor& packed, int64_t max_code,
                          const Tensor& a_scale, const OptTensor& row_scale, Tensor& acc) {
  packed_matrix(packed);
  TORCH_CHECK(a.size(1) == packed.size(1), "packed_mm_accumulate inner dimensions must match");
  const int64_t m = a.size(0), n = packed.size(0);
  check_residual(acc, m, n);
  GemmOperands g = gemm_operands(a, packed, a_scale, row_scale, n);
  const c10::DeviceGuard guard(a.device());
  residual_launch(g, packed, max_code, acc, acc);
}

Tensor packed_mm_t(const Tensor& a, const Tensor& packed, int64_t max_code,
                   const Tensor& a_scale, const OptTensor& row_scale,
                   at::ScalarType out_dtype) {
  packed_matrix(packed);
  TORCH_CHECK(a.size(1) == packed.size(0), "packed_mm_t: A has ", a.size(1),
              " columns, the packed state ", packed.size(0), " rows");
  const int64_t m = a.size(0), k = a.size(1), n = packed.size(1);
  GemmOperands g = gemm_operands(a, packed, a_scale, row_scale, n);
  const c10::DeviceGuard guard(a.device());
  Tensor out = at::empty({m, n}, a.options().dtype(out_dtype));
  if (m == 0 || n == 0) return out;
  check_status(rk_int8_gemm_packed_t(g.a.data_ptr<int8_t>(), ld(g.a), packed.data_ptr<uint8_t>(),
                                     ld(packed), static_cast<int>(max_code),
                                     g.ls.data_ptr<float>(), ptr<const float>(g.rs),
                                     out.data_ptr(), dtype_code(out_dtype), n, m, n, k,
                                     stream_of(a)),
               "rk_int8_gemm_packed_t");
  return out;
}

// ---------------------------------------------------------------------------------------
// Packed-state transforms (ratchet.py:52, 61, 73-75, 140, 195-199)
// ---------------------------------------------------------------------------------------
Tensor unpack_transpose(const Tensor& packed, int64_t max_code) {
  require_gpu(packed, "unpack_transpose");
  packed_matrix(packed);
  const c10::DeviceGuard guard(packed.device());
  const int64_t n = packed.size(0), k = packed.size(1);
  Tensor out = at::empty({k, n}, packed.options().dtype(at::kChar));
  if (n == 0 || k == 0) return out;
  check_status(rk_unpack_transpose(packed.data_ptr<uint8_t>(), ld(packed),
                                   static_cast<int>(max_code), out.data_ptr<int8_t>(), n, n, k,
                                   stream_of(packed)),
               "rk_unpack_transpose");
  return out;
}

std::tuple<Tensor, Tensor> unpack(const Tensor& packed, int64_t max_code) {
  require_gpu(packed, "unpack");
  TORCH_CHECK(packed.scalar_type() == at::kByte, "packed ratchet state must be uint8");
  const c10::DeviceGuard guard(packed.device());
  const Tensor flat = packed.contiguous();
  Tensor code = at::empty(packed.sizes(), packed.options().dtype(at::kChar));
  Tensor pressure = at::empty(packed.sizes(), packed.options().dtype(at::kChar));
  if (flat.numel() == 0) return {code, pressure};
  check_status(rk_unpack(flat.data_ptr<uint8_t>(), flat.numel(), static_cast<int>(max_code),
                         code.data_ptr<int8_t>(), pressure.data_ptr<int8_t>(), stream_of(flat)),
               "rk_unpack");
  return {code, pressure};
}

Tensor effective_bf16(const Tensor& packed, int64_t max_code, const Tensor& scale) {
  require_gpu(packed, "effective_bf16");
  packed_matrix(packed);
  const int64_t n = packed.size(0), k = packed.size(1);
  const Tensor s = f32_vector(scale, n, "row scale");
  const c10::DeviceGuard guard(packed.device());
  Tensor out = at::empty({n, k}, packed.options().dtype(at::kBFloat16));
  if (n == 0 || k == 0) return out;
  check_status(rk_effective_bf16(packed.data_ptr<uint8_t>(), ld(packed),
                                 static_cast<int>(max_code), s.data_ptr<float>(),
                                 static_cast<uint16_t*>(out.data_ptr()), k, n, k,
                                 stream_of(packed)),
               "rk_effective_bf16");
  return out;
}

// The bf16 grad_input against the packed state (rk_grad_input_bf16): out =
// bf16(g @ (bf16(code) * bf16(scale)[:, None])), the effective weight decoded into a
// workspace from torch's allocator in the GEMM's operand order.
Tensor grad_input_bf16(const Tensor& g_in, const Tensor& packed, int64_t max_code,
                       const Tensor& scale, at::ScalarType out_dtype) {
  require_gpu(g_in, "bf16 grad_input");
  packed_matrix(packed);
  same_device(g_in, packed, "bf16 grad_input");
  TORCH_CHECK(g_in.scalar_type() == at::kBFloat16 && g_in.dim() == 2,
              "bf16 grad_input: the gradient must be a bfloat16 matrix");
  TORCH_CHECK(out_dtype == at::kFloat || out_dtype == at::kBFloat16,
              "bf16 grad_input: output dtype must be float32 or bfloat16");
  const Tensor g = unit_columns(g_in);
  const int64_t m = g.size(0), n = g.size(1), k = packed.size(1);
  TORCH_CHECK(packed.size(0) == n, "bf16 grad_input: the gradient has ", n,
              " columns, the packed state ", packed.size(0), " rows");
  const Tensor s = f32_vector(scale, n, "row scale");
  const c10::DeviceGuard guard(g.device());
  Tensor out = at::empty({m, k}, g.options().dtype(out_dtype));
  if (m == 0 || k == 0) return out;
  const int64_t work_bytes = rk_grad_input_bf16_workspace(n, k);
  const Tensor work = at::empty({work_bytes > 0 ? work_bytes : 1}, g.options().dtype(at::kByte));
  check_status(rk_grad_input_bf16(static_cast<const uint16_t*>(g.data_ptr()), ld(g),
                                  packed.data_ptr<uint8_t>(), ld(packed),
                                  static_cast<int>(max_code), s.data_ptr<float>(),
                                  out.data_ptr(), dtype_code(out_dtype), k, m, n, k,
                                  work.data_ptr(), work_bytes, stream_of(g)),
               "rk_grad_input_bf16");
  return out;
}

Tensor dequant_bf16(const Tensor& q_in, const Tensor& s_in) {
  require_gpu(q_in, "dequant_bf16");
  int8_matrix(q_in, "q");
  const Tensor q = unit_columns(q_in);
  const int64_t m = q.size(0), k = q.size(1);
  const Tensor s = f32_vector(s_in, m, "row scale");
  const c10::DeviceGuard guard(q.device());
  Tensor out = at::empty({m, k}, q.options().dtype(at::kBFloat16));
  if (m == 0 || k == 0) return out;
  check_status(rk_dequant_bf16(q.data_ptr<int8_t>(), ld(q), s.data_ptr<float>(),
                               static_cast<uint16_t*>(out.data_ptr()), k, m, k, stream_of(q)),
               "rk_dequant_bf16");
  return out;
}

Tensor transpose_bf16(const Tensor& x_in) {
  require_gpu(x_in, "transpose_bf16");
  TORCH_CHECK(x_in.dim() == 2, "transpose_bf16 takes a 2-D tensor");
  const Tensor x = unit_columns(x_in);
  const int code = dtype_code(x, "transpose_bf16 input");
  const c10::DeviceGuard guard(x.device());
  const int64_t m = x.size(0), n = x.size(1);
  Tensor out = at::empty({n, m}, x.options().dtype(at::kBFloat16));
  if (m == 0 || n == 0) return out;
  check_status(rk_transpose_bf16(x.data_ptr(), code, ld(x),
                                 static_cast<uint16_t*>(out.data_ptr()), m, m, n, stream_of(x)),
               "rk_transpose_bf16");
  return out;
}

Tensor dequant_transpose_bf16(const Tensor& q_in, const Tensor& s_in) {
  require_gpu(q_in, "dequant_transpose_bf16");
  int8_matrix(q_in, "q");
  const Tensor q = unit_columns(q_in);
  const int64_t m = q.size(0), k = q.size(1);
  const Tensor s = f32_vector(s_in, m, "row scale");
  const c10::DeviceGuard guard(q.device());
  Tensor out = at::empty({k, m}, q.options().dtype(at::kBFloat16));
  if (m == 0 || k == 0) return out;
  check_status(rk_dequant_transpose_bf16(q.data_ptr<int8_t>(), ld(q), s.data_ptr<float>(),
                                         static_cast<uint16_t*>(out.data_ptr()), m, m, k,
                                         stream_of(q)),
               "rk_dequant_transpose_bf16");
  return out;
}

// ---------------------------------------------------------------------------------------
// BF16 grad_weight (ratchet.py:148-163)
// ---------------------------------------------------------------------------------------
int64_t grad_weight_splits(int64_t m, int64_t n, int64_t k) {
  return rk_grad_weight_splits(m, n, k);
}

void check_gradient(const Tensor& g, int64_t m) {
  TORCH_CHECK(g.dim() == 2 && g.size(0) == m, "upstream gradient must be [M, N] with M = ", m);
}

void check_workspace(const Tensor& work, int64_t n, int64_t k) {
  TORCH_CHECK(work.scalar_type() == at::kFloat && work.dim() == 3 && work.size(1) == n &&
                  work.size(2) == k && work.is_contiguous() && work.size(0) >= 1,
              "grad_weight workspace must be a contiguous float32 [nsplit, N, K] tensor");
}

// The work tensor of the partials operators: float32 [nsplit, N, K] split partials, or a
// bfloat16 [1, N, K] tensor that receives the gradient itself (one split, written by the
// GEMM's epilogue: the values rk_ratchet_update_partials would form from one split).
bool direct_workspace(const Tensor& work, int64_t n, int64_t k) {
  if (work.scalar_type() != at::kBFloat16) {
    check_workspace(work, n, k);
    return false;
  }
  TORCH_CHECK(work.dim() == 3 && work.size(0) == 1 && work.size(1) == n && work.size(2) == k &&
                  work.is_contiguous(),
              "a bfloat16 grad_weight work tensor must be a contiguous [1, N, K] tensor");
  return true;
}

// work: float32 split partials (out, when given, receives their bf16 sum), or null with one
// split and out given (the bf16 gradient written directly)
void grad_weight_launch(const Tensor& g_in, const Tensor& act, bool int8_act,
                        const OptTensor& s, float* work, int nsplit, uint16_t* out) {
  const Tensor g = unit_columns(g_in);
  const Tensor x = unit_columns(act);
  const int64_t m = g.size(0), n = g.size(1), k = x.size(1);
  const int gcode = dtype_code(g, "upstream gradient");
  if (int8_act) {
    const Tensor sv = f32_vector(*s, m, "activation row scale");
    check_status(rk_grad_weight_bf16(g.data_ptr(), gcode, ld(g), x.data_ptr<int8_t>(), ld(x),
                                     sv.data_ptr<float>(), m, n, k, work, nsplit, out, k,
                                     stream_of(g)),
                 "rk_grad_weight_bf16");
  } else {
    check_status(rk_grad_weight_bf16_x(g.data_ptr(), gcode, ld(g), x.data_ptr(),
                                       dtype_code(x, "activations"), ld(x), m, n, k, work,
                                       nsplit, out, k, stream_of(g)),
                 "rk_grad_weight_bf16_x");
  }
}

Tensor grad_weight_common(const Tensor& g, const Tensor& act, bool int8_act, const OptTensor& s,
                          int64_t nsplit) {
  require_gpu(g, "grad_weight");
  same_device(g, act, "grad_weight");
  check_gradient(g, act.size(0));
  const c10::DeviceGuard guard(g.device());
  const int64_t m = g.size(0), n = g.size(1), k = act.size(1);
  Tensor out = at::empty({n, k}, g.options().dtype(at::kBFloat16));
  if (n == 0 || k == 0) return out;
  const int64_t splits = nsplit > 0 ? nsplit : grad_weight_splits(m, n, k);
  // one split writes the bf16 gradient directly and needs no float32 workspace
  Tensor work = splits > 1 ? at::empty({splits, n, k}, g.options().dtype(at::kFloat)) : Tensor();
  grad_weight_launch(g, act, int8_act, s, splits > 1 ? work.data_ptr<float>() : nullptr,
                     static_cast<int>(splits), static_cast<uint16_t*>(out.data_ptr()));
  return out;
}

Tensor grad_weight(const Tensor& g, const Tensor& q, const Tensor& s, int64_t nsplit) {
  int8_matrix(q, "q");
  return grad_weight_common(g, q, true, s, nsplit);
}

Tensor grad_weight_x(const Tensor& g, const Tensor& x, int64_t nsplit) {
  TORCH_CHECK(x.dim() == 2, "activations must be a 2-D matrix");
  return grad_weight_common(g, x, false, std::nullopt, nsplit);
}

void grad_weight_partials_common(const Tensor& g, const Tensor& act, bool int8_act,
                                 const OptTensor& s, Tensor& work) {
  require_gpu(g, "grad_weight");
  same_device(g, act, "grad_weight");
  check_gradient(g, act.size(0));
  const bool direct = direct_workspace(work, g.size(1), act.size(1));
  const c10::DeviceGuard guard(g.device());
  if (g.size(1) == 0 || act.size(1) == 0) return;
  if (direct)
    grad_weight_launch(g, act, int8_act, s, nullptr, 1, static_cast<uint16_t*>(work.data_ptr()));
  else
    grad_weight_launch(g, act, int8_act, s, work.data_ptr<float>(),
                       static_cast<int>(work.size(0)), nullptr);
}

void grad_weight_partials(const Tensor& g, const Tensor& q, const Tensor& s, Tensor& work) {
  int8_matrix(q, "q");
  grad_weight_partials_common(g, q, true, s, work);
}

// The parts of one gradient row split by columns (the attention's q, k, v gradients), each
// [M, C] with unit column stride and one shared row stride.
struct Parts {
  const void* p[3] = {nullptr, nullptr, nullptr};
  int n = 0;
  int64_t cols = 0, ld = 0, rows = 0;
  int dtype = RK_F32;
};

Parts gradient_parts(const std::vector<Tensor>& parts, const char* what) {
  TORCH_CHECK(parts.size() >= 1 && parts.size() <= 3, what, ": 1 to 3 parts");
  Parts r;
  r.n = static_cast<int>(parts.size());
  for (int i = 0; i < r.n; ++i) {
    const Tensor& t = parts[i];
    require_gpu(t, what);
    TORCH_CHECK(t.dim() == 2 && t.stride(1) == 1, what, ": parts must be [M, C] with unit column stride");
    if (i == 0) {
      r.rows = t.size(0);
      r.cols = t.size(1);
      r.ld = t.size(0) > 1 ? t.stride(0) : t.size(1);
      r.dtype = dtype_code(t, what);
    } else {
      TORCH_CHECK(t.size(0) == r.rows && t.size(1) == r.cols && t.device() == parts[0].device() &&
                      t.scalar_type() == parts[0].scalar_type() &&
                      (t.size(0) <= 1 || t.stride(0) == r.ld),
                  what, ": parts must share shape, dtype, device and row stride");
    }
    r.p[i] = t.data_ptr();
  }
  return r;
}

std::tuple<Tensor, Tensor> quantize_rows_parts(const std::vector<Tensor>& parts,
                                               const OptTensor& col_scale, bool stochastic,
                                               int64_t seed, const OptTensor& seed_slot,
                                               int64_t row_offset) {
  const Parts g = gradient_parts(parts, "row quantization");
  const int64_t m = g.rows, k = g.n * g.cols;
  const c10::DeviceGuard guard(parts[0].device());
  Tensor q = at::empty({m, k}, parts[0].options().dtype(at::kChar));
  Tensor scale = at::empty({m}, parts[0].options().dtype(at::kFloat));
  const OptTensor cs = f32_vector(col_scale, k, "col_scale");
  if (m == 0 || k == 0) return {q, scale};
  const int64_t* slot = nullptr;
  if (seed_slot.has_value()) {
    TORCH_CHECK(stochastic, "a device seed applies to stochastic rounding only");
    TORCH_CHECK(seed_slot->scalar_type() == at::kLong && seed_slot->numel() == 1 &&
                    seed_slot->device() == parts[0].device(),
                "seed_slot must be one int64 on the input's device");
    slot = static_cast<const int64_t*>(seed_slot->data_ptr());
  }
  check_status(rk_quantize_rows_parts(g.p[0], g.p[1], g.p[2], g.n, g.cols, g.dtype, m, g.ld,
                                      ptr<const float>(cs), stochastic ? 1 : 0,
                                      static_cast<uint64_t>(seed), slot, row_offset,
                                      q.data_ptr<int8_t>(), k, scale.data_ptr<float>(),
                                      stream_of(parts[0])),
               "rk_quantize_rows_parts");
  return {q, scale};
}

// x: int8 activations with their row scale s, or float32 / bfloat16 activations (s None)
void grad_weight_partials_parts(const std::vector<Tensor>& parts, const Tensor& x_in,
                                const OptTensor& s, Tensor& work) {
  const Parts g = gradient_parts(parts, "grad_weight");
  TORCH_CHECK(x_in.dim() == 2, "activations must be a 2-D matrix");
  const bool int8_act = x_in.scalar_type() == at::kChar;
  TORCH_CHECK(int8_act == s.has_value(),
              "grad_weight: int8 activations take a row scale, float activations none");
  const Tensor x = unit_columns(x_in);
  TORCH_CHECK(x.size(0) == g.rows, "activations must have the gradient's rows");
  same_device(parts[0], x, "grad_weight");
  const int64_t m = g.rows, n = g.n * g.cols, k = x.size(1);
  const bool direct = direct_workspace(work, n, k);
  const c10::DeviceGuard guard(x.device());
  if (n == 0 || k == 0) return;
  const OptTensor sv = int8_act ? OptTensor(f32_vector(*s, m, "activation row scale"))
                                : OptTensor();
  check_status(rk_grad_weight_bf16_parts(g.p[0], g.p[1], g.p[2], g.n, g.cols, g.dtype, g.ld,
                                         x.data_ptr(),
                                         int8_act ? RK_I8 : dtype_code(x, "activations"), ld(x),
                                         ptr<const float>(sv), m, n, k,
                                         direct ? nullptr : work.data_ptr<float>(),
                                         direct ? 1 : static_cast<int>(work.size(0)),
                                         direct ? static_cast<uint16_t*>(work.data_ptr()) : nullptr,
                                         k, stream_of(x)),
               "rk_grad_weight_bf16_parts");
}

void grad_weight_partials_x(const Tensor& g, const Tensor& x, Tensor& work) {
  TORCH_CHECK(x.dim() == 2, "activations must be a 2-D matrix");
  grad_weight_partials_common(g, x, false, std::nullopt, work);
}

// ---------------------------------------------------------------------------------------
// The ratchet update (ratchet.py:248-301, 487-556, 613-625, 672-679)
// ---------------------------------------------------------------------------------------
void check_counts(const Tensor& counts) {
  TORCH_CHECK(counts.scalar_type() == at::kLong && counts.numel() == 4 && counts.is_contiguous(),
              "counts must be a contiguous int64 tensor of 4 entries");
}

void check_rows_f32(const OptTensor& t, int64_t rows, const char* what) {
  if (!t.has_value()) return;
  TORCH_CHECK(t->scalar_type() == at::kFloat && t->numel() == rows && t->is_contiguous(), what,
              " must be a contiguous float32 tensor of ", rows, " entries");
}

void check_update_outputs(const Tensor& packed, const OptTensor& rms_ema, const Tensor& counts,
                          const OptTensor& row_rms, const OptTensor& grad_scale,
                          const OptTensor& nonfinite, const OptTensor& rms_mean) {
  const int64_t rows = packed.size(0);
  check_counts(counts);
  check_rows_f32(rms_ema, rows, "rms_ema");
  check_rows_f32(row_rms, rows, "row_rms");
  check_rows_f32(grad_scale, rows, "grad_scale");
  if (nonfinite.has_value())
    TORCH_CHECK(nonfinite->scalar_type() == at::kInt && nonfinite->numel() >= 1,
                "nonfinite must be an int32 flag");
  if (rms_mean.has_value())
    TORCH_CHECK(rms_mean->scalar_type() == at::kFloat && rms_mean->numel() == 1,
                "rms_mean must be one float32");
  TORCH_CHECK(!rms_mean.has_value() || row_rms.has_value(), "rms_mean needs row_rms");
}

void update_from_z(Tensor& packed, const Tensor& z_in, int64_t max_code, int64_t threshold,
                   double low, double high, Tensor& counts) {
  require_gpu(packed, "the ratchet update");
  packed_matrix(packed);
  check_counts(counts);
  TORCH_CHECK(z_in.sizes() == packed.sizes(), "normalized gradient shape mismatch");
  const Tensor z = z_in.to(at::kFloat).contiguous();
  const c10::DeviceGuard guard(packed.device());
  const int64_t rows = packed.size(0), k = packed.size(1);
  if (rows == 0 || k == 0) return;
  check_status(rk_ratchet_update(packed.data_ptr<uint8_t>(), ld(packed), z.data_ptr<float>(), k,
                                 rows, k, static_cast<int>(max_code),
                                 static_cast<int>(threshold), static_cast<float>(low),
                                 static_cast<float>(high), counts.data_ptr<int64_t>(),
                                 stream_of(packed)),
               "rk_ratchet_update");
}

void update_from_grad(Tensor& packed, const Tensor& g_in, int64_t max_code, int64_t threshold,
                      double low, double high, double eps, const OptTensor& rms_ema, double beta,
                      Tensor& counts, const OptTensor& row_rms, const OptTensor& grad_scale,
                      const OptTensor& nonfinite, const OptTensor& rms_mean) {
  require_gpu(packed, "the ratchet update");
  packed_matrix(packed);
  TORCH_CHECK(g_in.sizes() == packed.sizes(), "weight gradient shape mismatch");
  check_update_outputs(packed, rms_ema, counts, row_rms, grad_scale, nonfinite, rms_mean);
  const Tensor g = unit_columns(g_in.scalar_type() == at::kFloat ||
                                        g_in.scalar_type() == at::kBFloat16
                                    ? g_in
                                    : g_in.to(at::kFloat));
  const c10::DeviceGuard guard(packed.device());
  const int64_t rows = packed.size(0), k = packed.size(1);
  if (rows == 0 || k == 0) return;
  check_status(rk_ratchet_update_grad(
                   packed.data_ptr<uint8_t>(), ld(packed), g.data_ptr(),
                   dtype_code(g, "weight gradient"), ld(g), rows, k, static_cast<int>(max_code),
                   static_cast<int>(threshold), static_cast<float>(low),
                   static_cast<float>(high), static_cast<float>(eps), ptr<float>(rms_ema),
                   static_cast<float>(beta), 1.0f - static_cast<float>(beta),
                   counts.data_ptr<int64_t>(), ptr<float>(row_rms), ptr<float>(grad_scale),
                   ptr<int32_t>(nonfinite), ptr<float>(rms_mean), stream_of(packed)),
               "rk_ratchet_update_grad");
}

void update_from_partials(Tensor& packed, const Tensor& partials, int64_t max_code,
                          int64_t threshold, double low, double high, double eps,
                          const OptTensor& rms_ema, double beta, Tensor& counts,
                          const OptTensor& row_rms, const OptTensor& grad_scale,
                          const OptTensor& nonfinite, const OptTensor& rms_mean,
                          const OptTensor& grad_out) {
  require_gpu(packed, "the ratchet update");
  packed_matrix(packed);
  const int64_t rows = packed.size(0), k = packed.size(1);
  check_workspace(partials, rows, k);
  check_update_outputs(packed, rms_ema, counts, row_rms, grad_scale, nonfinite, rms_mean);
  if (grad_out.has_value())
    TORCH_CHECK(grad_out->scalar_type() == at::kBFloat16 && grad_out->sizes() == packed.sizes() &&
                    grad_out->is_contiguous(),
                "grad_out must be a contiguous bfloat16 tensor of the state's shape");
  const c10::DeviceGuard guard(packed.device());
  if (rows == 0 || k == 0) return;
  check_status(rk_ratchet_update_partials(
                   packed.data_ptr<uint8_t>(), ld(packed), partials.data_ptr<float>(),
                   static_cast<int>(partials.size(0)), rows, k, static_cast<int>(max_code),
                   static_cast<int>(threshold), static_cast<float>(low),
                   static_cast<float>(high), static_cast<float>(eps), ptr<float>(rms_ema),
                   static_cast<float>(beta), 1.0f - static_cast<float>(beta),
                   counts.data_ptr<int64_t>(), ptr<float>(row_rms), ptr<float>(grad_scale),
                   ptr<int32_t>(nonfinite), ptr<float>(rms_mean), ptr<uint16_t>(grad_out), k,
                   stream_of(packed)),
               "rk_ratchet_update_partials");
}

Tensor normalize_rows(const Tensor& g_in, double eps, const OptTensor& rms_ema, double beta) {
  require_gpu(g_in, "ratchet normalization");
  TORCH_CHECK(g_in.dim() == 2, "normalization takes a 2-D gradient");
  const Tensor g = (g_in.scalar_type() == at::kFloat || g_in.scalar_type() == at::kBFloat16
                        ? g_in
                        : g_in.to(at::kFloat))
                       .contiguous();
  const int64_t rows = g.size(0), k = g.size(1);
  check_rows_f32(rms_ema, rows, "rms_ema");
  const c10::DeviceGuard guard(g.device());
  Tensor z = at::empty({rows, k}, g.options().dtype(at::kFloat));
  if (rows == 0 || k == 0) return z;
  check_status(rk_normalize_rows(g.data_ptr(), dtype_code(g, "gradient"), k, rows, k,
                                 static_cast<float>(eps), ptr<float>(rms_ema),
                                 static_cast<float>(beta), 1.0f - static_cast<float>(beta),
                                 z.data_ptr<float>(), k, nullptr, stream_of(g)),
               "rk_normalize_rows");
  return z;
}

// Several layers' fused updates in one launch. table_host (CPU) and table_dev (on the
// layers' device) hold the same rk_update_layer entries; `written` lists every tensor the
// launch writes (each layer's packed state, counts, row_rms, rms_ema, grad_scale, nonfinite),
// and every address the table writes through is checked to lie inside one of them.
void update_multi(const Tensor& table_host, const Tensor& table_dev, int64_t src,
                  at::TensorList written) {
  constexpr int64_t kEntry = sizeof(rk_update_layer);
  TORCH_CHECK(table_host.device().is_cpu() && table_host.scalar_type() == at::kByte &&
                  table_host.is_contiguous(),
              "table_host must be a contiguous CPU uint8 tensor");
  require_gpu(table_dev, "the multi-layer ratchet update");
  TORCH_CHECK(table_dev.scalar_type() == at::kByte && table_dev.is_contiguous() &&
                  table_dev.numel() == table_host.numel(),
              "table_dev must be a contiguous uint8 tensor the size of table_host");
  TORCH_CHECK(table_host.numel() > 0 && table_host.numel() % kEntry == 0,
              "the tables must hold whole rk_update_layer entries");
  TORCH_CHECK(reinterpret_cast<uintptr_t>(table_dev.data_ptr()) % 16 == 0,
              "table_dev must be 16-byte aligned");
  const int64_t n = table_host.numel() / kEntry;
  TORCH_CHECK(n <= 0x7fffffff, "too many layers");
  std::vector<std::pair<uintptr_t, uintptr_t>> ranges;
  for (const Tensor& t : written) {
    TORCH_CHECK(t.device() == table_dev.device(),
                "written tensors must be on the device of table_dev");
    const uintptr_t b = reinterpret_cast<uintptr_t>(t.data_ptr());
    ranges.emplace_back(b, b + static_cast<uintptr_t>(t.numel() * t.element_size()));
  }
  std::sort(ranges.begin(), ranges.end());
  auto covered = [&](uint64_t p, int64_t bytes) {
    if (p == 0 || bytes <= 0) return true;
    auto it = std::upper_bound(ranges.begin(), ranges.end(),
                               std::make_pair(static_cast<uintptr_t>(p), UINTPTR_MAX));
    while (it != ranges.begin()) {
      --it;
      if (it->first <= p && p + static_cast<uint64_t>(bytes) <= it->second) return true;
    }
    return false;
  };
  const auto* tab = reinterpret_cast<const rk_update_layer*>(table_host.data_ptr());
  for (int64_t i = 0; i < n; ++i) {
    const rk_update_layer& d = tab[i];
    if (d.rows <= 0) continue;
    TORCH_CHECK(covered(d.packed, (d.rows - 1) * d.ldp + d.K), "layer ", i,
                ": its packed state is not among the written tensors");
    TORCH_CHECK(covered(d.counts, 32), "layer ", i, ": counts not among the written tensors");
    TORCH_CHECK(covered(d.row_rms, d.rows * 4), "layer ", i,
                ": row_rms not among the written tensors");
    TORCH_CHECK(covered(d.rms_ema, d.rows * 4), "layer ", i,
                ": rms_ema not among the written tensors");
    TORCH_CHECK(covered(d.grad_scale, d.rows * 4), "layer ", i,
                ": grad_scale not among the written tensors");
    TORCH_CHECK(covered(d.nonfinite, 4), "layer ", i,
                ": nonfinite not among the written tensors");
  }
  const c10::DeviceGuard guard(table_dev.device());
  check_status(rk_ratchet_update_multi(tab,
                                       reinterpret_cast<const rk_update_layer*>(table_dev.data_ptr()),
                                       static_cast<int>(n), static_cast<int>(src),
                                       stream_of(table_dev)),
               "rk_ratchet_update_multi");
}

void pressure_leak(Tensor& packed, int64_t max_code) {
  require_gpu(packed, "the pressure leak");
  TORCH_CHECK(packed.scalar_type() == at::kByte && packed.is_contiguous(),
              "packed ratchet state must be contiguous uint8");
  const c10::DeviceGuard guard(packed.device());
  if (packed.numel() == 0) return;
  check_status(rk_pressure_leak(packed.data_ptr<uint8_t>(), packed.numel(),
                                static_cast<int>(max_code), stream_of(packed)),
               "rk_pressure_leak");
}

Tensor validate_state(const Tensor& packed_in, int64_t max_code, const OptTensor& scale_in) {
  require_gpu(packed_in, "ratchet state validation");
  TORCH_CHECK(packed_in.scalar_type() == at::kByte, "packed ratchet state must be uint8");
  const Tensor packed = packed_in.contiguous();
  OptTensor scale;
  if (scale_in.has_value()) scale = scale_in->to(at::kFloat).contiguous();
  const c10::DeviceGuard guard(packed.device());
  Tensor flags = at::zeros({3}, packed.options().dtype(at::kInt));
  check_status(rk_validate_state(packed.data_ptr<uint8_t>(), packed.numel(),
                                 static_cast<int>(max_code), ptr<const float>(scale),
                                 scale.has_value() ? scale->numel() : 0,
                                 flags.data_ptr<int32_t>(), stream_of(packed)),
               "rk_validate_state");
  return flags;
}

// ---------------------------------------------------------------------------------------
// Prologues and their backward (int8_fused.py:14-151, int8_backward.py:7-89)
// ---------------------------------------------------------------------------------------
Tensor float_rows(const Tensor& x) {
  TORCH_CHECK(x.dim() == 2, "expected a 2-D [rows, K] tensor");
  const Tensor f = (x.scalar_type() == at::kFloat || x.scalar_type() == at::kBFloat16)
                       ? x
                       : x.to(at::kFloat);
  return unit_columns(f);
}

std::tuple<Tensor, Tensor> rmsnorm_quantize(const Tensor& x_in, const Tensor& w_in, double eps) {
  require_gpu(x_in, "fused RMSNorm quantization");
  const Tensor x = float_rows(x_in);
  const int64_t m = x.size(0), k = x.size(1);
  const Tensor w = f32_vector(w_in.to(at::kFloat), k, "RMSNorm weight");
  const c10::DeviceGuard guard(x.device());
  Tensor q = at::empty({m, k}, x.options().dtype(at::kChar));
  Tensor s = at::empty({m}, x.options().dtype(at::kFloat));
  if (m == 0 || k == 0) return {q, s};
  check_status(rk_rmsnorm_quantize(x.data_ptr(), dtype_code(x, "RMSNorm input"), ld(x),
                                   w.data_ptr<float>(), static_cast<float>(eps),
                                   q.data_ptr<int8_t>(), k, s.data_ptr<float>(), m, k,
                                   stream_of(x)),
               "rk_rmsnorm_quantize");
  return {q, s};
}

std::tuple<Tensor, Tensor> gelu_quantize(const Tensor& x_in) {
  require_gpu(x_in, "fused GELU quantization");
  const Tensor x = float_rows(x_in);
  const int64_t m = x.size(0), k = x.size(1);
  const c10::DeviceGuard guard(x.device());
  Tensor q = at::empty({m, k}, x.options().dtype(at::kChar));
  Tensor s = at::empty({m}, x.options().dtype(at::kFloat));
  if (m == 0 || k == 0) return {q, s};
  check_status(rk_gelu_quantize(x.data_ptr(), dtype_code(x, "GELU input"), ld(x),
                                q.data_ptr<int8_t>(), k, s.data_ptr<float>(), m, k, stream_of(x)),
               "rk_gelu_quantize");
  return {q, s};
}

std::tuple<Tensor, Tensor> transpose_quantize(const Tensor& x_in) {
  require_gpu(x_in, "fused transpose quantization");
  TORCH_CHECK(x_in.dim() == 4, "transpose quantization takes [B, H, S, D]");
  const Tensor x = (x_in.scalar_type() == at::kFloat || x_in.scalar_type() == at::kBFloat16)
                       ? x_in
                       : x_in.to(at::kFloat);
  const int64_t b = x.size(0), h = x.size(1), s = x.size(2), d = x.size(3);
  const c10::DeviceGuard guard(x.device());
  Tensor q = at::empty({b * s, h * d}, x.options().dtype(at::kChar));
  Tensor scale = at::empty({b * s}, x.options().dtype(at::kFloat));
  if (b * s == 0 || h * d == 0) return {q, scale};
  check_status(rk_transpose_quantize(x.data_ptr(), dtype_code(x, "attention output"), b, h, s, d,
                                     x.stride(0), x.stride(1), x.stride(2), x.stride(3),
                                     q.data_ptr<int8_t>(), h * d, scale.data_ptr<float>(),
                                     stream_of(x)),
               "rk_transpose_quantize");
  return {q, scale};
}

std::tuple<Tensor, Tensor> rmsnorm_backward(const Tensor& gy_in, const Tensor& x_in,
                                            const Tensor& w_in, double eps,
                                            const OptTensor& residual_grad) {
  require_gpu(x_in, "RMSNorm backward");
  const Tensor x = float_rows(x_in);
  const Tensor gy = float_rows(gy_in);
  TORCH_CHECK(gy.sizes() == x.sizes(), "grad_y ", gy.sizes(), " does not match x ", x.sizes());
  const int64_t m = x.size(0), k = x.size(1);
  const Tensor w = f32_vector(w_in.to(at::kFloat), k, "RMSNorm weight");
  const c10::DeviceGuard guard(x.device());
  Tensor grad_x = at::empty({m, k}, x.options());
  Tensor grad_w = at::empty({k}, x.options().dtype(at::kFloat));
  if (k == 0) return {grad_x, grad_w};
  const int64_t parts = std::max<int64_t>(rk_rmsnorm_backward_parts(m), 1);
  Tensor work = at::empty({parts, k}, x.options().dtype(at::kFloat));
  if (residual_grad.has_value()) {
    // grad_x = bf16(dx) + residual_grad in one pass (float32 x: the residual stream)
    TORCH_CHECK(x.scalar_type() == at::kFloat,
                "RMSNorm backward with a residual gradient needs float32 x");
    TORCH_CHECK(residual_grad->scalar_type() == at::kFloat && residual_grad->numel() == m * k,
                "residual_grad must be float32 with x's shape");
    same_device(*residual_grad, x, "RMSNorm backward");
    const Tensor r = unit_columns(residual_grad->reshape({m, k}));
    check_status(rk_rmsnorm_backward_residual(
                     gy.data_ptr(), dtype_code(gy, "grad_y"), ld(gy), x.data_ptr<float>(), ld(x),
                     w.data_ptr<float>(), static_cast<float>(eps), m, k, r.data_ptr<float>(),
                     ld(r), static_cast<float*>(grad_x.data_ptr()), k, grad_w.data_ptr<float>(),
                     work.data_ptr<float>(), work.numel(), stream_of(x)),
                 "rk_rmsnorm_backward_residual");
    return {grad_x, grad_w};
  }
  check_status(rk_rmsnorm_backward(gy.data_ptr(), dtype_code(gy, "grad_y"), ld(gy),
                                   x.data_ptr(), dtype_code(x, "x"), ld(x), w.data_ptr<float>(),
                                   static_cast<float>(eps), m, k, grad_x.data_ptr(), k,
                                   grad_w.data_ptr<float>(), work.data_ptr<float>(),
                                   work.numel(), stream_of(x)),
               "rk_rmsnorm_backward");
  return {grad_x, grad_w};
}

Tensor gelu_backward(const Tensor& gy_in, const Tensor& x_in) {
  require_gpu(x_in, "GELU backward");
  const Tensor x = float_rows(x_in);
  const Tensor gy = float_rows(gy_in);
  TORCH_CHECK(gy.sizes() == x.sizes(), "grad_y ", gy.sizes(), " does not match x ", x.sizes());
  const int64_t m = x.size(0), k = x.size(1);
  const c10::DeviceGuard guard(x.device());
  Tensor grad_x = at::empty({m, k}, x.options());
  if (m == 0 || k == 0) return grad_x;
  check_status(rk_gelu_backward(gy.data_ptr(), dtype_code(gy, "grad_y"), ld(gy), x.data_ptr(),
                                dtype_code(x, "x"), ld(x), m, k, grad_x.data_ptr(), k,
                                stream_of(x)),
               "rk_gelu_backward");
  return grad_x;
}

Tensor embedding_backward(const Tensor& grad_in, const Tensor& ids_in, int64_t num_weights) {
  require_gpu(grad_in, "embedding backward");
  same_device(grad_in, ids_in, "embedding backward");
  TORCH_CHECK(ids_in.scalar_type() == at::kLong || ids_in.scalar_type() == at::kInt,
              "embedding backward: ids must be int64 or int32, got ", ids_in.scalar_type());
  TORCH_CHECK(num_weights >= 0, "embedding backward: num_weights must be non-negative");
  const int64_t d = grad_in.size(-1);
  const Tensor ids = ids_in.reshape({-1}).contiguous();
  Tensor grad = grad_in.reshape({-1, d});
  TORCH_CHECK(grad.size(0) == ids.size(0), "embedding backward: grad has ", grad.size(0),
              " rows for ", ids.size(0), " ids");
  if (grad.scalar_type() != at::kFloat && grad.scalar_type() != at::kBFloat16)
    grad = grad.to(at::kFloat);
  if (grad.stride(-1) != 1 || (grad.size(0) > 1 && grad.stride(0) % 4 != 0) ||
      reinterpret_cast<uintptr_t>(grad.data_ptr()) % (4 * grad.element_size()) != 0)
    grad = grad.contiguous();
  const int64_t t = grad.size(0);
  const c10::DeviceGuard guard(grad.device());
  Tensor out = at::empty({num_weights, d}, grad.options().dtype(at::kFloat));
  const int64_t bytes = rk_embedding_backward_workspace(t, num_weights, d);
  Tensor work = at::empty({std::max<int64_t>(bytes, 16)}, grad.options().dtype(at::kByte));
  check_status(rk_embedding_backward(grad.data_ptr(), dtype_code(grad, "grad"),
                                     t > 1 ? grad.stride(0) : d, ids.data_ptr(),
                                     ids.scalar_type() == at::kLong ? 1 : 0, t, num_weights, d,
                                     static_cast<float*>(out.data_ptr()), d, work.data_ptr(),
                                     work.numel(), stream_of(grad)),
               "rk_embedding_backward");
  return out;
}

// Causal attention forward (rk_attention_forward) on bf16 q, k, v [B, H, S, D]: returns
// (o, lse), o as a [B, H, S, D] view of [B, S, H, D] memory (rows of the heads' outputs side
// by side, the layout torch's memory-efficient forward writes), lse float32 [B, H, S].
std::tuple<Tensor, Tensor> attention_forward(const Tensor& q, const Tensor& k, const Tensor& v,
                                             double scale) {
  require_gpu(q, "attention");
  same_device(q, k, "attention");
  same_device(q, v, "attention");
  TORCH_CHECK(q.dim() == 4 && k.sizes() == q.sizes() && v.sizes() == q.sizes(),
              "attention: q, k, v must share a [B, H, S, D] shape");
  TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16 &&
                  v.scalar_type() == at::kBFloat16,
              "attention: q, k, v must be bfloat16");
  const auto unit = [](const Tensor& t) { return t.stride(3) == 1 ? t : t.contiguous(); };
  const Tensor qq = unit(q), kk = unit(k), vv = unit(v);
  const int64_t B = q.size(0), H = q.size(1), S = q.size(2), D = q.size(3);
  const c10::DeviceGuard guard(q.device());
  Tensor o = at::empty({B, S, H, D}, q.options()).permute({0, 2, 1, 3});
  Tensor lse = at::empty({B, H, S}, q.options().dtype(at::kFloat));
  const auto p16 = [](const Tensor& t) { return static_cast<const uint16_t*>(t.data_ptr()); };
  check_status(rk_attention_forward(p16(qq), qq.stride(0), qq.stride(1), qq.stride(2), p16(kk),
                                    kk.stride(0), kk.stride(1), kk.stride(2), p16(vv),
                                    vv.stride(0), vv.stride(1), vv.stride(2), B, H, S, D,
                                    static_cast<float>(scale),
                                    static_cast<uint16_t*>(o.data_ptr()), o.stride(0),
                                    o.stride(1), o.stride(2), lse.data_ptr<float>(),
                                    stream_of(q)),
               "rk_attention_forward");
  return {o, lse};
}

// Means of segments [offsets[s], offsets[s + 1]) of a float32 row-rms buffer (rk_row_rms_means).
Tensor row_rms_means(const Tensor& row_rms, const Tensor& offsets) {
  require_gpu(row_rms, "row rms means");
  same_device(row_rms, offsets, "row rms means");
  TORCH_CHECK(row_rms.scalar_type() == at::kFloat && row_rms.dim() == 1 && row_rms.is_contiguous(),
              "row rms means: row_rms must be a contiguous float32 vector");
  TORCH_CHECK(offsets.scalar_type() == at::kLong && offsets.dim() == 1 && offsets.size(0) >= 1 &&
                  offsets.is_contiguous(),
              "row rms means: offsets must be a contiguous int64 vector of nseg + 1 entries");
  const int64_t nseg = offsets.size(0) - 1;
  const c10::DeviceGuard guard(row_rms.device());
  Tensor means = at::empty({nseg}, row_rms.options());
  check_status(rk_row_rms_means(row_rms.data_ptr<float>(), row_rms.numel(),
                                offsets.data_ptr<int64_t>(), nseg, means.data_ptr<float>(),
                                stream_of(row_rms)),
               "rk_row_rms_means");
  return means;
}

// F.cross_entropy(logits, targets) (mean, ignore_index) in two launches: per-row max, log
// of the sum of exponentials and loss (kept in `stats` for the backward), then the mean in
// a fixed order. Returns (loss, stats [3, M], count), loss and count 0-d float32.
std::tuple<Tensor, Tensor, Tensor> cross_entropy_forward(const Tensor& logits_in,
                                                         const Tensor& targets_in,
                                                         int64_t ignore_index) {
  require_gpu(logits_in, "cross entropy");
  same_device(logits_in, targets_in, "cross entropy");
  TORCH_CHECK(logits_in.dim() == 2, "cross entropy: logits must be 2-D, got ",
              logits_in.sizes());
  TORCH_CHECK(targets_in.scalar_type() == at::kLong, "cross entropy: targets must be int64");
  TORCH_CHECK(targets_in.dim() == 1 && targets_in.size(0) == logits_in.size(0),
              "cross entropy: targets must be 1-D with one entry per row");
  const Tensor logits = unit_columns(logits_in);
  const Tensor targets = targets_in.contiguous();
  const int64_t m = logits.size(0), v = logits.size(1);
  const c10::DeviceGuard guard(logits.device());
  const auto f32 = logits.options().dtype(at::kFloat);
  Tensor stats = at::empty({3, m}, f32);
  Tensor loss = at::empty({}, f32);
  Tensor count = at::empty({}, f32);
  check_status(rk_cross_entropy_forward(logits.data_ptr(), dtype_code(logits, "logits"),
                                        ld(logits), targets.data_ptr<int64_t>(), m, v,
                                        ignore_index, stats.data_ptr<float>(),
                                        loss.data_ptr<float>(), count.data_ptr<float>(),
                                        stream_of(logits)),
               "rk_cross_entropy_forward");
  return {loss, stats, count};
}

// The gradient of cross_entropy_forward's loss with respect to the logits, in the logits'
// dtype (for bfloat16 logits: the float32 gradient rounded once, as a bfloat16 consumer
// casts it).
Tensor cross_entropy_backward(const Tensor& grad_loss_in, const Tensor& logits_in,
                              const Tensor& targets_in, const Tensor& stats,
                              const Tensor& count, int64_t ignore_index) {
  require_gpu(logits_in, "cross entropy backward");
  TORCH_CHECK(logits_in.dim() == 2, "cross entropy backward: logits must be 2-D");
  TORCH_CHECK(targets_in.scalar_type() == at::kLong, "cross entropy backward: targets must be int64");
  const Tensor logits = unit_columns(logits_in);
  const Tensor targets = targets_in.contiguous();
  const int64_t m = logits.size(0), v = logits.size(1);
  TORCH_CHECK(targets.numel() == m, "cross entropy backward: one target per row");
  TORCH_CHECK(stats.scalar_type() == at::kFloat && stats.is_contiguous() && stats.numel() == 3 * m,
              "cross entropy backward: stats must be the forward's float32 [3, M]");
  TORCH_CHECK(count.numel() == 1 && count.scalar_type() == at::kFloat,
              "cross entropy backward: count must be the forward's float32 scalar");
  const Tensor grad_loss = grad_loss_in.to(at::kFloat).reshape({}).contiguous();
  const c10::DeviceGuard guard(logits.device());
  Tensor grad = at::empty({m, v}, logits.options());
  check_status(rk_cross_entropy_backward(logits.data_ptr(), dtype_code(logits, "logits"),
                                         ld(logits), targets.data_ptr<int64_t>(), m, v,
                                         ignore_index, stats.data_ptr<float>(),
                                         count.data_ptr<float>(), grad_loss.data_ptr<float>(),
                                         grad.data_ptr(), dtype_code(grad, "grad"), v,
                                         stream_of(logits)),
               "rk_cross_entropy_backward");
  return grad;
}

}  // namespace

TORCH_LIBRARY(ratchet, m) {
  m.def(
      "quantize_rows(Tensor x, Tensor? col_scale=None, bool stochastic=False, int seed=0, "
      "Tensor? seed_slot=None, int row_offset=0, Tensor(a!)? x_bf16=None, "
      "bool round_bf16=False) -> (Tensor, Tensor)");
  m.def(
      "int8_mm_nt(Tensor a, Tensor b, Tensor a_scale, Tensor? b_scale, ScalarType out_dtype) "
      "-> Tensor");
  m.def(
      "packed_mm(Tensor a, Tensor packed, int max_code, Tensor a_scale, Tensor? row_scale, "
      "ScalarType out_dtype) -> Tensor");
  m.def(
      "packed_mm_residual(Tensor a, Tensor packed, int max_code, Tensor a_scale, "
      "Tensor? row_scale, Tensor residual) -> Tensor");
  m.def(
      "packed_mm_accumulate(Tensor a, Tensor packed, int max_code, Tensor a_scale, "
      "Tensor? row_scale, Tensor(a!) acc) -> ()");
  m.def(
      "packed_mm_t(Tensor a, Tensor packed, int max_code, Tensor a_scale, Tensor? row_scale, "
      "ScalarType out_dtype) -> Tensor");
  m.def("unpack_transpose(Tensor packed, int max_code) -> Tensor");
  m.def("unpack(Tensor packed, int max_code) -> (Tensor, Tensor)");
  m.def("effective_bf16(Tensor packed, int max_code, Tensor scale) -> Tensor");
  m.def(
      "grad_input_bf16(Tensor g, Tensor packed, int max_code, Tensor scale, "
      "ScalarType out_dtype=bfloat16) -> Tensor");
  m.def("dequant_bf16(Tensor q, Tensor s) -> Tensor");
  m.def("transpose_bf16(Tensor x) -> Tensor");
  m.def("dequant_transpose_bf16(Tensor q, Tensor s) -> Tensor");
  m.def("grad_weight_splits(int m, int n, int k) -> int", &grad_weight_splits);
  m.def("grad_weight(Tensor g, Tensor q, Tensor s, int nsplit=0) -> Tensor");
  m.def("grad_weight_x(Tensor g, Tensor x, int nsplit=0) -> Tensor");
  m.def("grad_weight_partials(Tensor g, Tensor q, Tensor s, Tensor(a!) work) -> ()");
  m.def("grad_weight_partials_x(Tensor g, Tensor x, Tensor(a!) work) -> ()");
  m.def(
      "grad_weight_partials_parts(Tensor[] parts, Tensor x, Tensor? s, Tensor(a!) work) -> ()");
  m.def(
      "quantize_rows_parts(Tensor[] parts, Tensor? col_scale=None, bool stochastic=False, "
      "int seed=0, Tensor? seed_slot=None, int row_offset=0) -> (Tensor, Tensor)");
  m.def(
      "update_from_z(Tensor(a!) packed, Tensor z, int max_code, int threshold, float low, "
      "float high, Tensor(b!) counts) -> ()");
  m.def(
      "update_from_grad(Tensor(a!) packed, Tensor g, int max_code, int threshold, float low, "
      "float high, float eps, Tensor(b!)? rms_ema, float beta, Tensor(c!) counts, "
      "Tensor(d!)? row_rms, Tensor(e!)? grad_scale, Tensor(f!)? nonfinite, "
      "Tensor(g!)? rms_mean) -> ()");
  m.def(
      "update_from_partials(Tensor(a!) packed, Tensor partials, int max_code, int threshold, "
      "float low, float high, float eps, Tensor(b!)? rms_ema, float beta, Tensor(c!) counts, "
      "Tensor(d!)? row_rms, Tensor(e!)? grad_scale, Tensor(f!)? nonfinite, "
      "Tensor(g!)? rms_mean, Tensor(h!)? grad_out) -> ()");
  m.def("update_multi(Tensor table_host, Tensor table_dev, int src, Tensor(a!)[] written) -> ()");
  m.def("normalize_rows(Tensor g, float eps, Tensor(a!)? rms_ema, float beta) -> Tensor");
  m.def("pressure_leak(Tensor(a!) packed, int max_code) -> ()");
  m.def("validate_state(Tensor packed, int max_code, Tensor? scale) -> Tensor");
  m.def("rmsnorm_quantize(Tensor x, Tensor w, float eps) -> (Tensor, Tensor)");
  m.def("gelu_quantize(Tensor x) -> (Tensor, Tensor)");
  m.def("transpose_quantize(Tensor x) -> (Tensor, Tensor)");
  m.def(
      "rmsnorm_backward(Tensor grad_y, Tensor x, Tensor w, float eps, "
      "Tensor? residual_grad=None) -> (Tensor, Tensor)");
  m.def("gelu_backward(Tensor grad_y, Tensor x) -> Tensor");
  m.def("embedding_backward(Tensor grad, Tensor ids, int num_weights) -> Tensor");
  m.def("row_rms_means(Tensor row_rms, Tensor offsets) -> Tensor");
  m.def("attention_forward(Tensor q, Tensor k, Tensor v, float scale) -> (Tensor, Tensor)");
  m.def("cross_entropy_forward(Tensor logits, Tensor targets, int ignore_index=-100) -> "
        "(Tensor, Tensor, Tensor)");
  m.def("cross_entropy_backward(Tensor grad_loss, Tensor logits, Tensor targets, Tensor stats, "
        "Tensor count, int ignore_index=-100) -> Tensor");
}

TORCH_LIBRARY_IMPL(ratchet, CUDA, m) {
  m.impl("quantize_rows", &quantize_rows);
  m.impl("int8_mm_nt", &int8_mm_nt);
  m.impl("packed_mm", &packed_mm);
  m.impl("packed_mm_residual", &packed_mm_residual);
  m.impl("packed_mm_accumulate", &packed_mm_accumulate);
  m.impl("packed_mm_t", &packed_mm_t);
  m.impl("unpack_transpose", &unpack_transpose);
  m.impl("unpack", &unpack);
  m.impl("grad_input_bf16", &grad_input_bf16);
  m.impl("effective_bf16", &effective_bf16);
  m.impl("dequant_bf16", &dequant_bf16);
  m.impl("transpose_bf16", &transpose_bf16);
  m.impl("dequant_transpose_bf16", &dequant_transpose_bf16);
  m.impl("grad_weight", &grad_weight);
  m.impl("grad_weight_x", &grad_weight_x);
  m.impl("grad_weight_partials", &grad_weight_partials);
  m.impl("grad_weight_partials_x", &grad_weight_partials_x);
  m.impl("grad_weight_partials_parts", &grad_weight_partials_parts);
  m.impl("quantize_rows_parts", &quantize_rows_parts);
  m.impl("update_from_z", &update_from_z);
  m.impl("update_from_grad", &update_from_grad);
  m.impl("update_from_partials", &update_from_partials);
  m.impl("update_multi", &update_multi);
  m.impl("normalize_rows", &normalize_rows);
  m.impl("pressure_leak", &pressure_leak);
  m.impl("validate_state", &validate_state);
  m.impl("rmsnorm_quantize", &rmsnorm_quantize);
  m.impl("gelu_quantize", &gelu_quantize);
  m.impl("transpose_quantize", &transpose_quantize);
  m.impl("rmsnorm_backward", &rmsnorm_backward);
  m.impl("gelu_backward", &gelu_backward);
  m.impl("embedding_backward", &embedding_backward);
  m.impl("row_rms_means", &row_rms_means);
  m.impl("attention_forward", &attention_forward);
  m.impl("cross_entropy_forward", &cross_entropy_forward);
  m.impl("cross_entropy_backward", &cross_entropy_backward);
}
