// Row-quantization arithmetic shared by the training quant kernels and the decode
// kernels: tanh-GELU and the rounding of x / s to an integer (nearest-even, or floor
// after adding a uniform for stochastic rounding).
#pragma once

#include "rk_common.h"

namespace rk {

__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3))), evaluated in the
  // operation order of int8_fused.py:72-75. tanh_fast's absolute error (< 3e-7) moves the
  // result by under 1.5e-7 |x|, a ten-thousandth of an int8 step for rows whose absmax
  // exceeds 0.2 |x|: quantized values change only where they sit on a rounding boundary.
  const float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  const float t = tanh_fast(inner);
  return 0.5f * x * (1.0f + t);
}

// Margin of the reciprocal fast path (2^-12). With r = RN(1/s) and |x/s| <= 127.00002,
// ya = RN(x * r) differs from x/s by at most |x/s| * 2^-23 < 2^-16, and the correctly
// rounded quotient Y = RN(x / s) by at most 2^-16 + 2^-18 < 2^-15. For stochastic
// rounding the sums RN(Y + u) and RN(ya + u) then differ by less than 2^-14 (each add
// rounds by at most half an ulp of a value below 128). So whenever ya (or ya + u) lies
// more than the margin away from a rounding boundary (a half-integer for rint, an
// integer for floor), the fast result equals the one computed from Y; otherwise, and
// for non-finite inputs, the lane takes the IEEE division x / s (int8_matmul.py:142,
// div_rn) and rounds that.
constexpr float kAmbiguity = 0.000244140625f;

// The fast path of round_quotient alone: the rounded value from ya = y * r, with `exact`
// set (never cleared) where that value may differ from the one computed from y / s (the
// same test as round_quotient's). Callers round a group of values this way and redo the
// group with round_quotient only when some value set the flag, so the common case runs
// without a branch per value.
template <bool SR>
__device__ __forceinline__ float round_fast(float y, float r, float u, bool& exact) {
  const float ya = y * r;
  if constexpr (SR) {
    const float v = ya + u;
    const float f = floorf(v);
    const float d = v - f;
    exact = exact || !(fabsf(ya) <= 128.0f) || d < kAmbiguity || d > 1.0f - kAmbiguity;
    return f;
  } else {
    const float t = __builtin_rintf(ya);
    exact = exact || !(fabsf(ya) <= 128.0f) || fabsf(ya - t) > 0.5f - kAmbiguity;
    return t;
  }
}

// Four int32 values in [-128, 127] as the bytes of one word (byte i from the i-th).
__device__ __forceinline__ uint32_t pack_bytes4(int b0, int b1, int b2, int b3) {
  // v_perm_b32 selects bytes of {S0, S1} (S1 = bytes 0-3, S0 = bytes 4-7; 0x0c = zero)
  const uint32_t lo = __builtin_amdgcn_perm(static_cast<uint32_t>(b1), static_cast<uint32_t>(b0),
                                            0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(static_cast<uint32_t>(b3), static_cast<uint32_t>(b2),
                                            0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

template <bool SR>
__device__ __forceinline__ float round_quotient(float y, float s, float r, float u) {
  const float ya = y * r;
  if constexpr (SR) {
    const float v = ya + u;
    const float f = floorf(v);
    const float d = v - f;
    if (!(fabsf(ya) <= 128.0f) || d < kAmbiguity || d > 1.0f - kAmbiguity) {
      return floorf(y / s + u);
    }
    return f;
  } else {
    const float t = __builtin_rintf(ya);
    if (!(fabsf(ya) <= 128.0f) || fabsf(ya - t) > 0.5f - kAmbiguity) {
      return __builtin_rintf(y / s);
    }
    return t;
  }
}

}  // namespace rk
