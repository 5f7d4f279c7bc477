// Shared device/host helpers for the gfx950 ratchet-linear kernels.
//
// Numerics contract (all kernels are compiled with -ffp-contract=off and without
// fast-math, so every fp32 multiply, add, divide and square root is a separately,
// correctly rounded IEEE operation, matching the reference's torch formulas and
// its libdevice div_rn / rint call sites, int8_matmul.py:90-95, 142).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "ratchet_hip.h"

namespace rk {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local last message, never throws).
// ---------------------------------------------------------------------------
int fail(int code, const char* fmt, ...);
int launch_status(const char* what);
void clear_error();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int dtype_size(int dt) { return dt == RK_F32 ? 4 : (dt == RK_BF16 ? 2 : 0); }

// ---------------------------------------------------------------------------
// bf16 <-> fp32 (round-to-nearest-even; NaN -> 0x7FC0 as torch's c10::BFloat16).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Raw buffer descriptor (stride 0) over [base, base + bytes), gfx9 data format word.
// Loads past `bytes` return zeros and stores past it are dropped, which replaces
// per-lane bounds checks at tile edges. The inputs are made wave-uniform explicitly:
// 64-bit address arithmetic runs on the vector unit, and a descriptor left in vector
// registers turns every buffer access into a waterfall loop. bytes < 2^31.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buffer(const void* base, int64_t bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32));
  const int n = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  void* p = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, n, 0x00020000);
}

// Four packed ratchet bytes -> four int8 codes: (byte & 15) - max_code per byte,
// computed without inter-byte borrows (each byte biased by 0x80). mc4 = max_code *
// 0x01010101.
__device__ __forceinline__ uint32_t decode4(uint32_t w, uint32_t mc4) {
  return (((w & 0x0F0F0F0Fu) | 0x80808080u) - mc4) ^ 0x80808080u;
}

// Elements per 16-byte vector for a dtype code.
template <int DT>
struct Vec;
template <>
struct Vec<RK_F32> {
  static constexpr int N = 4;
  using Elem = float;
};
template <>
struct Vec<RK_BF16> {
  static constexpr int N = 8;
  using Elem = uint16_t;
};

template <int DT>
__device__ __forceinline__ float load_elem(const void* base, int64_t idx) {
  if constexpr (DT == RK_F32) {
    return static_cast<const float*>(base)[idx];
  } else {
    return bf16_to_f32(static_cast<const uint16_t*>(base)[idx]);
  }
}

// Loads one 16-byte vector (Vec<DT>::N elements) at element index idx (must be
// 16-byte aligned) and widens it to fp32.
template <int DT>
__device__ __forceinline__ void load_vec16(const void* base, int64_t idx, float* out) {
  const uint4 raw = *reinterpret_cast<const uint4*>(
      static_cast<const char*>(base) + idx * (DT == RK_F32 ? 4 : 2));
  if constexpr (DT == RK_F32) {
    out[0] = __uint_as_float(raw.x);
    out[1] = __uint_as_float(raw.y);
    out[2] = __uint_as_float(raw.z);
    out[3] = __uint_as_float(raw.w);
  } else {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
}

// tanh(u) = 1 - 2 / (exp(2u) + 1) from the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32), about 5 instructions against ~25 for the correctly rounded tanhf. Absolute
// error below 3e-7 everywhere (the exponent argument's rounding, one ulp each of exp2 and
// rcp, the final subtraction); exp overflow gives 1, underflow -1, NaN stays NaN.
__device__ __forceinline__ float tanh_fast(float u) {
  const float e = __builtin_amdgcn_exp2f(u * 2.8853900817779268f);  // 2 log2(e) u
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
}

// ---------------------------------------------------------------------------
// Wavefront reductions (xor butterfly; every lane ends with the same value).
// The float sum's association order is fixed: offsets 32, 16, 8, 4, 2, 1 with
// v = v + v[lane ^ offset].
//
// The partner values move without the LDS crossbar: v_permlane32_swap / v_permlane16_swap
// of a register with itself leave, in their two results, a lane's own value and its
// lane ^ 32 (^ 16) partner's (which of the two is which depends on the half, and the sum
// or max does not care: a + b and b + a are the same bits); DPP row_ror:8 gives lane ^ 8
// inside a 16-lane row; lane ^ 4 is the half-row mirror (7 - i) of the quad-reversed
// register (i ^ 3); quad_perm gives ^ 2 and ^ 1.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, 0xf, 0xf, false));
}

// op(v, v[lane ^ off]) for off = 32, 16, 8, 4, 2, 1 on the raw 32-bit values
template <typename T, typename Op>
__device__ __forceinline__ T wave_butterfly(T v, Op op) {
  auto bits = [](T x) { return __builtin_bit_cast(uint32_t, x); };
  auto val = [](uint32_t x) { return __builtin_bit_cast(T, x); };
  {
    const auto r = __builtin_amdgcn_permlane32_swap(bits(v), bits(v), false, false);
    v = op(val(r[0]), val(r[1]));
  }
  {
    const auto r = __builtin_amdgcn_permlane16_swap(bits(v), bits(v), false, false);
    v = op(val(r[0]), val(r[1]));
  }
  v = op(v, val(dpp_u32<0x128>(bits(v))));                    // row_ror:8   -> lane ^ 8
  v = op(v, val(dpp_u32<0x141>(dpp_u32<0x1b>(bits(v)))));     // half-row mirror of quad
                                                              // reversal  -> lane ^ 4
  v = op(v, val(dpp_u32<0x4e>(bits(v))));                     // quad_perm -> lane ^ 2
  v = op(v, val(dpp_u32<0xb1>(bits(v))));                     // quad_perm -> lane ^ 1
  return v;
}

__device__ __forceinline__ float wave_sum_butterfly(float v) {
  return wave_butterfly(v, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ float wave_max(float v) {
  return wave_butterfly(v, [](float a, float b) { return fmaxf(a, b); });
}

__device__ __forceinline__ int wave_sum_int(int v) {
  return wave_butterfly(v, [](int a, int b) { return a + b; });
}

__device__ __forceinline__ int wave_or_int(int v) {
  return wave_butterfly(v, [](int a, int b) { return a | b; });
}

// ---------------------------------------------------------------------------
// Counter-based Philox4x32-10 (Salmon et al., SC'11), first output word for the
// counter (c0, 0, 0, 0) and key (k0, k1); then the int32 -> [0, 1) map of
// Triton's 32-bit `rand` (x < 0 ? ~x : x, times float32 0x2FFFFFFF).
// ---------------------------------------------------------------------------
constexpr uint32_t kPhiloxM0 = 0xD2511F53u;
constexpr uint32_t kPhiloxM1 = 0xCD9E8D57u;
constexpr uint32_t kPhiloxW0 = 0x9E3779B9u;
constexpr uint32_t kPhiloxW1 = 0xBB67AE85u;

// Three-input XOR in one gfx950 v_bitop3_b32 (truth table 0x96 = a ^ b ^ c).
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ void mul_wide(uint32_t m, uint32_t x, uint32_t& hi, uint32_t& lo) {
  const uint64_t p = static_cast<uint64_t>(m) * x;  // one v_mad_u64_u32
  hi = static_cast<uint32_t>(p >> 32);
  lo = static_cast<uint32_t>(p);
}

// Philox4x32-10 round: (c0, c1, c2, c3) <- (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2),
// hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)), then the key is bumped by (W0, W1).
//
// Per-launch constants of the first output word for key (k0, k1): the round keys and
// the products that depend only on the key. With the counter (x, 0, 0, 0):
//   round 0 leaves (k0, 0, hi(M0 x) ^ k1, lo(M0 x));
//   round 1 multiplies the key word k0 by M0, a constant (hi sh, lo sl);
//   the last round needs only hi(M1 c2).
// 17 wide multiplies per draw instead of 20; the xors fold into v_bitop3_b32.
struct PhiloxKey {
  uint32_t k0[10], k1[10];
  uint32_t r1c2;  // hi(M0 k0) ^ k1 of round 1
  uint32_t r2c2;  // lo(M0 k0) ^ k1 of round 2
};

__device__ __forceinline__ PhiloxKey philox_key(uint32_t k0, uint32_t k1) {
  PhiloxKey k;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    k.k0[r] = k0 + static_cast<uint32_t>(r) * kPhiloxW0;
    k.k1[r] = k1 + static_cast<uint32_t>(r) * kPhiloxW1;
  }
  uint32_t sh, sl;
  mul_wide(kPhiloxM0, k0, sh, sl);
  k.r1c2 = sh ^ k.k1[1];
  k.r2c2 = sl ^ k.k1[2];
  return k;
}

__device__ __forceinline__ uint32_t philox_word0(uint32_t x, const PhiloxKey& k) {
  uint32_t h, l;
  // round 0 on (x, 0, 0, 0)
  mul_wide(kPhiloxM0, x, h, l);
  const uint32_t c2 = h ^ k.k1[0];
  const uint32_t c3 = l;
  // round 1 on (k0, 0, c2, c3)
  mul_wide(kPhiloxM1, c2, h, l);
  uint32_t c0 = h ^ k.k0[1];
  uint32_t c1 = l;
  uint32_t d2 = c3 ^ k.r1c2;
  // round 2 on (c0, c1, d2, lo(M0 k0))
  uint32_t h0, l0, h1, l1;
  mul_wide(kPhiloxM0, c0, h0, l0);
  mul_wide(kPhiloxM1, d2, h1, l1);
  c0 = xor3(h1, c1, k.k0[2]);
  d2 = h0 ^ k.r2c2;
  c1 = l1;
  uint32_t d3 = l0;
  // rounds 3..8
#pragma unroll
  for (int r = 3; r < 9; ++r) {
    mul_wide(kPhiloxM0, c0, h0, l0);
    mul_wide(kPhiloxM1, d2, h1, l1);
    c0 = xor3(h1, c1, k.k0[r]);
    d2 = xor3(h0, d3, k.k1[r]);
    c1 = l1;
    d3 = l0;
  }
  // round 9: first word only
  return xor3(__umulhi(kPhiloxM1, d2), c1, k.k0[9]);
}

__device__ __forceinline__ float uniform_from_word(uint32_t w) {
  const int32_t x = static_cast<int32_t>(w);
  const int32_t y = x ^ (x >> 31);  // x < 0 ? ~x : x
  return static_cast<float>(y) * __uint_as_float(0x2FFFFFFFu);
}

}  // namespace rk
