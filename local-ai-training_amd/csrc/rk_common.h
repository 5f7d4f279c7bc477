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

// ---------------------------------------------------------------------------
// Wavefront reductions (xor butterfly; every lane ends with the same value).
// The float sum's association order is fixed: offsets 32, 16, 8, 4, 2, 1 with
// v = v + v[lane ^ offset].
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ int wave_or_int(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v |= __shfl_xor(v, off, kWave);
  return v;
}

// ---------------------------------------------------------------------------
// Counter-based Philox4x32-10 (Salmon et al., SC'11), first output word for the
// counter (c0, 0, 0, 0) and key (k0, k1); then the int32 -> [0, 1) map of
// Triton's 32-bit `rand` (x < 0 ? ~x : x, times float32 0x2FFFFFFF).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t philox_word0(uint32_t c0, uint32_t k0, uint32_t k1) {
  uint32_t c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
    const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
    const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c1 ^ k0;
    const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c3 ^ k1;
    c1 = static_cast<uint32_t>(p1);
    c3 = static_cast<uint32_t>(p0);
    c0 = n0;
    c2 = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c0;
}

__device__ __forceinline__ float uniform_from_word(uint32_t w) {
  int32_t x = static_cast<int32_t>(w);
  x = x < 0 ? ~x : x;
  return static_cast<float>(x) * __uint_as_float(0x2FFFFFFFu);
}

}  // namespace rk
