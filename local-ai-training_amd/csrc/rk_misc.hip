// Host error plumbing and the small elementwise kernels of the ratchet path
// (unpack, transposed unpack, BF16 effective weight, BF16 dequant, pressure leak,
// state validation).
#include <cstring>

#include "rk_common.h"

namespace rk {

static thread_local char g_last_error[512] = {0};

void clear_error() { g_last_error[0] = 0; }

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RK_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return RK_OK;
}

static unsigned flat_grid(int64_t n, int per_thread) {
  const int64_t threads = (n + per_thread - 1) / per_thread;
  const int64_t blocks = (threads + 255) / 256;
  return static_cast<unsigned>(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

// ---------------------------------------------------------------------------
__global__ void unpack_kernel(const uint8_t* packed, int64_t n, int mc, int8_t* code,
                              int8_t* pressure) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int b = packed[i];
    if (code) code[i] = static_cast<int8_t>((b & 15) - mc);
    if (pressure) pressure[i] = static_cast<int8_t>((b >> 4) - 7);
  }
}

// 64x64 tiles through LDS: packed[n, k] -> codeT[k, n].
__global__ __launch_bounds__(256) void unpack_transpose_kernel(const uint8_t* packed,
                                                               int64_t ldp, int mc,
                                                               int8_t* codeT, int64_t ldt,
                                                               int64_t N, int64_t K) {
  __shared__ int8_t tile[64][65];
  const int64_t tiles_k = (K + 63) / 64;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) / tiles_k) * 64;
  const int64_t k0 = (static_cast<int64_t>(blockIdx.x) % tiles_k) * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t n = n0 + r, k = k0 + tx;
    tile[r][tx] = (n < N && k < K) ? static_cast<int8_t>((packed[n * ldp + k] & 15) - mc) : 0;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t k = k0 + r, n = n0 + tx;
    if (k < K && n < N) codeT[k * ldt + n] = tile[tx][r];
  }
}

// Aligned form (N % 16 == 0, K % 16 == 0, 16-byte aligned rows): a 64 x 64 tile per
// block; each thread loads one 16-byte piece of a packed row (16 k values of one n),
// decodes it four bytes at a time, and after the tile is in LDS gathers one 16-byte
// piece of a codeT row (16 n values of one k). LDS rows are 68 bytes: the 16 rows a
// wave gathers from at once (16 c + i, c = 0..3) then start 16 banks apart.
__global__ __launch_bounds__(256) void unpack_transpose_vec_kernel(const uint8_t* packed,
                                                                   int64_t ldp, uint32_t mc4,
                                                                   int8_t* codeT, int64_t ldt,
                                                                   int64_t N, int64_t K) {
  constexpr int P = 68;
  __shared__ __attribute__((aligned(16))) uint8_t tile[64 * P];
  const int64_t tiles_k = (K + 63) / 64;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) / tiles_k) * 64;
  const int64_t k0 = (static_cast<int64_t>(blockIdx.x) % tiles_k) * 64;
  const int t = threadIdx.x;
  {
    const int r = t >> 2, seg = t & 3;
    const int64_t n = n0 + r, k = k0 + 16 * seg;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (n < N && k < K) {
      v = *reinterpret_cast<const uint4*>(packed + n * ldp + k);
      v = make_uint4(decode4(v.x, mc4), decode4(v.y, mc4), decode4(v.z, mc4),
                     decode4(v.w, mc4));
    }
    uint32_t* row = reinterpret_cast<uint32_t*>(tile + r * P + 16 * seg);
    row[0] = v.x;
    row[1] = v.y;
    row[2] = v.z;
    row[3] = v.w;
  }
  __syncthreads();
  const int kk = t >> 2, c = t & 3;
  const int64_t k = k0 + kk, n = n0 + 16 * c;
  if (k < K && n < N) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t x = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b)
        x |= static_cast<uint32_t>(tile[(16 * c + 4 * q + b) * P + kk]) << (8 * b);
      w[q] = x;
    }
    *reinterpret_cast<uint4*>(codeT + k * ldt + n) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

__global__ void effective_bf16_kernel(const uint8_t* packed, int64_t ldp, int mc,
                                      const float* scale, uint16_t* W, int64_t ldw, int64_t N,
                                      int64_t K) {
  const int64_t total = N * K;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = i / K, k = i - n * K;
    const float c = static_cast<float>((packed[n * ldp + k] & 15) - mc);
    const float s = round_bf16(scale[n]);
    W[n * ldw + k] = f32_to_bf16(c * s);
  }
}

__global__ void dequant_bf16_kernel(const int8_t* q, int64_t ldq, const float* s, uint16_t* X,
                                    int64_t ldx, int64_t M, int64_t K) {
  const int64_t total = M * K;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t m = i / K, k = i - m * K;
    X[m * ldx + k] = f32_to_bf16(static_cast<float>(q[m * ldq + k]) * round_bf16(s[m]));
  }
}

// 64 x 64 tiles through LDS: X[m, n] (f32 or bf16, row stride ldx) -> T[n, m] bf16
// (row stride ldt), each element rounded to bf16 (RNE) on the way. With DEQUANT the
// source is int8 q[m, n] and the value is bf16(q) * bf16(s[m]) rounded to bf16.
// Reads and writes are both row-contiguous 128-byte (or wider) wave accesses.
template <int DT, bool DEQUANT>
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const void* X, int64_t ldx,
                                                             const float* s, uint16_t* T,
                                                             int64_t ldt, int64_t M, int64_t N) {
  __shared__ uint16_t tile[64][66];
  const int64_t tiles_n = (N + 63) / 64;
  const int64_t m0 = (static_cast<int64_t>(blockIdx.x) / tiles_n) * 64;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) % tiles_n) * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t m = m0 + r, n = n0 + tx;
    uint16_t v = 0;
    if (m < M && n < N) {
      if constexpr (DEQUANT) {
        const int8_t q = static_cast<const int8_t*>(X)[m * ldx + n];
        v = f32_to_bf16(static_cast<float>(q) * round_bf16(s[m]));
      } else if constexpr (DT == RK_F32) {
        v = f32_to_bf16(static_cast<const float*>(X)[m * ldx + n]);
      } else {
        v = static_cast<const uint16_t*>(X)[m * ldx + n];
      }
    }
    tile[r][tx] = v;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t n = n0 + r, m = m0 + tx;
    if (n < N && m < M) T[n * ldt + m] = tile[tx][r];
  }
}

__global__ void pressure_leak_kernel(uint8_t* packed, int64_t n, int mc) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int b = packed[i];
    const int c = (b & 15) - mc;
    int p = (b >> 4) - 7;
    p -= (p > 0) - (p < 0);
    packed[i] = static_cast<uint8_t>(((c + mc) & 15) | (((p + 7) & 15) << 4));
  }
}

__global__ void validate_kernel(const uint8_t* packed, int64_t n, int mc, const float* scale,
                                int64_t n_rows, int32_t* flags) {
  int bad_code = 0, bad_p = 0, bad_s = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride) {
    const int b = packed[i];
    const int c = (b & 15) - mc, p = (b >> 4) - 7;
    bad_code |= (c < -mc) | (c > mc);
    bad_p |= (p < -7) | (p > 7);
  }
  if (scale) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_rows;
         i += stride) {
      const float s = scale[i];
      bad_s |= !((__float_as_uint(s) & 0x7f800000u) != 0x7f800000u && s > 0.0f);
    }
  }
  bad_code = wave_or_int(bad_code);
  bad_p = wave_or_int(bad_p);
  bad_s = wave_or_int(bad_s);
  if ((threadIdx.x & 63) == 0) {
    if (bad_code) atomicOr(&flags[0], 1);
    if (bad_p) atomicOr(&flags[1], 1);
    if (bad_s) atomicOr(&flags[2], 1);
  }
}

}  // namespace rk

using namespace rk;

extern "C" int rk_version(void) { return 100; }

extern "C" const char* rk_last_error(void) { return g_last_error; }

extern "C" int rk_unpack(const uint8_t* packed, int64_t n, int max_code, int8_t* code,
                         int8_t* pressure, void* stream) {
  clear_error();
  if (n < 0) return fail(RK_ERR_ARG, "negative size");
  if (n == 0) return RK_OK;
  if (!packed) return fail(RK_ERR_ARG, "null packed state");
  unpack_kernel<<<flat_grid(n, 1), 256, 0, as_stream(stream)>>>(packed, n, max_code, code,
                                                                 pressure);
  return launch_status("unpack");
}

extern "C" int rk_unpack_transpose(const uint8_t* packed, int64_t ldp, int max_code,
                                   int8_t* codeT, int64_t ldt, int64_t N, int64_t K,
                                   void* stream) {
  clear_error();
  if (N < 0 || K < 0) return fail(RK_ERR_ARG, "negative size");
  if (N == 0 || K == 0) return RK_OK;
  if (!packed || !codeT) return fail(RK_ERR_ARG, "null pointer");
  if (ldp < K || ldt < N) return fail(RK_ERR_ARG, "leading dimension too small");
  const int64_t tiles = ((N + 63) / 64) * ((K + 63) / 64);
  if (tiles > 0x7fffffff) return fail(RK_ERR_ARG, "grid too large");
  if (N % 16 == 0 && K % 16 == 0 && ldp % 16 == 0 && ldt % 16 == 0 && aligned16(packed) &&
      aligned16(codeT)) {
    unpack_transpose_vec_kernel<<<static_cast<unsigned>(tiles), 256, 0, as_stream(stream)>>>(
        packed, ldp, static_cast<uint32_t>(max_code) * 0x01010101u, codeT, ldt, N, K);
  } else {
    unpack_transpose_kernel<<<static_cast<unsigned>(tiles), 256, 0, as_stream(stream)>>>(
        packed, ldp, max_code, codeT, ldt, N, K);
  }
  return launch_status("unpack_transpose");
}

extern "C" int rk_effective_bf16(const uint8_t* packed, int64_t ldp, int max_code,
                                 const float* scale, uint16_t* W, int64_t ldw, int64_t N,
                                 int64_t K, void* stream) {
  clear_error();
  if (N < 0 || K < 0) return fail(RK_ERR_ARG, "negative size");
  if (N == 0 || K == 0) return RK_OK;
  if (!packed || !scale || !W) return fail(RK_ERR_ARG, "null pointer");
  if (ldp < K || ldw < K) return fail(RK_ERR_ARG, "leading dimension too small");
  effective_bf16_kernel<<<flat_grid(N * K, 4), 256, 0, as_stream(stream)>>>(
      packed, ldp, max_code, scale, W, ldw, N, K);
  return launch_status("effective_bf16");
}

extern "C" int rk_dequant_bf16(const int8_t* q, int64_t ldq, const float* s, uint16_t* Xh,
                               int64_t ldx, int64_t M, int64_t K, void* stream) {
  clear_error();
  if (M < 0 || K < 0) return fail(RK_ERR_ARG, "negative size");
  if (M == 0 || K == 0) return RK_OK;
  if (!q || !s || !Xh) return fail(RK_ERR_ARG, "null pointer");
  if (ldq < K || ldx < K) return fail(RK_ERR_ARG, "leading dimension too small");
  dequant_bf16_kernel<<<flat_grid(M * K, 4), 256, 0, as_stream(stream)>>>(q, ldq, s, Xh, ldx,
                                                                           M, K);
  return launch_status("dequant_bf16");
}

extern "C" int rk_pressure_leak(uint8_t* packed, int64_t n, int max_code, void* stream) {
  clear_error();
  if (n < 0) return fail(RK_ERR_ARG, "negative size");
  if (n == 0) return RK_OK;
  if (!packed) return fail(RK_ERR_ARG, "null packed state");
  pressure_leak_kernel<<<flat_grid(n, 1), 256, 0, as_stream(stream)>>>(packed, n, max_code);
  return launch_status("pressure_leak");
}

extern "C" int rk_validate_state(const uint8_t* packed, int64_t n, int max_code,
                                 const float* scale, int64_t n_rows, int32_t* flags,
                                 void* stream) {
  clear_error();
  if (n < 0 || n_rows < 0) return fail(RK_ERR_ARG, "negative size");
  if (!flags) return fail(RK_ERR_ARG, "null flags");
  if (n > 0 && !packed) return fail(RK_ERR_ARG, "null packed state");
  const int64_t work = n > n_rows ? n : n_rows;
  validate_kernel<<<flat_grid(work > 0 ? work : 1, 1), 256, 0, as_stream(stream)>>>(
      packed, n, max_code, scale, n_rows, flags);
  return launch_status("validate_state");
}

extern "C" int rk_transpose_bf16(const void* x, int x_dtype, int64_t ldx, uint16_t* t,
                                 int64_t ldt, int64_t M, int64_t N, void* stream) {
  clear_error();
  if (x_dtype != RK_F32 && x_dtype != RK_BF16) return fail(RK_ERR_ARG, "unsupported dtype");
  if (M < 0 || N < 0) return fail(RK_ERR_ARG, "negative size");
  if (M == 0 || N == 0) return RK_OK;
  if (!x || !t) return fail(RK_ERR_ARG, "null pointer");
  if (ldx < N || ldt < M) return fail(RK_ERR_ARG, "leading dimension too small");
  const int64_t tiles = ((M + 63) / 64) * ((N + 63) / 64);
  if (tiles > 0x7fffffff) return fail(RK_ERR_ARG, "grid too large");
  hipStream_t s = as_stream(stream);
  if (x_dtype == RK_F32)
    transpose_bf16_kernel<RK_F32, false><<<static_cast<unsigned>(tiles), 256, 0, s>>>(x, ldx, nullptr, t, ldt, M, N);
  else
    transpose_bf16_kernel<RK_BF16, false><<<static_cast<unsigned>(tiles), 256, 0, s>>>(x, ldx, nullptr, t, ldt, M, N);
  return launch_status("transpose_bf16");
}

extern "C" int rk_dequant_transpose_bf16(const int8_t* q, int64_t ldq, const float* scale,
                                         uint16_t* t, int64_t ldt, int64_t M, int64_t K,
                                         void* stream) {
  clear_error();
  if (M < 0 || K < 0) return fail(RK_ERR_ARG, "negative size");
  if (M == 0 || K == 0) return RK_OK;
  if (!q || !scale || !t) return fail(RK_ERR_ARG, "null pointer");
  if (ldq < K || ldt < M) return fail(RK_ERR_ARG, "leading dimension too small");
  const int64_t tiles = ((M + 63) / 64) * ((K + 63) / 64);
  if (tiles > 0x7fffffff) return fail(RK_ERR_ARG, "grid too large");
  transpose_bf16_kernel<RK_BF16, true><<<static_cast<unsigned>(tiles), 256, 0, as_stream(stream)>>>(
      q, ldq, scale, t, ldt, M, K);
  return launch_status("dequant_transpose_bf16");
}
