// Scaled int8 GEMM on gfx950 int8 MFMA (v_mfma_i32_16x16x64_i8).
//
//   C[m, n] = bf16_RNE( (float(sum_k A[m,k] * B[n,k]) * ls[m]) * rs[n] )
//
// A: int8 [M, K] (k contiguous); B: int8 [N, K] or the packed ratchet state
// [N, K] uint8 whose low nibble is code + max_code (decoded while staging).
// This is the "NT" form: both operands are K-contiguous, which is how the
// persistent codes are stored (packed[n, k]), so the forward GEMM needs no
// transposed copy of the weights (the reference makes one, ratchet.py:52).
//
// Tiling: 256 threads (4 wavefronts, 2x2), block tile 128x128, k-step 64 bytes.
// Each wavefront owns a 64x64 sub-tile = 4x4 MFMA 16x16 tiles (64 int32
// accumulators per lane). Tiles are double-buffered in LDS with rows padded to
// 80 bytes so the 16-byte fragment reads of 8 consecutive rows hit disjoint banks.
//
// MFMA operand roles are swapped (the B tile feeds the MFMA "A" operand) so that
// the accumulator layout gives every lane 4 consecutive output columns n of one
// row m: the epilogue stores 8 bytes (bf16) or 16 bytes (f32) per lane.
//
// Block order is XCD-aware: consecutive tile indices (which share an A row panel)
// are kept on one XCD's L2.
#include "rk_common.h"

namespace rk {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kLdsRow = kBK + 16;  // bytes

enum { B_INT8 = 0, B_PACKED = 1 };

struct GemmArgs {
  const int8_t* A;
  int64_t lda;
  const uint8_t* B;
  int64_t ldb;
  uint32_t mc4;  // max_code replicated in 4 bytes (packed B only)
  int max_code;
  const float* ls;
  const float* rs;
  void* C;
  int64_t ldc;
  int64_t M, N, K;
};

// Four packed bytes -> four int8 codes: byte - max_code on the low nibble,
// computed without inter-byte borrows (each lane biased by 0x80).
__device__ __forceinline__ uint32_t decode4(uint32_t w, uint32_t mc4) {
  return (((w & 0x0F0F0F0Fu) | 0x80808080u) - mc4) ^ 0x80808080u;
}

// Loads the 16-byte segment (row, k0 .. k0+15) of an operand; zeros outside
// [0, rows) x [0, K). FAST: K % 64 == 0, ld % 16 == 0, 16-byte aligned base.
template <bool FAST, int KIND>
__device__ __forceinline__ uint4 load_seg(const uint8_t* base, int64_t ld, int64_t row,
                                          int64_t rows, int64_t k0, int64_t K, uint32_t mc4,
                                          int max_code) {
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row >= rows) return v;
  if constexpr (FAST) {
    v = *reinterpret_cast<const uint4*>(base + row * ld + k0);
    if constexpr (KIND == B_PACKED) {
      v.x = decode4(v.x, mc4);
      v.y = decode4(v.y, mc4);
      v.z = decode4(v.z, mc4);
      v.w = decode4(v.w, mc4);
    }
  } else {
    uint32_t w[4] = {0, 0, 0, 0};
    const uint8_t* p = base + row * ld;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const int64_t k = k0 + b;
      uint32_t byte = 0;
      if (k < K) {
        byte = p[k];
        if constexpr (KIND == B_PACKED) byte = static_cast<uint8_t>((byte & 15u) - max_code);
      }
      w[b >> 2] |= byte << (8 * (b & 3));
    }
    v = make_uint4(w[0], w[1], w[2], w[3]);
  }
  return v;
}

template <int CDT>
__device__ __forceinline__ void store_out4(void* C, int64_t ldc, int64_t m, int64_t n,
                                           int64_t M, int64_t N, const float* v,
                                           bool vec_ok) {
  if (m >= M) return;
  if constexpr (CDT == RK_BF16) {
    uint16_t* row = static_cast<uint16_t*>(C) + m * ldc;
    uint16_t h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) h[r] = f32_to_bf16(v[r]);
    if (vec_ok && n + 3 < N) {
      uint2 pk;
      pk.x = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
      pk.y = static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16);
      *reinterpret_cast<uint2*>(row + n) = pk;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) row[n + r] = h[r];
    }
  } else {
    float* row = static_cast<float*>(C) + m * ldc;
    float f[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) f[r] = round_bf16(v[r]);
    if (vec_ok && n + 3 < N) {
      *reinterpret_cast<float4*>(row + n) = make_float4(f[0], f[1], f[2], f[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) row[n + r] = f[r];
    }
  }
}

template <int KIND, bool FAST, int CDT>
__global__ __launch_bounds__(256) void int8_gemm_nt_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t As[2][kBM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][kBN * kLdsRow];

  const int64_t tiles_n = (g.N + kBN - 1) / kBN;
  int64_t b = blockIdx.x;
  const int64_t nb = gridDim.x;
  if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);
  const int64_t m0 = (b / tiles_n) * kBM;
  const int64_t n0 = (b % tiles_n) * kBN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int g4 = lane >> 4, r16 = lane & 15;

  // Staging assignment: 512 16-byte segments per operand tile, 2 per thread.
  int srow[2], sseg[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = tid + 256 * j;
    srow[j] = c >> 2;
    sseg[j] = c & 3;
  }

  const uint8_t* Abase = reinterpret_cast<const uint8_t*>(g.A);
  uint4 ra[2], rb[2];
  auto load_tiles = [&](int64_t k0) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      ra[j] = load_seg<FAST, B_INT8>(Abase, g.lda, m0 + srow[j], g.M, k0 + 16 * sseg[j], g.K,
                                     0, 0);
      rb[j] = load_seg<FAST, KIND>(g.B, g.ldb, n0 + srow[j], g.N, k0 + 16 * sseg[j], g.K,
                                   g.mc4, g.max_code);
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      *reinterpret_cast<uint4*>(&As[buf][srow[j] * kLdsRow + 16 * sseg[j]]) = ra[j];
      *reinterpret_cast<uint4*>(&Bs[buf][srow[j] * kLdsRow + 16 * sseg[j]]) = rb[j];
    }
  };

  v4i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  const int64_t nk = (g.K + kBK - 1) / kBK;
  load_tiles(0);
  store_tiles(0);
  __syncthreads();

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = static_cast<int>(kt & 1);
    if (kt + 1 < nk) load_tiles((kt + 1) * kBK);

    v4i fa[4], fb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[i] = *reinterpret_cast<const v4i*>(
          &As[cur][(wm * 64 + i * 16 + r16) * kLdsRow + 16 * g4]);
      fb[i] = *reinterpret_cast<const v4i*>(
          &Bs[cur][(wn * 64 + i * 16 + r16) * kLdsRow + 16 * g4]);
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        acc[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[ni], fa[mi], acc[mi][ni], 0, 0, 0);

    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds rows m = .. + r16 and columns n = .. + 4*g4 + r.
  const bool vec_ok =
      (g.ldc % 4) == 0 && (reinterpret_cast<uintptr_t>(g.C) % (CDT == RK_BF16 ? 8 : 16)) == 0;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int64_t m = m0 + wm * 64 + mi * 16 + r16;
    const float lsm = m < g.M ? g.ls[m] : 0.0f;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const int64_t n = n0 + wn * 64 + ni * 16 + 4 * g4;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = static_cast<float>(acc[mi][ni][r]) * lsm;
        if (g.rs) t = t * (n + r < g.N ? g.rs[n + r] : 0.0f);
        v[r] = t;
      }
      store_out4<CDT>(g.C, g.ldc, m, n, g.M, g.N, v, vec_ok);
    }
  }
}

template <int KIND, int CDT>
static int launch_gemm(const GemmArgs& g, hipStream_t stream) {
  const int64_t tiles = ((g.M + kBM - 1) / kBM) * ((g.N + kBN - 1) / kBN);
  if (tiles > 0x7fffffff) return fail(RK_ERR_ARG, "GEMM grid too large");
  const bool fast = (g.K % kBK) == 0 && (g.lda % 16) == 0 && (g.ldb % 16) == 0 &&
                    aligned16(g.A) && aligned16(g.B);
  const dim3 grid(static_cast<unsigned>(tiles)), block(256);
  if (fast) {
    int8_gemm_nt_kernel<KIND, true, CDT><<<grid, block, 0, stream>>>(g);
  } else {
    int8_gemm_nt_kernel<KIND, false, CDT><<<grid, block, 0, stream>>>(g);
  }
  return launch_status("int8_gemm");
}

static int gemm_entry(const int8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, int kind,
                      int max_code, const float* ls, const float* rs, void* C, int c_dtype,
                      int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream) {
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(RK_ERR_ARG, "negative GEMM extent");
  if (c_dtype != RK_F32 && c_dtype != RK_BF16) return fail(RK_ERR_ARG, "bad output dtype");
  // |acc| <= K * 127 * 127 must fit int32.
  if (K > 133144) return fail(RK_ERR_ARG, "K too large for an int32 accumulator");
  if (M == 0 || N == 0) return RK_OK;
  if (!A || !B || !ls || !C) return fail(RK_ERR_ARG, "null GEMM operand");
  if (lda < K || ldb < K || ldc < N) return fail(RK_ERR_ARG, "leading dimension too small");
  if (kind == B_PACKED && (max_code < 1 || max_code > 7))
    return fail(RK_ERR_ARG, "max_code must be in 1..7");
  GemmArgs g{};
  g.A = A;
  g.lda = lda;
  g.B = B;
  g.ldb = ldb;
  g.max_code = max_code;
  g.mc4 = static_cast<uint32_t>(max_code) * 0x01010101u;
  g.ls = ls;
  g.rs = rs;
  g.C = C;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  hipStream_t s = as_stream(stream);
  if (kind == B_PACKED) {
    return c_dtype == RK_BF16 ? launch_gemm<B_PACKED, RK_BF16>(g, s)
                              : launch_gemm<B_PACKED, RK_F32>(g, s);
  }
  return c_dtype == RK_BF16 ? launch_gemm<B_INT8, RK_BF16>(g, s)
                            : launch_gemm<B_INT8, RK_F32>(g, s);
}

}  // namespace rk

using namespace rk;

extern "C" int rk_int8_gemm_nt(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                               const float* ls, const float* rs, void* C, int c_dtype,
                               int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream) {
  return gemm_entry(A, lda, reinterpret_cast<const uint8_t*>(B), ldb, B_INT8, 0, ls, rs, C,
                    c_dtype, ldc, M, N, K, stream);
}

extern "C" int rk_int8_gemm_packed(const int8_t* A, int64_t lda, const uint8_t* packed,
                                   int64_t ldp, int max_code, const float* ls, const float* rs,
                                   void* C, int c_dtype, int64_t ldc, int64_t M, int64_t N,
                                   int64_t K, void* stream) {
  return gemm_entry(A, lda, packed, ldp, B_PACKED, max_code, ls, rs, C, c_dtype, ldc, M, N, K,
                    stream);
}
