// Per-token absmax int8 quantization kernels (gfx950).
//
// One 64-lane wavefront owns one row; a 256-thread block covers 4 rows. Lane l
// handles 16-byte vectors at element offsets c*64*V + l*V (V = 4 fp32 / 8 bf16),
// so every pass over a row is one fully coalesced sweep. Rows of up to
// kMaxChunks*64*V elements (4*64*8 for stochastic rounding of bf16) stay in registers
// between the amax pass and the quantize pass (HBM read once); longer rows are re-read
// (L2-resident).
//
// The same template serves four row sources:
//   SRC_PLAIN     x[m, k] (+ optional per-column scale), int8_matmul.py:106-150
//   SRC_RMSNORM   x * rsqrt(mean x^2 + eps) * w,          int8_fused.py:14-39
//   SRC_GELU      tanh-GELU(x),                           int8_fused.py:58-84
//   SRC_TRANSPOSE [B,H,S,D] read as [B*S, H*D],           int8_fused.py:103-131
#include "rk_common.h"
#include "rk_rowquant.h"

namespace rk {

enum { SRC_PLAIN = 0, SRC_RMSNORM = 1, SRC_GELU = 2, SRC_TRANSPOSE = 3 };

struct QuantArgs {
  const void* x;
  int64_t M, K;
  int64_t sxm, sxk;           // plain / rmsnorm / gelu addressing
  int64_t H, S, D;            // transpose addressing
  int64_t sb, sh, ss, sd;
  const float* col_scale;     // plain only, may be null
  const float* w;             // rmsnorm weight
  float eps;
  uint32_t key0, key1;        // Philox key (SR only)
  const int64_t* seed_dev;    // SR only: when set, the key is read here at kernel time
  int64_t row_offset;         // SR counter row offset
  int8_t* q;
  int64_t ldq;
  float* scale;
  uint16_t* xb;               // plain only: bf16 side output, may be null
  int64_t ldxb;
  int vec_ok;                 // 16-byte vector loads are legal for every chunk
  int round_bf16;             // plain float32 source: each value is taken as bf16(x) first
  // plain source split by columns over up to three [M, part_cols] tensors (row stride sxm,
  // unit column stride), nparts > 0; part_cols is a multiple of 8, so no vector or element
  // group crosses a part
  const void* xp[3];
  int64_t part_cols;
  int nparts;
};

constexpr int kMaxChunks = 12;

template <int DT, int SRC>
__device__ __forceinline__ int64_t src_offset(const QuantArgs& a, int64_t row, int64_t e) {
  if constexpr (SRC == SRC_TRANSPOSE) {
    const int64_t b = row / a.S, s = row - b * a.S;
    const int64_t h = e / a.D, d = e - h * a.D;
    return b * a.sb + s * a.ss + h * a.sh + d * a.sd;
  } else {
    return row * a.sxm + e * a.sxk;
  }
}

// Loads the raw chunk starting at element e0 (V elements; zeros past K). VEC: the
// chunk is inside the row and 16-byte vector loads are legal.
template <int DT, int SRC, bool VEC>
__device__ __forceinline__ void load_chunk(const QuantArgs& a, int64_t row, int64_t e0,
                                           float* v) {
  constexpr int V = Vec<DT>::N;
  if constexpr (SRC == SRC_PLAIN) {
    if (a.nparts > 0) {
      const int64_t p = e0 / a.part_cols;
      const void* base = p == 0 ? a.xp[0] : (p == 1 ? a.xp[1] : a.xp[2]);
      const int64_t idx = row * a.sxm + (e0 - p * a.part_cols);
      if (VEC || (a.vec_ok && e0 + V <= a.K)) {
        load_vec16<DT>(base, idx, v);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = e0 + i < a.K ? load_elem<DT>(base, idx + i) : 0.0f;
      }
      return;
    }
  }
  if (VEC || (a.vec_ok && e0 + V <= a.K)) {
    load_vec16<DT>(a.x, src_offset<DT, SRC>(a, row, e0), v);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int64_t e = e0 + i;
      v[i] = e < a.K ? load_elem<DT>(a.x, src_offset<DT, SRC>(a, row, e)) : 0.0f;
    }
  }
}

// Row transform applied to a raw value at column e (row_factor = rsqrt for rmsnorm).
template <int DT, int SRC>
__device__ __forceinline__ float transform(const QuantArgs& a, float x, int64_t e,
                                           float row_factor) {
  if constexpr (SRC == SRC_PLAIN) {
    if constexpr (DT == RK_F32) {
      if (a.round_bf16) x = round_bf16(x);
    }
    return a.col_scale ? x * a.col_scale[e] : x;
  } else if constexpr (SRC == SRC_RMSNORM) {
    return x * row_factor * a.w[e];
  } else if constexpr (SRC == SRC_GELU) {
    return gelu_tanh(x);
  } else {
    return x;
  }
}

template <int DT>
__device__ __forceinline__ void store_bf16_chunk(uint16_t* dst, int64_t e0, int64_t K,
                                                 const float* v) {
  constexpr int V = Vec<DT>::N;
#pragma unroll
  for (int i = 0; i < V; ++i)
    if (e0 + i < K) dst[e0 + i] = f32_to_bf16(v[i]);
}

// Quantizes V transformed values y (row scale s, r = 1/s) at columns e0.. and stores
// them. ALL: every one of the V columns is inside the row (no per-element checks).
template <int DT, bool SR, bool ALL>
__device__ __forceinline__ void quant_store_chunk(const QuantArgs& a, uint32_t ctr_row,
                                                  const PhiloxKey& key, int64_t e0,
                                                  const float* y, float s, float r,
                                                  int8_t* qrow, bool vec_store) {
  constexpr int V = Vec<DT>::N;
  float t[V], u[V];
  bool exact = false;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    u[i] = 0.0f;
    if constexpr (SR) {
      // counter = (row_offset + m) * K + k, wrapped to 32 bits like the int32 offsets
      // of int8_matmul.py:143
      u[i] = uniform_from_word(philox_word0(ctr_row + static_cast<uint32_t>(e0 + i), key));
    }
    t[i] = round_fast<SR>(y[i], r, u[i], exact);
  }
  if (exact) {
    // a value of this lane's chunk lies within the margin of a rounding boundary (or is
    // not finite): round the chunk through round_quotient, which divides where needed
#pragma unroll
    for (int i = 0; i < V; ++i) t[i] = round_quotient<SR>(y[i], s, r, u[i]);
  }
  int qi[V];
#pragma unroll
  for (int i = 0; i < V; ++i) qi[i] = static_cast<int>(fminf(fmaxf(t[i], -127.0f), 127.0f));
  if (vec_store && (ALL || e0 + V <= a.K)) {
    uint32_t w[V / 4];
#pragma unroll
    for (int j = 0; j < V / 4; ++j)
      w[j] = pack_bytes4(qi[4 * j], qi[4 * j + 1], qi[4 * j + 2], qi[4 * j + 3]);
    if constexpr (V == 8) {
      *reinterpret_cast<uint2*>(qrow + e0) = make_uint2(w[0], w[1]);
    } else {
      *reinterpret_cast<uint32_t*>(qrow + e0) = w[0];
    }
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (e0 + i < a.K) qrow[e0 + i] = static_cast<int8_t>(qi[i]);
  }
}

// Transformed values of one chunk (VEC: the whole chunk is inside the row and the
// per-column scale, if any, is 16-byte aligned).
template <int DT, int SRC, bool VEC>
__device__ __forceinline__ void transform_chunk(const QuantArgs& a, int64_t e0, float* v,
                                                float row_factor) {
  constexpr int V = Vec<DT>::N;
  if constexpr (VEC && SRC == SRC_PLAIN) {
    if constexpr (DT == RK_F32) {
      if (a.round_bf16) {
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = round_bf16(v[i]);
      }
    }
    if (a.col_scale) {
#pragma unroll
      for (int j = 0; j < V / 4; ++j) {
        const float4 cs = *reinterpret_cast<const float4*>(a.col_scale + e0 + 4 * j);
        v[4 * j] = v[4 * j] * cs.x;
        v[4 * j + 1] = v[4 * j + 1] * cs.y;
        v[4 * j + 2] = v[4 * j + 2] * cs.z;
        v[4 * j + 3] = v[4 * j + 3] * cs.w;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i)
      v[i] = (VEC || e0 + i < a.K) ? transform<DT, SRC>(a, v[i], e0 + i, row_factor) : 0.0f;
  }
}

// P wavefronts per row (1, or 4: one row per block, wavefront w holding chunks w NC ..
// w NC + NC - 1 in registers, the partial absmax of each met in LDS). The max is exact in
// any order, so P changes no result.
template <int DT, int SRC, bool SR, int NC, bool VEC, int P = 1>
__global__ __launch_bounds__(256) void quant_rows_kernel(QuantArgs a) {
  static_assert(P == 1 || (P == 4 && NC > 0 && SRC != SRC_RMSNORM),
                "row slices: register-resident rows, one row per block, no row norm");
  constexpr int V = Vec<DT>::N;
  constexpr int SPAN = kWave * V;
  const int lane = threadIdx.x & (kWave - 1);
  const int slice = P == 1 ? 0 : static_cast<int>(threadIdx.x >> 6);
  const int64_t row = P == 1 ? static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)
                             : static_cast<int64_t>(blockIdx.x);
  if (row >= a.M) return;  // with P == 4 the whole block returns together
  const int64_t lane0 = static_cast<int64_t>(lane) * V;
  const int64_t nchunks = (a.K + SPAN - 1) / SPAN;
  int8_t* qrow = a.q + row * a.ldq;
  const bool vec_store = (a.ldq % V) == 0 && ((reinterpret_cast<uintptr_t>(a.q) % V) == 0);
  uint16_t* xbrow = (SRC == SRC_PLAIN && a.xb) ? a.xb + row * a.ldxb : nullptr;
  PhiloxKey key{};
  if constexpr (SR) {
    uint32_t k0 = a.key0, k1 = a.key1;
    if (a.seed_dev) {
      const uint64_t seed = static_cast<uint64_t>(*a.seed_dev);
      k0 = static_cast<uint32_t>(seed & 0xffffffffu);
      k1 = static_cast<uint32_t>(seed >> 32);
    }
    key = philox_key(k0, k1);
  }
  const uint32_t ctr_row =
      static_cast<uint32_t>(a.row_offset + row) * static_cast<uint32_t>(a.K);

  if constexpr (NC > 0) {
    // Register-resident row (or row slice): one HBM read.
    const int c0 = slice * NC;  // this wavefront's first chunk
    float xr[NC][V];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t e0 = (c0 + c) * SPAN + lane0;
      if (c0 + c < nchunks && (!VEC || e0 < a.K)) {
        load_chunk<DT, SRC, VEC>(a, row, e0, xr[c]);
        if (xbrow && e0 < a.K) store_bf16_chunk<DT>(xbrow, e0, a.K, xr[c]);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) xr[c][i] = 0.0f;
      }
    }
    float row_factor = 1.0f;
    if constexpr (SRC == SRC_RMSNORM) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int i = 0; i < V; ++i) acc = acc + xr[c][i] * xr[c][i];
      acc = wave_sum_butterfly(acc);
      row_factor = 1.0f / sqrtf(acc / static_cast<float>(a.K) + a.eps);
    }
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t e0 = (c0 + c) * SPAN + lane0;
      if (c0 + c < nchunks && e0 < a.K) {
        transform_chunk<DT, SRC, VEC>(a, e0, xr[c], row_factor);
#pragma unroll
        for (int i = 0; i < V; ++i) amax = fmaxf(amax, fabsf(xr[c][i]));
      }
    }
    amax = wave_max(amax);
    if constexpr (P > 1) {
      __shared__ float slice_max[P];
      if (lane == 0) slice_max[slice] = amax;
      __syncthreads();
#pragma unroll
      for (int w = 0; w < P; ++w) amax = fmaxf(amax, slice_max[w]);
    }
    const float s = fmaxf(amax / 127.0f, 1.17549435e-38f);
    const float r = 1.0f / s;
    if (lane == 0 && slice == 0) a.scale[row] = s;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t e0 = (c0 + c) * SPAN + lane0;
      if (c0 + c < nchunks && e0 < a.K)
        quant_store_chunk<DT, SR, VEC>(a, ctr_row, key, e0, xr[c], s, r, qrow, vec_store);
    }
  } else {
    // Streaming row: re-read per pass (the row stays cache-resident).
    float row_factor = 1.0f;
    if constexpr (SRC == SRC_RMSNORM) {
      float acc = 0.0f;
      for (int64_t c = 0; c < nchunks; ++c) {
        float v[V];
        load_chunk<DT, SRC, VEC>(a, row, c * SPAN + lane0, v);
#pragma unroll
        for (int i = 0; i < V; ++i) acc = acc + v[i] * v[i];
      }
      acc = wave_sum_butterfly(acc);
      row_factor = 1.0f / sqrtf(acc / static_cast<float>(a.K) + a.eps);
    }
    float amax = 0.0f;
    for (int64_t c = 0; c < nchunks; ++c) {
      const int64_t e0 = c * SPAN + lane0;
      if (e0 >= a.K) break;
      float v[V];
      load_chunk<DT, SRC, VEC>(a, row, e0, v);
      transform_chunk<DT, SRC, VEC>(a, e0, v, row_factor);
#pragma unroll
      for (int i = 0; i < V; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
    amax = wave_max(amax);
    const float s = fmaxf(amax / 127.0f, 1.17549435e-38f);
    const float r = 1.0f / s;
    if (lane == 0) a.scale[row] = s;
    for (int64_t c = 0; c < nchunks; ++c) {
      const int64_t e0 = c * SPAN + lane0;
      if (e0 >= a.K) break;
      float v[V];
      load_chunk<DT, SRC, VEC>(a, row, e0, v);
      if (xbrow) store_bf16_chunk<DT>(xbrow, e0, a.K, v);
      transform_chunk<DT, SRC, VEC>(a, e0, v, row_factor);
      quant_store_chunk<DT, SR, VEC>(a, ctr_row, key, e0, v, s, r, qrow, vec_store);
    }
  }
}

template <int DT, int SRC, bool SR, int NC, int P = 1>
static void launch_quant_nc(const QuantArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  if (a.vec_ok) {
    quant_rows_kernel<DT, SRC, SR, NC, true, P><<<grid, block, 0, stream>>>(a);
  } else {
    quant_rows_kernel<DT, SRC, SR, NC, false, P><<<grid, block, 0, stream>>>(a);
  }
}

template <int DT, int SRC, bool SR>
static int launch_quant(const QuantArgs& a, hipStream_t stream) {
  constexpr int SPAN = kWave * Vec<DT>::N;
  const int64_t nchunks = (a.K + SPAN - 1) / SPAN;
  const dim3 grid(static_cast<unsigned>((a.M + 3) / 4));
  const dim3 block(256);
  // Stochastic rounding of bf16 rows keeps at most 4 chunks in registers: with 8 or 12 the
  // compiler leaves the row array in scratch (the Philox draws of a chunk are too large to
  // unroll over every chunk), and the re-reading streaming form measured faster (8192 x
  // 6144: 103 us streaming against 157 us with 12 chunks; 8192 x 4096: 89 us with 8).
  constexpr bool kLongRows = !(SR && DT == RK_BF16);
  if (nchunks <= 1) {
    launch_quant_nc<DT, SRC, SR, 1>(a, grid, block, stream);
  } else if (nchunks <= 2) {
    launch_quant_nc<DT, SRC, SR, 2>(a, grid, block, stream);
  } else if (nchunks <= 4) {
    launch_quant_nc<DT, SRC, SR, 4>(a, grid, block, stream);
  } else {
    if constexpr (SRC != SRC_RMSNORM) {
      if (nchunks <= 16 && a.M <= (int64_t{1} << 23)) {  // one block per row: grid in range
        // rows of 5 to 16 chunks: the four wavefronts of a block share one row, 2-4 chunks
        // each in registers (one wavefront holding 8 or 12 chunks ran at 2-3 wavefronts
        // per SIMD, or for stochastic bf16 rows kept them in scratch)
        const dim3 rows(static_cast<unsigned>(a.M));
        if (nchunks <= 8) launch_quant_nc<DT, SRC, SR, 2, 4>(a, rows, block, stream);
        else if (nchunks <= 12) launch_quant_nc<DT, SRC, SR, 3, 4>(a, rows, block, stream);
        else launch_quant_nc<DT, SRC, SR, 4, 4>(a, rows, block, stream);
        return launch_status("quantize_rows");
      }
    }
    if constexpr (kLongRows) {
      if (nchunks <= 8) {
        launch_quant_nc<DT, SRC, SR, 8>(a, grid, block, stream);
        return launch_status("quantize_rows");
      }
      if (nchunks <= kMaxChunks) {
        launch_quant_nc<DT, SRC, SR, kMaxChunks>(a, grid, block, stream);
        return launch_status("quantize_rows");
      }
    }
    launch_quant_nc<DT, SRC, SR, 0>(a, grid, block, stream);
  }
  return launch_status("quantize_rows");
}

template <int SRC, bool SR>
static int dispatch_dtype(int dt, const QuantArgs& a, hipStream_t stream) {
  if (dt == RK_F32) return launch_quant<RK_F32, SRC, SR>(a, stream);
  return launch_quant<RK_BF16, SRC, SR>(a, stream);
}

static bool rows_vec_ok(const void* x, int dt, int64_t K, int64_t sxm, int64_t sxk) {
  const int V = 16 / dtype_size(dt);
  return sxk == 1 && aligned16(x) && (sxm % V) == 0 && (K % V) == 0;
}

static int check_common(const void* x, int dt, int64_t M, int64_t K, const int8_t* q,
                        int64_t ldq, const float* scale) {
  if (dt != RK_F32 && dt != RK_BF16) return fail(RK_ERR_ARG, "unsupported input dtype %d", dt);
  if (M < 0 || K <= 0) return fail(RK_ERR_ARG, "invalid shape M=%lld K=%lld", (long long)M, (long long)K);
  if (M > 0 && (!x || !q || !scale)) return fail(RK_ERR_ARG, "null pointer argument");
  if (ldq < K) return fail(RK_ERR_ARG, "ldq (%lld) < K (%lld)", (long long)ldq, (long long)K);
  if (M > (int64_t(1) << 33)) return fail(RK_ERR_ARG, "too many rows");
  return RK_OK;
}

// The dequantized output of the activation quantizations: NULL, or a 16-byte aligned
// bf16 matrix with a row stride that is a multiple of 8 elements and at least K.

}  // namespace rk

using namespace rk;

static int quantize_rows_entry(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                               int64_t sxk, const float* col_scale, int stochastic,
                               uint64_t seed, const int64_t* seed_dev, int64_t row_offset,
                               int8_t* q, int64_t ldq, float* scale, uint16_t* x_bf16,
                               int64_t ld_xb, void* stream) {
  clear_error();
  const int round_bf16 = x_dtype == RK_F32_AS_BF16 ? 1 : 0;
  if (round_bf16) x_dtype = RK_F32;
  if (int st = check_common(x, x_dtype, M, K, q, ldq, scale)) return st;
  if (x_bf16 && ld_xb < K) return fail(RK_ERR_ARG, "ld_xb < K");
  if (M == 0) return RK_OK;
  QuantArgs a{};
  a.round_bf16 = round_bf16;
  a.x = x;
  a.M = M;
  a.K = K;
  a.sxm = sxm;
  a.sxk = sxk;
  a.col_scale = col_scale;
  a.key0 = static_cast<uint32_t>(seed & 0xffffffffu);
  a.key1 = static_cast<uint32_t>(seed >> 32);
  a.seed_dev = seed_dev;
  a.row_offset = row_offset;
  a.q = q;
  a.ldq = ldq;
  a.scale = scale;
  a.xb = x_bf16;
  a.ldxb = ld_xb;
  a.vec_ok = (rows_vec_ok(x, x_dtype, K, sxm, sxk) && (!col_scale || aligned16(col_scale))) ? 1 : 0;
  if (stochastic) return dispatch_dtype<SRC_PLAIN, true>(x_dtype, a, as_stream(stream));
  return dispatch_dtype<SRC_PLAIN, false>(x_dtype, a, as_stream(stream));
}

extern "C" int rk_quantize_rows_parts(const void* x0, const void* x1, const void* x2, int nparts,
                                      int64_t part_cols, int x_dtype, int64_t M, int64_t ldx,
                                      const float* col_scale, int stochastic, uint64_t seed,
                                      const int64_t* seed_dev, int64_t row_offset, int8_t* q,
                                      int64_t ldq, float* scale, void* stream) {
  clear_error();
  if (nparts < 1 || nparts > 3) return fail(RK_ERR_ARG, "nparts must be 1, 2 or 3");
  if (part_cols <= 0 || part_cols % 8 != 0)
    return fail(RK_ERR_ARG, "part columns must be a positive multiple of 8");
  if (ldx < part_cols) return fail(RK_ERR_ARG, "ldx < part columns");
  if (seed_dev && !stochastic) return fail(RK_ERR_ARG, "a device seed applies to stochastic rounding only");
  const void* parts[3] = {x0, x1, x2};
  const int64_t K = nparts * part_cols;
  const int dt = x_dtype == RK_F32_AS_BF16 ? RK_F32 : x_dtype;
  if (int st = check_common(x0, dt, M, K, q, ldq, scale)) return st;
  if (M == 0) return RK_OK;
  bool vec = (!col_scale || aligned16(col_scale));
  for (int i = 0; i < nparts; ++i) {
    if (!parts[i]) return fail(RK_ERR_ARG, "null part");
    vec = vec && rows_vec_ok(parts[i], dt, part_cols, ldx, 1);
  }
  QuantArgs a{};
  a.x = x0;
  a.M = M;
  a.K = K;
  a.sxm = ldx;
  a.sxk = 1;
  a.col_scale = col_scale;
  a.key0 = static_cast<uint32_t>(seed & 0xffffffffu);
  a.key1 = static_cast<uint32_t>(seed >> 32);
  a.seed_dev = seed_dev;
  a.row_offset = row_offset;
  a.q = q;
  a.ldq = ldq;
  a.scale = scale;
  a.vec_ok = vec ? 1 : 0;
  a.round_bf16 = x_dtype == RK_F32_AS_BF16 ? 1 : 0;
  a.nparts = nparts;
  a.part_cols = part_cols;
  for (int i = 0; i < nparts; ++i) a.xp[i] = parts[i];
  if (stochastic) return dispatch_dtype<SRC_PLAIN, true>(dt, a, as_stream(stream));
  return dispatch_dtype<SRC_PLAIN, false>(dt, a, as_stream(stream));
}

extern "C" int rk_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                                int64_t sxk, const float* col_scale, int stochastic,
                                uint64_t seed, int64_t row_offset, int8_t* q, int64_t ldq,
                                float* scale, uint16_t* x_bf16, int64_t ld_xb, void* stream) {
  return quantize_rows_entry(x, x_dtype, M, K, sxm, sxk, col_scale, stochastic, seed, nullptr,
                             row_offset, q, ldq, scale, x_bf16, ld_xb, stream);
}

extern "C" int rk_quantize_rows_devseed(const void* x, int x_dtype, int64_t M, int64_t K,
                                        int64_t sxm, int64_t sxk, const float* col_scale,
                                        const int64_t* seed, int64_t row_offset, int8_t* q,
                                        int64_t ldq, float* scale, uint16_t* x_bf16,
                                        int64_t ld_xb, void* stream) {
  if (!seed) {
    clear_error();
    return fail(RK_ERR_ARG, "null device seed");
  }
  return quantize_rows_entry(x, x_dtype, M, K, sxm, sxk, col_scale, 1, 0, seed, row_offset, q,
                             ldq, scale, x_bf16, ld_xb, stream);
}

static int rmsnorm_quantize_entry(const void* x, int x_dtype, int64_t ldx, const float* w,
                                  float eps, int8_t* q, int64_t ldq, float* scale, int64_t M,
                                  int64_t K, void* stream) {
  clear_error();
  if (int st = check_common(x, x_dtype, M, K, q, ldq, scale)) return st;
  if (M > 0 && !w) return fail(RK_ERR_ARG, "null RMSNorm weight");
  if (M == 0) return RK_OK;
  QuantArgs a{};
  a.x = x;
  a.M = M;
  a.K = K;
  a.sxm = ldx;
  a.sxk = 1;
  a.w = w;
  a.eps = eps;
  a.q = q;
  a.ldq = ldq;
  a.scale = scale;
  a.vec_ok = rows_vec_ok(x, x_dtype, K, ldx, 1) ? 1 : 0;
  return dispatch_dtype<SRC_RMSNORM, false>(x_dtype, a, as_stream(stream));
}

extern "C" int rk_rmsnorm_quantize(const void* x, int x_dtype, int64_t ldx, const float* w,
                                   float eps, int8_t* q, int64_t ldq, float* scale, int64_t M,
                                   int64_t K, void* stream) {
  return rmsnorm_quantize_entry(x, x_dtype, ldx, w, eps, q, ldq, scale, M, K, stream);
}

static int gelu_quantize_entry(const void* x, int x_dtype, int64_t ldx, int8_t* q, int64_t ldq,
                               float* scale, int64_t M, int64_t K, void* stream) {
  clear_error();
  if (int st = check_common(x, x_dtype, M, K, q, ldq, scale)) return st;
  if (M == 0) return RK_OK;
  QuantArgs a{};
  a.x = x;
  a.M = M;
  a.K = K;
  a.sxm = ldx;
  a.sxk = 1;
  a.q = q;
  a.ldq = ldq;
  a.scale = scale;
  a.vec_ok = rows_vec_ok(x, x_dtype, K, ldx, 1) ? 1 : 0;
  return dispatch_dtype<SRC_GELU, false>(x_dtype, a, as_stream(stream));
}

extern "C" int rk_gelu_quantize(const void* x, int x_dtype, int64_t ldx, int8_t* q,
                                int64_t ldq, float* scale, int64_t M, int64_t K, void* stream) {
  return gelu_quantize_entry(x, x_dtype, ldx, q, ldq, scale, M, K, stream);
}

static int transpose_quantize_entry(const void* x, int x_dtype, int64_t B, int64_t H,
                                    int64_t S, int64_t D, int64_t sb, int64_t sh, int64_t ss,
                                    int64_t sd, int8_t* q, int64_t ldq, float* scale,
                                    void* stream) {
  clear_error();
  if (B < 0 || H <= 0 || S < 0 || D <= 0) return fail(RK_ERR_ARG, "invalid [B,H,S,D] shape");
  const int64_t M = B * S, K = H * D;
  if (int st = check_common(x, x_dtype, M, K, q, ldq, scale)) return st;
  if (M == 0) return RK_OK;
  QuantArgs a{};
  a.x = x;
  a.M = M;
  a.K = K;
  a.H = H;
  a.S = S;
  a.D = D;
  a.sb = sb;
  a.sh = sh;
  a.ss = ss;
  a.sd = sd;
  a.q = q;
  a.ldq = ldq;
  a.scale = scale;
  const int V = 16 / dtype_size(x_dtype);
  a.vec_ok = (sd == 1 && aligned16(x) && D % V == 0 && sb % V == 0 && sh % V == 0 &&
              ss % V == 0)
                 ? 1
                 : 0;
  return dispatch_dtype<SRC_TRANSPOSE, false>(x_dtype, a, as_stream(stream));
}

extern "C" int rk_transpose_quantize(const void* x, int x_dtype, int64_t B, int64_t H,
                                     int64_t S, int64_t D, int64_t sb, int64_t sh, int64_t ss,
                                     int64_t sd, int8_t* q, int64_t ldq, float* scale,
                                     void* stream) {
  return transpose_quantize_entry(x, x_dtype, B, H, S, D, sb, sh, ss, sd, q, ldq, scale, stream);
}

namespace rk {

__global__ __launch_bounds__(256) void philox_word0_kernel(uint32_t key0, uint32_t key1,
                                                           uint32_t counter0, int64_t n,
                                                           uint32_t* out) {
  const PhiloxKey key = philox_key(key0, key1);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    out[i] = philox_word0(counter0 + static_cast<uint32_t>(i), key);
  }
}

}  // namespace rk

extern "C" int rk_philox_word0(uint64_t seed, uint32_t counter0, int64_t n, uint32_t* out,
                               void* stream) {
  clear_error();
  if (n < 0) return fail(RK_ERR_ARG, "negative count");
  if (n == 0) return RK_OK;
  if (!out) return fail(RK_ERR_ARG, "null output");
  const int64_t blocks = (n + 255) / 256;
  const unsigned grid = static_cast<unsigned>(blocks < 8192 ? blocks : 8192);
  philox_word0_kernel<<<grid, 256, 0, as_stream(stream)>>>(
      static_cast<uint32_t>(seed & 0xffffffffu), static_cast<uint32_t>(seed >> 32), counter0, n,
      out);
  return launch_status("philox_word0");
}
