// Fused integer ratchet update (gfx950).
//
// Persistent state is one byte per weight: low nibble code + max_code, high nibble
// pressure + 7 (ratchet.py:185-199). The update never materializes a float weight:
// it reads the byte and the (normalized) gradient, writes the byte back, and
// accumulates the four move counts. Everything is one HBM sweep:
//   z path:    1 B packed read + 4 B z read + 1 B write per weight
//   grad path: 1 B packed read + 2|4 B gradient read + 1 B write per weight,
//              the row RMS normalization fused in (one wavefront per row).
//
// Row reduction order for mean(g^2) (fixed, reproduced by the oracle): lane l owns
// 16-byte vectors at c*64*V + l*V; it accumulates acc = acc + g*g over chunks c
// ascending and vector slots ascending (separately rounded fp32 ops); the 64 lane
// sums are combined by the xor butterfly of wave_sum_butterfly.
#include "rk_update_row.h"

namespace rk {

// ---------------------------------------------------------------------------
// Update on a normalized gradient z (apply_normalized_gradient).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ratchet_update_z_kernel(
    uint8_t* packed, int64_t ldp, const float* z, int64_t ldz, int64_t rows, int64_t K,
    int mc, int T, float low, float high, int64_t* counts, int vec_z, int vec_p) {
  constexpr int V = 4;
  const int lane = threadIdx.x & 63;
  MoveCounts cnt;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < rows;
       row += static_cast<int64_t>(gridDim.x) * 4) {
    uint8_t* prow = packed + row * ldp;
    const float* zrow = z + row * ldz;
    for (int64_t e0 = static_cast<int64_t>(lane) * V; e0 < K; e0 += 64 * V) {
      float zv[V];
      if (vec_z && e0 + V <= K) {
        load_vec16<RK_F32>(zrow, e0, zv);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) zv[i] = e0 + i < K ? zrow[e0 + i] : 0.0f;
      }
      uint32_t w[1];
      load_bytes<V>(prow, e0, K, vec_p, w);
      uint32_t out = 0;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        if (e0 + i < K) {
          out |= ratchet_byte((w[0] >> (8 * i)) & 0xffu, zv[i], mc, T, low, high, cnt) << (8 * i);
        }
      }
      store_bytes<V>(prow, e0, K, vec_p, &out);
    }
  }
  flush_counts(cnt, counts);
}


// Mean of rows values with one 256-thread block, in a fixed order: thread t adds rows t,
// t + 256, ... in order, then a halving tree (t += t + w for w = 128 .. 1). Thread 0 gets it.
__device__ __forceinline__ float block_mean_256(const float* x, int64_t rows, float* part) {
  float acc = 0.0f;
  for (int64_t r = threadIdx.x; r < rows; r += 256) acc = acc + x[r];
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) part[threadIdx.x] = part[threadIdx.x] + part[threadIdx.x + w];
    __syncthreads();
  }
  return part[0] / static_cast<float>(rows);
}

__global__ __launch_bounds__(256) void row_rms_mean_kernel(const float* row_rms, int64_t rows,
                                                            float* mean) {
  __shared__ float part[256];
  const float m = block_mean_256(row_rms, rows, part);
  if (threadIdx.x == 0) mean[0] = m;
}

// One block per segment [offsets[s], offsets[s + 1]) of a buffer holding several layers'
// row rms: the same order as row_rms_mean_kernel, so each mean equals that kernel's. The
// bounds are clamped to [0, n] (and e >= b), so offsets past the buffer read nothing outside.
__global__ __launch_bounds__(256) void row_rms_segment_means_kernel(const float* row_rms,
                                                                     int64_t n,
                                                                     const int64_t* offsets,
                                                                     float* means) {
  __shared__ float part[256];
  int64_t b = offsets[blockIdx.x], e = offsets[blockIdx.x + 1];
  b = b < 0 ? 0 : (b > n ? n : b);
  e = e < b ? b : (e > n ? n : e);
  const float m = block_mean_256(row_rms + b, e - b, part);
  if (threadIdx.x == 0) means[blockIdx.x] = m;
}
// Element i of a 16-byte gradient vector held as four words (4 fp32, or 8 bf16 in pairs,
// element 2j in the low half of word j).

template <int DT, int NC, bool ZONLY, bool ONE_SPLIT = false>
__global__ __launch_bounds__(256) void ratchet_update_grad_kernel(GradUpdateArgs a) {
  MoveCounts cnt;
  // K opaque per row: the compiler would otherwise hoist every chunk's per-element tail
  // tests out of the row loop and hold them in registers for the whole kernel
  auto opaque_k = [&]() {
    int64_t K = a.K;
    asm volatile("" : "+s"(K));
    return K;
  };
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < a.rows;
       row += static_cast<int64_t>(gridDim.x) * 4) {
    update_row<DT, NC, ZONLY, ONE_SPLIT>(a, row, opaque_k(), cnt);
  }
  flush_counts(cnt, a.counts);
}

static unsigned row_grid(int64_t rows) {
  // Enough blocks to fill 256 CUs several times over; rows beyond that loop.
  const int64_t want = (rows + 3) / 4;
  return static_cast<unsigned>(want < 4096 ? (want > 0 ? want : 1) : 4096);
}

static int check_update_common(const uint8_t* packed, int64_t ldp, int64_t rows, int64_t K,
                               int mc, int T, float low, float high) {
  if (rows < 0 || K <= 0) return fail(RK_ERR_ARG, "invalid update shape");
  if (rows > 0 && !packed) return fail(RK_ERR_ARG, "null packed state");
  if (ldp < K) return fail(RK_ERR_ARG, "ldp < K");
  if (mc < 1 || mc > 7) return fail(RK_ERR_ARG, "max_code must be in 1..7");
  if (T < 1 || T > 127) return fail(RK_ERR_ARG, "pressure_threshold must be in [1, 127]");
  if (!(low >= 0.0f && low < high)) return fail(RK_ERR_ARG, "bucket thresholds must satisfy 0 <= low < high");
  return RK_OK;
}

template <int DT, int NC, bool ZONLY>
static void launch_rows(const GradUpdateArgs& a, hipStream_t s) {
  if constexpr (DT == SRC_SPLITS && NC > 0) {
    if (a.nsplit == 1) {
      ratchet_update_grad_kernel<DT, NC, ZONLY, true><<<row_grid(a.rows), 256, 0, s>>>(a);
      return;
    }
  }
  ratchet_update_grad_kernel<DT, NC, ZONLY><<<row_grid(a.rows), 256, 0, s>>>(a);
}

template <bool ZONLY>
static int launch_grad_kernel(const GradUpdateArgs& a, int g_dtype, hipStream_t s) {
  const int V = g_dtype == RK_F32 ? 4 : 8;
  const int64_t nchunks = (a.K + 64 * V - 1) / (64 * V);
  if (g_dtype == RK_F32) {
    if (nchunks <= 2) launch_rows<RK_F32, 2, ZONLY>(a, s);
    else if (nchunks <= 8) launch_rows<RK_F32, 8, ZONLY>(a, s);
    else launch_rows<RK_F32, 0, ZONLY>(a, s);
  } else if (g_dtype == RK_BF16) {
    if (nchunks <= 1) launch_rows<RK_BF16, 1, ZONLY>(a, s);
    else if (nchunks <= 4) launch_rows<RK_BF16, 4, ZONLY>(a, s);
    else if (nchunks <= 12) launch_rows<RK_BF16, 12, ZONLY>(a, s);
    else launch_rows<RK_BF16, 0, ZONLY>(a, s);
  } else if constexpr (!ZONLY) {
    if (nchunks <= 1) launch_rows<SRC_SPLITS, 1, false>(a, s);
    else if (nchunks <= 4) launch_rows<SRC_SPLITS, 4, false>(a, s);
    else if (nchunks <= 12) launch_rows<SRC_SPLITS, 12, false>(a, s);
    else launch_rows<SRC_SPLITS, 0, false>(a, s);
  }
  return launch_status(ZONLY ? "normalize_rows" : "ratchet_update_grad");
}

}  // namespace rk

using namespace rk;

extern "C" int rk_ratchet_update(uint8_t* packed, int64_t ldp, const float* z, int64_t ldz,
                                 int64_t rows, int64_t K, int max_code, int threshold,
                                 float low, float high, int64_t* counts, void* stream) {
  clear_error();
  if (int st = check_update_common(packed, ldp, rows, K, max_code, threshold, low, high)) return st;
  if (rows == 0) return RK_OK;
  if (!z) return fail(RK_ERR_ARG, "null gradient");
  if (ldz < K) return fail(RK_ERR_ARG, "ldz < K");
  const int vec_z = aligned16(z) && (ldz % 4) == 0 && (K % 4) == 0;
  const int vec_p = (reinterpret_cast<uintptr_t>(packed) % 4) == 0 && (ldp % 4) == 0 && (K % 4) == 0;
  ratchet_update_z_kernel<<<row_grid(rows), 256, 0, as_stream(stream)>>>(
      packed, ldp, z, ldz, rows, K, max_code, threshold, low, high, counts, vec_z, vec_p);
  return launch_status("ratchet_update");
}

extern "C" int rk_ratchet_update_grad(uint8_t* packed, int64_t ldp, const void* g, int g_dtype,
                                      int64_t ldg, int64_t rows, int64_t K, int max_code,
                                      int threshold, float low, float high, float eps,
                                      float* rms_ema, float beta1, float beta2, int64_t* counts,
                                      float* row_rms, float* grad_scale, int32_t* nonfinite,
                                      float* rms_mean, void* stream) {
  clear_error();
  if (int st = check_update_common(packed, ldp, rows, K, max_code, threshold, low, high)) return st;
  if (g_dtype != RK_F32 && g_dtype != RK_BF16) return fail(RK_ERR_ARG, "unsupported gradient dtype");
  if (rows == 0) return RK_OK;
  if (!g) return fail(RK_ERR_ARG, "null gradient");
  if (ldg < K) return fail(RK_ERR_ARG, "ldg < K");
  if (!(eps > 0.0f)) return fail(RK_ERR_ARG, "eps must be positive");
  GradUpdateArgs a{};
  a.packed = packed;
  a.ldp = ldp;
  a.g = g;
  a.ldg = ldg;
  a.rows = rows;
  a.K = K;
  a.mc = max_code;
  a.T = threshold;
  a.low = low;
  a.high = high;
  a.eps = eps;
  a.rms_ema = rms_ema;
  a.beta1 = beta1;
  a.beta2 = beta2;
  a.counts = counts;
  a.row_rms = row_rms;
  a.grad_scale = grad_scale;
  a.nonfinite = nonfinite;
  if (rms_mean && !row_rms) return fail(RK_ERR_ARG, "rms_mean needs row_rms");
  const int V = g_dtype == RK_F32 ? 4 : 8;
  a.vec_g = aligned16(g) && (ldg % V) == 0 && (K % V) == 0;
  a.vec_p = (reinterpret_cast<uintptr_t>(packed) % V) == 0 && (ldp % V) == 0 && (K % V) == 0;
  if (int e = launch_grad_kernel<false>(a, g_dtype, as_stream(stream))) return e;
  if (!rms_mean) return RK_OK;
  row_rms_mean_kernel<<<1, 256, 0, as_stream(stream)>>>(row_rms, rows, rms_mean);
  return launch_status("row_rms_mean");
}

extern "C" int rk_ratchet_update_partials(uint8_t* packed, int64_t ldp, const float* partials,
                                          int nsplit, int64_t rows, int64_t K, int max_code,
                                          int threshold, float low, float high, float eps,
                                          float* rms_ema, float beta1, float beta2,
                                          int64_t* counts, float* row_rms, float* grad_scale,
                                          int32_t* nonfinite, float* rms_mean,
                                          uint16_t* grad_out, int64_t ld_grad_out,
                                          void* stream) {
  clear_error();
  if (int st = check_update_common(packed, ldp, rows, K, max_code, threshold, low, high)) return st;
  if (nsplit < 1 || nsplit > 64) return fail(RK_ERR_ARG, "nsplit must be in 1..64");
  if (rows == 0) return RK_OK;
  if (!partials) return fail(RK_ERR_ARG, "null partials");
  if (K % 8 != 0 || !aligned16(partials))
    return fail(RK_ERR_UNSUPPORTED, "partials need K %% 8 == 0 and 16-byte alignment");
  if (grad_out && (ld_grad_out < K || ld_grad_out % 8 != 0 || !aligned16(grad_out)))
    return fail(RK_ERR_ARG, "grad_out needs ld >= K, ld %% 8 == 0, 16-byte alignment");
  if (!(eps > 0.0f)) return fail(RK_ERR_ARG, "eps must be positive");
  if (rms_mean && !row_rms) return fail(RK_ERR_ARG, "rms_mean needs row_rms");
  GradUpdateArgs a{};
  a.packed = packed;
  a.ldp = ldp;
  a.part = partials;
  a.nsplit = nsplit;
  a.part_stride = rows * K;
  a.g_out = grad_out;
  a.ldgo = ld_grad_out;
  a.rows = rows;
  a.K = K;
  a.mc = max_code;
  a.T = threshold;
  a.low = low;
  a.high = high;
  a.eps = eps;
  a.rms_ema = rms_ema;
  a.beta1 = beta1;
  a.beta2 = beta2;
  a.counts = counts;
  a.row_rms = row_rms;
  a.grad_scale = grad_scale;
  a.nonfinite = nonfinite;
  a.vec_p = (reinterpret_cast<uintptr_t>(packed) % 8) == 0 && (ldp % 8) == 0;
  if (int e = launch_grad_kernel<false>(a, SRC_SPLITS, as_stream(stream))) return e;
  if (!rms_mean) return RK_OK;
  row_rms_mean_kernel<<<1, 256, 0, as_stream(stream)>>>(row_rms, rows, rms_mean);
  return launch_status("row_rms_mean");
}

extern "C" int rk_normalize_rows(const void* g, int g_dtype, int64_t ldg, int64_t rows, int64_t K,
                                 float eps, float* rms_ema, float beta1, float beta2, float* z,
                                 int64_t ldz, float* row_rms, void* stream) {
  clear_error();
  if (g_dtype != RK_F32 && g_dtype != RK_BF16) return fail(RK_ERR_ARG, "unsupported gradient dtype");
  if (rows < 0 || K <= 0) return fail(RK_ERR_ARG, "invalid normalize shape");
  if (rows == 0) return RK_OK;
  if (!g || !z) return fail(RK_ERR_ARG, "null pointer");
  if (ldg < K || ldz < K) return fail(RK_ERR_ARG, "leading dimension too small");
  if (!(eps > 0.0f)) return fail(RK_ERR_ARG, "eps must be positive");
  GradUpdateArgs a{};
  a.g = g;
  a.ldg = ldg;
  a.rows = rows;
  a.K = K;
  a.eps = eps;
  a.rms_ema = rms_ema;
  a.beta1 = beta1;
  a.beta2 = beta2;
  a.row_rms = row_rms;
  a.z_out = z;
  a.ldz = ldz;
  const int V = g_dtype == RK_F32 ? 4 : 8;
  a.vec_g = aligned16(g) && (ldg % V) == 0 && (K % V) == 0;
  return launch_grad_kernel<true>(a, g_dtype, as_stream(stream));
}

extern "C" int rk_row_rms_means(const float* row_rms, int64_t n, const int64_t* offsets,
                                int64_t nseg, float* means, void* stream) {
  clear_error();
  if (nseg < 0 || nseg > 0x7fffffff) return fail(RK_ERR_ARG, "segment count out of range");
  if (n < 0) return fail(RK_ERR_ARG, "negative row rms length");
  if (nseg == 0) return RK_OK;
  if (!offsets || !means || (n > 0 && !row_rms)) return fail(RK_ERR_ARG, "null pointer");
  row_rms_segment_means_kernel<<<static_cast<unsigned>(nseg), 256, 0, as_stream(stream)>>>(
      row_rms, n, offsets, means);
  return launch_status("row_rms_means");
}
