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

// ---------------------------------------------------------------------------
// Several layers in one launch (rk_ratchet_update_multi). The layers' rows form one row
// space; wavefront w takes the contiguous rows [w R, (w + 1) R) and walks the layer table
// forward as it crosses layer boundaries, each row through update_row with that layer's
// arguments (the same code as the per-layer kernel, so the same results). Move counts add
// up per wavefront and go to a layer's counters, four 64-bit atomics, when the wavefront
// leaves the layer.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void flush_wave_counts(MoveCounts& cnt, int64_t* counts) {
  const int p = wave_sum_int(cnt.pos), n = wave_sum_int(cnt.neg);
  const int bp = wave_sum_int(cnt.bpos), bn = wave_sum_int(cnt.bneg);
  if ((threadIdx.x & 63) == 0 && counts) {
    unsigned long long* c = reinterpret_cast<unsigned long long*>(counts);
    if (p) atomicAdd(c + 0, static_cast<unsigned long long>(p));
    if (n) atomicAdd(c + 1, static_cast<unsigned long long>(n));
    if (bp) atomicAdd(c + 2, static_cast<unsigned long long>(bp));
    if (bn) atomicAdd(c + 3, static_cast<unsigned long long>(bn));
  }
  cnt = MoveCounts{};
}

// A table entry read into wave-uniform registers: the entry's address is the same for every
// lane, but the compiler does not know the loaded words are, so each goes through
// readfirstlane (a descriptor or row bound left in vector registers would turn every buffer
// access of the row into a waterfall loop).
__device__ __forceinline__ rk_update_layer load_layer(const rk_update_layer* p) {
  static_assert(sizeof(rk_update_layer) % 16 == 0, "16-byte table entries");
  rk_update_layer d;
  const uint4* src = reinterpret_cast<const uint4*>(p);
  uint32_t* dst = reinterpret_cast<uint32_t*>(&d);
#pragma unroll
  for (int i = 0; i < static_cast<int>(sizeof(rk_update_layer) / 16); ++i) {
    const uint4 v = src[i];
    dst[4 * i + 0] = __builtin_amdgcn_readfirstlane(v.x);
    dst[4 * i + 1] = __builtin_amdgcn_readfirstlane(v.y);
    dst[4 * i + 2] = __builtin_amdgcn_readfirstlane(v.z);
    dst[4 * i + 3] = __builtin_amdgcn_readfirstlane(v.w);
  }
  return d;
}

__device__ __forceinline__ int64_t uniform_row_begin(const rk_update_layer* p) {
  const int64_t v = p->row_begin;
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <int DT>
__device__ __forceinline__ GradUpdateArgs layer_args(const rk_update_layer& d) {
  constexpr int V = DT == RK_F32 ? 4 : 8;
  GradUpdateArgs a{};
  a.packed = reinterpret_cast<uint8_t*>(d.packed);
  a.ldp = d.ldp;
  if constexpr (DT == SRC_SPLITS) {
    a.part = reinterpret_cast<const float*>(d.g);
    a.nsplit = d.nsplit;
    a.part_stride = d.rows * d.K;
    a.vec_p = (d.packed % 8) == 0 && (d.ldp % 8) == 0;
  } else {
    a.g = reinterpret_cast<const void*>(d.g);
    a.ldg = d.ldg;
    a.vec_g = (d.g % 16) == 0 && (d.ldg % V) == 0 && (d.K % V) == 0;
    a.vec_p = (d.packed % V) == 0 && (d.ldp % V) == 0 && (d.K % V) == 0;
  }
  a.rows = d.rows;
  a.K = d.K;
  a.mc = d.max_code;
  a.T = d.threshold;
  a.low = d.low;
  a.high = d.high;
  a.eps = d.eps;
  a.rms_ema = reinterpret_cast<float*>(d.rms_ema);
  a.beta1 = d.beta1;
  a.beta2 = d.beta2;
  a.counts = reinterpret_cast<int64_t*>(d.counts);
  a.row_rms = reinterpret_cast<float*>(d.row_rms);
  a.grad_scale = reinterpret_cast<float*>(d.grad_scale);
  a.nonfinite = reinterpret_cast<int32_t*>(d.nonfinite);
  return a;
}

template <int DT, int NC, bool ONE_SPLIT>
__global__ __launch_bounds__(256) void ratchet_update_multi_kernel(const rk_update_layer* tab,
                                                                   int nlayers, int64_t total_rows,
                                                                   int64_t rows_per_wave) {
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 +
                    __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  int64_t r = w * rows_per_wave;
  const int64_t r_end = r + rows_per_wave < total_rows ? r + rows_per_wave : total_rows;
  if (r >= r_end) return;
  // the last layer whose rows start at or before r (an empty layer shares its row_begin with
  // the next one and is passed over)
  int lo = 0, hi = nlayers - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (uniform_row_begin(tab + mid) <= r) lo = mid;
    else hi = mid - 1;
  }
  int l = lo;
  rk_update_layer d = load_layer(tab + l);
  GradUpdateArgs a = layer_args<DT>(d);
  int64_t lbeg = d.row_begin, lend = lbeg + d.rows;
  MoveCounts cnt;
  for (; r < r_end; ++r) {
    if (r >= lend) {
      flush_wave_counts(cnt, a.counts);
      do {
        ++l;
        d = load_layer(tab + l);
        lbeg = d.row_begin;
        lend = lbeg + d.rows;
      } while (r >= lend);
      a = layer_args<DT>(d);
    }
    // K opaque per row, as in ratchet_update_grad_kernel
    int64_t K = a.K;
    asm volatile("" : "+s"(K));
    update_row<DT, NC, false, ONE_SPLIT>(a, r - lbeg, K, cnt);
  }
  flush_wave_counts(cnt, a.counts);
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

// Grid of the multi-layer update: as many blocks as stay resident (the kernel's occupancy
// times the device's CUs), each wavefront a contiguous share of the rows.
template <int DT, int NC, bool ONE_SPLIT>
static void launch_multi(const rk_update_layer* tab, int nl, int64_t total, hipStream_t s) {
  static const int per_cu = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, ratchet_update_multi_kernel<DT, NC, ONE_SPLIT>, 256, 0) != hipSuccess || n < 1)
      n = 1;
    return n;
  }();
  // the device's CU count, looked up once per device (the attribute query is a driver call)
  static int cu_cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int cus = __atomic_load_n(&cu_cache[dev], __ATOMIC_RELAXED);
  if (cus < 1) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
      cus = 256;
    __atomic_store_n(&cu_cache[dev], cus, __ATOMIC_RELAXED);
  }
  const int64_t want = (total + 3) / 4;
  const int64_t cap = static_cast<int64_t>(per_cu) * cus;
  const int64_t blocks = want < cap ? want : cap;
  const int64_t rpw = (total + 4 * blocks - 1) / (4 * blocks);
  ratchet_update_multi_kernel<DT, NC, ONE_SPLIT>
      <<<static_cast<unsigned>(blocks), 256, 0, s>>>(tab, nl, total, rpw);
}

template <int DT>
static void launch_multi_nc(const rk_update_layer* tab, int nl, int64_t total, int64_t kmax,
                            bool one_split, hipStream_t s) {
  constexpr int V = DT == RK_F32 ? 4 : 8;
  const int64_t nchunks = (kmax + 64 * V - 1) / (64 * V);
  if constexpr (DT == RK_F32) {
    if (nchunks <= 2) launch_multi<DT, 2, false>(tab, nl, total, s);
    else if (nchunks <= 8) launch_multi<DT, 8, false>(tab, nl, total, s);
    else launch_multi<DT, 0, false>(tab, nl, total, s);
  } else if constexpr (DT == RK_BF16) {
    if (nchunks <= 1) launch_multi<DT, 1, false>(tab, nl, total, s);
    else if (nchunks <= 4) launch_multi<DT, 4, false>(tab, nl, total, s);
    else if (nchunks <= 12) launch_multi<DT, 12, false>(tab, nl, total, s);
    else launch_multi<DT, 0, false>(tab, nl, total, s);
  } else {
    if (one_split) {
      if (nchunks <= 1) launch_multi<DT, 1, true>(tab, nl, total, s);
      else if (nchunks <= 4) launch_multi<DT, 4, true>(tab, nl, total, s);
      else if (nchunks <= 12) launch_multi<DT, 12, true>(tab, nl, total, s);
      else launch_multi<DT, 0, false>(tab, nl, total, s);
    } else {
      if (nchunks <= 1) launch_multi<DT, 1, false>(tab, nl, total, s);
      else if (nchunks <= 4) launch_multi<DT, 4, false>(tab, nl, total, s);
      else if (nchunks <= 12) launch_multi<DT, 12, false>(tab, nl, total, s);
      else launch_multi<DT, 0, false>(tab, nl, total, s);
    }
  }
}

}  // namespace rk

using namespace rk;

extern "C" int rk_ratchet_update_multi(const rk_update_layer* table_host,
                                       const rk_update_layer* table_dev, int nlayers, int src,
                                       void* stream) {
  clear_error();
  static_assert(sizeof(rk_update_layer) == 160, "rk_update_layer layout");
  if (nlayers < 1) return fail(RK_ERR_ARG, "nlayers must be positive");
  if (!table_host || !table_dev) return fail(RK_ERR_ARG, "null layer table");
  if (src != RK_F32 && src != RK_BF16 && src != RK_UPDATE_SRC_SPLITS)
    return fail(RK_ERR_ARG, "unsupported gradient source");
  int64_t total = 0, kmax = 0;
  bool one_split = true;
  for (int i = 0; i < nlayers; ++i) {
    const rk_update_layer& d = table_host[i];
    if (d.row_begin != total)
      return fail(RK_ERR_ARG, "layer %d: row_begin %lld where its rows start at %lld", i,
                  static_cast<long long>(d.row_begin), static_cast<long long>(total));
    if (int st = check_update_common(reinterpret_cast<const uint8_t*>(d.packed), d.ldp, d.rows,
                                     d.K, d.max_code, d.threshold, d.low, d.high)) {
      char msg[256];
      snprintf(msg, sizeof msg, "%s", rk_last_error());
      return fail(st, "layer %d: %s", i, msg);
    }
    if (!(d.eps > 0.0f)) return fail(RK_ERR_ARG, "layer %d: eps must be positive", i);
    if (d.rows > 0 && !d.g) return fail(RK_ERR_ARG, "layer %d: null gradient", i);
    if (src == RK_UPDATE_SRC_SPLITS) {
      if (d.nsplit < 1 || d.nsplit > 64) return fail(RK_ERR_ARG, "layer %d: nsplit must be in 1..64", i);
      if (d.K % 8 != 0 || d.g % 16 != 0)
        return fail(RK_ERR_UNSUPPORTED, "layer %d: partials need K %% 8 == 0 and 16-byte alignment", i);
      if (d.nsplit != 1) one_split = false;
    } else if (d.ldg < d.K) {
      return fail(RK_ERR_ARG, "layer %d: ldg < K", i);
    }
    if (d.rows > 0 && d.K > kmax) kmax = d.K;
    total += d.rows;
  }
  if (total == 0) return RK_OK;
  hipStream_t s = as_stream(stream);
  if (src == RK_F32) launch_multi_nc<RK_F32>(table_dev, nlayers, total, kmax, false, s);
  else if (src == RK_BF16) launch_multi_nc<RK_BF16>(table_dev, nlayers, total, kmax, false, s);
  else launch_multi_nc<SRC_SPLITS>(table_dev, nlayers, total, kmax, one_split, s);
  return launch_status("ratchet_update_multi");
}

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
