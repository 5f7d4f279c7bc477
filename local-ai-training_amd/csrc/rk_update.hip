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
#include "rk_common.h"

namespace rk {

struct MoveCounts {
  int pos = 0, neg = 0, bpos = 0, bneg = 0;
};

// One weight: ratchet.py:248-262 (bucket) and 277-294 (update + repack).
__device__ __forceinline__ uint32_t ratchet_byte(uint32_t byte, float z, int mc, int T,
                                                 float low, float high, MoveCounts& cnt) {
  const float a = fabsf(z);
  const int mag = a >= high ? 2 : (a >= low ? 1 : 0);
  const int sgn = (z > 0.0f) - (z < 0.0f);
  const int c = static_cast<int>(byte & 15u) - mc;
  int p = static_cast<int>(byte >> 4) - 7 - sgn * mag;
  const int pr = p >= T, nr = p <= -T;
  const int pm = pr & (c < mc), nm = nr & (c > -mc);
  p = p - pr * T + nr * T;
  p = min(max(p, -128), 127);
  cnt.pos += pm;
  cnt.neg += nm;
  cnt.bpos += pr & (pm ^ 1);
  cnt.bneg += nr & (nm ^ 1);
  const int cn = c + pm - nm;
  return static_cast<uint32_t>((cn + mc) & 15) | (static_cast<uint32_t>((p + 7) & 15) << 4);
}

// Smallest float t >= 0 with RN(t / d) >= c, for c > 0 and 0 < d < inf (+inf if no finite t
// qualifies). RN(x / d) is non-decreasing in x, so for every float g:
//   RN(|g| / d) >= c  <=>  |g| >= t,
// which turns the update's bucket tests on z = g / d into compares on |g| with no division
// per weight. The search starts at RN(c * d), within a few ulps of the boundary; `ok` is
// cleared if it does not settle within 8 steps (the caller then divides per weight).
__device__ __forceinline__ float bucket_threshold(float c, float d, bool& ok) {
  constexpr float kMax = 3.40282347e38f;
  float t = c * d;
  if (!(t < kMax)) t = kMax;
  int i = 0;
  for (; i < 8 && !(t / d >= c); ++i) {
    if (t == kMax) return INFINITY;
    t = __uint_as_float(__float_as_uint(t) + 1u);
  }
  if (i == 8) ok = false;
  int j = 0;
  for (; j < 8; ++j) {
    const float prev = __uint_as_float(__float_as_uint(t) - 1u);
    if (!(prev / d >= c)) break;
    t = prev;
  }
  if (j == 8) ok = false;
  return t;
}

// Per-launch byte constants of ratchet_word (ratchet.py:248-301 on four packed weights).
struct SwarConsts {
  uint32_t ge_pr;    // + x: bit 7 of a byte set iff x >= T + 9 (pressure reset up)
  uint32_t ge_nr;    // + x: bit 7 set iff x >= 10 - T (clear: pressure reset down)
  uint32_t ge_cmax;  // + code: bit 7 set iff code byte >= 2 * max_code
  uint32_t T;
};

__device__ __forceinline__ SwarConsts swar_consts(int T, int mc) {
  const int c_pr = T + 9 < 20 ? T + 9 : 20;   // x <= 19: thresholds above never fire
  const int c_nr = 10 - T > 0 ? 10 - T : 0;
  SwarConsts k;
  k.ge_pr = static_cast<uint32_t>(128 - c_pr) * 0x01010101u;
  k.ge_nr = static_cast<uint32_t>(128 - c_nr) * 0x01010101u;
  k.ge_cmax = static_cast<uint32_t>(128 - 2 * mc) * 0x01010101u;
  k.T = static_cast<uint32_t>(T);
  return k;
}

// The update of four weights in one packed word, byte i holding weight i, and e holding
// per byte 2 - sign(z) * mag(z) in [0, 4] (from the bucket compares). With the pressure
// biased by 9 (x = (p + 7) + 2 - sign * mag = p_new + 9 in [0, 19]) every per-byte step
// stays inside its byte: the compares add (128 - bound) and read bit 7, the resets
// subtract / add T only where x >= T + 9 / x <= 9 - T (never both, T >= 1), codes move
// only inside [0, 2 max_code]. Bit-identical to ratchet_byte on each byte: the pressure
// nibble wraps the same way and the int8 clamp never binds for |p| <= 10. A byte 0x70
// (pressure 0) with e = 2 changes nothing and counts nothing, which is how the bytes
// past the end of a row are filled.
__device__ __forceinline__ uint32_t ratchet_word(uint32_t w, uint32_t e, const SwarConsts& k,
                                                 MoveCounts& cnt) {
  const uint32_t cb = w & 0x0F0F0F0Fu;
  const uint32_t x = ((w >> 4) & 0x0F0F0F0Fu) + e;
  const uint32_t pr = ((x + k.ge_pr) >> 7) & 0x01010101u;
  const uint32_t nr = (((x + k.ge_nr) >> 7) & 0x01010101u) ^ 0x01010101u;
  const uint32_t cmax = ((cb + k.ge_cmax) >> 7) & 0x01010101u;
  const uint32_t cpos = ((cb + 0x7F7F7F7Fu) >> 7) & 0x01010101u;
  const uint32_t pm = pr & (cmax ^ 0x01010101u);
  const uint32_t nm = nr & cpos;
  const uint32_t y = x - pr * k.T + nr * k.T;
  cnt.pos += __builtin_popcount(pm);
  cnt.neg += __builtin_popcount(nm);
  cnt.bpos += __builtin_popcount(pr & cmax);
  cnt.bneg += __builtin_popcount(nr & (cpos ^ 0x01010101u));
  const uint32_t cn = cb + pm - nm;
  const uint32_t pn = (y + 0x0E0E0E0Eu) & 0x0F0F0F0Fu;
  return cn | (pn << 4);
}

// Block-level count reduction and one 64-bit atomic per counter per block.
__device__ __forceinline__ void flush_counts(MoveCounts cnt, int64_t* counts) {
  __shared__ int sc[4];
  if (threadIdx.x < 4) sc[threadIdx.x] = 0;
  __syncthreads();
  const int p = wave_sum_int(cnt.pos), n = wave_sum_int(cnt.neg);
  const int bp = wave_sum_int(cnt.bpos), bn = wave_sum_int(cnt.bneg);
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&sc[0], p);
    atomicAdd(&sc[1], n);
    atomicAdd(&sc[2], bp);
    atomicAdd(&sc[3], bn);
  }
  __syncthreads();
  if (threadIdx.x < 4 && counts) {
    const int v = sc[threadIdx.x];
    if (v) atomicAdd(reinterpret_cast<unsigned long long*>(counts) + threadIdx.x,
                     static_cast<unsigned long long>(v));
  }
}

__device__ __forceinline__ bool finite_f32(float x) {
  return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u;
}

// Loads V packed bytes (FILL past K) into one word per 4 bytes.
template <int V, uint32_t FILL = 0u>
__device__ __forceinline__ void load_bytes(const uint8_t* p, int64_t e0, int64_t K, bool vec,
                                           uint32_t* w) {
  if (vec && e0 + V <= K) {
    if constexpr (V == 8) {
      const uint2 t = *reinterpret_cast<const uint2*>(p + e0);
      w[0] = t.x;
      w[1] = t.y;
    } else {
      w[0] = *reinterpret_cast<const uint32_t*>(p + e0);
    }
  } else {
#pragma unroll
    for (int j = 0; j < V / 4; ++j) w[j] = FILL * 0x01010101u;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (e0 + i < K)
        w[i >> 2] = (w[i >> 2] & ~(0xffu << (8 * (i & 3)))) |
                    (static_cast<uint32_t>(p[e0 + i]) << (8 * (i & 3)));
  }
}

template <int V>
__device__ __forceinline__ void store_bytes(uint8_t* p, int64_t e0, int64_t K, bool vec,
                                            const uint32_t* w) {
  if (vec && e0 + V <= K) {
    if constexpr (V == 8) {
      *reinterpret_cast<uint2*>(p + e0) = make_uint2(w[0], w[1]);
    } else {
      *reinterpret_cast<uint32_t*>(p + e0) = w[0];
    }
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (e0 + i < K) p[e0 + i] = static_cast<uint8_t>(w[i >> 2] >> (8 * (i & 3)));
  }
}

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

// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t upd_pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const bf2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// Fused normalize + update from the raw weight gradient (one wavefront per row).
// NC > 0: the row's gradient stays in registers between the two passes.
// ---------------------------------------------------------------------------
// Gradient source of the fused kernel besides RK_F32 / RK_BF16 tensors: the fp32 split
// partials of the grad_weight GEMM, part[s][row][k] (split stride part_stride), added in
// split order and rounded to bf16 exactly as grad_weight_reduce_kernel does, then consumed
// with the bf16 source's vector width (so every later operation, including the
// sum-of-squares order, is the one the bf16 gradient would see).
constexpr int SRC_SPLITS = 2;

struct GradUpdateArgs {
  uint8_t* packed;
  int64_t ldp;
  const void* g;
  int64_t ldg;
  const float* part;      // SRC_SPLITS: partials and their count / split stride
  int nsplit;
  int64_t part_stride;
  uint16_t* g_out;        // SRC_SPLITS: optional copy of the bf16 gradient consumed
  int64_t ldgo;
  int64_t rows, K;
  int mc, T;
  float low, high, eps;
  float* rms_ema;
  float beta1, beta2;
  int64_t* counts;
  float* row_rms;
  float* grad_scale;
  int32_t* nonfinite;
  float* z_out;  // normalize-only mode: z[row, k] (row stride ldz)
  int64_t ldz;
  int vec_g, vec_p;
};

// mean[0] = mean of row_rms[0 .. rows): one block, each thread a strided partial in
// fixed order, then a fixed LDS tree, so the result is reproducible.
__global__ __launch_bounds__(256) void row_rms_mean_kernel(const float* row_rms, int64_t rows,
                                                            float* mean) {
  __shared__ float part[256];
  float acc = 0.0f;
  for (int64_t r = threadIdx.x; r < rows; r += 256) acc = acc + row_rms[r];
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) part[threadIdx.x] = part[threadIdx.x] + part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) mean[0] = part[0] / static_cast<float>(rows);
}
// ZONLY = true: write z = g / (rms + eps) instead of updating (the reference's
// _normalize, ratchet.py:539-556), with the identical reduction order.
template <int DT, int NC, bool ZONLY>
__global__ __launch_bounds__(256) void ratchet_update_grad_kernel(GradUpdateArgs a) {
  constexpr int V = DT == RK_F32 ? 4 : 8;
  constexpr int SPAN = 64 * V;
  constexpr int NW = V / 4;
  const int lane = threadIdx.x & 63;
  const int64_t lane0 = static_cast<int64_t>(lane) * V;
  const int64_t nchunks = (a.K + SPAN - 1) / SPAN;
  MoveCounts cnt;

  for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < a.rows;
       row += static_cast<int64_t>(gridDim.x) * 4) {
    const char* grow =
        static_cast<const char*>(a.g) + row * a.ldg * (DT == RK_F32 ? 4 : 2);
    uint8_t* prow = a.packed + row * a.ldp;

    auto load_g = [&](int64_t e0, float* v) {
      if constexpr (DT == SRC_SPLITS) {
        // K % 8 == 0 (checked on the host): a vector is wholly inside or past the row
        if (e0 < a.K) {
          const float* p = a.part + row * a.K + e0;
          float4 lo = *reinterpret_cast<const float4*>(p);
          float4 hi = *reinterpret_cast<const float4*>(p + 4);
#pragma unroll 8
          for (int s = 1; s < a.nsplit; ++s) {
            const float4 l2 = *reinterpret_cast<const float4*>(p + s * a.part_stride);
            const float4 h2 = *reinterpret_cast<const float4*>(p + s * a.part_stride + 4);
            lo.x = lo.x + l2.x;
            lo.y = lo.y + l2.y;
            lo.z = lo.z + l2.z;
            lo.w = lo.w + l2.w;
            hi.x = hi.x + h2.x;
            hi.y = hi.y + h2.y;
            hi.z = hi.z + h2.z;
            hi.w = hi.w + h2.w;
          }
          const uint32_t w[4] = {upd_pack_bf16x2(lo.x, lo.y), upd_pack_bf16x2(lo.z, lo.w),
                                 upd_pack_bf16x2(hi.x, hi.y), upd_pack_bf16x2(hi.z, hi.w)};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i) v[i] = 0.0f;
        }
      } else if (a.vec_g && e0 + V <= a.K) {
        load_vec16<DT>(grow, e0, v);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = e0 + i < a.K ? load_elem<DT>(grow, e0 + i) : 0.0f;
      }
    };
    // SRC_SPLITS with a gradient copy requested: written once, from pass 1
    auto keep_g = [&](int64_t e0, const float* v) {
      if constexpr (DT == SRC_SPLITS) {
        if (a.g_out && e0 < a.K) {
          uint4 w;
          w.x = (__float_as_uint(v[0]) >> 16) | (__float_as_uint(v[1]) & 0xffff0000u);
          w.y = (__float_as_uint(v[2]) >> 16) | (__float_as_uint(v[3]) & 0xffff0000u);
          w.z = (__float_as_uint(v[4]) >> 16) | (__float_as_uint(v[5]) & 0xffff0000u);
          w.w = (__float_as_uint(v[6]) >> 16) | (__float_as_uint(v[7]) & 0xffff0000u);
          *reinterpret_cast<uint4*>(a.g_out + row * a.ldgo + e0) = w;
        }
      }
    };

    // Pass 1: sum of squares (fixed order). A non-finite gradient element makes the sum
    // non-finite, so only a row whose sum is not finite (overflow of finite values
    // included) is searched element by element.
    float xr[NC > 0 ? NC : 1][V];
    float acc = 0.0f;
    if constexpr (NC > 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (c < nchunks) {
          load_g(c * SPAN + lane0, xr[c]);
          keep_g(c * SPAN + lane0, xr[c]);
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i) xr[c][i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < V; ++i) acc = acc + xr[c][i] * xr[c][i];
      }
    } else {
      for (int64_t c = 0; c < nchunks; ++c) {
        float v[V];
        load_g(c * SPAN + lane0, v);
        keep_g(c * SPAN + lane0, v);
#pragma unroll
        for (int i = 0; i < V; ++i) acc = acc + v[i] * v[i];
      }
    }
    acc = wave_sum_butterfly(acc);
    int bad = 0;
    if (!finite_f32(acc)) {
      if constexpr (NC > 0) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int i = 0; i < V; ++i) bad |= !finite_f32(xr[c][i]);
      } else {
        for (int64_t c = 0; c < nchunks; ++c) {
          float v[V];
          load_g(c * SPAN + lane0, v);
#pragma unroll
          for (int i = 0; i < V; ++i) bad |= !finite_f32(v[i]);
        }
      }
      bad = wave_or_int(bad);
    }

    const float ms = acc / static_cast<float>(a.K);
    const float rms_inst = sqrtf(ms);
    float rms = rms_inst;
    if (a.rms_ema) {
      const float ema = a.rms_ema[row];
      const float upd = ema == 0.0f ? ms : a.beta1 * ema + a.beta2 * ms;
      const float ema_new = ms > 0.0f ? upd : ema;
      rms = sqrtf(ema_new);
      if ((ZONLY || !bad) && lane == 0) a.rms_ema[row] = ema_new;
    }
    if (a.row_rms && lane == 0) a.row_rms[row] = rms_inst;
    if constexpr (ZONLY) {
      const float dz = rms + a.eps;
      float* zrow = a.z_out + row * a.ldz;
      for (int64_t c = 0; c < nchunks; ++c) {
        const int64_t e0 = c * SPAN + lane0;
        if (e0 >= a.K) break;
        float v[V];
        if constexpr (NC > 0) {
#pragma unroll
          for (int cc = 0; cc < NC; ++cc)
            if (cc == c) {
#pragma unroll
              for (int i = 0; i < V; ++i) v[i] = xr[cc][i];
            }
        } else {
          load_g(e0, v);
        }
#pragma unroll
        for (int i = 0; i < V; ++i)
          if (e0 + i < a.K) zrow[e0 + i] = v[i] / dz;
      }
      continue;
    }
    if (bad) {
      if (lane == 0 && a.nonfinite) a.nonfinite[0] = 1;
      continue;
    }
    const float d = rms + a.eps;

    // Pass 2: normalize, update, repack; optional sum_k g * code (pre-update code).
    // z = g / d is never formed on the fast path: with tl / th the smallest floats whose
    // quotient by d reaches low / high, |z| >= low <=> |g| >= tl and likewise for high
    // (division is monotone), and for low > 0 a weight that moves has z != 0, so
    // sign(z) = sign(g). The per-weight division stays for low == 0 (where an underflowed
    // z of sign 0 still buckets), d not finite and positive, or an unsettled search.
    bool fast = a.low > 0.0f && d > 0.0f && d < INFINITY;
    float tl = 0.0f, th = 0.0f;
    if (fast) {
      tl = bucket_threshold(a.low, d, fast);
      th = bucket_threshold(a.high, d, fast);
    }
    const SwarConsts kc = swar_consts(a.T, a.mc);
    float gs = 0.0f;
    auto do_chunk = [&](int64_t e0, const float* v) {
      uint32_t w[NW], out[NW];
      load_bytes<V, 0x70u>(prow, e0, a.K, a.vec_p, w);
      if (a.grad_scale) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const uint32_t byte = (w[i >> 2] >> (8 * (i & 3))) & 0xffu;
          gs = gs + v[i] * static_cast<float>(static_cast<int>(byte & 15u) - a.mc);
        }
      }
      if (fast) {
#pragma unroll
        for (int j = 0; j < NW; ++j) {
          uint32_t e = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float g = v[4 * j + q];
            const uint32_t m = (fabsf(g) >= tl ? 1u : 0u) + (fabsf(g) >= th ? 1u : 0u);
            e |= (__float_as_uint(g) >> 31 ? 2u + m : 2u - m) << (8 * q);
          }
          out[j] = ratchet_word(w[j], e, kc, cnt);
        }
      } else {
#pragma unroll
        for (int j = 0; j < NW; ++j) out[j] = 0;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          if (e0 + i < a.K) {
            const uint32_t byte = (w[i >> 2] >> (8 * (i & 3))) & 0xffu;
            out[i >> 2] |=
                ratchet_byte(byte, v[i] / d, a.mc, a.T, a.low, a.high, cnt) << (8 * (i & 3));
          }
        }
      }
      store_bytes<V>(prow, e0, a.K, a.vec_p, out);
    };
    if constexpr (NC > 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int64_t e0 = c * SPAN + lane0;
        if (c < nchunks && e0 < a.K) do_chunk(e0, xr[c]);
      }
    } else {
      for (int64_t c = 0; c < nchunks; ++c) {
        const int64_t e0 = c * SPAN + lane0;
        if (e0 >= a.K) break;
        float v[V];
        load_g(e0, v);
        do_chunk(e0, v);
      }
    }
    if (a.grad_scale) {
      gs = wave_sum_butterfly(gs);
      if (lane == 0) a.grad_scale[row] = gs;
    }
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

template <bool ZONLY>
static int launch_grad_kernel(const GradUpdateArgs& a, int g_dtype, hipStream_t s) {
  const int V = g_dtype == RK_F32 ? 4 : 8;
  const int64_t nchunks = (a.K + 64 * V - 1) / (64 * V);
  const dim3 grid(row_grid(a.rows)), block(256);
  if (g_dtype == RK_F32) {
    if (nchunks <= 2) ratchet_update_grad_kernel<RK_F32, 2, ZONLY><<<grid, block, 0, s>>>(a);
    else if (nchunks <= 8) ratchet_update_grad_kernel<RK_F32, 8, ZONLY><<<grid, block, 0, s>>>(a);
    else ratchet_update_grad_kernel<RK_F32, 0, ZONLY><<<grid, block, 0, s>>>(a);
  } else if (g_dtype == RK_BF16) {
    if (nchunks <= 1) ratchet_update_grad_kernel<RK_BF16, 1, ZONLY><<<grid, block, 0, s>>>(a);
    else if (nchunks <= 4) ratchet_update_grad_kernel<RK_BF16, 4, ZONLY><<<grid, block, 0, s>>>(a);
    else if (nchunks <= 12) ratchet_update_grad_kernel<RK_BF16, 12, ZONLY><<<grid, block, 0, s>>>(a);
    else ratchet_update_grad_kernel<RK_BF16, 0, ZONLY><<<grid, block, 0, s>>>(a);
  } else if constexpr (!ZONLY) {
    if (nchunks <= 1) ratchet_update_grad_kernel<SRC_SPLITS, 1, false><<<grid, block, 0, s>>>(a);
    else if (nchunks <= 4) ratchet_update_grad_kernel<SRC_SPLITS, 4, false><<<grid, block, 0, s>>>(a);
    else if (nchunks <= 12) ratchet_update_grad_kernel<SRC_SPLITS, 12, false><<<grid, block, 0, s>>>(a);
    else ratchet_update_grad_kernel<SRC_SPLITS, 0, false><<<grid, block, 0, s>>>(a);
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
