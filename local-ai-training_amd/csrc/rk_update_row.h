// Device code of the fused integer ratchet update (gfx950), shared by the update kernels
// (rk_update.hip) and the grad_weight kernel that runs the update of its last row block
// (rk_gradw.hip).
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
#pragma once

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
    const int64_t rem = K - e0;
#pragma unroll
    for (int j = 0; j < V / 4; ++j) w[j] = FILL * 0x01010101u;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (i < rem)
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
    const int64_t rem = K - e0;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (i < rem) p[e0 + i] = static_cast<uint8_t>(w[i >> 2] >> (8 * (i & 3)));
  }
}


// ---------------------------------------------------------------------------
typedef float upd_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

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

template <int DT>
__device__ __forceinline__ float vec_elem(const uint32_t* w, int i) {
  if constexpr (DT == RK_F32) {
    return __uint_as_float(w[i]);
  } else {
    return __uint_as_float((i & 1) ? (w[i >> 1] & 0xffff0000u) : (w[i >> 1] << 16));
  }
}

// Smallest bf16 bit pattern whose value is >= t, for t >= 0 (+inf -> 0x7f80): for a bf16
// g, |g| >= t <=> bits(|g|) >= bf16_ceil_bits(t).
__device__ __forceinline__ uint32_t bf16_ceil_bits(float t) {
  const uint32_t b = __float_as_uint(t);
  return (b >> 16) + ((b & 0xffffu) != 0u ? 1u : 0u);
}

// Bucket bytes (2 - sign(g) * mag(g), byte q for element q) of four bf16 gradients held in
// two words, from 16-bit compares: kl / kh = (0x8000 - threshold bits) in both halves, so
// bit 15 of a half of |g| + k is set iff |g| >= threshold (|g| <= 0x7fff: no carry between
// halves). v_perm selectors 8..11 replicate bits 15 / 31 of its second and first source
// into a byte: 0x0b0a0908 lays out elements 0..3.
__device__ __forceinline__ uint32_t bucket_bytes_bf16(uint32_t w0, uint32_t w1, uint32_t kl,
                                                      uint32_t kh) {
  constexpr uint32_t kSel = 0x0b0a0908u;
  const uint32_t a0 = w0 & 0x7fff7fffu, a1 = w1 & 0x7fff7fffu;
  const uint32_t gel = __builtin_amdgcn_perm(a1 + kl, a0 + kl, kSel);
  const uint32_t geh = __builtin_amdgcn_perm(a1 + kh, a0 + kh, kSel);
  const uint32_t neg = __builtin_amdgcn_perm(w1, w0, kSel);
  const uint32_t m = (gel & 0x01010101u) + (geh & 0x01010101u);
  return 0x02020202u - m + (neg & (m << 1));
}

// Bucket bytes of four fp32 gradients from float compares against the thresholds.
__device__ __forceinline__ uint32_t bucket_bytes_f32(const uint32_t* w, float tl, float th) {
  uint32_t e = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float g = __uint_as_float(w[q]);
    const uint32_t m = (fabsf(g) >= tl ? 1u : 0u) + (fabsf(g) >= th ? 1u : 0u);
    e |= ((w[q] >> 31) ? 2u + m : 2u - m) << (8 * q);
  }
  return e;
}

// ZONLY = true: write z = g / (rms + eps) instead of updating (the reference's
// _normalize, ratchet.py:539-556), with the identical reduction order.
//
// A lane holds a row's gradient as 16-byte vectors (four words: 4 fp32 or 8 bf16), chunk c
// covering elements c * 64 * V + lane * V. NC > 0: the whole row stays in registers between
// the passes, the packed bytes are fetched with the gradient, and every load of the row is
// in flight before the first is consumed. NC == 0: rows longer than the register chunks
// stream twice.

// One row of the fused normalize + update (the body of ratchet_update_grad_kernel, shared
// with the grad_weight kernel that runs the update of its last row block): one wavefront
// processes row `row` of K columns and adds its move counts into `cnt`. NC > 0 holds the
// row's gradient in registers between the two passes; NC == 0 streams it twice.
template <int DT, int NC, bool ZONLY, bool ONE_SPLIT = false>
__device__ __forceinline__ void update_row(const GradUpdateArgs& a, int64_t row, int64_t K,
                                           MoveCounts& cnt) {
  constexpr int V = DT == RK_F32 ? 4 : 8;
  constexpr int SPAN = 64 * V;
  constexpr int NW = V / 4;
  constexpr int NCR = NC > 0 ? NC : 1;
  constexpr bool BF16W = DT != RK_F32;  // words hold bf16 pairs
  constexpr int ES = DT == RK_F32 ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const int64_t lane0 = static_cast<int64_t>(lane) * V;

  // Registers of one row between its loads and its arithmetic.
  struct Stage {
    upd_f32x4 lo[NCR], hi[NCR];  // SRC_SPLITS: split 0
    uint32_t xg[NCR][4];          // other sources: the gradient words
    uint32_t xp[NCR][NW];         // packed bytes
  };

  auto add4 = [](float4& x, const float4& y) {
    x.x = x.x + y.x;
    x.y = x.y + y.y;
    x.z = x.z + y.z;
    x.w = x.w + y.w;
  };

  // Issues every unconditional load of row `row` into `st`.
  auto issue = [&](int64_t row, int64_t K, Stage& st) {
    if constexpr (NC > 0) {
      if constexpr (DT == SRC_SPLITS) {
        const __amdgpu_buffer_rsrc_t rs = make_buffer(a.part + row * K, K * 4);
        const uint32_t voff = static_cast<uint32_t>(lane0) * 4u;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          st.lo[c] = __builtin_bit_cast(
              upd_f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, c * SPAN * 4, 0));
          st.hi[c] = __builtin_bit_cast(
              upd_f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, c * SPAN * 4 + 16, 0));
        }
      } else {
        // a vector wholly past K, or every vector when the gradient is not vector-aligned,
        // reads as zero (the unaligned case is re-read element by element in `body`)
        const char* grow = static_cast<const char*>(a.g) + row * a.ldg * ES;
        const __amdgpu_buffer_rsrc_t rg =
            make_buffer(grow, a.vec_g ? static_cast<int>(K) * ES : 0);
        const uint32_t voff = static_cast<uint32_t>(lane0) * ES;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const u32x4_t t = __builtin_bit_cast(
              u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rg, voff, c * SPAN * ES, 0));
          st.xg[c][0] = t.x;
          st.xg[c][1] = t.y;
          st.xg[c][2] = t.z;
          st.xg[c][3] = t.w;
        }
      }
      if constexpr (!ZONLY) {
        // K % V == 0 whenever vec_p, so a vector is wholly inside or past the row; without
        // vec_p every load reads zero and `body` reads the bytes one by one
        const __amdgpu_buffer_rsrc_t rp =
            make_buffer(a.packed + row * a.ldp, a.vec_p ? static_cast<int>(K) : 0);
        const uint32_t voff = static_cast<uint32_t>(lane0);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          if constexpr (V == 8) {
            const u32x2_t t = __builtin_bit_cast(
                u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rp, voff, c * SPAN, 0));
            st.xp[c][0] = t.x;
            st.xp[c][NW - 1] = t.y;
          } else {
            st.xp[c][0] = __builtin_amdgcn_raw_buffer_load_b32(rp, voff, c * SPAN, 0);
          }
        }
      }
    }
  };

  // Everything after the loads for one row.
  auto body = [&](int64_t row, int64_t K, Stage& st) {
    const int64_t nchunks = (K + SPAN - 1) / SPAN;
    const char* grow = static_cast<const char*>(a.g) + row * a.ldg * ES;
    uint8_t* prow = a.packed + row * a.ldp;
    const float* prt = a.part + row * K;

    // One vector of the gradient as words (zeros past K).
    auto load_words = [&](int64_t e0, uint32_t* w) {
      if constexpr (DT == SRC_SPLITS) {
        // K % 8 == 0 (checked on the host): a vector is wholly inside or past the row
        if (e0 < K) {
          float4 lo = *reinterpret_cast<const float4*>(prt + e0);
          float4 hi = *reinterpret_cast<const float4*>(prt + e0 + 4);
#pragma unroll 8
          for (int s = 1; s < a.nsplit; ++s) {
            add4(lo, *reinterpret_cast<const float4*>(prt + s * a.part_stride + e0));
            add4(hi, *reinterpret_cast<const float4*>(prt + s * a.part_stride + e0 + 4));
          }
          w[0] = upd_pack_bf16x2(lo.x, lo.y);
          w[1] = upd_pack_bf16x2(lo.z, lo.w);
          w[2] = upd_pack_bf16x2(hi.x, hi.y);
          w[3] = upd_pack_bf16x2(hi.z, hi.w);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = 0;
        }
      } else if (a.vec_g && e0 + V <= K) {
        const uint4 raw = *reinterpret_cast<const uint4*>(grow + e0 * ES);
        w[0] = raw.x;
        w[1] = raw.y;
        w[2] = raw.z;
        w[3] = raw.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = 0;
        const int64_t rem = K - e0;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          if (i < rem) {
            const uint32_t b = __float_as_uint(load_elem<DT>(grow, e0 + i));
            if constexpr (BF16W) w[i >> 1] |= (i & 1) ? (b & 0xffff0000u) : (b >> 16);
            else w[i] = b;
          }
        }
      }
    };
    // SRC_SPLITS with a gradient copy requested: the bf16 words, written once, in pass 1
    auto keep_words = [&](int64_t e0, const uint32_t* w) {
      if constexpr (DT == SRC_SPLITS) {
        if (a.g_out && e0 < K)
          *reinterpret_cast<uint4*>(a.g_out + row * a.ldgo + e0) = make_uint4(w[0], w[1], w[2], w[3]);
      }
    };
    auto sumsq = [&](float acc, const uint32_t* w) {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float x = vec_elem<DT>(w, i);
        acc = acc + x * x;
      }
      return acc;
    };

    // Pass 1: the remaining loads, then the sum of squares in fixed order. A non-finite
    // gradient element makes the sum non-finite, so only a row whose sum is not finite
    // (overflow of finite values included) is searched element by element.
    uint32_t (&xg)[NCR][4] = st.xg;
    float acc = 0.0f;
    if constexpr (NC > 0) {
      if constexpr (DT == SRC_SPLITS) {
        // later splits (buffer loads, one descriptor per split), GS splits of every chunk
        // in flight at a time, added in split order
        constexpr int GS = NC >= 8 ? 1 : (NC >= 4 ? 2 : (NC >= 2 ? 4 : 8));
        const uint32_t voff = static_cast<uint32_t>(lane0) * 4u;
        auto ld = [&](__amdgpu_buffer_rsrc_t r, int c, int half) {
          return __builtin_bit_cast(
              upd_f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, c * SPAN * 4 + 16 * half, 0));
        };
        // (ONE_SPLIT: the caller guarantees nsplit == 1, and no registers are set aside for
        // later splits)
        for (int s = 1; !ONE_SPLIT && s < a.nsplit; s += GS) {
          upd_f32x4 l[GS][NC], h[GS][NC];
#pragma unroll
          for (int q = 0; q < GS; ++q) {
            if (s + q < a.nsplit) {
              const __amdgpu_buffer_rsrc_t r = make_buffer(prt + (s + q) * a.part_stride, K * 4);
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                l[q][c] = ld(r, c, 0);
                h[q][c] = ld(r, c, 1);
              }
            }
          }
#pragma unroll
          for (int q = 0; q < GS; ++q) {
            if (s + q < a.nsplit) {
#pragma unroll
              for (int c = 0; c < NC; ++c) {
                st.lo[c] = st.lo[c] + l[q][c];
                st.hi[c] = st.hi[c] + h[q][c];
              }
            }
          }
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          xg[c][0] = upd_pack_bf16x2(st.lo[c].x, st.lo[c].y);
          xg[c][1] = upd_pack_bf16x2(st.lo[c].z, st.lo[c].w);
          xg[c][2] = upd_pack_bf16x2(st.hi[c].x, st.hi[c].y);
          xg[c][3] = upd_pack_bf16x2(st.hi[c].z, st.hi[c].w);
        }
      } else if (!a.vec_g) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          if (c < nchunks) {
            load_words(c * SPAN + lane0, xg[c]);
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) xg[c][j] = 0;
          }
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (c < nchunks) keep_words(c * SPAN + lane0, xg[c]);
        acc = sumsq(acc, xg[c]);
      }
    } else {
      for (int64_t c = 0; c < nchunks; ++c) {
        uint32_t w[4];
        load_words(c * SPAN + lane0, w);
        keep_words(c * SPAN + lane0, w);
        acc = sumsq(acc, w);
      }
    }
    acc = wave_sum_butterfly(acc);
    int bad = 0;
    if (!finite_f32(acc)) {
      auto scan = [&](const uint32_t* w) {
#pragma unroll
        for (int i = 0; i < V; ++i) bad |= !finite_f32(vec_elem<DT>(w, i));
      };
      if constexpr (NC > 0) {
#pragma unroll
        for (int c = 0; c < NC; ++c) scan(xg[c]);
      } else {
        for (int64_t c = 0; c < nchunks; ++c) {
          uint32_t w[4];
          load_words(c * SPAN + lane0, w);
          scan(w);
        }
      }
      bad = wave_or_int(bad);
    }

    const float ms = acc / static_cast<float>(K);
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
        if (e0 >= K) break;
        uint32_t w[4];
        if constexpr (NC > 0) {
#pragma unroll
          for (int cc = 0; cc < NC; ++cc)
            if (cc == c) {
#pragma unroll
              for (int j = 0; j < 4; ++j) w[j] = xg[cc][j];
            }
        } else {
          load_words(e0, w);
        }
        const int64_t rem = K - e0;
#pragma unroll
        for (int i = 0; i < V; ++i)
          if (i < rem) zrow[e0 + i] = vec_elem<DT>(w, i) / dz;
      }
      return;
    }
    if (bad) {
      if (lane == 0 && a.nonfinite) a.nonfinite[0] = 1;
      return;
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
    const uint32_t kl = (0x8000u - bf16_ceil_bits(tl)) * 0x00010001u;
    const uint32_t kh = (0x8000u - bf16_ceil_bits(th)) * 0x00010001u;
    const SwarConsts kc = swar_consts(a.T, a.mc);
    float gs = 0.0f;
    auto scale_terms = [&](const uint32_t* g, const uint32_t* w) {
      if (a.grad_scale) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const uint32_t byte = (w[i >> 2] >> (8 * (i & 3))) & 0xffu;
          gs = gs + vec_elem<DT>(g, i) * static_cast<float>(static_cast<int>(byte & 15u) - a.mc);
        }
      }
    };
    auto fast_chunk = [&](int64_t e0, const uint32_t* g, const uint32_t* wp) {
      uint32_t w[NW];
#pragma unroll
      for (int j = 0; j < NW; ++j) w[j] = wp[j];
      if (NC > 0 && !a.vec_p) load_bytes<V, 0x70u>(prow, e0, K, false, w);
      scale_terms(g, w);
      uint32_t out[NW];
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        uint32_t e;
        if constexpr (BF16W) e = bucket_bytes_bf16(g[2 * j], g[2 * j + 1], kl, kh);
        else e = bucket_bytes_f32(g, tl, th);
        out[j] = ratchet_word(w[j], e, kc, cnt);
      }
      store_bytes<V>(prow, e0, K, a.vec_p, out);
    };
    if (fast && NC > 0) {
#pragma unroll
      for (int c = 0; c < NCR; ++c) {
        const int64_t e0 = c * SPAN + lane0;
        if (c < nchunks && e0 < K) fast_chunk(e0, xg[c], st.xp[c]);
      }
    } else {
      // streaming rows, and the division path (re-read from memory: nothing has been
      // written yet), one chunk at a time
      for (int64_t c = 0; c < nchunks; ++c) {
        const int64_t e0 = c * SPAN + lane0;
        if (e0 >= K) break;
        uint32_t g[4], w[NW];
        load_words(e0, g);
        load_bytes<V, 0x70u>(prow, e0, K, a.vec_p, w);
        if (fast) {
          fast_chunk(e0, g, w);
        } else {
          scale_terms(g, w);
          uint32_t out[NW];
#pragma unroll
          for (int j = 0; j < NW; ++j) out[j] = 0;
          const int64_t rem = K - e0;
#pragma unroll
          for (int i = 0; i < V; ++i) {
            if (i < rem) {
              const uint32_t byte = (w[i >> 2] >> (8 * (i & 3))) & 0xffu;
              out[i >> 2] |= ratchet_byte(byte, vec_elem<DT>(g, i) / d, a.mc, a.T, a.low,
                                          a.high, cnt) << (8 * (i & 3));
            }
          }
          store_bytes<V>(prow, e0, K, a.vec_p, out);
        }
      }
    }
    if (a.grad_scale) {
      gs = wave_sum_butterfly(gs);
      if (lane == 0) a.grad_scale[row] = gs;
    }
  };

  Stage st;
  issue(row, K, st);
  body(row, K, st);
}

}  // namespace rk
