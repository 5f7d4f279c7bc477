// Causal self-attention forward of the training step (flash form, gfx950), for the model's
// F.scaled_dot_product_attention(q, k, v, is_causal=True) (model.py:117-123): bf16 q, k, v
// [B, H, S, D] (any batch / head / position strides, unit feature stride), D = 64 or 128.
// Writes o (bf16) and the per-query log-sum-exp lse = log(sum_j exp(s_j)) of the scaled
// scores s_j = (q . k_j) * scale, float32 [B, H, S], the pair torch's memory-efficient
// attention backward takes (so the backward stays torch's).
//
// One workgroup = 4 wavefronts = 128 queries of one (batch, head); key blocks (64 keys for
// D = 64, 32 for D = 128) are staged in LDS (K row-major, V transposed). Each wavefront owns 32 queries and computes
// S^T = K . Q^T with v_mfma_f32_32x32x16_bf16, K rows as the first operand and its Q rows
// (held in registers) as the second, so a lane holds all the scores of ONE query (its
// lane index mod 32) for 16 keys of each 32-key tile (the partner lane l ^ 32 holds the
// other 16): the softmax's row max and row sum are a lane's own values plus one xor-32
// exchange. The online softmax runs in base 2 (scores times scale * log2 e, exp2). The
// output accumulates transposed, O^T = V^T . P^T: the 8 probabilities a lane holds for
// one 16-key MFMA step are exactly the second operand that step needs, once the
// operand's k slots are mapped to keys {16 s + 4 h + 0..3, 16 s + 8 + 4 h + 0..3}
// (h = lane / 32, the accumulator's own row order), and the first operand reads V^T with
// the same slot order. The probabilities enter the product rounded to bf16; their sum
// stays float32. Causal blocks above a wavefront's diagonal are skipped; the diagonal
// block is masked per element. Every global load goes through a buffer descriptor bounded
// by the (batch, head) extent, so positions past S read zeros without a test.
#include "rk_common.h"

namespace rk {

typedef float v16f_a __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf_a __attribute__((ext_vector_type(8)));

constexpr int kAttnBM = 128;  // queries per workgroup (4 wavefronts x 32)

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t sqb, sqh, sqs;  // element strides (feature stride 1)
  int64_t skb, skh, sks;
  int64_t svb, svh, svs;
  uint16_t* o;
  int64_t sob, soh, sos;
  float* lse;  // [B, H, S]
  int64_t B, H, S;
  float scale_log2;  // scale * log2(e)
};

__device__ __forceinline__ v8bf_a as_v8bf(uint4 r) { return __builtin_bit_cast(v8bf_a, r); }

typedef __bf16 bf16x2_a __attribute__((ext_vector_type(2)));

// Two finite floats -> a bf16 pair (low half first), round to nearest even: gfx950's
// packed conversion, one instruction per pair.
__device__ __forceinline__ uint32_t bf16x2_of(float lo, float hi) {
  const bf16x2_a v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// BN keys per block: 64 for D = 64; 32 for D = 128, which keeps the scores, probabilities
// and staging registers small enough for two wavefronts per SIMD.
template <int D, int BN>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs a) {
  constexpr int BM = kAttnBM, KT = BN / 32;
  constexpr int KP = D * 2 + 16;  // K row pitch (bytes): 16 rows of a fragment read cover all banks
  constexpr int VP = BN * 2 + 8;  // V^T row pitch (bytes): the 32 rows of a fragment read are
                                  // 34 dwords apart, 32 distinct even banks
  constexpr int PIECES = BN * D / 8 / 256;  // 16-byte pieces of K per thread
  constexpr int VKEYS = 4, DG = D / 4;       // V staging: 4 keys x 4 features per thread
  static_assert((BN / VKEYS) * DG == 256, "one 4 x 4 V piece per thread");
  // two buffers: block kb + 1 is written while block kb is read
  __shared__ __attribute__((aligned(16))) uint8_t sk2[2][BN * KP];
  __shared__ __attribute__((aligned(16))) uint8_t sv2[2][D * VP];

  // positions fit 32 bits (checked by the host, with the row offsets of S + BN rows)
  const int S = static_cast<int>(a.S);
  const int sqs = static_cast<int>(a.sqs), sks = static_cast<int>(a.sks),
            svs = static_cast<int>(a.svs);
  const int nqb = (S + BM - 1) / BM;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x);  // longest causal rows first
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int tid = threadIdx.x, lane = tid & 63, hh = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q0 = qb * BM;
  const int qw0 = q0 + 32 * wave;  // this wavefront's first query
  const int qi = qw0 + l32;        // this lane's query

  // descriptors end at the head's last position: rows past S read zeros (their offsets,
  // up to S + BN rows, stay below 2^31)
  const __amdgpu_buffer_rsrc_t qbuf =
      make_buffer(a.q + b * a.sqb + h * a.sqh, (static_cast<int64_t>(S - 1) * sqs + D) * 2);
  const __amdgpu_buffer_rsrc_t kbuf =
      make_buffer(a.k + b * a.skb + h * a.skh, (static_cast<int64_t>(S - 1) * sks + D) * 2);
  const __amdgpu_buffer_rsrc_t vbuf =
      make_buffer(a.v + b * a.svb + h * a.svh, (static_cast<int64_t>(S - 1) * svs + D) * 2);

  // Q of this lane's query, features 16 s + 8 hh .. + 7: the second MFMA operand
  v8bf_a qf[D / 16];
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
    qf[s] = as_v8bf(__builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  qbuf, (qi * sqs + 16 * s + 8 * hh) * 2, 0, 0)));

  // staging. K: piece c = tid + 256 i is row c / (D / 8), features 8 (c % (D / 8)) .. + 7.
  // V: thread tid takes keys 4 (tid / DG) .. + 3, features 4 (tid % DG) .. + 3 (8-byte loads),
  // and writes them transposed as 4 rows of V^T, 4 keys (8 bytes) each.
  uint4 kr[PIECES];
  uint2 vr[VKEYS];
  const int vd0 = 4 * (tid % DG), vk0 = VKEYS * (tid / DG);
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < PIECES; ++i) {
      const int c = tid + 256 * i, row = c / (D / 8), col = 8 * (c % (D / 8));
      kr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                            kbuf, ((kb * BN + row) * sks + col) * 2, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < VKEYS; ++i)
      vr[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                            vbuf, ((kb * BN + vk0 + i) * svs + vd0) * 2, 0, 0));
  };
  auto lstore = [&](int buf) {
    uint8_t* sk = sk2[buf];
    uint8_t* sv = sv2[buf];
#pragma unroll
    for (int i = 0; i < PIECES; ++i) {
      const int c = tid + 256 * i, row = c / (D / 8), col = 8 * (c % (D / 8));
      *reinterpret_cast<uint4*>(sk + row * KP + col * 2) = kr[i];
    }
    // feature j of keys vk0 .. vk0 + 3: the low / high halves of word j / 2 of each key
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;  // high or low bf16 halves
      const uint32_t w0 = (j < 2) ? vr[0].x : vr[0].y, w1 = (j < 2) ? vr[1].x : vr[1].y;
      const uint32_t w2 = (j < 2) ? vr[2].x : vr[2].y, w3 = (j < 2) ? vr[3].x : vr[3].y;
      *reinterpret_cast<uint2*>(sv + (vd0 + j) * VP + vk0 * 2) =
          make_uint2(__builtin_amdgcn_perm(w1, w0, sel), __builtin_amdgcn_perm(w3, w2, sel));
    }
  };

  float m = -INFINITY, l = 0.0f;
  v16f_a o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) o[dt] = v16f_a{};

  const int last_key = (q0 + BM - 1 < S - 1) ? q0 + BM - 1 : S - 1;
  const int nkb = last_key / BN + 1;
  gload(0);
  lstore(0);
  if (nkb > 1) gload(1);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const uint8_t* sk = sk2[kb & 1];
    const uint8_t* sv = sv2[kb & 1];
    const int k0 = kb * BN;
    if (k0 <= qw0 + 31) {  // else the block lies above this wavefront's diagonal

      // S^T for two 32-key tiles: lane holds keys k0 + 32 kt + 8 (e / 4) + 4 hh + e % 4
      v16f_a st[KT];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        st[kt] = v16f_a{};
#pragma unroll
        for (int s = 0; s < D / 16; ++s) {
          const v8bf_a kf = as_v8bf(*reinterpret_cast<const uint4*>(
              sk + (32 * kt + l32) * KP + (16 * s + 8 * hh) * 2));
          st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], st[kt], 0, 0, 0);
        }
      }
      const bool diag = k0 + BN - 1 > qw0;  // some key of the block lies past some query
      float mx = -INFINITY;
      if (diag) {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = k0 + 32 * kt + 8 * (e / 4) + 4 * hh + (e % 4);
            if (key > qi) st[kt][e] = -INFINITY;
          }
      }
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, st[kt][e]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      // the running max in base-2 units (scale * log2 e > 0 commutes with max)
      const float mnew = fmaxf(m, mx * a.scale_log2);
      const float mref = mnew == -INFINITY ? 0.0f : mnew;  // a row with no key yet
      const float alpha = __builtin_amdgcn_exp2f(m - mref);
      float ps = 0.0f;
      uint4 pf[KT][2];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        float p[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kt][e], a.scale_log2, -mref));
          ps = ps + p[e];
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
          pf[kt][s2] = make_uint4(bf16x2_of(p[8 * s2], p[8 * s2 + 1]),
                                  bf16x2_of(p[8 * s2 + 2], p[8 * s2 + 3]),
                                  bf16x2_of(p[8 * s2 + 4], p[8 * s2 + 5]),
                                  bf16x2_of(p[8 * s2 + 6], p[8 * s2 + 7]));
      }
      ps = ps + __shfl_xor(ps, 32, kWave);
      l = l * alpha + ps;
      m = mnew;
      // rescale only when some query's running max grew (alpha == 1 exactly otherwise:
      // exp2(0) = 1), which after the first blocks is rare
      const bool rescale = __any(alpha != 1.0f);
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        if (rescale) {
#pragma unroll
          for (int e = 0; e < 16; ++e) o[dt][e] = o[dt][e] * alpha;
        }
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const uint8_t* row = sv + (32 * dt + l32) * VP + (32 * kt + 16 * s2 + 4 * hh) * 2;
            const uint2 lo = *reinterpret_cast<const uint2*>(row);
            const uint2 hi = *reinterpret_cast<const uint2*>(row + 16);
            const v8bf_a vf = as_v8bf(make_uint4(lo.x, lo.y, hi.x, hi.y));
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, as_v8bf(pf[kt][s2]), o[dt], 0, 0,
                                                            0);
          }
      }
    }
    // block kb + 1 (in registers since the last iteration) goes to the other buffer, whose
    // reads all ended before the last barrier; block kb + 2's loads go out
    if (kb + 1 < nkb) {
      lstore((kb + 1) & 1);
      if (kb + 2 < nkb) gload(kb + 2);
    }
    __syncthreads();
  }

  // o[dt][e] = O[qi][32 dt + 8 (e / 4) + 4 hh + e % 4] * l
  if (qi < S) {
    const float inv = 1.0f / l;
    uint16_t* orow = a.o + b * a.sob + h * a.soh + static_cast<int64_t>(qi) * a.sos;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d0 = 32 * dt + 8 * r + 4 * hh;
        *reinterpret_cast<uint2*>(orow + d0) =
            make_uint2(bf16x2_of(o[dt][4 * r] * inv, o[dt][4 * r + 1] * inv),
                       bf16x2_of(o[dt][4 * r + 2] * inv, o[dt][4 * r + 3] * inv));
      }
    if (hh == 0) a.lse[bh * S + qi] = (m + __log2f(l)) * 0.69314718055994531f;
  }
}

}  // namespace rk

using namespace rk;

extern "C" int rk_attention_forward(const uint16_t* q, int64_t sqb, int64_t sqh, int64_t sqs,
                                    const uint16_t* k, int64_t skb, int64_t skh, int64_t sks,
                                    const uint16_t* v, int64_t svb, int64_t svh, int64_t svs,
                                    int64_t B, int64_t H, int64_t S, int64_t D, float scale,
                                    uint16_t* o, int64_t sob, int64_t soh, int64_t sos,
                                    float* lse, void* stream) {
  clear_error();
  if (B < 0 || H < 0 || S < 0) return fail(RK_ERR_ARG, "negative size");
  if (D != 64 && D != 128) return fail(RK_ERR_UNSUPPORTED, "head size %lld (64 or 128 only)",
                                       static_cast<long long>(D));
  if (B == 0 || H == 0 || S == 0) return RK_OK;
  if (!q || !k || !v || !o || !lse) return fail(RK_ERR_ARG, "null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || (reinterpret_cast<uintptr_t>(o) & 7))
    return fail(RK_ERR_UNSUPPORTED, "q, k, v need 16-byte and o 8-byte alignment");
  const int64_t strides[] = {sqb, sqh, sqs, skb, skh, sks, svb, svh, svs, sob, soh, sos};
  for (int64_t st : strides)
    if (st < 0 || st % 8 != 0)
      return fail(RK_ERR_UNSUPPORTED, "strides must be non-negative multiples of 8 elements");
  // buffer offsets are 32-bit: the rows of one (batch, head) up to S + 128 (the last key
  // block's padding) must lie below 2^31 bytes
  const int64_t rows = S + 128;
  if ((rows * sqs + D) * 2 >= (int64_t{1} << 31) || (rows * sks + D) * 2 >= (int64_t{1} << 31) ||
      (rows * svs + D) * 2 >= (int64_t{1} << 31))
    return fail(RK_ERR_UNSUPPORTED, "sequence extent exceeds 2^31 bytes per head");
  if (B * H > 0x7fffffff || (S + kAttnBM - 1) / kAttnBM > 0x7fffffff)
    return fail(RK_ERR_ARG, "grid too large");
  AttnArgs a{q, k, v, sqb, sqh, sqs, skb, skh, sks, svb, svh, svs, o, sob, soh, sos, lse,
             B, H, S, scale * 1.4426950408889634f};
  const dim3 grid(static_cast<unsigned>((S + kAttnBM - 1) / kAttnBM),
                  static_cast<unsigned>(B * H));
  if (D == 64) attn_fwd_kernel<64, 64><<<grid, 256, 0, as_stream(stream)>>>(a);
  else attn_fwd_kernel<128, 32><<<grid, 256, 0, as_stream(stream)>>>(a);
  return launch_status("attention_forward");
}
