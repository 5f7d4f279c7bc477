// KV-cached decode kernels (gfx950): one token per sequence, M <= 16 rows, for the
// ratchet transformer's incremental generation (the reference recomputes the whole
// window per token instead, generate.py:183-201).
//
// A decode step is bounded by the fixed cost of each dependent launch (a few
// microseconds on MI355X: dispatch plus the cross-XCD cache release at kernel end)
// more than by HBM, so a transformer layer runs in six launches:
//
//   decode_gemv_kernel  (qkv)      RMSNorm+quant prologue, bf16 store
//   decode_attn_partial_kernel     split-position attention, appends k/v at `pos`
//   decode_attn_combine_kernel     merges the splits into the float32 [B, H*D] row
//   decode_gemv_kernel  (proj)     per-token quant prologue, residual-add epilogue
//   decode_gemv_kernel  (expand)   RMSNorm+quant prologue, tanh-GELU epilogue
//   decode_gemv_kernel  (contract) per-token quant prologue, residual-add epilogue
//
// decode_gemv_kernel: a block owns 16 (or 32) weight rows (n) and up to 16 token rows. It requests
// the activation rows first and then its packed code pieces (one 16-byte piece per
// lane per 64-wide k-block, every k-block of the wave's K range at once), so the
// prologue runs while the codes are still in flight. The prologue quantizes the M
// activation rows into LDS with the
// arithmetic of quant_rows_kernel lane for lane (one wavefront per row, the same
// per-lane accumulation order and butterfly, the same rounding), so q and s equal what
// the training kernels produce for those rows. v_mfma_i32_16x16x64_i8 takes the
// decoded codes as its first operand and the LDS rows as its second; the waves'
// int32 partial sums meet in LDS and the epilogue applies (acc * s_m) * row_scale_n,
// rounds to bf16 and then stores it (bf16 or widened f32), stores tanh-GELU of it
// (f32), or adds it to the f32 residual row (y += value: the torch `hidden + out`).
#include "rk_common.h"
#include "rk_rowquant.h"

namespace rk {

typedef int dec_v4i __attribute__((ext_vector_type(4)));
typedef unsigned int dec_u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 dec_bf16x2 __attribute__((ext_vector_type(2)));

enum { DEC_PRO_INT8 = 0, DEC_PRO_PLAIN = 1, DEC_PRO_RMSNORM = 2 };
enum { DEC_EPI_STORE = 0, DEC_EPI_GELU = 1, DEC_EPI_ADD = 2 };

constexpr int kDecMaxK = 6144;           // longest activation row (24 chunks of 256 f32)
constexpr int kDecMaxM = 16;
constexpr int kDecMaxSplits = 64;        // position splits per (sequence, head)

struct DecodeGemvArgs {
  const float* x;       // float rows (PLAIN / RMSNORM prologue)
  int64_t ldx;
  const int8_t* xq;     // int8 rows and their scales (INT8 prologue)
  int64_t ldxq;
  const float* xs;
  const float* w;       // RMSNorm weight
  float eps;
  const uint8_t* packed;
  int64_t ldp;
  uint32_t mc4;
  const float* rs;      // per-output-row code scale
  void* y;
  int64_t ldy;
  int M, N, K;
};

__device__ __forceinline__ uint32_t dec_pack_bf16x2(float lo, float hi) {
  const dec_bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// Loads of one f32 activation row (and the RMSNorm weight): V = 4 elements per lane per
// 256-element chunk, chunk c at c*256 + lane*4 as in quant_rows_kernel. The loads are
// unconditional (offsets past K re-read the row's last vector and are zeroed after the
// load), so the compiler can keep later loads in flight while it waits for these.
template <int NCH>
__device__ __forceinline__ void dec_load_row(const float* row, int K, int lane,
                                             float (&v)[NCH][4]) {
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e0 = c * kWave * 4 + lane * 4;
    const bool in = e0 < K;
    const float4 t = *reinterpret_cast<const float4*>(row + (in ? e0 : K - 4));
    v[c][0] = in ? t.x : 0.0f;
    v[c][1] = in ? t.y : 0.0f;
    v[c][2] = in ? t.z : 0.0f;
    v[c][3] = in ? t.w : 0.0f;
  }
}

// Chunks c0 .. c0 + NC - 1 of a register-resident row (zeros past K) -> int8 values in
// LDS at dst (the row's start): x / s rounded to nearest even, through the reciprocal
// fast path for the lane's four values, redone through round_quotient (which divides
// where needed) only when one lies within the margin of a rounding boundary.
template <int NC>
__device__ __forceinline__ void dec_store_q(const float (&xr)[NC][4], int c0, int lane, int K,
                                            float s, float r, int8_t* dst) {
  constexpr int V = 4, SPAN = kWave * V;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e0 = (c0 + c) * SPAN + lane * V;
    if (e0 < K) {
      bool exact = false;
      float t[V];
#pragma unroll
      for (int i = 0; i < V; ++i) t[i] = round_fast<false>(xr[c][i], r, 0.0f, exact);
      if (exact) {
#pragma unroll
        for (int i = 0; i < V; ++i) t[i] = round_quotient<false>(xr[c][i], s, r, 0.0f);
      }
      int qi[V];
#pragma unroll
      for (int i = 0; i < V; ++i) qi[i] = static_cast<int>(fminf(fmaxf(t[i], -127.0f), 127.0f));
      *reinterpret_cast<uint32_t*>(dst + e0) = pack_bytes4(qi[0], qi[1], qi[2], qi[3]);
    }
  }
}

// Register-resident row -> int8 row in LDS + its scale, with quant_rows_kernel's
// arithmetic for an f32 row: the per-lane sum of squares in chunk order, the xor
// butterfly, x * rsqrt-factor * w, the absmax scale and round_quotient. WREG: the
// RMSNorm weight is in wr (else it is read from the LDS copy wsh).
template <int PRO, int NCH, bool WREG = true>
__device__ __forceinline__ void dec_quant_row(const DecodeGemvArgs& a, int lane,
                                              float (&xr)[NCH][4], const float (&wr)[NCH][4],
                                              const float* wsh, int8_t* dst, float* s_out) {
  constexpr int V = 4, SPAN = kWave * V;
  const int K = a.K;
  float row_factor = 1.0f;
  if constexpr (PRO == DEC_PRO_RMSNORM) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < V; ++i) acc = acc + xr[c][i] * xr[c][i];
    acc = wave_sum_butterfly(acc);
    row_factor = 1.0f / sqrtf(acc / static_cast<float>(K) + a.eps);
  }
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if constexpr (PRO == DEC_PRO_RMSNORM) {
      float wv[V];
      if constexpr (WREG) {
#pragma unroll
        for (int i = 0; i < V; ++i) wv[i] = wr[c][i];
      } else {
        const int e0 = c * SPAN + lane * V;
        const float4 t = *reinterpret_cast<const float4*>(wsh + (e0 < K ? e0 : K - V));
        wv[0] = t.x;
        wv[1] = t.y;
        wv[2] = t.z;
        wv[3] = t.w;
      }
#pragma unroll
      for (int i = 0; i < V; ++i) xr[c][i] = xr[c][i] * row_factor * wv[i];
    }
#pragma unroll
    for (int i = 0; i < V; ++i) amax = fmaxf(amax, fabsf(xr[c][i]));  // zeros past K
  }
  amax = wave_max(amax);
  const float s = fmaxf(amax / 127.0f, 1.17549435e-38f);
  const float r = 1.0f / s;
  if (lane == 0) *s_out = s;
  dec_store_q<NCH>(xr, 0, lane, K, s, r, dst);
}

// MM: capacity in token rows; WV: wavefronts (K is split across them, and the prologue
// rows: wavefront w quantizes rows w, w + WV, ...); KBW: k-blocks a wavefront holds in
// registers (>= ceil(K / 64 / WV)); NCH: 256-element chunks of a register-resident row
// (>= ceil(K / 256)). Both are checked on the host. NT: 16-row output tiles per workgroup,
// all behind one prologue (the next tile's codes are requested before the current tile's
// MFMAs). Token rows: blockIdx.y selects rows blockIdx.y * MM onward, so that more token
// rows than MM, or a grid of twice the workgroups with half the prologue rows each, run
// as several row groups over the same codes. RS (plain prologue only): wavefronts per
// prologue row, each holding NCH / RS of its chunks; the slices' absmax values meet in LDS
// (a max, so the scale is the one a whole-row wavefront computes) and each wavefront
// quantizes its own slice.
//
// Load order: the activation rows (and RMSNorm weight) are requested first, then the
// packed codes, so the prologue waits only for the small activation loads while the
// code loads stay in flight (loads return in order). With two prologue rows per
// wavefront both are preloaded when they fit the register budget (NCH <= 8).
// (16-row variants with 512 threads and short K: 4 waves per SIMD, two workgroups per
// CU; with 1024 threads: 4 waves per SIMD, one workgroup)
template <int PRO, int EPI, int YDT, int MM, int WV, int KBW, int NCH, int NT = 1, int RS = 1>
__global__ __launch_bounds__(64 * WV, (MM >= 8 && (NCH <= 8 || WV == 16)) ? 4 : 1)
void decode_gemv_kernel(DecodeGemvArgs a) {
  constexpr int NB = 16, KB = 64;
  static_assert(RS == 1 || (PRO != DEC_PRO_INT8 && MM * RS == WV && NCH % RS == 0),
                "row slices: float prologue rows, one slice per wavefront");
  constexpr bool kSlicedNorm = RS > 1 && PRO == DEC_PRO_RMSNORM;
  constexpr int NCHL = NCH / RS;  // row chunks a wavefront holds
  if (blockIdx.y > 0) {  // this workgroup's token rows (uniform)
    const int mb = static_cast<int>(blockIdx.y) * MM;
    if constexpr (PRO == DEC_PRO_INT8) {
      a.xq += mb * a.ldxq;
      a.xs += mb;
    } else {
      a.x += mb * a.ldx;
    }
    a.y = static_cast<char*>(a.y) + mb * a.ldy * (YDT == RK_BF16 ? 2 : 4);
    a.M -= mb;
  }
  if (a.M > MM) a.M = MM;
  constexpr int RPW = (MM + WV - 1) / WV;                 // prologue rows per wavefront
  constexpr bool PRE = RPW == 1 || NCH <= 8;              // all prologue rows preloaded
  // RMSNorm weight: preloaded per wavefront with one prologue row; with two it is
  // staged once in LDS (one float4 per thread, requested ahead of the codes), which
  // keeps two-row wavefronts under 128 VGPRs
  constexpr bool WPRE = RPW == 1;
  constexpr bool WLDS = PRO == DEC_PRO_RMSNORM && !WPRE;
  constexpr int XR = PRE ? RPW : 1;
  constexpr int KP = NCH * 256 + 16;                      // LDS pitch (16-byte skew)
  constexpr int IPT = (MM * (KP / 16) + 64 * WV - 1) / (64 * WV);  // int8 pieces
  constexpr int WPT = (NCH * 64 + 64 * WV - 1) / (64 * WV);        // weight float4s
  __shared__ __align__(16) int8_t qa[MM * KP];
  __shared__ __align__(16) float wsh[WLDS ? NCH * 256 : 4];
  __shared__ float sc[MM];
  __shared__ float part[RS > 1 ? MM : 1][RS];  // slice absmax values
  __shared__ float rfac[kSlicedNorm ? MM : 1];  // RMSNorm factors of sliced rows
  __shared__ dec_v4i red[WV][kWave];
  // wave index made scalar: the code loads' k offset is then an SGPR (a value the
  // compiler takes as divergent would turn each buffer load into a waterfall loop)
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g4 = lane >> 4;
  const int M = a.M, K = a.K;
  int64_t n0 = static_cast<int64_t>(blockIdx.x) * NT * NB;

  // 0. epilogue operands (wavefront 0 writes the outputs): row scales and, for the
  //    residual add, the rows being added to; requested first, needed last
  const int em = r16 < M ? r16 : M - 1;
  float4 rs4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), old = rs4;
  auto load_epilogue = [&](int64_t tile_n0) {
    if (wave == 0) {
      const int64_t en = tile_n0 + 4 * g4;
      rs4 = *reinterpret_cast<const float4*>(a.rs + en);
      if constexpr (EPI == DEC_EPI_ADD)
        old = *reinterpret_cast<const float4*>(static_cast<const float*>(a.y) + em * a.ldy + en);
    }
  };
  load_epilogue(n0);

  // 1. activation rows of the prologue (the first row only when they do not all fit)
  float xr[PRO == DEC_PRO_INT8 ? 1 : XR][NCHL][4];
  float wr[NCH][4];  // RMSNorm weight (unread by the other prologues)
  dec_u32x4 xq_r[PRO == DEC_PRO_INT8 ? IPT : 1];
  int xq_lds[PRO == DEC_PRO_INT8 ? IPT : 1];
  const int pieces = K / 16;
  const int srow = wave / RS, slice = wave - srow * RS;  // row slice (RS > 1)
  // sliced RMSNorm rows: the first slice's wavefront also holds the whole row, whose sum of
  // squares it takes in the unsliced order; every slice holds its piece of the norm weight
  float xf[kSlicedNorm ? NCH : 1][4];
  float wsl[kSlicedNorm ? NCHL : 1][4];
  if constexpr (RS > 1) {
    const float* row = a.x + (srow < M ? srow : M - 1) * a.ldx;
    if constexpr (kSlicedNorm) {
      if (slice == 0) dec_load_row<NCH>(row, K, lane, xf);
    }
#pragma unroll
    for (int c = 0; c < NCHL; ++c) {
      const int e0 = (slice * NCHL + c) * kWave * 4 + lane * 4;
      const bool in = e0 < K;
      const float4 t = *reinterpret_cast<const float4*>(row + (in ? e0 : K - 4));
      xr[0][c][0] = in ? t.x : 0.0f;
      xr[0][c][1] = in ? t.y : 0.0f;
      xr[0][c][2] = in ? t.z : 0.0f;
      xr[0][c][3] = in ? t.w : 0.0f;
      if constexpr (kSlicedNorm) {
        const float4 w = *reinterpret_cast<const float4*>(a.w + (in ? e0 : K - 4));
        wsl[c][0] = in ? w.x : 0.0f;
        wsl[c][1] = in ? w.y : 0.0f;
        wsl[c][2] = in ? w.z : 0.0f;
        wsl[c][3] = in ? w.w : 0.0f;
      }
    }
  } else if constexpr (PRO == DEC_PRO_INT8) {
    // pieces past the M rows re-load piece 0 of row 0 (and store it back unchanged)
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      const int idx = tid + i * 64 * WV;
      const int id = idx < M * pieces ? idx : 0;
      const int m = id / pieces, c = id - m * pieces;
      xq_r[i] = *reinterpret_cast<const dec_u32x4*>(a.xq + m * a.ldxq + 16 * c);
      xq_lds[i] = m * KP + 16 * c;
    }
  } else if constexpr (PRE) {
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int m = wave + r * WV < M ? wave + r * WV : M - 1;
      dec_load_row<NCH>(a.x + m * a.ldx, K, lane, xr[r]);
    }
    if constexpr (PRO == DEC_PRO_RMSNORM && WPRE) dec_load_row<NCH>(a.w, K, lane, wr);
  }
  float4 wpiece[WLDS ? WPT : 1];
  if constexpr (WLDS) {
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int e = 4 * (tid + i * 64 * WV);
      wpiece[i] = *reinterpret_cast<const float4*>(a.w + (e < K ? e : K - 4));
    }
  }

  // keep the activation loads ahead of the code loads in the instruction stream
  __builtin_amdgcn_sched_barrier(0);

  // 2. this wavefront's packed code pieces of a 16-row tile, every k-block of its range at
  //    once (positions past the range re-load its last k-block; their MFMAs are skipped)
  const int b_voff = r16 * static_cast<int>(a.ldp) + 16 * g4;
  const int nkb = K / KB;
  const int per = (nkb + WV - 1) / WV;
  const int kb_begin = wave * per;
  const int kb_cnt = nkb - kb_begin < per ? (nkb - kb_begin > 0 ? nkb - kb_begin : 0) : per;
  const int kb_last = kb_cnt > 0 ? kb_begin + kb_cnt - 1 : 0;
  auto load_codes = [&](int64_t tile_n0, dec_u32x4 (&bw)[KBW]) {
    const __amdgpu_buffer_rsrc_t b_rsrc =
        make_buffer(a.packed + tile_n0 * a.ldp, (NB - 1) * a.ldp + K);
#pragma unroll
    for (int j = 0; j < KBW; ++j) {
      const int kb = kb_begin + j < kb_last ? kb_begin + j : kb_last;
      bw[j] = __builtin_bit_cast(
          dec_u32x4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, b_voff, kb * KB, 0));
    }
  };
  dec_u32x4 bw[KBW], bn[KBW];
  load_codes(n0, bw);

  // 3. prologue: int8 rows (or quantized activation rows) and their scales into LDS
  if constexpr (RS > 1) {
    if constexpr (kSlicedNorm) {
      // dec_quant_row's factor: the per-lane sum of squares in chunk order over the whole
      // row, the xor butterfly, 1 / sqrt(mean + eps); then (x * factor) * w per slice
      if (slice == 0) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc = acc + xf[c][i] * xf[c][i];
        acc = wave_sum_butterfly(acc);
        if (lane == 0) rfac[srow] = 1.0f / sqrtf(acc / static_cast<float>(K) + a.eps);
      }
      __syncthreads();
      const float rf = rfac[srow];
#pragma unroll
      for (int c = 0; c < NCHL; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) xr[0][c][i] = xr[0][c][i] * rf * wsl[c][i];
    }
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NCHL; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(xr[0][c][i]));  // zeros past K
    amax = wave_max(amax);
    if (lane == 0) part[srow][slice] = amax;
    __syncthreads();
    amax = part[srow][0];
#pragma unroll
    for (int j = 1; j < RS; ++j) amax = fmaxf(amax, part[srow][j]);
    const float s = fmaxf(amax / 127.0f, 1.17549435e-38f);
    const float r = 1.0f / s;
    if (srow < M) {
      if (slice == 0 && lane == 0) sc[srow] = s;
      dec_store_q<NCHL>(xr[0], slice * NCHL, lane, K, s, r, qa + srow * KP);
    }
  } else if constexpr (PRO == DEC_PRO_INT8) {
#pragma unroll
    for (int i = 0; i < IPT; ++i) *reinterpret_cast<dec_u32x4*>(qa + xq_lds[i]) = xq_r[i];
    if (tid < M) sc[tid] = a.xs[tid];
  } else {
    if constexpr (WLDS) {
#pragma unroll
      for (int i = 0; i < WPT; ++i) {
        const int e = 4 * (tid + i * 64 * WV);
        if (e < K) *reinterpret_cast<float4*>(wsh + e) = wpiece[i];
      }
      __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int m = wave + r * WV;
      if constexpr (PRE) {
        if (m < M)
          dec_quant_row<PRO, NCH, WPRE>(a, lane, xr[r], wr, wsh, qa + m * KP, sc + m);
      } else {
        if (m < M) {
          dec_load_row<NCH>(a.x + m * a.ldx, K, lane, xr[0]);
          dec_quant_row<PRO, NCH, false>(a, lane, xr[0], wr, wsh, qa + m * KP, sc + m);
        }
      }
    }
  }
  __syncthreads();

  // 4. per tile: MFMA over the wavefront's k-blocks (token rows past M read row MM-1: their
  //    results are never stored), the next tile's codes requested first; the wavefronts'
  //    sums meet in LDS and wavefront 0 writes the tile
  const int8_t* arow = qa + (r16 < MM ? r16 : MM - 1) * KP + 16 * g4;
  auto tile = [&](dec_u32x4 (&cur)[KBW], dec_u32x4 (&nxt)[KBW], int t) {
    if (t + 1 < NT) load_codes(n0 + NB, nxt);
    dec_v4i acc = dec_v4i{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < KBW; ++j) {
      if (j < kb_cnt) {
        dec_u32x4 v = cur[j];
        v.x = decode4(v.x, a.mc4);
        v.y = decode4(v.y, a.mc4);
        v.z = decode4(v.z, a.mc4);
        v.w = decode4(v.w, a.mc4);
        const dec_v4i av = *reinterpret_cast<const dec_v4i*>(arow + (kb_begin + j) * KB);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(dec_v4i, v), av, acc, 0,
                                                    0, 0);
      }
    }
    red[wave][lane] = acc;
    __syncthreads();
    const int m = r16;
    if (wave == 0 && m < M) {
      dec_v4i sum = red[0][lane];
#pragma unroll
      for (int w = 1; w < WV; ++w) {
        const dec_v4i q = red[w][lane];
        sum = dec_v4i{sum[0] + q[0], sum[1] + q[1], sum[2] + q[2], sum[3] + q[3]};
      }
      // 5. epilogue: lane holds out[m = r16][n0 + 4*g4 + 0..3]
      const int64_t n = n0 + 4 * g4;
      const float lsm = sc[m];
      const float v0 = static_cast<float>(sum[0]) * lsm * rs4.x;
      const float v1 = static_cast<float>(sum[1]) * lsm * rs4.y;
      const float v2 = static_cast<float>(sum[2]) * lsm * rs4.z;
      const float v3 = static_cast<float>(sum[3]) * lsm * rs4.w;
      const uint32_t lo = dec_pack_bf16x2(v0, v1), hi = dec_pack_bf16x2(v2, v3);
      if constexpr (EPI == DEC_EPI_STORE && YDT == RK_BF16) {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.y) + m * a.ldy + n) =
            make_uint2(lo, hi);
      } else {
        float f[4] = {__uint_as_float(lo << 16), __uint_as_float(lo & 0xffff0000u),
                      __uint_as_float(hi << 16), __uint_as_float(hi & 0xffff0000u)};
        float* yrow = static_cast<float*>(a.y) + m * a.ldy + n;
        if constexpr (EPI == DEC_EPI_GELU) {
#pragma unroll
          for (int r = 0; r < 4; ++r) f[r] = gelu_tanh(f[r]);
        } else if constexpr (EPI == DEC_EPI_ADD) {
          f[0] = old.x + f[0];
          f[1] = old.y + f[1];
          f[2] = old.z + f[2];
          f[3] = old.w + f[3];
        }
        *reinterpret_cast<float4*>(yrow) = make_float4(f[0], f[1], f[2], f[3]);
      }
    }
    n0 += NB;
    if (t + 1 < NT) {
      load_epilogue(n0);
      __syncthreads();  // every wavefront read red before the next tile overwrites it
    }
  };
#pragma unroll
  for (int t = 0; t < NT; t += 2) {
    tile(bw, bn, t);
    if (t + 1 < NT) tile(bn, bw, t + 1);
  }
}

template <int PRO, int EPI, int YDT>
static int launch_decode_gemv(const DecodeGemvArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(a.N / 16));
  // Register and LDS footprints sized to K: rows of up to 2048 keep 8 chunks, longer rows
  // (<= 6144) 24. Plain prologue rows (no norm weight, whose sum of squares fixes the
  // order of a row's reduction) are sliced over several wavefronts.
  constexpr bool kPlain = PRO == DEC_PRO_PLAIN;
  const bool small_k = a.K <= 2048;
  const dim3 grid8(static_cast<unsigned>(a.N / 16), static_cast<unsigned>((a.M + 7) / 8));
  if (a.M <= 1) {
    // one token row; long rows split K over 8 wavefronts (twice the code loads in flight
    // per CU: 14.7 -> 12.5 us for N 2048 x K 5632), short ones over 4 (8 were slower)
    // (float rows sliced over all the wavefronts: plain ones by absmax alone, RMSNorm ones
    // after the first wavefront's whole-row sum of squares)
    constexpr bool kSlice1 = PRO != DEC_PRO_INT8;
    if (small_k) {
      if constexpr (kSlice1)
        decode_gemv_kernel<PRO, EPI, YDT, 1, 4, 8, 8, 1, 4><<<grid, 256, 0, stream>>>(a);
      else
        decode_gemv_kernel<PRO, EPI, YDT, 1, 4, 8, 8><<<grid, 256, 0, stream>>>(a);
    } else {
      if constexpr (kSlice1)
        decode_gemv_kernel<PRO, EPI, YDT, 1, 8, 12, 24, 1, 8><<<grid, 512, 0, stream>>>(a);
      else
        decode_gemv_kernel<PRO, EPI, YDT, 1, 8, 12, 24><<<grid, 512, 0, stream>>>(a);
    }
  } else if (a.M <= 4) {
    if (small_k) decode_gemv_kernel<PRO, EPI, YDT, 4, 4, 8, 8><<<grid, 256, 0, stream>>>(a);
    else decode_gemv_kernel<PRO, EPI, YDT, 4, 4, 24, 24><<<grid, 256, 0, stream>>>(a);
  } else if (small_k && a.N >= 4096 && a.N % 32 == 0) {
    // wide layers: two 16-row tiles behind one prologue (the prologue's VALU work, repeated
    // by every workgroup, outweighs a second tile's code loads and MFMAs), token rows in
    // groups of 8
    const dim3 grid2(static_cast<unsigned>(a.N / 32), static_cast<unsigned>((a.M + 7) / 8));
    decode_gemv_kernel<PRO, EPI, YDT, 8, 8, 4, 8, 2><<<grid2, 512, 0, stream>>>(a);
  } else if (small_k) {
    // narrow layers (N / 16 workgroups would leave CUs idle): groups of 8 token rows, twice
    // the workgroups over the same codes
    if constexpr (kPlain)
      decode_gemv_kernel<PRO, EPI, YDT, 8, 16, 2, 8, 1, 2><<<grid8, 1024, 0, stream>>>(a);
    else
      decode_gemv_kernel<PRO, EPI, YDT, 8, 8, 4, 8><<<grid8, 512, 0, stream>>>(a);
  } else if constexpr (PRO == DEC_PRO_RMSNORM) {
    decode_gemv_kernel<PRO, EPI, YDT, 16, 8, 12, 24><<<grid, 512, 0, stream>>>(a);
  } else if constexpr (kPlain) {
    // long plain rows: groups of 8 token rows, two wavefronts per row
    decode_gemv_kernel<PRO, EPI, YDT, 8, 16, 6, 24, 1, 2><<<grid8, 1024, 0, stream>>>(a);
  } else {
    // long int8 rows: groups of 8 token rows
    decode_gemv_kernel<PRO, EPI, YDT, 8, 8, 12, 24><<<grid8, 512, 0, stream>>>(a);
  }
  return launch_status("decode_gemv");
}

// ---------------------------------------------------------------------------
// Attention of one query per (sequence, head) over the cache, positions 0..pos.
// ---------------------------------------------------------------------------
struct DecodeAttnArgs {
  const void* qkv;      // row b: q | k | v, each H*D (head h at h*D)
  int64_t ldqkv;
  void* kc;             // caches [B, H, L, D] (element strides sb, sh, sl; d contiguous)
  void* vc;
  int64_t sb, sh, sl;
  const int64_t* pos;
  int B, H, L, nsplit;
  float scale;
  float* work;          // [B, H, nsplit, D + 4]: max, sum, 2 pad, unnormalized output
                        // (records 16-byte aligned for the combine's vector loads)
  float* out;           // [B, H*D] attention rows (ldo)
  int64_t ldo;
};

// E consecutive elements (16-byte aligned for f32, 8 * E-byte aligned for bf16).
template <int DT, int E>
__device__ __forceinline__ void dec_load(const void* base, int64_t idx, float* out) {
  if constexpr (DT == RK_BF16 && E == 4) {
    const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + idx);
    out[0] = __uint_as_float(raw.x << 16);
    out[1] = __uint_as_float(raw.x & 0xffff0000u);
    out[2] = __uint_as_float(raw.y << 16);
    out[3] = __uint_as_float(raw.y & 0xffff0000u);
  } else {
    constexpr int P = Vec<DT>::N;
#pragma unroll
    for (int c = 0; c < E / P; ++c) load_vec16<DT>(base, idx + c * P, out + c * P);
  }
}

template <int DT, int E>
__device__ __forceinline__ void dec_store(void* base, int64_t idx, const float* v) {
  if constexpr (DT == RK_F32) {
#pragma unroll
    for (int c = 0; c < E; c += 4)
      *reinterpret_cast<float4*>(static_cast<float*>(base) + idx + c) =
          make_float4(v[c], v[c + 1], v[c + 2], v[c + 3]);
  } else {
#pragma unroll
    for (int c = 0; c < E; c += 4)
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + idx + c) =
          make_uint2(dec_pack_bf16x2(v[c], v[c + 1]), dec_pack_bf16x2(v[c + 2], v[c + 3]));
  }
}

// One position's E cache elements as loaded: float32 as is; bf16 as the raw 16-bit words
// (two per VGPR), widened where they are used, which halves the registers a loaded
// batch holds.
template <int CDT, int E>
struct KvPiece {
  float v[E];
  __device__ __forceinline__ void load(const void* base, int64_t idx) {
    dec_load<CDT, E>(base, idx, v);
  }
  __device__ __forceinline__ float operator[](int e) const { return v[e]; }
};

template <int E>
struct KvPiece<RK_BF16, E> {
  static_assert(E % 4 == 0, "whole 8-byte words");
  uint32_t w[E / 2];
  __device__ __forceinline__ void load(const void* base, int64_t idx) {
    const uint16_t* p = static_cast<const uint16_t*>(base) + idx;
    if constexpr (E % 8 == 0) {
#pragma unroll
      for (int c = 0; c < E / 8; ++c) {
        const uint4 r = *reinterpret_cast<const uint4*>(p + 8 * c);
        w[4 * c] = r.x;
        w[4 * c + 1] = r.y;
        w[4 * c + 2] = r.z;
        w[4 * c + 3] = r.w;
      }
    } else {
      const uint2 r = *reinterpret_cast<const uint2*>(p);
      w[0] = r.x;
      w[1] = r.y;
    }
  }
  __device__ __forceinline__ float operator[](int e) const {
    return __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
  }
  __device__ __forceinline__ void store(void* base, int64_t idx) const {
    uint16_t* p = static_cast<uint16_t*>(base) + idx;
    if constexpr (E % 8 == 0) {
#pragma unroll
      for (int c = 0; c < E / 8; ++c)
        *reinterpret_cast<uint4*>(p + 8 * c) =
            make_uint4(w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]);
    } else {
      *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    }
  }
};

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over each 16-lane row of the wavefront, every lane ending with its row's total, in
// DPP moves: lane i adds lane 15-i, then 7-i within its half-row, then its quad partners
// i^2 and i^1. Each step adds a symmetric pair (a + b on one lane, b + a on the other),
// so all 16 lanes hold the same bits.
__device__ __forceinline__ float row16_sum(float v) {
  v = v + dpp_mov<0x140>(v);  // row_mirror
  v = v + dpp_mov<0x141>(v);  // row_half_mirror
  v = v + dpp_mov<0x4e>(v);   // quad_perm [2, 3, 0, 1]
  v = v + dpp_mov<0xb1>(v);   // quad_perm [1, 0, 3, 2]
  return v;
}

typedef __bf16 dec_bf16x2v __attribute__((ext_vector_type(2)));

// a.bf16[0] * b.bf16[0] + a.bf16[1] * b.bf16[1] + c (v_dot2c_f32_bf16; the products of two
// bf16 values are exact in float32)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dec_bf16x2v, a),
                                         __builtin_bit_cast(dec_bf16x2v, b), c, false);
}

// Merge (m2, l2, o2) into (m, l, o): both are softmax states over disjoint position
// sets; an empty state has m = -inf, l = 0, o = 0.
template <int E>
__device__ __forceinline__ void dec_merge(float& m, float& l, float* o, float m2, float l2,
                                          const float* o2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  const float c1 = m == -INFINITY ? 0.0f : expf(m - mn);
  const float c2 = m2 == -INFINITY ? 0.0f : expf(m2 - mn);
  l = l * c1 + l2 * c2;
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = o[e] * c1 + o2[e] * c2;
  m = mn;
}

// grid (nsplit, H, B), 256 threads. 16 lanes share one position (E = D / 16 elements
// each); a wavefront takes 4 positions per pass, the block 16, unrolled by U.
template <int QDT, int CDT, int E, int U>
__global__ __launch_bounds__(256) void decode_attn_partial_kernel(DecodeAttnArgs a) {
  constexpr int D = 16 * E;
  __shared__ float sm[4], sl[4];
  __shared__ float so[4][D];
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int grp = lane >> 4, gl = lane & 15;
  const int64_t p = *a.pos;
  if (p < 0 || p >= a.L) return;  // the combine kernel flags the step
  const int n_valid = static_cast<int>(p) + 1;
  const int chunk = (((n_valid + a.nsplit - 1) / a.nsplit) + 15) & ~15;
  const int j0 = split * chunk;
  const int j1 = j0 + chunk < n_valid ? j0 + chunk : n_valid;

  const int64_t row = static_cast<int64_t>(b) * a.ldqkv + static_cast<int64_t>(h) * D + gl * E;
  const int64_t C = static_cast<int64_t>(a.H) * D;
  // bf16 projections over a bf16 cache: q and the keys stay packed and meet in bf16 dot
  // products (float32 accumulation), and a batch of positions shares one softmax rescale
  constexpr bool kDot2 = QDT == RK_BF16 && CDT == RK_BF16;
  float qv[E], kn[E], vn[E];
  KvPiece<RK_BF16, E> qp, knp, vnp;
  if constexpr (kDot2) {
    qp.load(a.qkv, row);
    knp.load(a.qkv, row + C);
    vnp.load(a.qkv, row + 2 * C);
  } else {
    dec_load<QDT, E>(a.qkv, row, qv);
    dec_load<QDT, E>(a.qkv, row + C, kn);
    dec_load<QDT, E>(a.qkv, row + 2 * C, vn);
  }
  const int64_t cbase = static_cast<int64_t>(b) * a.sb + static_cast<int64_t>(h) * a.sh + gl * E;

  float m = -INFINITY, l = 0.0f, o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = 0.0f;
  // U positions per group per batch; two register buffers alternate so the next
  // batch's loads are in flight while this one is reduced. Loads are unconditional
  // (positions past the split re-read position j0; position p takes the step's k, v
  // from registers), so waits count only the older batch.
  using Piece = KvPiece<CDT, E>;
  auto load = [&](int jb, Piece (&kk)[U], Piece (&vv)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = jb + 16 * u;
      const int64_t off = cbase + static_cast<int64_t>(j < j1 ? j : j0) * a.sl;
      kk[u].load(a.kc, off);
      vv[u].load(a.vc, off);
    }
  };
  auto reduce_dot2 = [&](int jb, const Piece (&kk)[U], const Piece (&vv)[U]) {
    if constexpr (kDot2) {
      // the batch's U scores (independent bf16 dot products, each summed over its 16
      // lanes), then one rescale; positions past the split score -inf (weight 0), and the
      // batch's first position is inside it, so the new maximum is finite
      float sc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool cur = jb + 16 * u == p;
        float d = 0.0f;
#pragma unroll
        for (int w = 0; w < E / 2; ++w) d = dot2_bf16(qp.w[w], cur ? knp.w[w] : kk[u].w[w], d);
        sc[u] = d;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) sc[u] = row16_sum(sc[u]);
      float mn = m;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        sc[u] = jb + 16 * u < j1 ? sc[u] * a.scale : -INFINITY;
        mn = fmaxf(mn, sc[u]);
      }
      const float c = expf(m - mn);  // 0 while m is -inf
      float pj[U], psum = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        pj[u] = expf(sc[u] - mn);
        psum = psum + pj[u];
      }
      l = l * c + psum;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float t = o[e] * c;
#pragma unroll
        for (int u = 0; u < U; ++u) t = t + pj[u] * (jb + 16 * u == p ? vnp[e] : vv[u][e]);
        o[e] = t;
      }
      m = mn;
    }
  };
  auto reduce = [&](int jb, const Piece (&kk)[U], const Piece (&vv)[U]) {
    if constexpr (kDot2) {
      reduce_dot2(jb, kk, vv);
      return;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = jb + 16 * u;
      if (j >= j1) break;
      const bool cur = j == p;
      float d = 0.0f;
#pragma unroll
      for (int e = 0; e < E; ++e) d = d + qv[e] * (cur ? kn[e] : kk[u][e]);
      d = d + __shfl_xor(d, 8, kWave);
      d = d + __shfl_xor(d, 4, kWave);
      d = d + __shfl_xor(d, 2, kWave);
      d = d + __shfl_xor(d, 1, kWave);
      const float s = d * a.scale;
      const float mn = fmaxf(m, s);
      const float c = expf(m - mn);
      const float pj = expf(s - mn);
      l = l * c + pj;
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = o[e] * c + pj * (cur ? vn[e] : vv[u][e]);
      m = mn;
    }
  };
  {
    Piece ka[U], va[U], kb[U], vb[U];
    int jb = j0 + wave * 4 + grp;
    load(jb, ka, va);
    while (jb < j1) {
      load(jb + 16 * U, kb, vb);
      reduce(jb, ka, va);
      jb += 16 * U;
      if (jb >= j1) break;
      load(jb + 16 * U, ka, va);
      reduce(jb, kb, vb);
      jb += 16 * U;
    }
  }
  // the wavefront's four position groups, then the block's four wavefronts
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    float o2[E];
#pragma unroll
    for (int e = 0; e < E; ++e) o2[e] = __shfl_xor(o[e], off, kWave);
    const float m2 = __shfl_xor(m, off, kWave), l2 = __shfl_xor(l, off, kWave);
    dec_merge<E>(m, l, o, m2, l2, o2);
  }
  if (grp == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) so[wave][gl * E + e] = o[e];
    if (gl == 0) {
      sm[wave] = m;
      sl[wave] = l;
    }
  }
  // the split holding p appends the step's k, v (its loop read them from registers, and
  // no other workgroup reads position p)
  if (j0 <= p && p < j1 && tid < 16) {
    if constexpr (kDot2) {
      knp.store(a.kc, cbase + p * a.sl);
      vnp.store(a.vc, cbase + p * a.sl);
    } else {
      dec_store<CDT, E>(a.kc, cbase + p * a.sl, kn);
      dec_store<CDT, E>(a.vc, cbase + p * a.sl, vn);
    }
  }
  __syncthreads();
  if (tid >= 16) return;
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    float o2[E];
#pragma unroll
    for (int e = 0; e < E; ++e) o2[e] = so[w][gl * E + e];
    dec_merge<E>(m, l, o, sm[w], sl[w], o2);
  }
  float* out = a.work + ((static_cast<int64_t>(b) * a.H + h) * a.nsplit + split) * (D + 4);
  if (gl == 0) {
    out[0] = m;
    out[1] = l;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) out[4 + gl * E + e] = o[e];
}

// grid (H, B), 256 threads: out[b, h*D + d] = sum_s w_s o_s[d] / sum_s w_s l_s with
// w_s = exp(m_s - max_s m_s). Threads (split group sg, 4-element piece) issue their
// splits' loads together, then the groups are summed in fixed order.
template <int E>
__global__ __launch_bounds__(256) void decode_attn_combine_kernel(DecodeAttnArgs a) {
  constexpr int D = 16 * E, P = D / 4, G = 256 / P, SPT = kDecMaxSplits / G;
  __shared__ float ws[kDecMaxSplits];
  __shared__ float lsum;
  __shared__ float4 red[G][P];
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int S = a.nsplit;
  const int64_t p = *a.pos;
  const float* base = a.work + (static_cast<int64_t>(b) * a.H + h) * S * (D + 4);
  const int piece = tid % P, sg = tid / P;
  float4 ov[SPT];
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const int sp = sg + i * G;
    ov[i] = *reinterpret_cast<const float4*>(base + (sp < S ? sp : 0) * (D + 4) + 4 + 4 * piece);
  }
  if (tid < kWave) {
    const float ms = tid < S ? base[tid * (D + 4)] : -INFINITY;
    const float ls = tid < S ? base[tid * (D + 4) + 1] : 0.0f;
    const float mx = wave_max(ms);
    const float w = ms == -INFINITY ? 0.0f : expf(ms - mx);
    const float l = wave_sum_butterfly(w * ls);
    ws[tid] = w;
    if (tid == 0) lsum = l;
  }
  __syncthreads();
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const int sp = sg + i * G;
    if (sp < S) {
      const float w = ws[sp];
      acc.x = acc.x + ov[i].x * w;
      acc.y = acc.y + ov[i].y * w;
      acc.z = acc.z + ov[i].z * w;
      acc.w = acc.w + ov[i].w * w;
    }
  }
  red[sg][piece] = acc;
  __syncthreads();
  if (tid >= P) return;
  float4 t = red[0][tid];
#pragma unroll
  for (int g = 1; g < G; ++g) {
    const float4 u = red[g][tid];
    t.x = t.x + u.x;
    t.y = t.y + u.y;
    t.z = t.z + u.z;
    t.w = t.w + u.w;
  }
  const bool ok = p >= 0 && p < a.L;
  const float l = ok ? lsum : __uint_as_float(0x7fc00000u);
  *reinterpret_cast<float4*>(a.out + static_cast<int64_t>(b) * a.ldo + h * D + 4 * tid) =
      make_float4(t.x / l, t.y / l, t.z / l, t.w / l);
}

template <int QDT, int CDT, int E>
static int launch_decode_attention(const DecodeAttnArgs& a, hipStream_t stream) {
  // splits of up to 32 positions (few sequence-head pairs) take batches of 2 positions per
  // lane group, one batch per block; longer splits 4 (measured on the 1B model: batch 1
  // 0.886 -> 0.878 ms per step with 2, batch 16 1.630 -> 1.647 with 2 and 1.638 with 8)
  const dim3 grid(a.nsplit, a.H, a.B);
  if (a.L <= 32 * a.nsplit)
    decode_attn_partial_kernel<QDT, CDT, E, 2><<<grid, 256, 0, stream>>>(a);
  else
    decode_attn_partial_kernel<QDT, CDT, E, 4><<<grid, 256, 0, stream>>>(a);
  if (int st = launch_status("decode_attention")) return st;
  decode_attn_combine_kernel<E><<<dim3(a.H, a.B), 256, 0, stream>>>(a);
  return launch_status("decode_attention");
}

template <int QDT, int CDT>
static int dispatch_head(const DecodeAttnArgs& a, int D, hipStream_t stream) {
  if (D == 64) return launch_decode_attention<QDT, CDT, 4>(a, stream);
  if (D == 128) return launch_decode_attention<QDT, CDT, 8>(a, stream);
  return launch_decode_attention<QDT, CDT, 16>(a, stream);
}

// grid B: hidden[b] = table[token_b] + pos_table[pos] (a NaN row for an id or position
// out of range, which is never read).
__global__ __launch_bounds__(256) void decode_embed_kernel(const int64_t* tokens,
                                                           const float* table, int64_t vocab,
                                                           int64_t C, const float* pos_table,
                                                           int64_t n_pos, const int64_t* pos,
                                                           float* hidden, int64_t ldh) {
  const int b = blockIdx.x;
  const int64_t t = tokens[b], p = *pos;
  const bool ok = t >= 0 && t < vocab && p >= 0 && p < n_pos;
  float* out = hidden + b * ldh;
  for (int64_t c = threadIdx.x; c < C; c += blockDim.x)
    out[c] = ok ? table[t * C + c] + pos_table[p * C + c] : __uint_as_float(0x7fc00000u);
}

// (v, i) ranks above (best, bi): the larger value, a NaN above every number, and among
// equal values (or NaNs) the smaller index, which makes the pick torch.argmax's.
__device__ __forceinline__ bool greedy_better(float v, int i, float best, int bi) {
  const bool vn = v != v, bn = best != best;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > best || (v == best && i < bi);
}

// grid B, 1024 threads: tokens[b * ldt] = the argmax of logits row b; block 0 then adds
// one to *pos (no kernel of the step reads pos after this one). Each thread issues all its
// loads of a pass before comparing (VEC: float4 pieces of 16-byte aligned rows).
template <bool VEC>
__global__ __launch_bounds__(1024) void decode_greedy_kernel(const float* logits, int64_t ldl,
                                                             int V, int64_t* tokens,
                                                             int64_t ldt, int64_t* pos) {
  constexpr int NT = 1024, UN = 4;
  __shared__ float sv[NT / kWave];
  __shared__ int si[NT / kWave];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const float* row = logits + b * ldl;
  float best = -INFINITY;
  int bi = V;  // no index yet: any value, -inf included, ranks above it
  auto take = [&](float v, int i) {
    if (greedy_better(v, i, best, bi)) {
      best = v;
      bi = i;
    }
  };
  if constexpr (VEC) {
    for (int base = 4 * tid; base < V; base += 4 * NT * UN) {
      float4 t[UN];
#pragma unroll
      for (int u = 0; u < UN; ++u) {
        const int i = base + 4 * NT * u;
        t[u] = i < V ? *reinterpret_cast<const float4*>(row + i)
                     : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      }
#pragma unroll
      for (int u = 0; u < UN; ++u) {
        const int i = base + 4 * NT * u;
        if (i < V) {
          take(t[u].x, i);
          take(t[u].y, i + 1);
          take(t[u].z, i + 2);
          take(t[u].w, i + 3);
        }
      }
    }
  } else {
    for (int base = tid; base < V; base += NT * UN) {
      float t[UN];
#pragma unroll
      for (int u = 0; u < UN; ++u) {
        const int i = base + NT * u;
        t[u] = i < V ? row[i] : -INFINITY;
      }
#pragma unroll
      for (int u = 0; u < UN; ++u)
        if (base + NT * u < V) take(t[u], base + NT * u);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) take(__shfl_xor(best, off, kWave), __shfl_xor(bi, off, kWave));
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int w = 1; w < NT / kWave; ++w) take(sv[w], si[w]);
    tokens[b * ldt] = bi;
    if (pos != nullptr && b == 0) *pos = *pos + 1;
  }
}

// Splits per (sequence, head), at least 16 positions per split, at most kDecMaxSplits.
// Workgroups in all: about 512 for few (sequence, head) pairs, where the combine's
// per-pair merge over the splits is on the critical path, and about 2048 for many, where
// the partial kernel streams the cache. Measured on the 1B model's 1024-position cache,
// 16 heads: batch 1 at 256/512/1024/2048 workgroups 976/968/995/994 us per step, batch
// 16 at 256/1024/2048/4096 workgroups 1.720/1.695/1.667/1.737 ms per step.
int64_t decode_splits(int64_t B, int64_t H, int64_t L) {
  const int64_t bh = B * H;
  const int64_t target = bh >= 128 ? 2048 : 512;
  int64_t s = (target + bh - 1) / bh;
  const int64_t by_len = L / 16 > 1 ? L / 16 : 1;
  if (s > by_len) s = by_len;
  if (s > kDecMaxSplits) s = kDecMaxSplits;
  return s < 1 ? 1 : s;
}

}  // namespace rk

using namespace rk;

extern "C" int rk_decode_gemv(const float* x, int64_t ldx, const int8_t* xq, int64_t ldxq,
                              const float* xs, int prologue, const float* norm_w, float eps,
                              const uint8_t* packed, int64_t ldp, int max_code,
                              const float* row_scale, void* y, int y_dtype, int64_t ldy,
                              int epilogue, int64_t M, int64_t N, int64_t K, void* stream) {
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(RK_ERR_ARG, "negative decode GEMV extent");
  if (M > kDecMaxM) return fail(RK_ERR_ARG, "decode GEMV takes at most %d rows", kDecMaxM);
  if (N % 16 != 0 || K % 64 != 0 || K > kDecMaxK)
    return fail(RK_ERR_UNSUPPORTED, "decode GEMV needs N %% 16 == 0, K %% 64 == 0, K <= %d",
                kDecMaxK);
  if (prologue < DEC_PRO_INT8 || prologue > DEC_PRO_RMSNORM)
    return fail(RK_ERR_ARG, "bad decode GEMV prologue %d", prologue);
  if (epilogue < DEC_EPI_STORE || epilogue > DEC_EPI_ADD)
    return fail(RK_ERR_ARG, "bad decode GEMV epilogue %d", epilogue);
  if (y_dtype != RK_F32 && y_dtype != RK_BF16) return fail(RK_ERR_ARG, "bad output dtype");
  if (epilogue != DEC_EPI_STORE && y_dtype != RK_F32)
    return fail(RK_ERR_ARG, "GELU and residual-add epilogues write float32");
  if (max_code < 1 || max_code > 7) return fail(RK_ERR_ARG, "max_code must be in 1..7");
  if (M == 0 || N == 0) return RK_OK;
  if (K == 0) return fail(RK_ERR_ARG, "decode GEMV needs K > 0");
  if (!packed || !row_scale || !y) return fail(RK_ERR_ARG, "null decode GEMV operand");
  if (ldp < K || ldy < N) return fail(RK_ERR_ARG, "leading dimension too small");
  if (ldp % 16 != 0 || !aligned16(packed) || !aligned16(row_scale) || !aligned16(y) ||
      ldy % 4 != 0)
    return fail(RK_ERR_UNSUPPORTED, "decode GEMV needs 16-byte aligned rows");
  if (16 * ldp + K >= (int64_t{1} << 31)) return fail(RK_ERR_ARG, "code rows too long");
  if (prologue == DEC_PRO_INT8) {
    if (!xq || !xs) return fail(RK_ERR_ARG, "null int8 activation rows");
    if (ldxq < K || ldxq % 16 != 0 || !aligned16(xq))
      return fail(RK_ERR_UNSUPPORTED, "int8 rows must be 16-byte aligned, ldxq >= K");
  } else {
    if (!x) return fail(RK_ERR_ARG, "null activation rows");
    if (ldx < K || ldx % 4 != 0 || !aligned16(x))
      return fail(RK_ERR_UNSUPPORTED, "activation rows must be 16-byte aligned, ldx >= K");
    if (prologue == DEC_PRO_RMSNORM && (!norm_w || !aligned16(norm_w)))
      return fail(RK_ERR_ARG, "RMSNorm prologue needs a 16-byte aligned weight");
    // every workgroup reads all activation rows while others write their output columns
    const char* xb = reinterpret_cast<const char*>(x);
    const char* yb = static_cast<const char*>(y);
    const int64_t ys = dtype_size(y_dtype);
    if (xb < yb + ((M - 1) * ldy + N) * ys && yb < xb + ((M - 1) * ldx + K) * 4)
      return fail(RK_ERR_ARG, "decode GEMV output must not overlap its activation rows");
  }
  DecodeGemvArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.xq = xq;
  a.ldxq = ldxq;
  a.xs = xs;
  a.w = norm_w;
  a.eps = eps;
  a.packed = packed;
  a.ldp = ldp;
  a.mc4 = static_cast<uint32_t>(max_code) * 0x01010101u;
  a.rs = row_scale;
  a.y = y;
  a.ldy = ldy;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  if (N / 16 > 0x7fffffff) return fail(RK_ERR_ARG, "decode GEMV grid too large");
  hipStream_t s = as_stream(stream);
#define RK_DEC_EPI(PRO)                                                            \
  switch (epilogue) {                                                              \
    case DEC_EPI_STORE:                                                            \
      return y_dtype == RK_BF16 ? launch_decode_gemv<PRO, DEC_EPI_STORE, RK_BF16>(a, s) \
                                : launch_decode_gemv<PRO, DEC_EPI_STORE, RK_F32>(a, s); \
    case DEC_EPI_GELU:                                                             \
      return launch_decode_gemv<PRO, DEC_EPI_GELU, RK_F32>(a, s);                  \
    default:                                                                       \
      return launch_decode_gemv<PRO, DEC_EPI_ADD, RK_F32>(a, s);                   \
  }
  if (prologue == DEC_PRO_INT8) {
    RK_DEC_EPI(DEC_PRO_INT8)
  } else if (prologue == DEC_PRO_PLAIN) {
    RK_DEC_EPI(DEC_PRO_PLAIN)
  } else {
    RK_DEC_EPI(DEC_PRO_RMSNORM)
  }
#undef RK_DEC_EPI
}

extern "C" int64_t rk_decode_attention_splits(int64_t B, int64_t H, int64_t max_len) {
  return decode_splits(B, H, max_len);
}

extern "C" int rk_decode_attention(const void* qkv, int qkv_dtype, int64_t ld_qkv,
                                   void* k_cache, void* v_cache, int cache_dtype, int64_t sb,
                                   int64_t sh, int64_t sl, const int64_t* pos, int64_t B,
                                   int64_t H, int64_t D, int64_t max_len, float scale,
                                   float* work, int64_t work_floats, float* out, int64_t ldo,
                                   void* stream) {
  clear_error();
  if (B < 0 || H <= 0 || max_len <= 0) return fail(RK_ERR_ARG, "invalid decode attention shape");
  if (D != 64 && D != 128 && D != 256)
    return fail(RK_ERR_UNSUPPORTED, "decode attention supports head size 64, 128 or 256");
  if ((qkv_dtype != RK_F32 && qkv_dtype != RK_BF16) ||
      (cache_dtype != RK_F32 && cache_dtype != RK_BF16))
    return fail(RK_ERR_ARG, "unsupported decode attention dtype");
  if (B == 0) return RK_OK;
  if (B > 65535 || H > 65535) return fail(RK_ERR_ARG, "decode attention grid too large");
  if (!qkv || !k_cache || !v_cache || !pos || !work || !out)
    return fail(RK_ERR_ARG, "null decode attention operand");
  if (ld_qkv < 3 * H * D || ldo < H * D) return fail(RK_ERR_ARG, "leading dimension too small");
  if (sl < D || sh < max_len * sl || sb < H * sh)
    return fail(RK_ERR_ARG, "cache strides do not describe [B, H, max_len, D]");
  const int qes = dtype_size(qkv_dtype), ces = dtype_size(cache_dtype);
  if (!aligned16(qkv) || (ld_qkv * qes) % 16 != 0 || !aligned16(k_cache) || !aligned16(v_cache) ||
      (sl * ces) % 16 != 0 || (sh * ces) % 16 != 0 || (sb * ces) % 16 != 0 || !aligned16(out) ||
      ldo % 4 != 0 || !aligned16(work))
    return fail(RK_ERR_UNSUPPORTED, "decode attention needs 16-byte aligned rows");
  const int64_t nsplit = decode_splits(B, H, max_len);
  if (work_floats < B * H * nsplit * (D + 4))
    return fail(RK_ERR_ARG, "decode attention workspace too small (%lld floats, need %lld)",
                (long long)work_floats, (long long)(B * H * nsplit * (D + 4)));
  DecodeAttnArgs a{};
  a.qkv = qkv;
  a.ldqkv = ld_qkv;
  a.kc = k_cache;
  a.vc = v_cache;
  a.sb = sb;
  a.sh = sh;
  a.sl = sl;
  a.pos = pos;
  a.B = static_cast<int>(B);
  a.H = static_cast<int>(H);
  a.L = static_cast<int>(max_len);
  a.nsplit = static_cast<int>(nsplit);
  a.scale = scale;
  a.work = work;
  a.out = out;
  a.ldo = ldo;
  hipStream_t s = as_stream(stream);
  if (qkv_dtype == RK_BF16) {
    return cache_dtype == RK_BF16 ? dispatch_head<RK_BF16, RK_BF16>(a, static_cast<int>(D), s)
                                  : dispatch_head<RK_BF16, RK_F32>(a, static_cast<int>(D), s);
  }
  return cache_dtype == RK_BF16 ? dispatch_head<RK_F32, RK_BF16>(a, static_cast<int>(D), s)
                                : dispatch_head<RK_F32, RK_F32>(a, static_cast<int>(D), s);
}

extern "C" int rk_decode_embed(const int64_t* tokens, int64_t B, const float* table,
                               int64_t vocab, int64_t C, const float* pos_table, int64_t n_pos,
                               const int64_t* pos, float* hidden, int64_t ldh, void* stream) {
  clear_error();
  if (B < 0 || vocab <= 0 || C <= 0 || n_pos <= 0) return fail(RK_ERR_ARG, "invalid embed shape");
  if (B == 0) return RK_OK;
  if (B > 65535) return fail(RK_ERR_ARG, "decode embed grid too large");
  if (!tokens || !table || !pos_table || !pos || !hidden)
    return fail(RK_ERR_ARG, "null decode embed operand");
  if (ldh < C) return fail(RK_ERR_ARG, "leading dimension too small");
  decode_embed_kernel<<<dim3(static_cast<unsigned>(B)), 256, 0, as_stream(stream)>>>(
      tokens, table, vocab, C, pos_table, n_pos, pos, hidden, ldh);
  return launch_status("decode_embed");
}

extern "C" int rk_decode_greedy(const float* logits, int64_t ldl, int64_t B, int64_t V,
                                int64_t* tokens, int64_t ld_tokens, int64_t* pos, void* stream) {
  clear_error();
  if (B < 0 || V <= 0 || V > (int64_t{1} << 30)) return fail(RK_ERR_ARG, "invalid greedy shape");
  if (B == 0) return RK_OK;
  if (B > 65535) return fail(RK_ERR_ARG, "greedy grid too large");
  if (!logits || !tokens) return fail(RK_ERR_ARG, "null greedy operand");
  if (ldl < V || ld_tokens < 1) return fail(RK_ERR_ARG, "leading dimension too small");
  const dim3 grid(static_cast<unsigned>(B));
  if (aligned16(logits) && V % 4 == 0 && ldl % 4 == 0)
    decode_greedy_kernel<true><<<grid, 1024, 0, as_stream(stream)>>>(
        logits, ldl, static_cast<int>(V), tokens, ld_tokens, pos);
  else
    decode_greedy_kernel<false><<<grid, 1024, 0, as_stream(stream)>>>(
        logits, ldl, static_cast<int>(V), tokens, ld_tokens, pos);
  return launch_status("decode_greedy");
}
