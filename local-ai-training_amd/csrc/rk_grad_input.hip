// The int8 grad_input of the ratchet backward with the gradient's stochastic-rounding
// quantization done while the GEMM stages its first operand (ratchet.py:125-134):
//
//   y[m, k]  = g[m, k] * col_scale[k]              (bf16(g) first for RK_F32_AS_BF16)
//   s[m]     = max(max_k |y[m, k]| / 127, FLT_MIN), r = 1 / s
//   q[m, k]  = clamp(floor(y[m, k] / s[m] + u), -127, 127),
//              u = Philox4x32-10 word 0 at counter (row_offset + m) * K + k (int8_matmul.py:142-144)
//   gx[m, n] = bf16(float(sum_k q[m, k] * code[k, n]) * s[m])   (int8_matmul.py:289-343)
//
// with code[k, n] the packed ratchet state [K, N] decoded in place (the layer's weight
// [out, in]: the backward contracts over its output features). The results are those of
// rk_quantize_rows(stochastic) followed by rk_int8_gemm_packed_t, bit for bit, but the int8
// gradient never reaches HBM and the Philox work (VALU) overlaps the GEMM's MFMAs.
//
// One block owns 64 gradient rows and every output column (N <= 512), so each row is
// quantized exactly once: phase 1 streams the block's rows for their absmax (the row scale
// must be known before any value is rounded); phase 2 walks the contraction in 64-column
// steps: each thread rounds 8 values of one row into the LDS A tile, the block stages the
// packed [64][N] codes as the B tile, and 8 wavefronts (2 x 4, 32 x N/4 wave tiles) run
// v_mfma_i32_32x32x32_i8 on them (the fragment step and layouts of rk_mfma32.h). The
// epilogue scales by s[m], rounds to bf16 and stores through an LDS staging tile, as the
// int8 GEMM does.
#include "rk_common.h"
#include "rk_mfma32.h"
#include "rk_rowquant.h"

namespace rk {

struct SrGiArgs {
  const void* g[3];        // gradient column parts (g[0] alone when nparts == 1)
  int64_t ldg;             // row stride of every part, elements
  int64_t part_cols;       // columns per part, a multiple of 64
  const float* col_scale;  // [K] or null
  uint32_t key0, key1;
  const int64_t* seed_dev;  // when set, the Philox key is read here at kernel time
  int64_t row_offset;
  const uint8_t* packed;   // [K, N] packed codes
  int64_t ldp;
  uint32_t mc4;            // max_code in each byte
  int64_t M, K, N;
  float* scale;            // [M] row scales
  int8_t* q;               // optional [M, K] codes
  int64_t ldq;
  uint16_t* xb;            // optional bf16(g) [M, K]
  int64_t ldxb;
  void* out;               // [M, N] bf16, or float32 holding bf16 values (out_f32)
  int64_t ldo;
  int out_f32;
  int nparts;
  int round_bf16;          // float32 gradient taken as bf16(g)
};

constexpr int kGiBM = 64;         // gradient rows per block
constexpr int kGiThreads = 512;   // 8 wavefronts
constexpr int kGiMaxK = 4096;     // col_scale staged in LDS

// 8 gradient values (one 16-byte bf16 piece, or two float32 pieces) of one row
template <int DT>
struct GiSlot {
  u32x4 g[DT == RK_F32 ? 2 : 1];
};

template <int DT>
__device__ __forceinline__ void gi_unpack(const GiSlot<DT>& s, float* v) {
  if constexpr (DT == RK_BF16) {
    const uint32_t w[4] = {s.g[0].x, s.g[0].y, s.g[0].z, s.g[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v[4 * h] = __uint_as_float(s.g[h].x);
      v[4 * h + 1] = __uint_as_float(s.g[h].y);
      v[4 * h + 2] = __uint_as_float(s.g[h].z);
      v[4 * h + 3] = __uint_as_float(s.g[h].w);
    }
  }
}

// NJ: 32-column MFMA blocks per wave (N = 128 NJ). CS: a column scale is given.
template <int DT, int NJ, bool CS>
__global__ __launch_bounds__(kGiThreads) void grad_input_sr_kernel(SrGiArgs a) {
  constexpr int N = 128 * NJ, BTP = N + 32, ES = DT == RK_F32 ? 4 : 2;
  constexpr int GV = DT == RK_F32 ? 2 : 1;  // 16-byte gradient pieces per thread and step
  constexpr int BSEG = NJ;                  // 16-byte code pieces per thread and step
  constexpr int ATILE = kGiBM * 64, BTILE = 64 * BTP;
  constexpr int EPITCH = N * 2 + 8;
  static_assert(kGiBM * EPITCH <= 2 * (ATILE + BTILE), "epilogue staging fits the tiles");
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * (ATILE + BTILE)];
  __shared__ __attribute__((aligned(16))) float cs_l[CS ? kGiMaxK : 4];
  __shared__ float s_l[kGiBM], r_l[kGiBM];
  uint8_t* As = smem;
  uint8_t* Bs = smem + 2 * ATILE;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kGiBM;
  const int64_t rows = a.M - m0 < kGiBM ? a.M - m0 : kGiBM;
  const int nk = static_cast<int>(a.K / 64);

  // this thread's 8 gradient values per step: row ra, columns ca .. ca + 7 of the step
  const int ra = tid >> 3, ca = (tid & 7) * 8;
  // Descriptors over the block's rows of each part (rows past M read zeros).
  __amdgpu_buffer_rsrc_t g_rsrc[3];
#pragma unroll
  for (int p = 0; p < 3; ++p) {
    const void* base = a.g[p < a.nparts ? p : 0];
    g_rsrc[p] = make_buffer(static_cast<const char*>(base) + m0 * a.ldg * ES,
                            ((rows - 1) * a.ldg + a.part_cols) * ES);
  }
  const int g_voff = (ra * static_cast<int>(a.ldg) + ca) * ES;
  const int steps_per_part = static_cast<int>(a.part_cols / 64);
  auto load_g = [&](GiSlot<DT>& s, int kt) {
    const int p = kt / steps_per_part;  // uniform
    const __amdgpu_buffer_rsrc_t r = p == 0 ? g_rsrc[0] : (p == 1 ? g_rsrc[1] : g_rsrc[2]);
    const int soff = (kt - p * steps_per_part) * 64 * ES;
#pragma unroll
    for (int h = 0; h < GV; ++h)
      s.g[h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             r, g_voff + 16 * h, soff, 0));
  };

  if constexpr (CS) {
    for (int k = tid * 4; k < a.K; k += kGiThreads * 4)
      *reinterpret_cast<float4*>(cs_l + k) = *reinterpret_cast<const float4*>(a.col_scale + k);
    __syncthreads();
  }
  // y = transform(g) for the 8 values at step column c0 (k = 64 kt + c0)
  auto transform = [&](float* v, int k) {
    if constexpr (DT == RK_F32) {
      if (a.round_bf16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = round_bf16(v[i]);
      }
    }
    if constexpr (CS) {
      const float4 c0 = *reinterpret_cast<const float4*>(cs_l + k);
      const float4 c1 = *reinterpret_cast<const float4*>(cs_l + k + 4);
      v[0] = v[0] * c0.x;
      v[1] = v[1] * c0.y;
      v[2] = v[2] * c0.z;
      v[3] = v[3] * c0.w;
      v[4] = v[4] * c1.x;
      v[5] = v[5] * c1.y;
      v[6] = v[6] * c1.z;
      v[7] = v[7] * c1.w;
    }
  };

  // ---- phase 1: row absmax -> s, r (the 8 threads of a row are 8 consecutive lanes) ----
  {
    float amax = 0.0f;
    constexpr int U = 4;
    int kt = 0;
    for (; kt + U <= nk; kt += U) {
      GiSlot<DT> sl[U];
#pragma unroll
      for (int u = 0; u < U; ++u) load_g(sl[u], kt + u);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float v[8];
        gi_unpack<DT>(sl[u], v);
        transform(v, 64 * (kt + u) + ca);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
      }
    }
    for (; kt < nk; ++kt) {
      GiSlot<DT> sl;
      load_g(sl, kt);
      float v[8];
      gi_unpack<DT>(sl, v);
      transform(v, 64 * kt + ca);
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    if ((tid & 7) == 0) {
      const float s = fmaxf(amax / 127.0f, 1.17549435e-38f);
      s_l[ra] = s;
      r_l[ra] = 1.0f / s;
      if (ra < rows) a.scale[m0 + ra] = s;
    }
  }

  PhiloxKey key;
  {
    uint32_t k0 = a.key0, k1 = a.key1;
    if (a.seed_dev) {
      const uint64_t seed = static_cast<uint64_t>(*a.seed_dev);
      k0 = static_cast<uint32_t>(seed & 0xffffffffu);
      k1 = static_cast<uint32_t>(seed >> 32);
    }
    key = philox_key(k0, k1);
  }
  // counter = (row_offset + m) * K + k, wrapped to 32 bits (int8_matmul.py:143)
  const uint32_t ctr_row =
      static_cast<uint32_t>(a.row_offset + m0 + ra) * static_cast<uint32_t>(a.K);
  __syncthreads();  // s_l, r_l
  const float s_row = s_l[ra], r_row = r_l[ra];
  const int a_st = ra * 64 + 16 * ((ca >> 4) ^ swz32(ra)) + (ca & 8);
  int8_t* qrow = a.q && ra < rows ? a.q + (m0 + ra) * a.ldq : nullptr;
  uint16_t* xbrow = a.xb && ra < rows ? a.xb + (m0 + ra) * a.ldxb : nullptr;

  // ---- phase 2 ----
  // packed [K, N] rows of one step: 64 rows x N bytes, BSEG 16-byte pieces per thread
  const __amdgpu_buffer_rsrc_t b_rsrc = make_buffer(a.packed, (a.K - 1) * a.ldp + N);
  const int b_step = 64 * static_cast<int>(a.ldp);
  int b_voff[BSEG], b_st[BSEG];
#pragma unroll
  for (int j = 0; j < BSEG; ++j) {
    const int c = tid + kGiThreads * j, krow = c / (N / 16), nseg = c % (N / 16);
    b_voff[j] = krow * static_cast<int>(a.ldp) + 16 * nseg;
    b_st[j] = krow * BTP + 16 * nseg;
  }
  struct Slot {
    GiSlot<DT> g;
    u32x4 b[BSEG];
  };
  auto load = [&](Slot& s, int kt) {
    load_g(s.g, kt);
#pragma unroll
    for (int j = 0; j < BSEG; ++j)
      s.b[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             b_rsrc, b_voff[j], kt * b_step, 0));
  };
  auto store = [&](Slot& s, int buf, int kt) {
#pragma unroll
    for (int h = 0; h < GV; ++h) asm volatile("" : "+v"(s.g.g[h]));
#pragma unroll
    for (int j = 0; j < BSEG; ++j) asm volatile("" : "+v"(s.b[j]));
    uint8_t* bt = Bs + buf * BTILE;
#pragma unroll
    for (int j = 0; j < BSEG; ++j) {
      u32x4 v = s.b[j];
      v.x = decode4(v.x, a.mc4);
      v.y = decode4(v.y, a.mc4);
      v.z = decode4(v.z, a.mc4);
      v.w = decode4(v.w, a.mc4);
      *reinterpret_cast<u32x4*>(bt + b_st[j]) = v;
    }
    const int k = 64 * kt + ca;
    float v[8];
    gi_unpack<DT>(s.g, v);
    if (xbrow) {
      if constexpr (DT == RK_BF16) {
        *reinterpret_cast<u32x4*>(xbrow + k) = s.g.g[0];
      } else {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[i] = static_cast<uint32_t>(f32_to_bf16(v[2 * i])) |
                 (static_cast<uint32_t>(f32_to_bf16(v[2 * i + 1])) << 16);
        *reinterpret_cast<u32x4*>(xbrow + k) = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
    transform(v, k);
    float t[8], u[8];
    bool exact = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      u[i] = uniform_from_word(philox_word0(ctr_row + static_cast<uint32_t>(k + i), key));
      t[i] = round_fast<true>(v[i], r_row, u[i], exact);
    }
    if (exact) {
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] = round_quotient<true>(v[i], s_row, r_row, u[i]);
    }
    int qi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) qi[i] = static_cast<int>(fminf(fmaxf(t[i], -127.0f), 127.0f));
    const uint2 w8 = make_uint2(pack_bytes4(qi[0], qi[1], qi[2], qi[3]),
                                pack_bytes4(qi[4], qi[5], qi[6], qi[7]));
    *reinterpret_cast<uint2*>(As + buf * ATILE + a_st) = w8;
    if (qrow) *reinterpret_cast<uint2*>(qrow + k) = w8;
  };

  const int wm = wave & 1, wn = wave >> 1;  // 2 x 4 wavefronts
  const int arow0 = 32 * wm, brow0 = wn * (N / 4);
  v16i acc[1][NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[0][j] = v16i{};

  // register ring of 2 steps over an LDS ping-pong (the int8 GEMM's schedule); loads past
  // the last step are never consumed and stay in bounds (zeros past each descriptor)
  Slot ring[2];
  load(ring[0], 0);
  __builtin_amdgcn_sched_barrier(0);
  load(ring[1], nk > 1 ? 1 : 0);
  __builtin_amdgcn_sched_barrier(0);
  const int nk_pairs = nk & ~1;
  for (int kb = 0; kb < nk_pairs; kb += 2) {
#pragma unroll
    for (int slot = 0; slot < 2; ++slot) {
      store(ring[slot], slot, kb + slot);
      load(ring[slot], kb + slot + 2 < nk ? kb + slot + 2 : nk - 1);
      __syncthreads();
      mfma32_step<true, 1, NJ, BTP>(acc, As + slot * ATILE, Bs + slot * BTILE, arow0, brow0,
                                    lane);
    }
  }
  if (nk & 1) {
    store(ring[0], 0, nk - 1);
    __syncthreads();
    mfma32_step<true, 1, NJ, BTP>(acc, As, Bs, arow0, brow0, lane);
  }
  __syncthreads();  // every fragment read done: the tiles become the staging buffer

  // ---- epilogue: gx = bf16(float(acc) * s[m]) staged in LDS, stored 16 bytes a lane ----
  const int r32 = lane & 31, hh = lane >> 5;
  {
    const float ls = s_l[arow0 + r32];
    uint8_t* srow = smem + (arow0 + r32) * EPITCH;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float v0 = static_cast<float>(acc[0][j][4 * q]) * ls;
        const float v1 = static_cast<float>(acc[0][j][4 * q + 1]) * ls;
        const float v2 = static_cast<float>(acc[0][j][4 * q + 2]) * ls;
        const float v3 = static_cast<float>(acc[0][j][4 * q + 3]) * ls;
        *reinterpret_cast<uint2*>(srow + (brow0 + 32 * j + 8 * q + 4 * hh) * 2) =
            make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
      }
  }
  __syncthreads();
  const int oes = a.out_f32 ? 4 : 2;
  constexpr int CHUNKS = N / 8, RSTEP = kGiThreads / CHUNKS;
  const int ch = tid % CHUNKS;
  const __amdgpu_buffer_rsrc_t o_rsrc =
      make_buffer(static_cast<char*>(a.out) + m0 * a.ldo * oes, ((rows - 1) * a.ldo + N) * oes);
#pragma unroll
  for (int it = 0; it < kGiBM / RSTEP; ++it) {
    const int row = tid / CHUNKS + RSTEP * it;
    const uint8_t* src = smem + row * EPITCH + 16 * ch;
    const uint2 lo = *reinterpret_cast<const uint2*>(src);
    const uint2 hi = *reinterpret_cast<const uint2*>(src + 8);
    const int voff = (row * static_cast<int>(a.ldo) + 8 * ch) * oes;
    if (!a.out_f32) {
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(v4i, make_uint4(lo.x, lo.y, hi.x, hi.y)), o_rsrc, voff, 0, 0);
    } else {
      const uint4 w0 = make_uint4(lo.x << 16, lo.x & 0xffff0000u, lo.y << 16, lo.y & 0xffff0000u);
      const uint4 w1 = make_uint4(hi.x << 16, hi.x & 0xffff0000u, hi.y << 16, hi.y & 0xffff0000u);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, w0), o_rsrc, voff, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, w1), o_rsrc, voff + 16, 0, 0);
    }
  }
}

template <int DT, int NJ>
static void launch_gi_cs(const SrGiArgs& a, dim3 grid, hipStream_t st) {
  if (a.col_scale) grad_input_sr_kernel<DT, NJ, true><<<grid, kGiThreads, 0, st>>>(a);
  else grad_input_sr_kernel<DT, NJ, false><<<grid, kGiThreads, 0, st>>>(a);
}

template <int DT>
static void launch_gi(const SrGiArgs& a, dim3 grid, hipStream_t st) {
  if (a.N == 128) launch_gi_cs<DT, 1>(a, grid, st);
  else if (a.N == 256) launch_gi_cs<DT, 2>(a, grid, st);
  else launch_gi_cs<DT, 4>(a, grid, st);
}

}  // namespace rk

using namespace rk;

extern "C" int rk_grad_input_sr(const void* g0, const void* g1, const void* g2, int nparts,
                                int64_t part_cols, int g_dtype, int64_t ldg,
                                const float* col_scale, uint64_t seed, const int64_t* seed_dev,
                                int64_t row_offset, const uint8_t* packed, int64_t ldp,
                                int max_code, int64_t M, int64_t K, int64_t N, float* scale,
                                int8_t* q, int64_t ldq, uint16_t* g_bf16, int64_t ld_gb,
                                void* out, int out_dtype, int64_t ldo, void* stream) {
  clear_error();
  const int round_bf16 = g_dtype == RK_F32_AS_BF16 ? 1 : 0;
  const int dt = round_bf16 ? RK_F32 : g_dtype;
  if (dt != RK_F32 && dt != RK_BF16) return fail(RK_ERR_ARG, "unsupported gradient dtype %d", g_dtype);
  if (out_dtype != RK_F32 && out_dtype != RK_BF16)
    return fail(RK_ERR_ARG, "unsupported output dtype %d", out_dtype);
  if (nparts < 1 || nparts > 3) return fail(RK_ERR_ARG, "nparts must be 1, 2 or 3");
  if (M < 0 || K <= 0 || N <= 0) return fail(RK_ERR_ARG, "invalid shape");
  if (max_code < 1 || max_code > 7) return fail(RK_ERR_ARG, "max_code must be in 1..7");
  if (part_cols * nparts != K) return fail(RK_ERR_ARG, "K must be nparts x part_cols");
  if (ldg < part_cols || ldp < N || ldo < N || (q && ldq < K) || (g_bf16 && ld_gb < K))
    return fail(RK_ERR_ARG, "leading dimension too small");
  if (M > 0 && (!scale || !packed || !out)) return fail(RK_ERR_ARG, "null pointer argument");
  const void* parts[3] = {g0, g1, g2};
  const int es = dtype_size(dt), oes = out_dtype == RK_F32 ? 4 : 2;
  bool ok = part_cols % 64 == 0 && (N == 128 || N == 256 || N == 512) && K <= kGiMaxK &&
            (ldg * es) % 16 == 0 && ldp % 16 == 0 && aligned16(packed) && aligned16(out) &&
            (ldo * oes) % 16 == 0 && (!col_scale || aligned16(col_scale)) &&
            (!q || (ldq % 8 == 0 && (reinterpret_cast<uintptr_t>(q) % 8) == 0)) &&
            (!g_bf16 || (ld_gb % 8 == 0 && aligned16(g_bf16))) &&
            int64_t{kGiBM} * ldg * es < (int64_t{1} << 31) && K * ldp < (int64_t{1} << 31) &&
            int64_t{kGiBM} * ldo * oes < (int64_t{1} << 31);
  for (int i = 0; i < nparts; ++i) {
    if (M > 0 && !parts[i]) return fail(RK_ERR_ARG, "null gradient part");
    ok = ok && aligned16(parts[i]);
  }
  if (!ok)
    return fail(RK_ERR_UNSUPPORTED,
                "fused SR grad_input needs N in {128, 256, 512}, K <= %d, parts of a multiple of "
                "64 columns and 16-byte aligned rows", kGiMaxK);
  if (M == 0) return RK_OK;
  if ((M + kGiBM - 1) / kGiBM > 0x7fffffff) return fail(RK_ERR_ARG, "too many rows");
  SrGiArgs a{};
  for (int i = 0; i < 3; ++i) a.g[i] = i < nparts ? parts[i] : parts[0];
  a.ldg = ldg;
  a.part_cols = part_cols;
  a.nparts = nparts;
  a.col_scale = col_scale;
  a.key0 = static_cast<uint32_t>(seed & 0xffffffffu);
  a.key1 = static_cast<uint32_t>(seed >> 32);
  a.seed_dev = seed_dev;
  a.row_offset = row_offset;
  a.packed = packed;
  a.ldp = ldp;
  a.mc4 = 0x01010101u * static_cast<uint32_t>(max_code);
  a.M = M;
  a.K = K;
  a.N = N;
  a.scale = scale;
  a.q = q;
  a.ldq = ldq;
  a.xb = g_bf16;
  a.ldxb = ld_gb;
  a.out = out;
  a.ldo = ldo;
  a.out_f32 = out_dtype == RK_F32 ? 1 : 0;
  a.round_bf16 = round_bf16;
  const dim3 grid(static_cast<unsigned>((M + kGiBM - 1) / kGiBM));
  if (dt == RK_F32) launch_gi<RK_F32>(a, grid, as_stream(stream));
  else launch_gi<RK_BF16>(a, grid, as_stream(stream));
  return launch_status("grad_input_sr");
}
