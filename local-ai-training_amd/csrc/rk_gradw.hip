// BF16 grad_weight of the ratchet backward on gfx950 (the "TN" product):
//
//   Gw[n, k] = bf16_RNE( sum_m bf16(g[m, n]) * xh[m, k] ),
//   xh[m, k] = bf16_RNE( bf16(q[m, k]) * bf16_RNE(s[m]) )        (ratchet.py:73-75, 159-163)
//
// g is the upstream gradient [M, N] (float32 or bfloat16, row-major), q / s the saved
// per-token int8 activations and scales. Both operands are read in their natural
// token-major layout: no transposed copies are made. Tiles are staged in LDS as
// [32 tokens][128 features] bf16 (xh is dequantized during staging) and the MFMA
// fragments, which need 8 consecutive tokens of one feature per lane, are gathered with
// gfx950's transposing LDS read ds_read_b64_tr_b16: within each 16-lane group, source
// lane s points at token row (s >> 2), features 4 (s & 3) .. +3, and lane l receives
// feature l of the four token rows.
//
// The token (contraction) axis is split into `nsplit` ranges; each block writes fp32
// partial sums of one 128 x 128 output tile for one range, and a second kernel adds the
// ranges in a fixed order and rounds to bf16, so results are reproducible run to run.
#include "rk_common.h"

namespace rk {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef unsigned int gw_u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s* lds_v4s_ptr;

struct GwArgs {
  const void* g;
  int64_t ldg;
  const int8_t* q;
  int64_t ldq;
  const float* s;
  float* part;  // [nsplit][N][K] fp32
  int64_t M, N, K;
  int64_t m_chunk;  // tokens per split, a multiple of 32
  int nsplit;
};

constexpr int GW_BN = 128;                 // output rows (n) per block
constexpr int GW_BK = 128;                 // output columns (k) per block
constexpr int GW_BM = 32;                  // tokens per pipeline step
constexpr int GW_PITCH = GW_BN * 2 + 32;   // LDS row pitch in bytes (conflict-free tr reads)
constexpr int GW_TILE = GW_BM * GW_PITCH;  // one staged operand tile

__device__ __forceinline__ uint32_t gw_pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const bf2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// Global data of one pipeline step held in registers (ring slot): the g tile piece
// (GV 16-byte loads) and the q tile piece (one 16-byte load) of this thread.
template <int GV>
struct GwSlot {
  gw_u32x4 g[GV];
  gw_u32x4 q;
};

// Fragment of 8 consecutive tokens for feature column `col0 + lane % 16` (+16 for the
// upper half of each 32-lane half) from a staged [token][feature] tile.
__device__ __forceinline__ v8bf gw_fragment(const uint8_t* tile, int tok0, int col0, int lane) {
  const int grp = lane >> 4, sl = lane & 15;
  const int row = tok0 + 8 * (grp >> 1) + (sl >> 2);
  const int col = col0 + 16 * (grp & 1) + 4 * (sl & 3);
  const uint8_t* p = tile + row * GW_PITCH + col * 2;
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)(p));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)(p + 4 * GW_PITCH));
  const v4s both[2] = {lo, hi};
  v8bf f;
  __builtin_memcpy(&f, both, sizeof(f));
  return f;
}

template <int GDT, int S>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 8)))
void grad_weight_partial_kernel(GwArgs a) {
  constexpr int GV = GDT == RK_F32 ? 4 : 2;  // 16-byte g loads per thread per step
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 2 * GW_TILE];

  const int64_t tiles_k = (a.K + GW_BK - 1) / GW_BK;
  const int64_t tiles = ((a.N + GW_BN - 1) / GW_BN) * tiles_k;
  int64_t b = blockIdx.x;
  const int64_t nb = gridDim.x;
  if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);  // one XCD per token range
  const int split = static_cast<int>(b / tiles);
  const int64_t t = b % tiles;
  const int64_t n0 = (t / tiles_k) * GW_BN, k0 = (t % tiles_k) * GW_BK;
  const int64_t m_begin = split * a.m_chunk;
  const int64_t m_end = min(a.M, m_begin + a.m_chunk);
  const int steps = m_end > m_begin ? static_cast<int>((m_end - m_begin + GW_BM - 1) / GW_BM) : 0;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wk = wave >> 1;

  // Staging geometry. g: 16-byte pieces of 8 bf16 (or 4 f32 -> 4 bf16 = 8 bytes) along n.
  // q: one 16-byte piece (16 tokens' ... 16 features of one token) per thread.
  int g_row[GV], g_col[GV];  // token row in the step, first feature column in the tile
#pragma unroll
  for (int j = 0; j < GV; ++j) {
    const int c = tid + 256 * j;
    if constexpr (GDT == RK_F32) {
      g_row[j] = c >> 5;         // 32 pieces of 4 floats per 128-feature row
      g_col[j] = 4 * (c & 31);
    } else {
      g_row[j] = c >> 4;         // 16 pieces of 8 bf16 per row
      g_col[j] = 8 * (c & 15);
    }
  }
  const int q_row = tid >> 3, q_col = 16 * (tid & 7);
  const int es = GDT == RK_F32 ? 4 : 2;
  const char* gbase = static_cast<const char*>(a.g);

  auto load_slot = [&](GwSlot<GV>& r, int step) {
    const int64_t m_base = m_begin + static_cast<int64_t>(step) * GW_BM;
#pragma unroll
    for (int j = 0; j < GV; ++j) {
      const int64_t m = m_base + g_row[j], n = n0 + g_col[j];
      r.g[j] = gw_u32x4{0, 0, 0, 0};
      if (m < m_end && n < a.N)
        r.g[j] = *reinterpret_cast<const gw_u32x4*>(gbase + (m * a.ldg + n) * es);
    }
    const int64_t m = m_base + q_row, k = k0 + q_col;
    r.q = gw_u32x4{0, 0, 0, 0};
    if (m < m_end && k < a.K) r.q = *reinterpret_cast<const gw_u32x4*>(a.q + m * a.ldq + k);
  };
  auto store_slot = [&](const GwSlot<GV>& r, int step, uint8_t* gt, uint8_t* xt) {
#pragma unroll
    for (int j = 0; j < GV; ++j) {
      uint8_t* dst = gt + g_row[j] * GW_PITCH + g_col[j] * 2;
      if constexpr (GDT == RK_F32) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(
            gw_pack_bf16x2(__uint_as_float(r.g[j].x), __uint_as_float(r.g[j].y)),
            gw_pack_bf16x2(__uint_as_float(r.g[j].z), __uint_as_float(r.g[j].w)));
      } else {
        *reinterpret_cast<gw_u32x4*>(dst) = r.g[j];
      }
    }
    // xh = bf16(bf16(q) * bf16(s)): q is exact in bf16, so this is one fp32 multiply
    // of q by the bf16-rounded scale, rounded to bf16.
    const int64_t m = m_begin + static_cast<int64_t>(step) * GW_BM + q_row;
    const float sm = m < m_end ? round_bf16(a.s[m]) : 0.0f;
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v0 = static_cast<float>(static_cast<int8_t>(w[i] & 0xff)) * sm;
      const float v1 = static_cast<float>(static_cast<int8_t>((w[i] >> 8) & 0xff)) * sm;
      const float v2 = static_cast<float>(static_cast<int8_t>((w[i] >> 16) & 0xff)) * sm;
      const float v3 = static_cast<float>(static_cast<int8_t>(w[i] >> 24)) * sm;
      o[2 * i] = gw_pack_bf16x2(v0, v1);
      o[2 * i + 1] = gw_pack_bf16x2(v2, v3);
    }
    uint8_t* dst = xt + q_row * GW_PITCH + q_col * 2;
    *reinterpret_cast<gw_u32x4*>(dst) = gw_u32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<gw_u32x4*>(dst + 16) = gw_u32x4{o[4], o[5], o[6], o[7]};
  };

  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};

  // Register ring of S steps: the global loads of step st + S are issued right after
  // step st is written to LDS, so S steps of g and q stream in while the MFMAs run.
  GwSlot<GV> ring[S];
#pragma unroll
  for (int i = 0; i < S; ++i)
    if (i < steps) load_slot(ring[i], i);
  for (int st = 0; st < steps; st += S) {
#pragma unroll
    for (int slot = 0; slot < S; ++slot) {
      const int step = st + slot;
      if (step < steps) {
        uint8_t* gt = smem + (step & 1) * 2 * GW_TILE;
        uint8_t* xt = gt + GW_TILE;
        store_slot(ring[slot], step, gt, xt);
        if (step + S < steps) load_slot(ring[slot], step + S);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          v8bf fa[2], fb[2];
#pragma unroll
          for (int i = 0; i < 2; ++i) fa[i] = gw_fragment(gt, 16 * u, wn * 64 + 32 * i, lane);
#pragma unroll
          for (int j = 0; j < 2; ++j) fb[j] = gw_fragment(xt, 16 * u, wk * 64 + 32 * j, lane);
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
      }
    }
  }

  // Partial sums: acc[i][j][e] is C[n][k] with k = k0 + wk*64 + 32 j + lane % 32 and
  // n = n0 + wn*64 + 32 i + 8 (e / 4) + 4 (lane / 32) + e % 4.
  float* out = a.part + static_cast<int64_t>(split) * a.N * a.K;
  const int lk = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t k = k0 + wk * 64 + 32 * j + lk;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t n = n0 + wn * 64 + 32 * i + 8 * (e >> 2) + 4 * lh + (e & 3);
        if (n < a.N && k < a.K) out[n * a.K + k] = acc[i][j][e];
      }
    }
}

// Gw[n, k] = bf16(sum over splits of part[s][n][k]), splits added in order 0, 1, ...
__global__ __launch_bounds__(256) void grad_weight_reduce_kernel(const float* part, int nsplit,
                                                                 int64_t N, int64_t K,
                                                                 uint16_t* out, int64_t ldo) {
  const int64_t total4 = N * K / 4;  // K % 4 == 0
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total4;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    float4 acc = reinterpret_cast<const float4*>(part)[i];
    for (int s = 1; s < nsplit; ++s) {
      const float4 v = reinterpret_cast<const float4*>(part + s * N * K)[i];
      acc.x = acc.x + v.x;
      acc.y = acc.y + v.y;
      acc.z = acc.z + v.z;
      acc.w = acc.w + v.w;
    }
    const int64_t e = 4 * i, n = e / K, k = e - n * K;
    *reinterpret_cast<uint2*>(out + n * ldo + k) =
        make_uint2(gw_pack_bf16x2(acc.x, acc.y), gw_pack_bf16x2(acc.z, acc.w));
  }
}

}  // namespace rk

using namespace rk;

extern "C" int rk_grad_weight_splits(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 1;
  const int64_t tiles = ((N + GW_BN - 1) / GW_BN) * ((K + GW_BK - 1) / GW_BK);
  int64_t splits = (512 + tiles - 1) / tiles;       // about two blocks per CU
  const int64_t max_by_m = (M + 511) / 512;         // at least 512 tokens per split
  if (splits > max_by_m) splits = max_by_m;
  if (splits > 64) splits = 64;
  return static_cast<int>(splits < 1 ? 1 : splits);
}

extern "C" int rk_grad_weight_bf16(const void* g, int g_dtype, int64_t ldg, const int8_t* q,
                                   int64_t ldq, const float* s, int64_t M, int64_t N, int64_t K,
                                   float* workspace, int nsplit, uint16_t* out, int64_t ldo,
                                   void* stream) {
  clear_error();
  if (g_dtype != RK_F32 && g_dtype != RK_BF16) return fail(RK_ERR_ARG, "unsupported gradient dtype");
  if (M < 0 || N < 0 || K < 0) return fail(RK_ERR_ARG, "negative size");
  if (N == 0 || K == 0) return RK_OK;
  if (!g || !q || !s || !workspace || !out) return fail(RK_ERR_ARG, "null pointer");
  if (nsplit < 1 || nsplit > 64) return fail(RK_ERR_ARG, "nsplit must be in 1..64");
  if (ldg < N || ldq < K || ldo < K) return fail(RK_ERR_ARG, "leading dimension too small");
  const int ge = g_dtype == RK_F32 ? 4 : 2;
  if ((N % 8) != 0 || (K % 16) != 0 || ((ldg * ge) % 16) != 0 || (ldq % 16) != 0 ||
      (ldo % 4) != 0 || !aligned16(g) || !aligned16(q) || !aligned16(workspace) ||
      (reinterpret_cast<uintptr_t>(out) % 8) != 0)
    return fail(RK_ERR_UNSUPPORTED,
                "grad_weight needs N %% 8 == 0, K %% 16 == 0 and 16-byte aligned rows");
  const int64_t tiles = ((N + GW_BN - 1) / GW_BN) * ((K + GW_BK - 1) / GW_BK);
  const int64_t chunk = ((M + nsplit - 1) / nsplit + GW_BM - 1) / GW_BM * GW_BM;
  GwArgs a{};
  a.g = g;
  a.ldg = ldg;
  a.q = q;
  a.ldq = ldq;
  a.s = s;
  a.part = workspace;
  a.M = M;
  a.N = N;
  a.K = K;
  a.m_chunk = chunk > 0 ? chunk : GW_BM;
  a.nsplit = nsplit;
  const int64_t blocks = tiles * nsplit;
  if (blocks > 0x7fffffff) return fail(RK_ERR_ARG, "grid too large");
  hipStream_t st = as_stream(stream);
  // Ring depth: 4 steps for a bf16 gradient, 2 for float32 (its wider staging would
  // drop the kernel to one wave per SIMD at depth 4). RK_GW_RING overrides (2, 4, 6).
  static const int ring_env = [] {
    const char* v = getenv("RK_GW_RING");
    return v ? atoi(v) : 0;
  }();
  const int ring = ring_env ? ring_env : (g_dtype == RK_F32 ? 2 : 4);
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  if (g_dtype == RK_F32) {
    if (ring == 4) grad_weight_partial_kernel<RK_F32, 4><<<grid, block, 0, st>>>(a);
    else if (ring == 6) grad_weight_partial_kernel<RK_F32, 6><<<grid, block, 0, st>>>(a);
    else grad_weight_partial_kernel<RK_F32, 2><<<grid, block, 0, st>>>(a);
  } else {
    if (ring == 2) grad_weight_partial_kernel<RK_BF16, 2><<<grid, block, 0, st>>>(a);
    else if (ring == 6) grad_weight_partial_kernel<RK_BF16, 6><<<grid, block, 0, st>>>(a);
    else grad_weight_partial_kernel<RK_BF16, 4><<<grid, block, 0, st>>>(a);
  }
  if (int e = launch_status("grad_weight_partial")) return e;
  const int64_t total4 = N * K / 4;
  const int64_t rblocks = (total4 + 255) / 256;
  grad_weight_reduce_kernel<<<static_cast<unsigned>(rblocks < 4096 ? rblocks : 4096), 256, 0, st>>>(
      workspace, nsplit, N, K, out, ldo);
  return launch_status("grad_weight_reduce");
}
