// BF16 grad_input against the packed ratchet state, on gfx950 bf16 MFMA:
//
//   out[m, k] = bf16_RNE( sum_n G[m, n] * E[n, k] ),
//   E[n, k]   = bf16_RNE( bf16(code[n, k]) * bf16_RNE(scale[n]) )            (ratchet.py:136-141)
//
// G is the bf16 upstream gradient [M, N] (the contraction axis N contiguous), packed the
// layer's state [N, K] (low nibble code + max_code), scale its fp32 row scales. This is the
// backward of every layer that keeps the bf16 grad_input: the lm_head always, the others
// with int8_backward off.
//
// Two kernels:
//  1. effective_fragments_kernel decodes E once into a workspace laid out in MFMA operand
//     order: for each 64-row contraction step s, 32-column block kb and 16-row sub-step q,
//     1 KB holds the 64 lanes' fragments, lane l = 8 values E[64 s + 16 q + 8 (l / 32) + j]
//     [32 kb + l % 32], j = 0..7. (code * bf16(scale) is exact in fp32 for a code in
//     [-7, 7], so the one conversion is the reference's rounded bf16 multiply.) A block
//     decodes a 64 x 128 tile into LDS and writes it out with gfx950's transposing LDS read.
//  2. grad_input_bf16_kernel: block tile 128 rows (m) x 256 columns (k), 4 wavefronts each
//     owning all 128 rows and 64 columns (4 x 2 v_mfma_f32_32x32x16_bf16 tiles, 128
//     accumulators). Per 64-row contraction step a wavefront reads its E fragments straight
//     from the workspace (1 KB contiguous per load instruction, so every lane's 16 bytes
//     share cache lines with its neighbours'), and G goes through LDS: the block stages the
//     step's [128][64] G tile with 8 lanes per 128-byte row (fragment loads straight from G
//     would put each lane on its own row, 4x the L1 requests per FLOP), XOR-swizzled by
//     (row / 2) % 8 so the 16-lane groups of a fragment read hit 16 distinct bank groups.
//     Loads run R = 4 steps ahead in a register ring, the LDS ring is R stages deep and a
//     step's G tile is staged two steps before it is read, so the first fragments of step
//     s + 1 are read before step s's barrier (their latency overlaps the barrier wait) and
//     the next sub-step's fragments are read during the current sub-step's MFMAs
//     (sched_group_barrier fixes that interleave). Every load of the main loop is issued
//     unconditionally (steps past the end read zeros through the buffer bounds), so the
//     compiler's wait counts see the same loads in flight on every path.
//  The epilogue stages the block's bf16 tile in LDS and stores 16-byte row pieces;
//  out-of-range columns go to an offset past the output descriptor (dropped).
//
// The contraction order inside a step (16 q + 8 h + j for lane half h) is the same for G and
// E, so each MFMA multiplies matching rows; accumulation is float32.
#include "rk_common.h"
#include "rk_mfma32.h"
#include "rk_tr16.h"

namespace rk {

typedef float gi_v16f __attribute__((ext_vector_type(16)));

constexpr int kGiBM = 128, kGiBN = 256, kGiBK = 64;  // block rows, columns, contraction/step
constexpr int kGiRing = 4;                           // register ring = LDS ring depth
constexpr int kGiGP = kGiBK * 2;                     // G stage row: 128 bytes
constexpr int kGiGStage = kGiBM * kGiGP;             // 16 KB
constexpr int kGiEPitch = kGiBN * 2 + 16;            // epilogue staging row (bf16)
constexpr int kGiLds = kGiRing * kGiGStage > kGiBM * kGiEPitch ? kGiRing * kGiGStage
                                                               : kGiBM * kGiEPitch;
constexpr int kEfPitch = 128 * 2 + 16;  // decoded [64][128] tile row of the first kernel

// 32-column blocks of the workspace per contraction step (a multiple of 8: whole k tiles)
__host__ __device__ inline int64_t gi_col_blocks(int64_t K) {
  return 8 * ((K + kGiBN - 1) / kGiBN);
}
__host__ __device__ inline int64_t gi_steps(int64_t N) { return (N + kGiBK - 1) / kGiBK; }

struct EfArgs {
  const uint8_t* packed;
  int64_t ldp;
  int mc;
  const float* scale;
  uint16_t* ef;
  int64_t N, K, KBP;
};

__global__ __launch_bounds__(256) void effective_fragments_kernel(EfArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[64 * kEfPitch];
  const int64_t groups = a.KBP / 4;  // 128-column groups per step
  const int64_t s = blockIdx.x / groups, grp = blockIdx.x % groups;
  const int tid = threadIdx.x;
  // decode: thread -> tile row tid / 4, columns 32 (tid % 4) .. +31; rows past N and
  // columns past K decode to zero
  const int row = tid >> 2, c32 = (tid & 3) * 32;
  const int64_t n = s * 64 + row, col0 = grp * 128 + c32;
  uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float sc = 0.0f;
  if (n < a.N) {
    sc = static_cast<float>(static_cast<__bf16>(a.scale[n]));
    const uint8_t* src = a.packed + n * a.ldp + col0;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int64_t c = col0 + 16 * h2;
      if (c + 16 <= a.K) {
        const uint4 v = *reinterpret_cast<const uint4*>(src + 16 * h2);
        w[4 * h2] = v.x;
        w[4 * h2 + 1] = v.y;
        w[4 * h2 + 2] = v.z;
        w[4 * h2 + 3] = v.w;
      } else if (c + 8 <= a.K) {  // K % 8 == 0: the row's last 8 columns
        const uint2 v = *reinterpret_cast<const uint2*>(src + 16 * h2);
        w[4 * h2] = v.x;
        w[4 * h2 + 1] = v.y;
      }
    }
  }
  const int mc = a.mc;
  uint32_t o[16];
#pragma unroll
  for (int e = 0; e < 32; e += 2) {
    float v[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int ee = e + t;
      const bool in = n < a.N && col0 + ee < a.K;
      const int code = static_cast<int>((w[ee >> 2] >> (8 * (ee & 3))) & 15u) - mc;
      v[t] = in ? static_cast<float>(code) * sc : 0.0f;
    }
    o[e >> 1] = pack_bf16x2(v[0], v[1]);
  }
  uint8_t* dst = tile + row * kEfPitch + c32 * 2;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<uint4*>(dst + 16 * i) =
        make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
  __syncthreads();
  // wavefront w writes column block 4 grp + w: for each sub-step q the 64 lanes' fragments
  // (rows 16 q + 8 (lane / 32) .. +7 of column 32 w + lane % 32), 1 KB contiguous
  const int wave = tid >> 6, lane = tid & 63;
  uint4* out = reinterpret_cast<uint4*>(a.ef) + ((s * a.KBP + grp * 4 + wave) * 4) * 64 + lane;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    out[q * 64] = __builtin_bit_cast(uint4, tr16_fragment<kEfPitch>(tile, 16 * q, 32 * wave, lane));
}

struct GiArgs {
  const uint16_t* g;
  int64_t ldg;
  const uint16_t* ef;
  int64_t KBP;
  void* out;
  int64_t ldo;
  int64_t M, N, K;
};

struct GiSlot {
  u32x4 g[4];     // this thread's 4 pieces of the step's [128][64] G tile
  u32x4 e[2][4];  // this wavefront's E fragments [column block][sub-step]
};

template <int CDT>
__global__ __launch_bounds__(256) void grad_input_bf16_kernel(GiArgs a) {
  constexpr int R = kGiRing;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kGiLds];
  const int64_t tiles_k = (a.K + kGiBN - 1) / kGiBN;
  int64_t b = blockIdx.x;
  const int64_t nb = gridDim.x;
  if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);  // a row panel's k tiles on one XCD
  const int64_t m0 = (b / tiles_k) * kGiBM, tk = b % tiles_k, k0 = tk * kGiBN;
  const int64_t rows_a = a.M - m0 < kGiBM ? a.M - m0 : kGiBM;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, h = lane >> 5;

  // G rows past M read zeros (descriptor bound), pieces past N an offset past it; the
  // workspace's steps past the end read zeros likewise.
  const __amdgpu_buffer_rsrc_t g_rsrc =
      make_buffer(a.g + m0 * a.ldg, ((rows_a - 1) * a.ldg + a.N) * 2);
  const int64_t ns = gi_steps(a.N);
  const __amdgpu_buffer_rsrc_t e_rsrc = make_buffer(a.ef, ns * a.KBP * 4096);
  int gv[4], gl[4], gn[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = tid + 256 * j, row = c >> 3, p = c & 7;  // 8 lanes per 128-byte row
    gv[j] = row * static_cast<int>(a.ldg) * 2 + 16 * p;
    gl[j] = row * kGiGP + 16 * (p ^ ((row >> 1) & 7));
    gn[j] = 8 * p;
  }
  const int e_base = static_cast<int>((tk * 8 + 2 * wave) * 4096) + 16 * lane;
  const int e_step = static_cast<int>(a.KBP * 4096);

  auto issue = [&](GiSlot& sl, int s) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = 64 * s + gn[j] < a.N;
      sl.g[j] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     g_rsrc, in ? gv[j] + 128 * s : static_cast<int>(0x80000000u), 0, 0));
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        sl.e[jj][q] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       e_rsrc, e_base + s * e_step + (jj * 4 + q) * 1024, 0, 0));
  };
  auto stage_g = [&](GiSlot& sl, int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4*>(smem + buf * kGiGStage + gl[j]) = sl.g[j];
  };
  // G fragment i of sub-step q: row 32 i + lane % 32, contraction 16 q + 8 h .. +7
  auto gfrag = [&](int buf, int q, int i) {
    const int row = 32 * i + r32, p = 2 * q + h;
    return *reinterpret_cast<const v8bf*>(smem + buf * kGiGStage + row * kGiGP +
                                          16 * (p ^ ((row >> 1) & 7)));
  };

  gi_v16f acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = gi_v16f{};

  v8bf g0[4];  // sub-step 0's G fragments, read before the previous step's barrier
  auto compute = [&](GiSlot& sl, int buf) {
    v8bf gf[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) gf[0][i] = g0[i];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q < 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i) gf[(q + 1) & 1][i] = gfrag(buf, q + 1, i);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(v8bf, sl.e[j][q]), gf[q & 1][i], acc[i][j], 0, 0, 0);
    }
  };
  // one step: sub-steps 0..2 each interleave the next sub-step's 4 fragment reads with its
  // first 4 MFMAs; sub-step 3 carries the G staging writes and the next issue's 12 loads;
  // the next step's first fragment reads close it
  auto schedule_step = [&]() {
#pragma unroll
    for (int q = 0; q < 3; ++q) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 3, 0);  // VMEM read
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
  };

  const int nsteps = static_cast<int>(ns);
  GiSlot ring[R];
#pragma unroll
  for (int r = 0; r < R; ++r) issue(ring[r], r);
  stage_g(ring[0], 0);
  stage_g(ring[1], 1);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) g0[i] = gfrag(0, 0, i);

  // Step s (ring slot and LDS stage s % R): compute from stage s % R, stage step s + 2's G
  // into stage (s + 2) % R (last read in step s - 2, before the previous barrier), refill
  // the slot with step s + R, read step s + 1's first fragments (staged in step s - 1,
  // visible since that step's barrier), then the barrier. Its wait leaves those 4 reads in
  // flight: LDS operations complete in order, so lgkmcnt(4) means this wavefront's staging
  // writes, issued before them, are done.
  int s0 = 0;
  for (; s0 + R <= nsteps; s0 += R) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int s = s0 + r;
      compute(ring[r], r);
      stage_g(ring[(r + 2) % R], (r + 2) % R);
      issue(ring[r], s + R);
#pragma unroll
      for (int i = 0; i < 4; ++i) g0[i] = gfrag((r + 1) % R, 0, i);
      schedule_step();
      asm volatile("s_waitcnt lgkmcnt(4)\n\ts_barrier" ::: "memory");
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int s = s0 + r;
    if (s < nsteps) {
      compute(ring[r], r);
      stage_g(ring[(r + 2) % R], (r + 2) % R);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 4; ++i) g0[i] = gfrag((r + 1) % R, 0, i);
    }
  }
  __syncthreads();  // every fragment read done: the stages become the staging buffer

  // Epilogue: acc[i][j][e] is row 32 i + lane % 32, column 64 wave + 32 j + 8 (e / 4) +
  // 4 h + e % 4; staged as bf16, stored as 16-byte pieces of the 512-byte tile rows.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint8_t* srow = smem + (32 * i + r32) * kGiEPitch;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<uint2*>(srow + (64 * wave + 32 * j + 8 * q + 4 * h) * 2) =
            make_uint2(pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                       pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]));
  }
  __syncthreads();
  constexpr int ES = CDT == RK_BF16 ? 2 : 4;
  const __amdgpu_buffer_rsrc_t c_rsrc =
      make_buffer(static_cast<char*>(a.out) + (m0 * a.ldo + k0) * ES,
                  ((rows_a - 1) * a.ldo + (a.K - k0)) * ES);
  const int ch = tid & 31;
  const bool col_in = k0 + 8 * ch < a.K;
#pragma unroll
  for (int it = 0; it < kGiBM / 8; ++it) {
    const int row = (tid >> 5) + 8 * it;
    const uint8_t* src = smem + row * kGiEPitch + 16 * ch;
    const uint2 lo = *reinterpret_cast<const uint2*>(src);
    const uint2 hi = *reinterpret_cast<const uint2*>(src + 8);
    const uint32_t off =
        col_in ? static_cast<uint32_t>((row * a.ldo + 8 * ch) * ES) : 0x80000000u;
    if constexpr (CDT == RK_BF16) {
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(v4i, make_uint4(lo.x, lo.y, hi.x, hi.y)), c_rsrc,
          static_cast<int>(off), 0, 0);
    } else {
      const uint4 w0 = make_uint4(lo.x << 16, lo.x & 0xffff0000u, lo.y << 16, lo.y & 0xffff0000u);
      const uint4 w1 = make_uint4(hi.x << 16, hi.x & 0xffff0000u, hi.y << 16, hi.y & 0xffff0000u);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, w0), c_rsrc,
                                             static_cast<int>(off), 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, w1), c_rsrc,
                                             static_cast<int>(off + 16u), 0, 0);
    }
  }
}

}  // namespace rk

using namespace rk;

extern "C" int64_t rk_grad_input_bf16_workspace(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 0;
  return gi_steps(N) * gi_col_blocks(K) * 4096;
}

extern "C" int rk_grad_input_bf16(const uint16_t* g, int64_t ldg, const uint8_t* packed,
                                  int64_t ldp, int max_code, const float* scale, void* out,
                                  int out_dtype, int64_t ldo, int64_t M, int64_t N, int64_t K,
                                  void* work, int64_t work_bytes, void* stream) {
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(RK_ERR_ARG, "negative size");
  if (out_dtype != RK_F32 && out_dtype != RK_BF16) return fail(RK_ERR_ARG, "bad output dtype");
  if (max_code < 1 || max_code > 7) return fail(RK_ERR_ARG, "max_code must be in 1..7");
  if (M == 0 || K == 0) return RK_OK;
  if (!g || !packed || !scale || !out || !work) return fail(RK_ERR_ARG, "null pointer");
  if (ldg < N || ldp < K || ldo < K) return fail(RK_ERR_ARG, "leading dimension too small");
  const int es = out_dtype == RK_BF16 ? 2 : 4;
  if (N == 0 || N % 8 != 0 || K % 8 != 0 || (ldg * 2) % 16 != 0 || ldp % 16 != 0 ||
      (ldo * es) % 16 != 0 || !aligned16(g) || !aligned16(packed) || !aligned16(out) ||
      !aligned16(work))
    return fail(RK_ERR_UNSUPPORTED,
                "bf16 grad_input needs N a positive multiple of 8, K %% 8 == 0 and 16-byte "
                "aligned rows");
  const int64_t need = rk_grad_input_bf16_workspace(N, K);
  if (work_bytes < need) return fail(RK_ERR_ARG, "bf16 grad_input workspace too small");
  // 32-bit buffer offsets: a block's G panel, the workspace with the ring's loads past its
  // last step, a block's output rows
  const int64_t ns = gi_steps(N), kbp = gi_col_blocks(K);
  if (kGiBM * ldg * 2 >= (int64_t{1} << 31) ||
      (ns + kGiRing) * kbp * 4096 >= (int64_t{1} << 31) || kGiBM * ldo * es >= (int64_t{1} << 31))
    return fail(RK_ERR_UNSUPPORTED, "bf16 grad_input operands too large for 32-bit offsets");
  const int64_t tiles = ((M + kGiBM - 1) / kGiBM) * ((K + kGiBN - 1) / kGiBN);
  if (tiles > 0x7fffffff || ns * kbp / 4 > 0x7fffffff) return fail(RK_ERR_ARG, "grid too large");
  EfArgs e{packed, ldp, max_code, scale, static_cast<uint16_t*>(work), N, K, kbp};
  effective_fragments_kernel<<<dim3(static_cast<unsigned>(ns * kbp / 4)), 256, 0,
                               as_stream(stream)>>>(e);
  const int st = launch_status("effective_fragments");
  if (st != RK_OK) return st;
  GiArgs a{g, ldg, static_cast<const uint16_t*>(work), kbp, out, ldo, M, N, K};
  const dim3 grid(static_cast<unsigned>(tiles));
  if (out_dtype == RK_BF16)
    grad_input_bf16_kernel<RK_BF16><<<grid, 256, 0, as_stream(stream)>>>(a);
  else
    grad_input_bf16_kernel<RK_F32><<<grid, 256, 0, as_stream(stream)>>>(a);
  return launch_status("grad_input_bf16");
}
