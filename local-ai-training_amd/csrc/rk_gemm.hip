// Scaled int8 GEMM on gfx950 int8 MFMA.
//
//   C[m, n] = bf16_RNE( (float(sum_k A[m,k] * B[n,k]) * ls[m]) * rs[n] )
//
// A: int8 [M, K] (k contiguous); B: int8 [N, K] or the packed ratchet state
// [N, K] uint8 whose low nibble is code + max_code (decoded while staging).
// This is the "NT" form: both operands are K-contiguous, which is how the
// persistent codes are stored (packed[n, k]), so the forward GEMM needs no
// transposed copy of the weights (the reference makes one, ratchet.py:52).
//
// Two kernels:
//  * int8_gemm_m32_kernel, for aligned shapes (K % 64 == 0, 16-byte aligned rows and
//    scales, N % 8 == 0): v_mfma_i32_32x32x32_i8, 128 x 128 or 256 x 256 block tiles, buffer
//    addressing, register ring + LDS ping-pong, LDS-staged coalesced epilogue;
//  * int8_gemm_nt_kernel, any shape and stride (ragged K, unaligned rows):
//    v_mfma_i32_16x16x64_i8 with bounds-checked staging.
// Block order is XCD-aware: consecutive tile indices (which share an A row panel)
// are kept on one XCD's L2.
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "rk_common.h"
#include "rk_mfma32.h"

namespace rk {

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kLdsRow = kBK + 16;  // bytes

// B_PACKED_T: the packed state read as the K x N operand, code[k, n] = packed[k, n]
// decoded (the grad_input GEMM contracts over the packed rows; aligned kernel only).
enum { B_INT8 = 0, B_PACKED = 1, B_PACKED_T = 2 };

struct GemmArgs {
  const int8_t* A;
  int64_t lda;
  const uint8_t* B;
  int64_t ldb;
  uint32_t mc4;  // max_code replicated in 4 bytes (packed B only)
  int max_code;
  const float* ls;
  const float* rs;
  void* C;
  int64_t ldc;
  int64_t M, N, K;
  const float* R;  // optional residual added to a float32 output (32x32x32 kernel only)
  int64_t ldr;
};

// Loads the 16-byte segment (row, k0 .. k0+15) of an operand; zeros outside
// [0, rows) x [0, K). FAST: K % 64 == 0, ld % 16 == 0, 16-byte aligned base.
template <bool FAST, int KIND>
__device__ __forceinline__ uint4 load_seg(const uint8_t* base, int64_t ld, int64_t row,
                                          int64_t rows, int64_t k0, int64_t K, uint32_t mc4,
                                          int max_code) {
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row >= rows) return v;
  if constexpr (FAST) {
    v = *reinterpret_cast<const uint4*>(base + row * ld + k0);
    if constexpr (KIND == B_PACKED) {
      v.x = decode4(v.x, mc4);
      v.y = decode4(v.y, mc4);
      v.z = decode4(v.z, mc4);
      v.w = decode4(v.w, mc4);
    }
  } else {
    uint32_t w[4] = {0, 0, 0, 0};
    const uint8_t* p = base + row * ld;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const int64_t k = k0 + b;
      uint32_t byte = 0;
      if (k < K) {
        byte = p[k];
        if constexpr (KIND == B_PACKED) byte = static_cast<uint8_t>((byte & 15u) - max_code);
      }
      w[b >> 2] |= byte << (8 * (b & 3));
    }
    v = make_uint4(w[0], w[1], w[2], w[3]);
  }
  return v;
}

template <int CDT>
__device__ __forceinline__ void store_out4(void* C, int64_t ldc, int64_t m, int64_t n,
                                           int64_t M, int64_t N, const float* v,
                                           bool vec_ok) {
  if (m >= M) return;
  if constexpr (CDT == RK_BF16) {
    uint16_t* row = static_cast<uint16_t*>(C) + m * ldc;
    uint16_t h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) h[r] = f32_to_bf16(v[r]);
    if (vec_ok && n + 3 < N) {
      uint2 pk;
      pk.x = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
      pk.y = static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16);
      *reinterpret_cast<uint2*>(row + n) = pk;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) row[n + r] = h[r];
    }
  } else {
    float* row = static_cast<float*>(C) + m * ldc;
    float f[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) f[r] = round_bf16(v[r]);
    if (vec_ok && n + 3 < N) {
      *reinterpret_cast<float4*>(row + n) = make_float4(f[0], f[1], f[2], f[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) row[n + r] = f[r];
    }
  }
}

template <int KIND, bool FAST, int CDT>
__global__ __launch_bounds__(256) void int8_gemm_nt_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t As[2][kBM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][kBN * kLdsRow];

  const int64_t tiles_n = (g.N + kBN - 1) / kBN;
  int64_t b = blockIdx.x;
  const int64_t nb = gridDim.x;
  if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);
  const int64_t m0 = (b / tiles_n) * kBM;
  const int64_t n0 = (b % tiles_n) * kBN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int g4 = lane >> 4, r16 = lane & 15;

  // Staging assignment: 512 16-byte segments per operand tile, 2 per thread.
  int srow[2], sseg[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = tid + 256 * j;
    srow[j] = c >> 2;
    sseg[j] = c & 3;
  }

  const uint8_t* Abase = reinterpret_cast<const uint8_t*>(g.A);
  uint4 ra[2], rb[2];
  auto load_tiles = [&](int64_t k0) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      ra[j] = load_seg<FAST, B_INT8>(Abase, g.lda, m0 + srow[j], g.M, k0 + 16 * sseg[j], g.K,
                                     0, 0);
      rb[j] = load_seg<FAST, KIND>(g.B, g.ldb, n0 + srow[j], g.N, k0 + 16 * sseg[j], g.K,
                                   g.mc4, g.max_code);
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      *reinterpret_cast<uint4*>(&As[buf][srow[j] * kLdsRow + 16 * sseg[j]]) = ra[j];
      *reinterpret_cast<uint4*>(&Bs[buf][srow[j] * kLdsRow + 16 * sseg[j]]) = rb[j];
    }
  };

  v4i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  const int64_t nk = (g.K + kBK - 1) / kBK;
  load_tiles(0);
  store_tiles(0);
  __syncthreads();

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = static_cast<int>(kt & 1);
    if (kt + 1 < nk) load_tiles((kt + 1) * kBK);

    v4i fa[4], fb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[i] = *reinterpret_cast<const v4i*>(
          &As[cur][(wm * 64 + i * 16 + r16) * kLdsRow + 16 * g4]);
      fb[i] = *reinterpret_cast<const v4i*>(
          &Bs[cur][(wn * 64 + i * 16 + r16) * kLdsRow + 16 * g4]);
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        acc[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[ni], fa[mi], acc[mi][ni], 0, 0, 0);

    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds rows m = .. + r16 and columns n = .. + 4*g4 + r.
  const bool vec_ok =
      (g.ldc % 4) == 0 && (reinterpret_cast<uintptr_t>(g.C) % (CDT == RK_BF16 ? 8 : 16)) == 0;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int64_t m = m0 + wm * 64 + mi * 16 + r16;
    const float lsm = m < g.M ? g.ls[m] : 0.0f;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const int64_t n = n0 + wn * 64 + ni * 16 + 4 * g4;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = static_cast<float>(acc[mi][ni][r]) * lsm;
        if (g.rs) t = t * (n + r < g.N ? g.rs[n + r] : 0.0f);
        v[r] = t;
      }
      store_out4<CDT>(g.C, g.ldc, m, n, g.M, g.N, v, vec_ok);
    }
  }
}

// Staging registers of one k-step (one slot of the register ring).
template <int NA, int NB>
struct RingSlot {
  u32x4 a[NA];
  u32x4 b[NB];
};

// ---------------------------------------------------------------------------
// 32x32x32 MFMA kernel (aligned shapes): block tile 128 x 128, 4 wavefronts in 2 x 2,
// wave tile 64 x 64 = 2 x 2 blocks of v_mfma_i32_32x32x32_i8 (two per 64-byte k-step),
// register ring of 2 k-steps, LDS ping-pong, one barrier per k-step. The fragment step
// and the LDS tile layouts are in rk_mfma32.h.
// ---------------------------------------------------------------------------
// Block configurations of the 32x32x32 kernel: BM x BN tile, WM x WN wavefronts, each a
// (BM / WM) x (BN / WN) wave tile of 32 x 32 MFMA blocks, MINW waves per SIMD.
//  * 128 x 128, 2 x 2 waves (64 x 64 wave tiles, 64 accumulator registers), two or more
//    blocks per CU: small grids;
//  * 256 x 256, 2 x 4 waves (128 x 64 wave tiles, 128 accumulator registers, one block
//    per CU): twice the MACs per byte fetched from L2 (a 128 x 128 tile needs 1 byte of
//    A or B per 128 int8 ops, which at MFMA peak is about the whole L2 bandwidth); used
//    for K >= 1024 when the grid still covers the chip (at K = 512 the single block per CU
//    leaves the prologue and epilogue exposed and the small tiles are faster).
template <int BM_, int BN_, int WM_, int WN_, int MINW_, int EROUNDS_, int RING_>
struct M32Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, MINW = MINW_;
  static constexpr int RING = RING_;  // k-steps of global loads held in registers (1 or 2)
  static constexpr int EROUNDS = EROUNDS_;  // epilogue staging rounds (LDS holds BM / EROUNDS rows)
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int MI = BM / WM / 32, NJ = BN / WN / 32;
  static constexpr int BTP = BN + 32;  // B_PACKED_T staging pitch: 8 rows cover 64 banks
};
using CfgSmall = M32Cfg<128, 128, 2, 2, 2, 1, 2>;
using CfgBig = M32Cfg<256, 256, 2, 4, 2, 2, 1>;

//
// The instructions outside the MFMAs bound this kernel at K = 512 (8 k-steps per tile),
// so it is written to keep them few:
//  * A, B, ls, rs and C are addressed through buffer descriptors over the block's rows:
//    rows past M or N read as zeros and their stores are dropped, so there are no
//    clamps or bounds branches, per-thread offsets are fixed and a k-step only moves a
//    scalar offset;
//  * the epilogue stages bf16 results in LDS rows of 264 bytes: the 32 rows of one
//    8-byte fragment write start 2 banks apart, and a 16-lane row of the 16-byte
//    copy-out covers 64 banks, so neither side needs a swizzle or a lane swap;
//  * each thread copies out a fixed 8-column chunk, so the column bound is one compare.
// ---------------------------------------------------------------------------
template <int KIND, int CDT, bool HAS_RS, class CFG>
__global__ __launch_bounds__(CFG::THREADS) __attribute__((amdgpu_waves_per_eu(CFG::MINW, 8)))
void int8_gemm_m32_kernel(GemmArgs g) {
  constexpr int BM = CFG::BM, BN = CFG::BN, BK = 64, S = CFG::RING;
  constexpr int THREADS = CFG::THREADS, MI = CFG::MI, NJ = CFG::NJ, BTP = CFG::BTP;
  constexpr bool BT = KIND == B_PACKED_T;
  constexpr int SEGS = BM * BK / 16 / THREADS;  // 16-byte pieces per thread per operand (2)
  static_assert(SEGS * 16 * THREADS == BM * BK && BN == BM, "square tiles");
  constexpr int EPITCH = BN * 2 + 8;  // epilogue staging row, bytes
  constexpr int EROWS = BM / CFG::EROUNDS;  // rows staged per epilogue round
  static_assert(CFG::WM % CFG::EROUNDS == 0, "whole wave rows per epilogue round");
  constexpr int BSTAGE = BT ? BK * BTP : BN * BK;  // bytes of one B stage
  constexpr int TILES = 2 * BM * BK + 2 * BSTAGE;
  constexpr int BODY = EROWS * EPITCH > TILES ? EROWS * EPITCH : TILES;
  constexpr int SMEM = BODY + BN * 4;  // + the tile's column scales
  static_assert(THREADS >= BN, "one column scale per thread");
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];
  uint8_t* As = smem;
  uint8_t* Bs = smem + 2 * BM * BK;
  float* const rs_lds = reinterpret_cast<float*>(smem + BODY);

  const int64_t tiles_n = (g.N + BN - 1) / BN;
  int64_t b = blockIdx.x;
  const int64_t nb = gridDim.x;
  if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);
  const int64_t m0 = (b / tiles_n) * BM;
  const int64_t n0 = (b % tiles_n) * BN;
  const int64_t rows_a = g.M - m0 < BM ? g.M - m0 : BM;
  const int64_t rows_b = g.N - n0 < BN ? g.N - n0 : BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % CFG::WM, wn = wave / CFG::WM;
  const int arow0 = wm * (BM / CFG::WM), brow0 = wn * (BN / CFG::WN);

  const __amdgpu_buffer_rsrc_t a_rsrc =
      make_buffer(g.A + m0 * g.lda, (rows_a - 1) * g.lda + g.K);
  // B_PACKED_T: the descriptor spans columns n0.. of all K rows (a k-step moves the
  // scalar offset by 64 rows); columns past N in the last row read zeros, elsewhere the
  // next columns (in bounds; their outputs are never stored)
  const __amdgpu_buffer_rsrc_t b_rsrc =
      BT ? make_buffer(g.B + n0, (g.K - 1) * g.ldb + (g.N - n0))
         : make_buffer(g.B + n0 * g.ldb, (rows_b - 1) * g.ldb + g.K);
  const int b_step = BT ? BK * static_cast<int>(g.ldb) : BK;
  int a_voff[SEGS], b_voff[SEGS], st_off[SEGS], bst_off[SEGS];
#pragma unroll
  for (int j = 0; j < SEGS; ++j) {
    const int c = tid + THREADS * j, row = c >> 2, seg = c & 3;
    a_voff[j] = row * static_cast<int>(g.lda) + 16 * seg;
    st_off[j] = row * BK + 16 * (seg ^ swz32(row));
    if constexpr (BT) {
      const int krow = c / (BN / 16), nseg = c % (BN / 16);  // 64 rows of BN bytes
      b_voff[j] = krow * static_cast<int>(g.ldb) + 16 * nseg;
      bst_off[j] = krow * BTP + 16 * nseg;
    } else {
      b_voff[j] = row * static_cast<int>(g.ldb) + 16 * seg;
      bst_off[j] = st_off[j];
    }
  }

  RingSlot<SEGS, SEGS> ring[S];
  auto load = [&](RingSlot<SEGS, SEGS>& r, int kt) {
#pragma unroll
    for (int j = 0; j < SEGS; ++j)
      r.a[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             a_rsrc, a_voff[j], kt * BK, 0));
#pragma unroll
    for (int j = 0; j < SEGS; ++j)
      r.b[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             b_rsrc, b_voff[j], kt * b_step, 0));
  };
  auto store = [&](RingSlot<SEGS, SEGS>& r, int buf) {
    // Pin the slot here (see the grad_weight kernel): otherwise the decode of every slot
    // is computed as soon as its load is issued and the wait covers the whole ring.
#pragma unroll
    for (int j = 0; j < SEGS; ++j) asm volatile("" : "+v"(r.a[j]), "+v"(r.b[j]));
    uint8_t* at = As + buf * BM * BK;
    uint8_t* bt = Bs + buf * BSTAGE;
#pragma unroll
    for (int j = 0; j < SEGS; ++j) *reinterpret_cast<u32x4*>(at + st_off[j]) = r.a[j];
#pragma unroll
    for (int j = 0; j < SEGS; ++j) {
      u32x4 v = r.b[j];
      if constexpr (KIND == B_PACKED || KIND == B_PACKED_T) {
        v.x = decode4(v.x, g.mc4);
        v.y = decode4(v.y, g.mc4);
        v.z = decode4(v.z, g.mc4);
        v.w = decode4(v.w, g.mc4);
      }
      *reinterpret_cast<u32x4*>(bt + bst_off[j]) = v;
    }
  };

  v16i acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = v16i{};

  // Ring of S = 2 k-steps (registers) over an LDS ping-pong: the loads of step kt + 2 are
  // issued right after step kt is written to LDS. Pairs of k-steps run without a branch;
  // an odd last step follows. Loads past the last k-step are never consumed (past the
  // last row's end they read zeros, elsewhere the next row: always in bounds).
  // The epilogue's row and column scales are requested first, so their latency passes
  // under the main loop's; the column scales go to LDS once the first k-steps are issued.
  const int r32 = lane & 31, hh = lane >> 5;
  const __amdgpu_buffer_rsrc_t ls_rsrc = make_buffer(g.ls + m0, rows_a * 4);
  float lsv[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
    lsv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           ls_rsrc, (arow0 + 32 * i + r32) * 4, 0, 0));
  float rsv = 1.0f;
  if constexpr (HAS_RS) {
    const __amdgpu_buffer_rsrc_t rs_rsrc = make_buffer(g.rs + n0, rows_b * 4);
    rsv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_rsrc, tid * 4, 0, 0));
  }
  const int nk = static_cast<int>(g.K / BK);
  if constexpr (S == 2) {
    load(ring[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    load(ring[1], 1);
    __builtin_amdgcn_sched_barrier(0);
    if (HAS_RS && tid < BN) rs_lds[tid] = rsv;
    const int nk_pairs = nk & ~1;
    for (int kb = 0; kb < nk_pairs; kb += S) {
#pragma unroll
      for (int slot = 0; slot < S; ++slot) {
        store(ring[slot], slot);
        load(ring[slot], kb + slot + S);
        __syncthreads();
        mfma32_step<BT, MI, NJ, BTP>(acc, As + slot * BM * BK, Bs + slot * BSTAGE, arow0,
                                     brow0, lane);
      }
    }
    if (nk & 1) {
      store(ring[0], 0);
      __syncthreads();
      mfma32_step<BT, MI, NJ, BTP>(acc, As, Bs, arow0, brow0, lane);
    }
  } else {
    // one k-step in registers: the loads of step kt + 1 are issued right after step kt is
    // written to LDS (the same LDS ping-pong and one barrier per step)
    load(ring[0], 0);
    if (HAS_RS && tid < BN) rs_lds[tid] = rsv;
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      store(ring[0], buf);
      load(ring[0], kt + 1);
      __syncthreads();
      mfma32_step<BT, MI, NJ, BTP>(acc, As + buf * BM * BK, Bs + buf * BSTAGE, arow0, brow0,
                                   lane);
    }
  }
  __syncthreads();  // all fragment reads done: the tiles become the staging buffer

  // Epilogue. acc[i][j][e]: row m = arow0 + 32 i + (lane & 31), columns
  // n = brow0 + 32 j + 8 q + 4 (lane >> 5) + (e % 4), q = e / 4. In round r the waves
  // whose rows lie in [r EROWS, (r + 1) EROWS) stage them as bf16, then the whole block
  // copies them out.
  constexpr int ES = CDT == RK_BF16 ? 2 : 4;
  constexpr int CHUNKS = BN / 8;             // 8-column chunks per row
  constexpr int RSTEP = THREADS / CHUNKS;    // rows copied per pass
  const int ch = tid % CHUNKS;               // 8-column chunk of this thread
  const __amdgpu_buffer_rsrc_t c_rsrc =
      make_buffer(static_cast<char*>(g.C) + (m0 * g.ldc + n0) * ES,
                  ((rows_a - 1) * g.ldc + (g.N - n0)) * ES);
  // float32 output with a residual: C = R + (the bf16 result widened), the same float32
  // add as adding the two tensors afterwards (R may be C itself: each thread reads its
  // residual before it stores over it)
  const bool has_r = CDT == RK_F32 && g.R != nullptr;
  const __amdgpu_buffer_rsrc_t r_rsrc =
      make_buffer(has_r ? g.R + m0 * g.ldr + n0 : g.ls,
                  has_r ? ((rows_a - 1) * g.ldr + (g.N - n0)) * 4 : 0);
#pragma unroll
  for (int round = 0; round < CFG::EROUNDS; ++round) {
    if (arow0 / EROWS == round) {
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        uint8_t* srow = smem + (arow0 - round * EROWS + 32 * i + r32) * EPITCH;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float4 rs4 = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            if constexpr (HAS_RS)
              rs4 = *reinterpret_cast<const float4*>(rs_lds + brow0 + 32 * j + 8 * q + 4 * hh);
            float v0 = static_cast<float>(acc[i][j][4 * q]) * lsv[i];
            float v1 = static_cast<float>(acc[i][j][4 * q + 1]) * lsv[i];
            float v2 = static_cast<float>(acc[i][j][4 * q + 2]) * lsv[i];
            float v3 = static_cast<float>(acc[i][j][4 * q + 3]) * lsv[i];
            if constexpr (HAS_RS) {
              v0 = v0 * rs4.x;
              v1 = v1 * rs4.y;
              v2 = v2 * rs4.z;
              v3 = v3 * rs4.w;
            }
            *reinterpret_cast<uint2*>(srow + (brow0 + 32 * j + 8 * q + 4 * hh) * 2) =
                make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
          }
      }
    }
    __syncthreads();
    if (n0 + 8 * ch < g.N) {
#pragma unroll
      for (int it = 0; it < EROWS / RSTEP; ++it) {
        const int srow = tid / CHUNKS + RSTEP * it;
        const int row = round * EROWS + srow;
        const uint8_t* src = smem + srow * EPITCH + 16 * ch;
        const uint2 lo = *reinterpret_cast<const uint2*>(src);
        const uint2 hi = *reinterpret_cast<const uint2*>(src + 8);
        const int voff = (row * static_cast<int>(g.ldc) + 8 * ch) * ES;
        if constexpr (CDT == RK_BF16) {
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(v4i, make_uint4(lo.x, lo.y, hi.x, hi.y)), c_rsrc, voff, 0, 0);
        } else {
          uint4 w0 = make_uint4(lo.x << 16, lo.x & 0xffff0000u, lo.y << 16, lo.y & 0xffff0000u);
          uint4 w1 = make_uint4(hi.x << 16, hi.x & 0xffff0000u, hi.y << 16, hi.y & 0xffff0000u);
          if (has_r) {
            const int roff = (row * static_cast<int>(g.ldr) + 8 * ch) * 4;
            const float4 r0 = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(r_rsrc, roff, 0, 0));
            const float4 r1 = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(r_rsrc, roff + 16, 0, 0));
            w0.x = __float_as_uint(r0.x + __uint_as_float(w0.x));
            w0.y = __float_as_uint(r0.y + __uint_as_float(w0.y));
            w0.z = __float_as_uint(r0.z + __uint_as_float(w0.z));
            w0.w = __float_as_uint(r0.w + __uint_as_float(w0.w));
            w1.x = __float_as_uint(r1.x + __uint_as_float(w1.x));
            w1.y = __float_as_uint(r1.y + __uint_as_float(w1.y));
            w1.z = __float_as_uint(r1.z + __uint_as_float(w1.z));
            w1.w = __float_as_uint(r1.w + __uint_as_float(w1.w));
          }
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, w0), c_rsrc, voff, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, w1), c_rsrc, voff + 16,
                                                 0, 0);
        }
      }
    }
    if (round + 1 < CFG::EROUNDS) __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Persistent LDS-ring kernel (aligned shapes, 256 x 256 tiles): the wide token GEMMs
// (N >= 4096: the lm_head, the 1B qkv / expand).
//
// Each of the 8 wavefronts (2 x 4) owns a 128 x 64 wave tile (4 x 2 blocks of
// v_mfma_i32_32x32x32_i8, accumulators in 128 registers). Operands reach LDS through
// gfx950's buffer_load_dwordx4 ... lds (16 bytes per lane straight into LDS, no
// registers, no VALU): one 32 KB stage per 64-byte k-step (A [256][64] + B [256][64], or
// for the packed [K, N] operand B [64][256]), S stages in a ring. The block is persistent:
// it walks its tiles in order and the ring runs across tile boundaries, so the loads of the
// next tile's first S - 1 k-steps are in flight during the current tile's last k-steps and
// its epilogue. The LDS-DMA destination is fixed by the lane (lane l writes bytes
// 16 l .. 16 l + 15 of the instruction's 1 KB), so the bank swizzles are applied to the
// source instead: lane l fetches the segment that belongs at its slot.
//  * [256][64] stages: slot (row, t) holds segment t ^ ((row >> 2) & 3) (the 32-row MFMA
//    fragment reads of the register-ring kernel above, conflict-free);
//  * the packed [64][256] stage: slot (row, t) of a 256-byte row holds segment
//    t ^ 2 (row & 7): the transposing fragment reads (8 rows x 2 adjacent segments per 32
//    lanes) then touch 16 distinct 16-byte bank groups.
// The row scales (and column scales) of each tile go to a double-buffered LDS area by the
// same DMA, ahead of the tile's first k-step, so the epilogue reads them with no vector
// memory wait. The epilogue stages the bf16 results in LDS, 64 rows per round, so every
// store writes 16 bytes of 32-lane-contiguous 512-byte rows (stores straight from the MFMA
// layout scatter 8 bytes over 32 rows per instruction and cost 18 of 45 us at
// 16384 x 2048 x 512). Out-of-range columns are stored to an offset past the output
// descriptor (2^31, dropped by the hardware) instead of behind a branch. Tiles are walked in
// groups of 8 row tiles (n-major inside a group), so the 32 tiles an XCD runs at once
// share 8 A panels and 4 B panels in its L2 (8192^3: 626 -> 534 us against row-major).
//
// Synchronization per k-step: each wavefront waits for its own DMA loads of the stage
// (vmcnt, and lgkmcnt(0): the LDS write of an LDS-DMA load is tracked on the LDS counter, and
// with vmcnt alone a wavefront on a busy CU was measured reading stale stage bytes), then
// one s_barrier makes every wavefront's part visible; the stage refilled after the barrier
// is the one every wavefront finished reading before it arrived. The DMA loads are inline assembly, which
// the compiler does not track: its own vmcnt waits (the residual loads) only become
// stricter, never too weak, with loads it cannot see in flight.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef unsigned int u32x2_v __attribute__((ext_vector_type(2)));

constexpr int kPipeBM = 256, kPipeBN = 256, kPipeBK = 64, kPipeStages = 3;
// epilogue staging: 64 rows of 256 bf16 at a 520-byte pitch (rows 2 banks apart)
constexpr int kEPitch = 520, kERows = 64;
constexpr int kPipeStage = (kPipeBM + kPipeBN) * kPipeBK;  // 32 KB
constexpr int kPipeScales = 2 * 2 * 1024;                  // ls + rs, two tiles

__host__ __device__ constexpr int vmcnt_imm(int n) {
  // s_waitcnt immediate that waits for vmcnt <= n only (expcnt 7, lgkmcnt 15)
  return 0x0F70 | (n & 15) | ((n >> 4) << 14);
}

// One LDS-DMA load: 16 bytes per lane at buffer offset voff + soff into LDS bytes
// lds + 16 lane .. + 15. M0 holds the LDS address (wave-uniform).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t lds, int voff, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}

struct PipeSched {
  int tiles, tiles_m, tiles_n, tiles_per_xcd;
};

template <int KIND, int CDT, bool HAS_RS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void int8_gemm_pipe_kernel(GemmArgs g, PipeSched p) {
  constexpr int BM = kPipeBM, BN = kPipeBN, BK = kPipeBK, S = kPipeStages;
  constexpr int NW = 8, THR = 64 * NW, CH = 16 / NW, WNT = BN / (NW / 2);
  constexpr int MI = 4, NJ = WNT / 32, ASZ = BM * BK, STAGE = kPipeStage;
  constexpr bool BT = KIND == B_PACKED_T;
  constexpr bool PACKED = KIND != B_INT8;
  constexpr int ES = CDT == RK_BF16 ? 2 : 4;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[S * STAGE + kPipeScales + kERows * kEPitch];
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_ptr)smem));

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int arow0 = (wave & 1) * 128, brow0 = (wave >> 1) * WNT;
  const int r32 = lane & 31, h = lane >> 5;

  // Tiles: row-major over (m tile, n tile), consecutive indices share an A row panel. The
  // blocks of one XCD (block b runs on XCD b % 8) take one contiguous range of tiles, so
  // the A panels and B of that range stay in the XCD's L2.
  const int xcd = blockIdx.x & 7, lb = blockIdx.x >> 3, bpx = gridDim.x >> 3;
  const int t_begin = xcd * p.tiles_per_xcd;
  const int t_span = min(p.tiles, t_begin + p.tiles_per_xcd) - t_begin;
  const int n_my = t_span > lb ? (t_span - lb + bpx - 1) / bpx : 0;
  const int nk = static_cast<int>(g.K / BK);
  const int total = n_my * nk;

  // Per-lane DMA source offsets (fixed for the kernel). Wave w fills 1 KB chunks 2w and
  // 2w + 1 of each operand's stage.
  const int lda = static_cast<int>(g.lda), ldb = static_cast<int>(g.ldb);
  const int sg = (lane & 3) ^ ((lane >> 4) & 3);  // [256][64] stage: 16 rows of 4 slots
  int a_v[CH], b_v[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int chunk = CH * wave + c;
    a_v[c] = (16 * chunk + (lane >> 2)) * lda + 16 * sg;
    if constexpr (BT) {
      const int r0 = 4 * chunk + (lane >> 4);
      b_v[c] = r0 * ldb + 16 * ((lane & 15) ^ (2 * (r0 & 7)));
    } else {
      b_v[c] = (16 * chunk + (lane >> 2)) * ldb + 16 * sg;
    }
  }
  const int b_kstep = BT ? BK * ldb : BK;  // B offset per k-step

  // Tile order: groups of GM row tiles, n-major inside a group, so the 32 tiles an XCD
  // runs at once span GM row panels of A and 32 / GM column panels of B.
  constexpr int GM = 8;
  auto tile_origin = [&](int ordinal, int64_t& m0, int64_t& n0) {
    const int tile = t_begin + lb + ordinal * bpx;
    const int group = GM * p.tiles_n;
    const int gidx = tile / group, first_m = gidx * GM;
    const int gm = p.tiles_m - first_m < GM ? p.tiles_m - first_m : GM;
    const int r = tile - gidx * group;
    m0 = static_cast<int64_t>(first_m + r % gm) * BM;
    n0 = static_cast<int64_t>(r / gm) * BN;
  };

  // Producer state: the current tile's descriptors, recomputed when the tile changes.
  int pt = 0, pk = 0, pstage = 0;
  __amdgpu_buffer_rsrc_t ar = make_buffer(g.A, 0), br = make_buffer(g.B, 0);
  int64_t pm0 = 0, pn0 = 0, prows = 0, pcols = 0;
  auto set_tile = [&]() {
    tile_origin(pt, pm0, pn0);
    prows = g.M - pm0 < BM ? g.M - pm0 : BM;
    pcols = g.N - pn0 < BN ? g.N - pn0 : BN;
    ar = make_buffer(g.A + pm0 * g.lda, (prows - 1) * g.lda + g.K);
    br = BT ? make_buffer(g.B + pn0, (g.K - 1) * g.ldb + (g.N - pn0))
            : make_buffer(g.B + pn0 * g.ldb, (pcols - 1) * g.ldb + g.K);
  };
  if (total > 0) set_tile();
  auto issue = [&]() {
    if (pk == 0 && wave < 2) {
      const uint32_t dst = lds0 + S * STAGE + (pt & 1) * 2048 + wave * 1024;
      if (wave == 0) {
        dma16(make_buffer(g.ls + pm0, prows * 4), dst, 16 * lane, 0);
      } else if (HAS_RS) {
        dma16(make_buffer(g.rs + pn0, pcols * 4), dst, 16 * lane, 0);
      }
    }
    const uint32_t st = lds0 + pstage * STAGE + 1024 * CH * wave;
    const int ak = pk * BK, bk = pk * b_kstep;
#pragma unroll
    for (int c = 0; c < CH; ++c) dma16(ar, st + 1024 * c, a_v[c] + ak, 0);
#pragma unroll
    for (int c = 0; c < CH; ++c) dma16(br, st + ASZ + 1024 * c, b_v[c] + bk, 0);
    if (++pstage == S) pstage = 0;
    if (++pk == nk) {
      pk = 0;
      ++pt;
      if (pt < n_my) set_tile();
    }
  };

  v16i acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = v16i{};

  for (int s = 0; s < S - 1 && s < total; ++s) issue();
  int ct = 0, ck = 0, cstage = 0;  // consumer: tile ordinal, k-step, stage
  for (int step = 0; step < total; ++step) {
    // this step's loads landed: at most the loads of the (up to S - 2) later steps in
    // flight (2 CH per step; the scale loads and stores issued after them only make the
    // wait stricter)
    const int ahead = total - 1 - step;
    if (ahead >= S - 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * CH * (S - 2)) & ~0x0F00);
    else if (ahead == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * CH) & ~0x0F00);
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & ~0x0F00);
    asm volatile("s_barrier" ::: "memory");
    if (step + S - 1 < total) issue();

    const uint8_t* at = smem + cstage * STAGE;
    if (++cstage == S) cstage = 0;
    const uint8_t* bt = at + ASZ;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      v4i fa[MI], fb[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int ra = arow0 + i * 32 + r32;
        fa[i] = *reinterpret_cast<const v4i*>(at + ra * 64 + 16 * ((h + 2 * kh) ^ swz32(ra)));
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        v4i v;
        if constexpr (BT) {
          // 16 consecutive k rows of output column `col` per lane (transposing read)
          const int sl = lane & 15;
          const int col = brow0 + j * 32 + 16 * ((lane >> 4) & 1) + 8 * (sl & 1);
          const int r0 = 16 * (h + 2 * kh) + (sl >> 1);  // r0 & 7 == (r0 + 8) & 7
          const int phys = 16 * ((col >> 4) ^ (2 * (r0 & 7))) + (col & 15);
          const v2i_t lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_ptr)(bt + r0 * 256 + phys));
          const v2i_t hi =
              __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_ptr)(bt + (r0 + 8) * 256 + phys));
          v = v4i{lo.x, lo.y, hi.x, hi.y};
        } else {
          const int rb = brow0 + j * 32 + r32;
          v = *reinterpret_cast<const v4i*>(bt + rb * 64 + 16 * ((h + 2 * kh) ^ swz32(rb)));
        }
        if constexpr (PACKED) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = static_cast<int>(decode4(static_cast<uint32_t>(v[e]), g.mc4));
        }
        fb[j] = v;
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[j], fa[i], acc[i][j], 0, 0, 0);
    }
    if (++ck < nk) continue;

    // Epilogue of tile ct: C = bf16((acc * ls) * rs), rows m = arow0 + 32 i + lane % 32,
    // columns n = brow0 + 32 j + 8 q + 4 (lane / 32) + e % 4 (e = 4 q .. 4 q + 3).
    ck = 0;
    int64_t m0, n0;
    tile_origin(ct, m0, n0);
    const int64_t rows_a = g.M - m0 < BM ? g.M - m0 : BM;
    const uint8_t* sc = smem + S * STAGE + (ct & 1) * 2048;
    ++ct;
    const __amdgpu_buffer_rsrc_t c_r =
        make_buffer(static_cast<char*>(g.C) + (m0 * g.ldc + n0) * ES,
                    ((rows_a - 1) * g.ldc + (g.N - n0)) * ES);
    const bool has_r = CDT == RK_F32 && g.R != nullptr;
    const __amdgpu_buffer_rsrc_t r_r =
        make_buffer(has_r ? g.R + m0 * g.ldr + n0 : g.ls,
                    has_r ? ((rows_a - 1) * g.ldr + (g.N - n0)) * 4 : 0);
    float lsv[MI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
      lsv[i] = *reinterpret_cast<const float*>(sc + (arow0 + 32 * i + r32) * 4);
    {
      uint8_t* stg = smem + S * STAGE + kPipeScales;
      const int wm = wave & 1;
#pragma unroll
      for (int round = 0; round < 4; ++round) {
        if (wm == (round >> 1)) {
#pragma unroll
          for (int ii = 0; ii < 2; ++ii) {
            const int i = 2 * (round & 1) + ii;
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int nl = brow0 + 32 * j + 8 * q + 4 * h;
                float4 rs4 = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
                if constexpr (HAS_RS) rs4 = *reinterpret_cast<const float4*>(sc + 1024 + nl * 4);
                float v0 = static_cast<float>(acc[i][j][4 * q]) * lsv[i];
                float v1 = static_cast<float>(acc[i][j][4 * q + 1]) * lsv[i];
                float v2 = static_cast<float>(acc[i][j][4 * q + 2]) * lsv[i];
                float v3 = static_cast<float>(acc[i][j][4 * q + 3]) * lsv[i];
                if constexpr (HAS_RS) {
                  v0 = v0 * rs4.x; v1 = v1 * rs4.y; v2 = v2 * rs4.z; v3 = v3 * rs4.w;
                }
                *reinterpret_cast<uint2*>(stg + (32 * ii + r32) * kEPitch + nl * 2) =
                    make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
                acc[i][j][4 * q] = 0; acc[i][j][4 * q + 1] = 0; acc[i][j][4 * q + 2] = 0; acc[i][j][4 * q + 3] = 0;
              }
          }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        asm volatile("s_barrier" ::: "memory");
#pragma unroll
        for (int it = 0; it < 2048 / THR; ++it) {
          const int c = tid + THR * it, row = c >> 5, seg = c & 31;
          const uint8_t* src = stg + row * kEPitch + 16 * seg;
          const uint2 lo = *reinterpret_cast<const uint2*>(src);
          const uint2 hi = *reinterpret_cast<const uint2*>(src + 8);
          const int ml = 64 * round + row;
          const bool in = n0 + 8 * seg < g.N;
          if constexpr (CDT == RK_BF16) {
            const uint32_t off = in ? static_cast<uint32_t>((ml * g.ldc + 8 * seg) * 2) : 0x80000000u;
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(v4i, make_uint4(lo.x, lo.y, hi.x, hi.y)), c_r,
                static_cast<int>(off), 0, 0);
          } else {
            const uint32_t off = in ? static_cast<uint32_t>((ml * g.ldc + 8 * seg) * 4) : 0x80000000u;
            uint4 w0 = make_uint4(lo.x << 16, lo.x & 0xffff0000u, lo.y << 16, lo.y & 0xffff0000u);
            uint4 w1 = make_uint4(hi.x << 16, hi.x & 0xffff0000u, hi.y << 16, hi.y & 0xffff0000u);
            if (has_r) {
              // C = R + widened bf16, the float add of adding the tensors afterwards (R may
              // be C itself: each thread reads the residual it then overwrites)
              const uint32_t roff = in ? static_cast<uint32_t>((ml * g.ldr + 8 * seg) * 4) : 0x80000000u;
              const float4 r0 = __builtin_bit_cast(
                  float4, __builtin_amdgcn_raw_buffer_load_b128(r_r, static_cast<int>(roff), 0, 0));
              const float4 r1 = __builtin_bit_cast(
                  float4, __builtin_amdgcn_raw_buffer_load_b128(r_r, static_cast<int>(roff + 16u), 0, 0));
              w0.x = __float_as_uint(r0.x + __uint_as_float(w0.x));
              w0.y = __float_as_uint(r0.y + __uint_as_float(w0.y));
              w0.z = __float_as_uint(r0.z + __uint_as_float(w0.z));
              w0.w = __float_as_uint(r0.w + __uint_as_float(w0.w));
              w1.x = __float_as_uint(r1.x + __uint_as_float(w1.x));
              w1.y = __float_as_uint(r1.y + __uint_as_float(w1.y));
              w1.z = __float_as_uint(r1.z + __uint_as_float(w1.z));
              w1.w = __float_as_uint(r1.w + __uint_as_float(w1.w));
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, w0), c_r,
                                                   static_cast<int>(off), 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, w1), c_r,
                                                   static_cast<int>(off + 16u), 0, 0);
          }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): staging reads done
        asm volatile("s_barrier" ::: "memory");
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Small-M kernel (M <= 16 tokens: decode steps): the weight matrix is read once, so the
// kernel is an HBM stream over B. One block = 16 output rows n, its 4 wavefronts split K;
// each wavefront issues its 16-byte loads in batches of 8 (all in flight before the
// first decode), multiplies with v_mfma_i32_16x16x64_i8 (B rows as the first operand:
// lane l then holds token m = l & 15 and outputs n = 4 (l >> 4) .. +3), and the four
// int32 partials are added through LDS (exact, so any order gives the same sum) before
// the same (acc * ls) * rs -> bf16 epilogue. Token rows past M read zeros through the
// descriptor; k-blocks past a wavefront's range re-read its last block (in bounds) and
// skip the MFMA.
// ---------------------------------------------------------------------------
template <int KIND, int CDT, bool HAS_RS>
__global__ __launch_bounds__(256) void int8_gemv_kernel(GemmArgs g) {
  constexpr int NB = 16, KB = 64, W = 4, BATCH = 8;
  __shared__ v4i red[W][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * NB;
  const int64_t rows_b = g.N - n0 < NB ? g.N - n0 : NB;
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_buffer(g.B + n0 * g.ldb, (rows_b - 1) * g.ldb + g.K);
  const __amdgpu_buffer_rsrc_t a_rsrc = make_buffer(g.A, (g.M - 1) * g.lda + g.K);
  const int b_voff = r16 * static_cast<int>(g.ldb) + 16 * g4;
  const int a_voff = r16 * static_cast<int>(g.lda) + 16 * g4;
  const int nkb = static_cast<int>(g.K / KB);
  const int per = (nkb + W - 1) / W;
  const int kb_begin = wave * per;
  const int kb_end = kb_begin + per < nkb ? kb_begin + per : nkb;

  v4i acc = v4i{0, 0, 0, 0};
  for (int kb0 = kb_begin; kb0 < kb_end; kb0 += BATCH) {
    u32x4 bw[BATCH], aw[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int kb = kb0 + j < kb_end ? kb0 + j : kb_end - 1;
      bw[j] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, b_voff, kb * KB, 0));
      aw[j] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_voff, kb * KB, 0));
    }
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      if (kb0 + j < kb_end) {
        u32x4 v = bw[j];
        if constexpr (KIND == B_PACKED) {
          v.x = decode4(v.x, g.mc4);
          v.y = decode4(v.y, g.mc4);
          v.z = decode4(v.z, g.mc4);
          v.w = decode4(v.w, g.mc4);
        }
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, v),
                                                    __builtin_bit_cast(v4i, aw[j]), acc, 0, 0, 0);
      }
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  v4i sum = red[0][lane];
#pragma unroll
  for (int w = 1; w < W; ++w) {
    const v4i t = red[w][lane];
    sum = v4i{sum[0] + t[0], sum[1] + t[1], sum[2] + t[2], sum[3] + t[3]};
  }
  const int m = r16;
  const int64_t n = n0 + 4 * g4;
  if (m >= g.M || n >= g.N) return;
  const float lsm = g.ls[m];
  float v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = static_cast<float>(sum[r]) * lsm;
  if constexpr (HAS_RS) {
    const float4 rs4 = *reinterpret_cast<const float4*>(g.rs + n);
    v[0] = v[0] * rs4.x;
    v[1] = v[1] * rs4.y;
    v[2] = v[2] * rs4.z;
    v[3] = v[3] * rs4.w;
  }
  const uint32_t lo = pack_bf16x2(v[0], v[1]), hi = pack_bf16x2(v[2], v[3]);
  if constexpr (CDT == RK_BF16) {
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(g.C) + m * g.ldc + n) = make_uint2(lo, hi);
  } else {
    *reinterpret_cast<uint4*>(static_cast<float*>(g.C) + m * g.ldc + n) =
        make_uint4(lo << 16, lo & 0xffff0000u, hi << 16, hi & 0xffff0000u);
  }
}

template <int KIND, int CDT, bool HAS_RS>
static void launch_gemv(const GemmArgs& g, hipStream_t stream) {
  const int64_t blocks = (g.N + 15) / 16;
  int8_gemv_kernel<KIND, CDT, HAS_RS><<<dim3(static_cast<unsigned>(blocks)), 256, 0, stream>>>(g);
}

// 256 x 256 tiles for K >= 1024 when they still give every CU a tile, 128 x 128
// otherwise.
static bool use_big_tiles(const GemmArgs& g) {
  const int64_t big = ((g.M + 255) / 256) * ((g.N + 255) / 256);
  return g.K >= 1024 && big >= 256;
}

// Kernel choice for aligned token-sized GEMMs: RATCHET_GEMM_KERNEL=ring forces the
// register-ring kernel, =pipe the persistent LDS-ring kernel (where its shape conditions
// hold); unset or anything else picks by shape.
static int gemm_kernel_override() {
  static const int mode = [] {
    const char* e = getenv("RATCHET_GEMM_KERNEL");
    if (!e) return 0;
    if (strcmp(e, "ring") == 0) return 1;
    if (strcmp(e, "pipe") == 0) return 2;
    return 0;
  }();
  return mode;
}

// The persistent kernel needs K % 64 == 0 and at least 4 k-steps (the scale buffers of two
// tiles are reused every other tile, refilled S - 1 = 2 steps ahead), and output offsets
// well inside 32 bits (stores of columns past N go to an offset past the descriptor).
static bool pipe_supported(const GemmArgs& g, int es) {
  return g.K >= 256 && g.M > 16 && 256 * g.ldc * es <= (int64_t{1} << 30) &&
         (g.R == nullptr || 256 * g.ldr * 4 <= (int64_t{1} << 30));
}

// By shape (MI355X, ring / pipe, us): wide outputs favour the persistent kernel (16384 x
// 8192 x 512 float32: 218.7 / 183.6; 8192 x 8192 x 2048: 207.0 / 191.2; 8192 x 6144 x 2048:
// 131.9 / 128.3), narrow ones the register ring (16384 x 2048 x 512: 34.2 / 36.9;
// grad_input 16384 x 512 x 2048: 25.6 / 37.4).
static bool use_pipe(const GemmArgs& g, int es) {
  if (!pipe_supported(g, es)) return false;
  const int mode = gemm_kernel_override();
  if (mode != 0) return mode == 2;
  const int64_t tiles = ((g.M + kPipeBM - 1) / kPipeBM) * ((g.N + kPipeBN - 1) / kPipeBN);
  return g.N >= 4096 && tiles >= 256;
}

template <int KIND, int CDT, bool HAS_RS>
static void launch_pipe(const GemmArgs& g, hipStream_t stream) {
  PipeSched p{};
  p.tiles_n = static_cast<int>((g.N + kPipeBN - 1) / kPipeBN);
  p.tiles_m = static_cast<int>((g.M + kPipeBM - 1) / kPipeBM);
  p.tiles = p.tiles_m * p.tiles_n;
  p.tiles_per_xcd = (p.tiles + 7) / 8;
  // one 512-thread block per CU (256 CUs), 8 per XCD at least; never more blocks than tiles
  const int per_xcd = p.tiles_per_xcd < 32 ? p.tiles_per_xcd : 32;
  int8_gemm_pipe_kernel<KIND, CDT, HAS_RS><<<dim3(8 * per_xcd), 512, 0, stream>>>(g, p);
}

template <int KIND, int CDT, bool HAS_RS>
static void launch_m32(const GemmArgs& g, hipStream_t stream) {
  if (use_pipe(g, CDT == RK_BF16 ? 2 : 4)) {
    launch_pipe<KIND, CDT, HAS_RS>(g, stream);
    return;
  }
  if (use_big_tiles(g)) {
    const int64_t tiles = ((g.M + 255) / 256) * ((g.N + 255) / 256);
    int8_gemm_m32_kernel<KIND, CDT, HAS_RS, CfgBig>
        <<<dim3(static_cast<unsigned>(tiles)), CfgBig::THREADS, 0, stream>>>(g);
  } else {
    const int64_t tiles = ((g.M + 127) / 128) * ((g.N + 127) / 128);
    int8_gemm_m32_kernel<KIND, CDT, HAS_RS, CfgSmall>
        <<<dim3(static_cast<unsigned>(tiles)), CfgSmall::THREADS, 0, stream>>>(g);
  }
}

template <int KIND, int CDT>
static int launch_gemm(const GemmArgs& g, hipStream_t stream) {
  const bool fast = (g.K % kBK) == 0 && (g.lda % 16) == 0 && (g.ldb % 16) == 0 &&
                    aligned16(g.A) && aligned16(g.B);
  const int es = CDT == RK_BF16 ? 2 : 4;
  const bool aligned_out = fast && (g.N % 8) == 0 && ((g.ldc * es) % 16) == 0 &&
                           aligned16(g.C) && (g.rs == nullptr || aligned16(g.rs));
  // Buffer offsets are 32-bit: a block's furthest A/B load (256 rows, prefetch two
  // k-steps past K) and C store (256 rows) must stay below 2^31 bytes.
  const bool fits32 = 256 * g.lda + g.K + 256 < (int64_t{1} << 31) &&
                      256 * g.ldb + g.K + 256 < (int64_t{1} << 31) &&
                      256 * g.ldc * es < (int64_t{1} << 31);
  if (g.R) {
    // the residual epilogue exists in the 32x32x32 kernel only
    const bool r_ok = CDT == RK_F32 && aligned_out && fits32 && g.M > 16 && aligned16(g.R) &&
                      (g.ldr % 4) == 0 && g.ldr >= g.N && 256 * g.ldr * 4 < (int64_t{1} << 31);
    if (!r_ok)
      return fail(RK_ERR_UNSUPPORTED,
                  "residual GEMM needs float32 output, M > 16, K %% 64 == 0, N %% 8 == 0 and "
                  "16-byte aligned rows");
    if (g.rs) launch_m32<KIND, CDT, true>(g, stream);
    else launch_m32<KIND, CDT, false>(g, stream);
    return launch_status("int8_gemm_residual");
  }
  if (aligned_out && fits32 && g.M <= 16) {
    // decode-sized M: one pass over B spread over the whole chip
    if ((g.N + 15) / 16 > 0x7fffffff) return fail(RK_ERR_ARG, "GEMM grid too large");
    if (g.rs) launch_gemv<KIND, CDT, true>(g, stream);
    else launch_gemv<KIND, CDT, false>(g, stream);
    return launch_status("int8_gemv");
  }
  if (aligned_out && fits32) {
    const int64_t tiles = ((g.M + 127) / 128) * ((g.N + 127) / 128);
    if (tiles > 0x7fffffff) return fail(RK_ERR_ARG, "GEMM grid too large");
    if (g.rs) launch_m32<KIND, CDT, true>(g, stream);
    else launch_m32<KIND, CDT, false>(g, stream);
    return launch_status("int8_gemm");
  }
  const int64_t tiles = ((g.M + kBM - 1) / kBM) * ((g.N + kBN - 1) / kBN);
  if (tiles > 0x7fffffff) return fail(RK_ERR_ARG, "GEMM grid too large");
  const dim3 grid(static_cast<unsigned>(tiles)), block(256);
  if (fast) {
    int8_gemm_nt_kernel<KIND, true, CDT><<<grid, block, 0, stream>>>(g);
  } else {
    int8_gemm_nt_kernel<KIND, false, CDT><<<grid, block, 0, stream>>>(g);
  }
  return launch_status("int8_gemm");
}

// C = (A @ code) * ls * rs with code = decode(packed) as the [K, N] operand: the m32
// kernel only (aligned shapes; RK_ERR_UNSUPPORTED otherwise).
template <int CDT>
static int launch_gemm_packed_t(const GemmArgs& g, hipStream_t stream) {
  const int es = CDT == RK_BF16 ? 2 : 4;
  const bool aligned = (g.K % 64) == 0 && (g.lda % 16) == 0 && (g.ldb % 16) == 0 &&
                       aligned16(g.A) && aligned16(g.B) && (g.N % 8) == 0 &&
                       ((g.ldc * es) % 16) == 0 && aligned16(g.C) &&
                       (g.rs == nullptr || aligned16(g.rs));
  if (!aligned)
    return fail(RK_ERR_UNSUPPORTED,
                "packed [K, N] GEMM needs K %% 64 == 0, N %% 8 == 0 and 16-byte aligned rows");
  // 32-bit buffer offsets: A as in the NT form; B's furthest scalar + vector offset is
  // (K + 2 k-steps) rows of ldb bytes
  const bool fits32 = 256 * g.lda + g.K + 256 < (int64_t{1} << 31) &&
                      (g.K + 128) * g.ldb + 256 < (int64_t{1} << 31) &&
                      256 * g.ldc * es < (int64_t{1} << 31);
  if (!fits32) return fail(RK_ERR_UNSUPPORTED, "packed [K, N] GEMM operands too large");
  const int64_t tiles = ((g.M + 127) / 128) * ((g.N + 127) / 128);
  if (tiles > 0x7fffffff) return fail(RK_ERR_ARG, "GEMM grid too large");
  if (g.rs) launch_m32<B_PACKED_T, CDT, true>(g, stream);
  else launch_m32<B_PACKED_T, CDT, false>(g, stream);
  return launch_status("int8_gemm_packed_t");
}

static int gemm_entry(const int8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, int kind,
                      int max_code, const float* ls, const float* rs, void* C, int c_dtype,
                      int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream,
                      const float* R = nullptr, int64_t ldr = 0) {
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(RK_ERR_ARG, "negative GEMM extent");
  if (c_dtype != RK_F32 && c_dtype != RK_BF16) return fail(RK_ERR_ARG, "bad output dtype");
  // |acc| <= K * 127 * 127 must fit int32.
  if (K > 133144) return fail(RK_ERR_ARG, "K too large for an int32 accumulator");
  if (M == 0 || N == 0) return RK_OK;
  if (!A || !B || !ls || !C) return fail(RK_ERR_ARG, "null GEMM operand");
  if (lda < K || ldb < K || ldc < N) return fail(RK_ERR_ARG, "leading dimension too small");
  if (kind == B_PACKED && (max_code < 1 || max_code > 7))
    return fail(RK_ERR_ARG, "max_code must be in 1..7");
  GemmArgs g{};
  g.A = A;
  g.lda = lda;
  g.B = B;
  g.ldb = ldb;
  g.max_code = max_code;
  g.mc4 = static_cast<uint32_t>(max_code) * 0x01010101u;
  g.ls = ls;
  g.rs = rs;
  g.C = C;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  g.R = R;
  g.ldr = ldr;
  hipStream_t s = as_stream(stream);
  if (kind == B_PACKED) {
    return c_dtype == RK_BF16 ? launch_gemm<B_PACKED, RK_BF16>(g, s)
                              : launch_gemm<B_PACKED, RK_F32>(g, s);
  }
  return c_dtype == RK_BF16 ? launch_gemm<B_INT8, RK_BF16>(g, s)
                            : launch_gemm<B_INT8, RK_F32>(g, s);
}

}  // namespace rk

using namespace rk;

extern "C" int rk_int8_gemm_nt(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                               const float* ls, const float* rs, void* C, int c_dtype,
                               int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream) {
  return gemm_entry(A, lda, reinterpret_cast<const uint8_t*>(B), ldb, B_INT8, 0, ls, rs, C,
                    c_dtype, ldc, M, N, K, stream);
}

extern "C" int rk_int8_gemm_packed(const int8_t* A, int64_t lda, const uint8_t* packed,
                                   int64_t ldp, int max_code, const float* ls, const float* rs,
                                   void* C, int c_dtype, int64_t ldc, int64_t M, int64_t N,
                                   int64_t K, void* stream) {
  return gemm_entry(A, lda, packed, ldp, B_PACKED, max_code, ls, rs, C, c_dtype, ldc, M, N, K,
                    stream);
}

extern "C" int rk_int8_gemm_packed_residual(const int8_t* A, int64_t lda,
                                            const uint8_t* packed, int64_t ldp, int max_code,
                                            const float* ls, const float* rs, const float* R,
                                            int64_t ldr, float* C, int64_t ldc, int64_t M,
                                            int64_t N, int64_t K, void* stream) {
  clear_error();
  if (!R) return fail(RK_ERR_ARG, "null residual");
  if (M > 0 && N > 0 && C) {
    // Each thread reads the residual element it then overwrites, so R may be C itself
    // (same rows, same stride); any other overlap lets one block overwrite rows another
    // block still has to read.
    const char* rb = reinterpret_cast<const char*>(R);
    const char* cb = reinterpret_cast<const char*>(C);
    const bool overlap = rb < cb + ((M - 1) * ldc + N) * int64_t{4} &&
                         cb < rb + ((M - 1) * ldr + N) * int64_t{4};
    if (overlap && !(R == C && ldr == ldc))
      return fail(RK_ERR_ARG, "residual overlaps the output without being the output itself");
  }
  return gemm_entry(A, lda, packed, ldp, B_PACKED, max_code, ls, rs, C, RK_F32, ldc, M, N, K,
                    stream, R, ldr);
}

extern "C" int rk_int8_gemm_packed_t(const int8_t* A, int64_t lda, const uint8_t* packed,
                                     int64_t ldp, int max_code, const float* ls,
                                     const float* rs, void* C, int c_dtype, int64_t ldc,
                                     int64_t M, int64_t N, int64_t K, void* stream) {
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(RK_ERR_ARG, "negative GEMM extent");
  if (c_dtype != RK_F32 && c_dtype != RK_BF16) return fail(RK_ERR_ARG, "bad output dtype");
  if (K > 133144) return fail(RK_ERR_ARG, "K too large for an int32 accumulator");
  if (max_code < 1 || max_code > 7) return fail(RK_ERR_ARG, "max_code must be in 1..7");
  if (M == 0 || N == 0) return RK_OK;
  if (!A || !packed || !ls || !C) return fail(RK_ERR_ARG, "null GEMM operand");
  if (lda < K || ldp < N || ldc < N) return fail(RK_ERR_ARG, "leading dimension too small");
  GemmArgs g{};
  g.A = A;
  g.lda = lda;
  g.B = packed;
  g.ldb = ldp;
  g.max_code = max_code;
  g.mc4 = static_cast<uint32_t>(max_code) * 0x01010101u;
  g.ls = ls;
  g.rs = rs;
  g.C = C;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  hipStream_t s = as_stream(stream);
  return c_dtype == RK_BF16 ? launch_gemm_packed_t<RK_BF16>(g, s)
                            : launch_gemm_packed_t<RK_F32>(g, s);
}
