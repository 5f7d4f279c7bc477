// BF16 grad_weight of the ratchet backward on gfx950 (the "TN" product):
//
//   Gw[n, k] = bf16_RNE( sum_m bf16(g[m, n]) * X[m, k] )                 (ratchet.py:159-163)
//
// g is the upstream gradient [M, N] (float32 or bfloat16, row-major). The activation
// operand X [M, K] comes in one of three forms:
//   int8 q + scale s : X = bf16_RNE(bf16(q) * bf16_RNE(s[m]))  (the dequantized saved
//                      activations of the fused int8 forward, ratchet.py:73-75),
//                      dequantized while staging;
//   bfloat16         : X as given (e.g. that dequantized copy, or bf16(inputs) of the
//                      non-fused forward, ratchet.py:161);
//   float32          : X = bf16_RNE(x), converted while staging.
// Both operands are read in their natural token-major layout: no transposed copies are
// made. Tiles are staged in LDS as [BM tokens][128 features] bf16 and the MFMA fragments,
// which need 8 consecutive tokens of one feature per lane, are gathered with gfx950's
// transposing LDS read ds_read_b64_tr_b16: within each 16-lane group, source lane s
// points at token row (s >> 2), features 4 (s & 3) .. +3, and lane l receives feature l
// of the four token rows.
//
// The token (contraction) axis is split into `nsplit` ranges; each block writes fp32
// partial sums of one 128 x 128 output tile for one range, and a second kernel adds the
// ranges in a fixed order and rounds to bf16, so results are reproducible run to run.
#include <mutex>

#include "rk_common.h"
#include "rk_tr16.h"
#include "rk_update_row.h"

namespace rk {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int gw_u32x4 __attribute__((ext_vector_type(4)));

// Forms of the activation operand X.
enum { GW_X_Q8 = 0, GW_X_BF16 = 1, GW_X_F32 = 2 };

struct GwArgs {
  const void* g;
  int64_t ldg;
  // the gradient's columns split over up to three separate [M, part_cols] tensors (row
  // stride ldg), nparts > 0; part_cols is a multiple of the output tile, so one tile's
  // columns lie in one part
  const void* g_parts[3];
  int64_t part_cols;
  int nparts;
  const void* x;    // int8 q, bf16 or f32 activations [M, K]
  int64_t ldx;
  const float* s;   // per-token scale (int8 form only)
  float* part;      // [nsplit][N][K] fp32
  uint16_t* out;    // one split: the bf16 gradient [N, K] (row stride ldo) written directly
  int64_t ldo;
  int64_t M, N, K;
  int64_t m_chunk;  // tokens per split, a multiple of the block's tokens per step
  int nsplit;
  // fused update (rk_grad_weight_update): the update's arguments over these partials, the
  // arrival counters (one per FEAT-row block, then one for the layer) and the arrivals that
  // complete a row block (its column tiles times the splits)
  GradUpdateArgs u;
  int32_t* counters;
  int arrivals;
  float* rms_mean;
};

constexpr int GW_BM = 32;                  // tokens per pipeline step
// LDS row pitch: FEAT * 2 + 64 bytes (320 or 576, 80 or 144 dwords: 16 banks mod 64), so
// consecutive token rows start 16 banks apart. A transposing read serves 32 lanes per pass
// (rows r..r+3, two 32-byte column halves): rows start at banks 0, 16, 32, 48 and the
// second half adds 8, so the eight 8-bank segments are disjoint.
constexpr int kGwMaxRing = 6;

__device__ __forceinline__ uint32_t gw_pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const bf2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// Block configurations: FEAT x FEAT output tiles (n x k) over WN x WK wavefronts, each a
// (FEAT / WN) x (FEAT / WK) wave tile of 32 x 32 MFMA blocks, times TG token groups; staged
// LDS rows of FEAT bf16 features plus 64 bytes (the pitch keeps consecutive token rows 16
// banks apart). With TG = 2 a pipeline step stages 2 x 32 tokens once for two sets of
// WN x WK wavefronts, each set contracting its own 32 tokens; the second set's sums are
// added to the first's through LDS at the end (one fixed add per output), so the block
// covers twice the tokens per split with the same MFMAs per wavefront between barriers.
//  * 128 x 128, 2 x 2 waves x 2 token groups: the op shape and small layers (one 8-wave
//    block per CU: half the split partials of two 4-wave blocks, and each staged tile -
//    its loads, its int8 -> bf16 conversion, its LDS writes - serves 8 wavefronts);
//  * 256 x 256, 2 x 4 waves: large layers. A 128 x 128 bf16 tile fetches 64 bytes of g and
//    X per token step for 1 MFLOP, about the whole L2 bandwidth at the bf16 MFMA peak; the
//    large tile halves the bytes per FLOP.
template <int FEAT_, int WN_, int WK_, int TG_ = 1>
struct GwCfg {
  static constexpr int FEAT = FEAT_, WN = WN_, WK = WK_, TG = TG_;
  static constexpr int THREADS = 64 * WN * WK * TG;
  static constexpr int PITCH = FEAT * 2 + 64;
  static constexpr int MI = FEAT / WN / 32, NJ = FEAT / WK / 32;
};
using GwSmall = GwCfg<128, 2, 2, 2>;
using GwBig = GwCfg<256, 2, 4>;

// A [BM tokens][FEAT features] tile of an operand with ES-byte elements is read as
// 16-byte pieces: FEAT * ES / 16 pieces per token row, 16 / ES elements each, spread over
// the block's THREADS (piece c = tid + THREADS j).
template <int ES, int BM, int FEAT, int THREADS>
struct GwPieces {
  static constexpr int kPerRow = FEAT * ES / 16;
  static constexpr int kElems = 16 / ES;
  static constexpr int kPerThread = BM * FEAT * ES / 16 / THREADS;
  static_assert(kPerThread * THREADS == BM * kPerRow, "whole pieces per thread");
  __device__ static int row(int c) { return c / kPerRow; }
  __device__ static int col(int c) { return (c % kPerRow) * kElems; }
};

// Writes one 16-byte piece of a float32 (4 values) or bfloat16 (8 values) operand into
// the bf16 LDS tile.
template <int ES>
__device__ __forceinline__ void gw_store_piece(uint8_t* dst, const gw_u32x4& v) {
  if constexpr (ES == 4) {
    *reinterpret_cast<uint2*>(dst) =
        make_uint2(gw_pack_bf16x2(__uint_as_float(v.x), __uint_as_float(v.y)),
                   gw_pack_bf16x2(__uint_as_float(v.z), __uint_as_float(v.w)));
  } else {
    *reinterpret_cast<gw_u32x4*>(dst) = v;
  }
}

// Global data of one pipeline step held in registers (ring slot): the g and X tile
// pieces of this thread, and (int8 form) the scales of its X rows.
template <int GV, int XV>
struct GwSlot {
  gw_u32x4 g[GV];
  gw_u32x4 x[XV];
  float s[XV];
};

// mean[0] = mean of row_rms[0 .. rows) by threads 0..255 of the block: each a strided
// partial sum in row order, then a fixed LDS tree (the order of row_rms_mean_kernel).
__device__ __forceinline__ void block_row_rms_mean(const float* row_rms, int64_t rows,
                                                   float* mean) {
  __shared__ float part[256];
  const int t = threadIdx.x;
  if (t < 256) {
    float acc = 0.0f;
    for (int64_t r = t; r < rows; r += 256) acc = acc + row_rms[r];
    part[t] = acc;
  }
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (t < w) part[t] = part[t] + part[t + w];
    __syncthreads();
  }
  if (t == 0) mean[0] = part[0] / static_cast<float>(rows);
}

// UNC < 0: partial sums only, or with BF16OUT (one split) the bf16 gradient itself, rounded
// by the reduce kernel's conversion. UNC >= 0 (rk_grad_weight_update): after writing its partial
// tile, each block publishes it (device-scope release: the XCDs' L2s are not coherent) and
// counts its arrival for its row block; the block that completes a row block acquires and
// runs the fused update (update_row with the split-partial source, UNC chunks in registers)
// on those rows, then resets the row block's counter for the next launch. The block that
// completes the last row block writes the mean row rms the same way.
template <int GDT, int XK, int S, int BM, class CFG, int UNC = -1, bool BF16OUT = false>
__global__ __launch_bounds__(CFG::THREADS) __attribute__((amdgpu_waves_per_eu(2, 8)))
void grad_weight_partial_kernel(GwArgs a) {
  static_assert(!BF16OUT || UNC < 0, "the fused update reads split partials");
  constexpr int GE = GDT == RK_F32 ? 4 : 2;                          // g element bytes
  constexpr int XE = XK == GW_X_Q8 ? 1 : (XK == GW_X_BF16 ? 2 : 4);  // X element bytes
  constexpr int FEAT = CFG::FEAT, THREADS = CFG::THREADS, PITCH = CFG::PITCH;
  constexpr int MI = CFG::MI, NJ = CFG::NJ;
  constexpr int SB = BM * CFG::TG;  // tokens per pipeline step (all token groups)
  using GP = GwPieces<GE, SB, FEAT, THREADS>;
  using XP = GwPieces<XE, SB, FEAT, THREADS>;
  constexpr int GV = GP::kPerThread, XV = XP::kPerThread;
  constexpr int TILE = SB * PITCH;  // one staged operand tile
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 2 * TILE];

  const int64_t tiles_k = (a.K + FEAT - 1) / FEAT;
  const int64_t tiles = ((a.N + FEAT - 1) / FEAT) * tiles_k;
  int64_t b = blockIdx.x;
  const int64_t nb = gridDim.x;
  if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);  // one XCD per token range
  const int split = static_cast<int>(b / tiles);
  const int64_t t = b % tiles;
  const int64_t n0 = (t / tiles_k) * FEAT, k0 = (t % tiles_k) * FEAT;
  const int64_t m_begin = split * a.m_chunk;
  const int64_t m_end = min(a.M, m_begin + a.m_chunk);
  const int steps = m_end > m_begin ? static_cast<int>((m_end - m_begin + SB - 1) / SB) : 0;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tg = wave / (CFG::WN * CFG::WK), wl = wave % (CFG::WN * CFG::WK);  // token group
  const int wn = wl % CFG::WN, wk = wl / CFG::WN;
  const int nw0 = wn * (FEAT / CFG::WN), kw0 = wk * (FEAT / CFG::WK);  // wave tile origin

  // Buffer descriptors over this block's token range. num_records ends at the last valid
  // byte (row m_end - 1, column N - 1 / K - 1), so every load past the range - token rows
  // of padded steps, feature columns past N or K in the last row - returns zeros without
  // a branch or a select. Loads stay unconditional, so the compiler counts outstanding
  // loads exactly and waits only for the ring slot it consumes. Per-thread offsets are
  // fixed; the step advances a scalar offset. The host guarantees offsets < 2^31.
  const int64_t rows = m_end - m_begin;
  const void* gbase = a.g;
  int64_t gcol0 = n0, gcols = a.N;
  if (a.nparts > 0) {
    const int64_t p = n0 / a.part_cols;  // uniform: scalar selects, no indexed kernarg array
    gbase = p == 0 ? a.g_parts[0] : (p == 1 ? a.g_parts[1] : a.g_parts[2]);
    gcol0 = n0 - p * a.part_cols;
    gcols = a.part_cols;
  }
  const __amdgpu_buffer_rsrc_t g_rsrc = make_buffer(
      static_cast<const char*>(gbase) + (m_begin * a.ldg + gcol0) * GE,
      rows > 0 ? ((rows - 1) * a.ldg + (gcols - gcol0)) * GE : 0);
  const __amdgpu_buffer_rsrc_t x_rsrc = make_buffer(
      static_cast<const char*>(a.x) + (m_begin * a.ldx + k0) * XE,
      rows > 0 ? ((rows - 1) * a.ldx + (a.K - k0)) * XE : 0);
  const __amdgpu_buffer_rsrc_t s_rsrc =
      make_buffer(XK == GW_X_Q8 ? a.s + m_begin : a.s, XK == GW_X_Q8 && rows > 0 ? rows * 4 : 0);
  int g_voff[GV], g_lds[GV], x_voff[XV], x_lds[XV], s_voff[XV];
#pragma unroll
  for (int j = 0; j < GV; ++j) {
    const int c = tid + THREADS * j;
    g_voff[j] = (GP::row(c) * static_cast<int>(a.ldg) + GP::col(c)) * GE;
    g_lds[j] = GP::row(c) * PITCH + GP::col(c) * 2;
  }
#pragma unroll
  for (int j = 0; j < XV; ++j) {
    const int c = tid + THREADS * j;
    x_voff[j] = (XP::row(c) * static_cast<int>(a.ldx) + XP::col(c)) * XE;
    x_lds[j] = TILE + XP::row(c) * PITCH + XP::col(c) * 2;
    s_voff[j] = XP::row(c) * 4;
  }
  const int g_step = SB * static_cast<int>(a.ldg) * GE;
  const int x_step = SB * static_cast<int>(a.ldx) * XE;

  auto load_slot = [&](GwSlot<GV, XV>& r, int step) {
#pragma unroll
    for (int j = 0; j < GV; ++j)
      r.g[j] = __builtin_bit_cast(
          gw_u32x4, __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, g_voff[j], step * g_step, 0));
#pragma unroll
    for (int j = 0; j < XV; ++j)
      r.x[j] = __builtin_bit_cast(
          gw_u32x4, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, x_voff[j], step * x_step, 0));
    if constexpr (XK == GW_X_Q8) {
#pragma unroll
      for (int j = 0; j < XV; ++j)
        r.s[j] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(s_rsrc, s_voff[j], step * SB * 4, 0));
    }
  };
  // `tile` is the g tile of one LDS buffer; the X tile follows it.
  auto store_slot = [&](GwSlot<GV, XV>& r, uint8_t* tile) {
    // Pin the slot's registers here: without this the compiler computes the conversions
    // of every slot as soon as its load is issued, which makes it wait for the whole
    // ring instead of the one slot being stored.
#pragma unroll
    for (int j = 0; j < GV; ++j) asm volatile("" : "+v"(r.g[j]));
#pragma unroll
    for (int j = 0; j < XV; ++j) asm volatile("" : "+v"(r.x[j]));
#pragma unroll
    for (int j = 0; j < GV; ++j) gw_store_piece<GE>(tile + g_lds[j], r.g[j]);
    if constexpr (XK == GW_X_Q8) {
      // X = bf16(bf16(q) * bf16(s)): q is exact in bf16, so this is one fp32 multiply of
      // q by the bf16-rounded scale (a positive finite value, so the hardware
      // conversion's round-to-nearest-even is the reference's cast), rounded to bf16.
      // Rows past the range load q = 0 and s = 0.
#pragma unroll
      for (int j = 0; j < XV; ++j) {
        asm volatile("" : "+v"(r.s[j]));
        const float sm = static_cast<float>(static_cast<__bf16>(r.s[j]));
        const uint32_t w[4] = {r.x[j].x, r.x[j].y, r.x[j].z, r.x[j].w};
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
        *reinterpret_cast<gw_u32x4*>(tile + x_lds[j]) = gw_u32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<gw_u32x4*>(tile + x_lds[j] + 16) = gw_u32x4{o[4], o[5], o[6], o[7]};
      }
    } else {
#pragma unroll
      for (int j = 0; j < XV; ++j) gw_store_piece<XE>(tile + x_lds[j], r.x[j]);
    }
  };

  v16f acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = v16f{};

  // Register ring of S steps over an LDS ping-pong, one barrier per step at its top. Step
  // st reads its tiles from buffer st % 2 (staged during step st - 1) and, in the same
  // barrier interval, stages step st + 1 (held in slot (st + 1) % S) into the other buffer,
  // whose last reader was step st - 1, and refills that slot with step st + 1 + S. So one
  // interval holds a step's MFMAs, the next step's staging writes and the loads S steps
  // ahead, and sched_group_barrier interleaves them: the second 16-token half's fragment
  // reads during the first half's MFMAs, the staging writes and the loads during the
  // second half's. The step count is padded to a multiple of S (even, so a slot's LDS
  // buffer is fixed); padded steps stage zeros, and adding +0 products to an accumulator
  // that started at +0 leaves it bit-for-bit unchanged, so no step branches.
  static_assert(S % 2 == 0 && S <= kGwMaxRing, "ring depth must be even and <= 6");
  if (steps > 0) {
    constexpr int U = BM / 16;                // 16-token halves per step
    constexpr int R = (MI + NJ) * 2;          // transposing reads per half
    constexpr int NM = MI * NJ;               // MFMAs per half
    constexpr int DSW = GV + XV * (XK == GW_X_Q8 ? 2 : 1);  // staging writes per step
    constexpr int VM = GV + XV * (XK == GW_X_Q8 ? 2 : 1);   // loads per step
    const int steps_pad = ((steps + S - 1) / S) * S;
    GwSlot<GV, XV> ring[S];
    // Issue the first S steps in slot order (the scheduler barrier keeps them so): the
    // loop body waits for a slot with the later slots still in flight only if its loads
    // are older than theirs on every path into the loop.
#pragma unroll
    for (int i = 0; i < S; ++i) {
      load_slot(ring[i], i);
      __builtin_amdgcn_sched_barrier(0);
    }
    store_slot(ring[0], smem);
    load_slot(ring[0], S);
    for (int st = 0; st < steps_pad; st += S) {
#pragma unroll
      for (int slot = 0; slot < S; ++slot) {
        const int step = st + slot;
        __syncthreads();
        const uint8_t* gt = smem + (slot & 1) * 2 * TILE;
        const uint8_t* xt = gt + TILE;
        v8bf fa[U][MI], fb[U][NJ];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
          for (int i = 0; i < MI; ++i)
            fa[u][i] = tr16_fragment<PITCH>(gt, BM * tg + 16 * u, nw0 + 32 * i, lane);
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            fb[u][j] = tr16_fragment<PITCH>(xt, BM * tg + 16 * u, kw0 + 32 * j, lane);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[u][i], fb[u][j], acc[i][j],
                                                                  0, 0, 0);
        store_slot(ring[(slot + 1) % S], smem + ((slot + 1) & 1) * 2 * TILE);
        load_slot(ring[(slot + 1) % S], step + 1 + S);
        __builtin_amdgcn_sched_group_barrier(0x100, R, 0);  // DS read: the first half
#pragma unroll
        for (int u = 1; u < U; ++u)
#pragma unroll
          for (int k = 0; k < NM; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, (R + NM - 1) / NM, 0);  // DS read
          }
#pragma unroll
        for (int k = 0; k < NM; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x200, (DSW + NM - 1) / NM, 0);  // DS write
          __builtin_amdgcn_sched_group_barrier(0x020, (VM + NM - 1) / NM, 0);   // VMEM read
        }
      }
    }
  }

  if constexpr (CFG::TG == 2) {
    // token group 1 hands its sums to group 0 through the (now idle) LDS tiles: float4
    // (i, j, e / 4) of lane l of wave tile wl at float4 index (wl (MI NJ 4) + (i NJ + j) 4 +
    // e / 4) 64 + l, so each write and read instruction covers 1 KB of consecutive words
    static_assert(4 * MI * NJ * 16 * 64 * 4 <= 2 * 2 * TILE, "exchange fits the LDS tiles");
    float4* xch = reinterpret_cast<float4*>(smem) + wl * (MI * NJ * 4 * 64) + lane;
    __syncthreads();  // every wavefront's last fragment reads are done
    if (tg == 1) {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            xch[((i * NJ + j) * 4 + q) * 64] = make_float4(
                acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
    }
    __syncthreads();
    if (tg == 0) {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 o = xch[((i * NJ + j) * 4 + q) * 64];
            acc[i][j][4 * q] = acc[i][j][4 * q] + o.x;
            acc[i][j][4 * q + 1] = acc[i][j][4 * q + 1] + o.y;
            acc[i][j][4 * q + 2] = acc[i][j][4 * q + 2] + o.z;
            acc[i][j][4 * q + 3] = acc[i][j][4 * q + 3] + o.w;
          }
    }
  }
  // token group 0 holds the block's sums; every wavefront stays for the fused update
  const bool owner = tg == 0;

  // Partial sums: acc[i][j][e] is C[n][k] with k = k0 + kw0 + 32 j + lane % 32 and
  // n = n0 + nw0 + 32 i + 8 (e / 4) + 4 (lane / 32) + e % 4.
  const int lk = lane & 31, lh = lane >> 5;
  if constexpr (BF16OUT) {
    // one split: the sum is complete; round it as grad_weight_reduce_kernel does (the same
    // packed conversion) and store the bf16 gradient, half the bytes of a float32 partial
    if (!owner) return;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t k = k0 + kw0 + 32 * j + lk;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int64_t n = n0 + nw0 + 32 * i + 8 * (e >> 2) + 4 * lh + (e & 3);
          if (n < a.N && k < a.K)
            a.out[n * a.ldo + k] = static_cast<uint16_t>(gw_pack_bf16x2(acc[i][j][e], 0.0f));
        }
      }
    return;
  }
  float* out = a.part + static_cast<int64_t>(split) * a.N * a.K;
  if (owner) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int64_t k = k0 + kw0 + 32 * j + lk;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int64_t n = n0 + nw0 + 32 * i + 8 * (e >> 2) + 4 * lh + (e & 3);
          if (n < a.N && k < a.K) out[n * a.K + k] = acc[i][j][e];
        }
      }
  }

  if constexpr (UNC >= 0) {
    __shared__ int finisher;
    const int64_t rblock = n0 / FEAT;
    const int64_t rblocks = (a.N + FEAT - 1) / FEAT;
    __threadfence();  // this thread's partial stores, device-wide, before the arrival
    __syncthreads();
    if (tid == 0) finisher = atomicAdd(a.counters + rblock, 1) == a.arrivals - 1;
    __syncthreads();
    if (!finisher) return;
    __threadfence();  // acquire: every split's partials of these rows
    MoveCounts cnt;
    const int64_t row_end = n0 + FEAT < a.N ? n0 + FEAT : a.N;
    for (int64_t row = n0 + wave; row < row_end; row += THREADS / 64)
      update_row<SRC_SPLITS, UNC, false>(a.u, row, a.K, cnt);
    flush_counts(cnt, a.u.counts);
    if (tid == 0) a.counters[rblock] = 0;  // every arrival of this launch is in
    if (a.rms_mean) {
      __threadfence();  // this block's row_rms stores, before the layer arrival
      __syncthreads();
      if (tid == 0) finisher = atomicAdd(a.counters + rblocks, 1) == rblocks - 1;
      __syncthreads();
      if (!finisher) return;
      __threadfence();
      block_row_rms_mean(a.u.row_rms, a.N, a.rms_mean);
      if (tid == 0) a.counters[rblocks] = 0;
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

// Ring depth 2 and 32-token steps: ring depths 4 and 6 and 64-token steps (BM = 64, 80 KB
// of LDS) measure the same or slower on MI355X at the op and model shapes.
template <int XK, class CFG, int UNC = -1, bool BF16OUT = false>
void launch_partial_g(const GwArgs& a, int g_dtype, dim3 grid, hipStream_t st) {
  if (g_dtype == RK_F32)
    grad_weight_partial_kernel<RK_F32, XK, 2, GW_BM, CFG, UNC, BF16OUT>
        <<<grid, CFG::THREADS, 0, st>>>(a);
  else
    grad_weight_partial_kernel<RK_BF16, XK, 2, GW_BM, CFG, UNC, BF16OUT>
        <<<grid, CFG::THREADS, 0, st>>>(a);
}

// The fused form: the update's row chunks in registers for rows of up to 512 columns (one
// 512-element chunk), streamed twice otherwise (the partials re-read from cache).
template <int XK, class CFG>
void launch_partial_upd(const GwArgs& a, int g_dtype, dim3 grid, hipStream_t st) {
  if (a.K <= 512) launch_partial_g<XK, CFG, 1>(a, g_dtype, grid, st);
  else launch_partial_g<XK, CFG, 0>(a, g_dtype, grid, st);
}

// The 256 x 256 tile where it still leaves at least 64 output tiles (the op shape's
// 2048 x 512 gradient keeps 128 x 128 tiles and fewer split partials).
static bool gw_big_tiles(int64_t N, int64_t K) {
  return N >= 256 && K >= 256 && ((N + 255) / 256) * ((K + 255) / 256) >= 64;
}

// Shared validation and launch of both entry points; x_kind is a GW_X_* form.
int grad_weight_launch(const void* g, int g_dtype, int64_t ldg, const void* x, int x_kind,
                       int64_t ldx, const float* s, int64_t M, int64_t N, int64_t K,
                       float* workspace, int nsplit, uint16_t* out, int64_t ldo, void* stream,
                       const GradUpdateArgs* upd = nullptr, int32_t* counters = nullptr,
                       float* rms_mean = nullptr, const void* const* g_parts = nullptr,
                       int nparts = 0, int64_t part_cols = 0) {
  if (g_dtype != RK_F32 && g_dtype != RK_BF16) return fail(RK_ERR_ARG, "unsupported gradient dtype");
  if (M < 0 || N < 0 || K < 0) return fail(RK_ERR_ARG, "negative size");
  if (N == 0 || K == 0) return RK_OK;
  // one split with an output needs no workspace: the kernel writes the bf16 gradient itself
  const bool direct = nsplit == 1 && out != nullptr && upd == nullptr;
  if (!g || !x || (x_kind == GW_X_Q8 && !s) || (!workspace && !direct))
    return fail(RK_ERR_ARG, "null pointer");
  if (nsplit < 1 || nsplit > 64) return fail(RK_ERR_ARG, "nsplit must be in 1..64");
  if ((nparts == 0 && ldg < N) || ldx < K || (out && ldo < K))
    return fail(RK_ERR_ARG, "leading dimension too small");
  const int ge = g_dtype == RK_F32 ? 4 : 2;
  const int xe = x_kind == GW_X_Q8 ? 1 : (x_kind == GW_X_BF16 ? 2 : 4);
  if ((N % 8) != 0 || (K % 16) != 0 || ((ldg * ge) % 16) != 0 || ((ldx * xe) % 16) != 0 ||
      (ldo % 4) != 0 || !aligned16(g) || !aligned16(x) || (workspace && !aligned16(workspace)) ||
      (reinterpret_cast<uintptr_t>(out) % 8) != 0)
    return fail(RK_ERR_UNSUPPORTED,
                "grad_weight needs N %% 8 == 0, K %% 16 == 0 and 16-byte aligned rows");
  const bool big = gw_big_tiles(N, K);
  const int64_t feat = big ? GwBig::FEAT : GwSmall::FEAT;
  if (nparts > 0) {
    if (nparts > 3 || part_cols <= 0 || nparts * part_cols != N || part_cols % feat != 0)
      return fail(RK_ERR_UNSUPPORTED,
                  "grad_weight parts: N must be parts x columns, columns a multiple of %lld",
                  static_cast<long long>(feat));
    for (int i = 0; i < nparts; ++i)
      if (!g_parts[i] || !aligned16(g_parts[i]))
        return fail(RK_ERR_ARG, "gradient parts must be non-null and 16-byte aligned");
    if (ldg < part_cols) return fail(RK_ERR_ARG, "leading dimension too small");
  }
  const int64_t tiles = ((N + feat - 1) / feat) * ((K + feat - 1) / feat);
  const int64_t sb = GW_BM * (big ? GwBig::TG : GwSmall::TG);  // tokens per pipeline step
  const int64_t chunk = ((M + nsplit - 1) / nsplit + sb - 1) / sb * sb;
  // Buffer offsets are 32-bit: the furthest load of a block (ring padding and prefetch
  // included) must stay below 2^31 bytes from the block's first row.
  const int64_t reach = chunk + (2 * kGwMaxRing + 1) * sb;
  if (reach * ldg * ge >= (int64_t{1} << 31) || reach * ldx * xe >= (int64_t{1} << 31))
    return fail(RK_ERR_UNSUPPORTED,
                "grad_weight token range too large for 32-bit offsets; raise nsplit");
  GwArgs a{};
  a.g = g;
  a.ldg = ldg;
  a.x = x;
  a.ldx = ldx;
  a.s = s;
  a.part = workspace;
  a.out = out;
  a.ldo = ldo;
  a.M = M;
  a.N = N;
  a.K = K;
  a.m_chunk = chunk > 0 ? chunk : sb;
  a.nsplit = nsplit;
  a.nparts = nparts;
  a.part_cols = part_cols;
  for (int i = 0; i < nparts; ++i) a.g_parts[i] = g_parts[i];
  const int64_t blocks = tiles * nsplit;
  if (blocks > 0x7fffffff) return fail(RK_ERR_ARG, "grid too large");
  hipStream_t st = as_stream(stream);
  const dim3 grid(static_cast<unsigned>(blocks));
  if (upd) {
    // the fused update: the caller's update arguments over these partials
    a.u = *upd;
    a.u.part = workspace;
    a.u.nsplit = nsplit;
    a.u.part_stride = N * K;
    a.u.rows = N;
    a.u.K = K;
    a.counters = counters;
    a.arrivals = static_cast<int>(((K + feat - 1) / feat) * nsplit);
    a.rms_mean = rms_mean;
    if (big) {
      if (x_kind == GW_X_Q8) launch_partial_upd<GW_X_Q8, GwBig>(a, g_dtype, grid, st);
      else if (x_kind == GW_X_BF16) launch_partial_upd<GW_X_BF16, GwBig>(a, g_dtype, grid, st);
      else launch_partial_upd<GW_X_F32, GwBig>(a, g_dtype, grid, st);
    } else {
      if (x_kind == GW_X_Q8) launch_partial_upd<GW_X_Q8, GwSmall>(a, g_dtype, grid, st);
      else if (x_kind == GW_X_BF16) launch_partial_upd<GW_X_BF16, GwSmall>(a, g_dtype, grid, st);
      else launch_partial_upd<GW_X_F32, GwSmall>(a, g_dtype, grid, st);
    }
    return launch_status("grad_weight_update");
  }
  if (direct) {
    if (big) {
      if (x_kind == GW_X_Q8) launch_partial_g<GW_X_Q8, GwBig, -1, true>(a, g_dtype, grid, st);
      else if (x_kind == GW_X_BF16) launch_partial_g<GW_X_BF16, GwBig, -1, true>(a, g_dtype, grid, st);
      else launch_partial_g<GW_X_F32, GwBig, -1, true>(a, g_dtype, grid, st);
    } else {
      if (x_kind == GW_X_Q8) launch_partial_g<GW_X_Q8, GwSmall, -1, true>(a, g_dtype, grid, st);
      else if (x_kind == GW_X_BF16) launch_partial_g<GW_X_BF16, GwSmall, -1, true>(a, g_dtype, grid, st);
      else launch_partial_g<GW_X_F32, GwSmall, -1, true>(a, g_dtype, grid, st);
    }
    return launch_status("grad_weight_bf16");
  }
  if (big) {
    if (x_kind == GW_X_Q8) launch_partial_g<GW_X_Q8, GwBig>(a, g_dtype, grid, st);
    else if (x_kind == GW_X_BF16) launch_partial_g<GW_X_BF16, GwBig>(a, g_dtype, grid, st);
    else launch_partial_g<GW_X_F32, GwBig>(a, g_dtype, grid, st);
  } else {
    if (x_kind == GW_X_Q8) launch_partial_g<GW_X_Q8, GwSmall>(a, g_dtype, grid, st);
    else if (x_kind == GW_X_BF16) launch_partial_g<GW_X_BF16, GwSmall>(a, g_dtype, grid, st);
    else launch_partial_g<GW_X_F32, GwSmall>(a, g_dtype, grid, st);
  }
  if (int e = launch_status("grad_weight_partial")) return e;
  if (!out) return RK_OK;  // partials only (rk_ratchet_update_partials reduces them)
  const int64_t total4 = N * K / 4;
  const int64_t rblocks = (total4 + 255) / 256;
  grad_weight_reduce_kernel<<<static_cast<unsigned>(rblocks < 4096 ? rblocks : 4096), 256, 0, st>>>(
      workspace, nsplit, N, K, out, ldo);
  return launch_status("grad_weight_reduce");
}

// ---------------------------------------------------------------------------
// Allocation-free form (rk_grad_weight_bf16_noalloc): the split partials live in one
// file-scope device array per GPU instead of a caller workspace, for callers that may not
// allocate (code under graph capture, serving loops). Host code never uses the array's name
// as an address: its device address is looked up once per device with hipGetSymbolAddress
// (that device current) and cached. Every call on a GPU shares the array, so calls that
// overlap on one GPU (two streams, two threads) race; each call overwrites every partial it
// reads, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
constexpr int64_t kScratchFloats = int64_t{16} << 20;  // 64 MB of float32 partials
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kScratchFloats];

static float* scratch_address(hipStream_t stream, int& status) {
  static std::mutex mu;
  static float* addr[kMaxDevices] = {};
  int dev = -1;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    status = fail(RK_ERR_ARG, "cannot resolve the stream's device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev]) return addr[dev];
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) {
    status = fail(RK_ERR_LAUNCH, "hipGetDevice failed");
    return nullptr;
  }
  if (cur != dev && hipSetDevice(dev) != hipSuccess) {
    status = fail(RK_ERR_LAUNCH, "hipSetDevice(%d) failed", dev);
    return nullptr;
  }
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (cur != dev) (void)hipSetDevice(cur);
  if (e != hipSuccess || p == nullptr) {
    status = fail(RK_ERR_LAUNCH, "scratch address: %s", hipGetErrorString(e));
    return nullptr;
  }
  addr[dev] = static_cast<float*>(p);
  return addr[dev];
}

}  // namespace rk

using namespace rk;

extern "C" int rk_grad_weight_splits(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 1;
  const bool big = gw_big_tiles(N, K);
  const int64_t feat = big ? GwBig::FEAT : GwSmall::FEAT;
  const int64_t tiles = ((N + feat - 1) / feat) * ((K + feat - 1) / feat);
  // small tiles: at most one 8-wave block per CU (their LDS and registers allow no
  // second), so the splits never make a second, mostly idle round of blocks (48 tiles x 6
  // splits = 288 blocks took twice the time of 5 splits). Large tiles: one split while the
  // tiles alone occupy half the CUs (each further split adds 4 B per weight of partials
  // that the update reads back, which costs more than the idle CUs: measured at the 1B
  // shapes), else about one 8-wave block per CU.
  int64_t splits = big ? (tiles >= 128 ? 1 : (256 + tiles - 1) / tiles) : 256 / tiles;
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
  return grad_weight_launch(g, g_dtype, ldg, q, GW_X_Q8, ldq, s, M, N, K, workspace, nsplit,
                            out, ldo, stream);
}

extern "C" int rk_grad_weight_bf16_parts(const void* g0, const void* g1, const void* g2,
                                         int nparts, int64_t part_cols, int g_dtype, int64_t ldg,
                                         const void* x, int x_dtype, int64_t ldx, const float* s,
                                         int64_t M, int64_t N, int64_t K, float* workspace,
                                         int nsplit, uint16_t* out, int64_t ldo, void* stream) {
  clear_error();
  if (nparts < 1 || nparts > 3) return fail(RK_ERR_ARG, "nparts must be 1, 2 or 3");
  if (x_dtype != RK_F32 && x_dtype != RK_BF16 && x_dtype != RK_I8)
    return fail(RK_ERR_ARG, "unsupported activation dtype");
  const int kind = x_dtype == RK_I8 ? GW_X_Q8 : (x_dtype == RK_BF16 ? GW_X_BF16 : GW_X_F32);
  const void* parts[3] = {g0, g1, g2};
  return grad_weight_launch(g0, g_dtype, ldg, x, kind, ldx, s, M, N, K, workspace, nsplit, out,
                            ldo, stream, nullptr, nullptr, nullptr, parts, nparts, part_cols);
}

extern "C" int rk_grad_weight_bf16_x(const void* g, int g_dtype, int64_t ldg, const void* x,
                                     int x_dtype, int64_t ldx, int64_t M, int64_t N, int64_t K,
                                     float* workspace, int nsplit, uint16_t* out, int64_t ldo,
                                     void* stream) {
  clear_error();
  if (x_dtype != RK_F32 && x_dtype != RK_BF16) return fail(RK_ERR_ARG, "unsupported x dtype");
  return grad_weight_launch(g, g_dtype, ldg, x, x_dtype == RK_F32 ? GW_X_F32 : GW_X_BF16, ldx,
                            nullptr, M, N, K, workspace, nsplit, out, ldo, stream);
}

extern "C" int rk_grad_weight_bf16_noalloc(const void* g, int g_dtype, int64_t ldg,
                                           const int8_t* q, int64_t ldq, const float* s,
                                           int64_t M, int64_t N, int64_t K, int nsplit,
                                           uint16_t* out, int64_t ldo, void* stream) {
  clear_error();
  if (N < 0 || K < 0 || nsplit < 1 || nsplit > 64)
    return fail(RK_ERR_ARG, "nsplit must be in 1..64 and sizes non-negative");
  if (N == 0 || K == 0) return RK_OK;
  if (!out) return fail(RK_ERR_ARG, "null output (the partials are not returned)");
  if (static_cast<int64_t>(nsplit) * N * K > kScratchFloats)
    return fail(RK_ERR_ARG,
                "nsplit * N * K = %lld float32 partials exceed the %lld-float scratch "
                "(use rk_grad_weight_bf16 with a workspace, or fewer splits)",
                static_cast<long long>(static_cast<int64_t>(nsplit) * N * K),
                static_cast<long long>(kScratchFloats));
  int status = RK_OK;
  float* partials = scratch_address(as_stream(stream), status);
  if (!partials) return status;
  return grad_weight_launch(g, g_dtype, ldg, q, GW_X_Q8, ldq, s, M, N, K, partials, nsplit,
                            out, ldo, stream);
}

extern "C" int rk_grad_weight_update(const void* g, int g_dtype, int64_t ldg, const void* x,
                                     int x_dtype, int64_t ldx, const float* s, int64_t M,
                                     int64_t N, int64_t K, float* workspace, int nsplit,
                                     int32_t* counters, uint8_t* packed, int64_t ldp,
                                     int max_code, int threshold, float low, float high,
                                     float eps, float* rms_ema, float beta1, float beta2,
                                     int64_t* counts, float* row_rms, int32_t* nonfinite,
                                     float* rms_mean, uint16_t* grad_out, int64_t ld_grad_out,
                                     void* stream) {
  clear_error();
  if (x_dtype != RK_F32 && x_dtype != RK_BF16 && x_dtype != RK_I8)
    return fail(RK_ERR_ARG, "unsupported activation dtype");
  if (N <= 0 || K <= 0 || M < 0) return fail(RK_ERR_ARG, "invalid shape");
  if (!packed || !counters) return fail(RK_ERR_ARG, "null packed state or counters");
  if (ldp < K) return fail(RK_ERR_ARG, "ldp < K");
  if (max_code < 1 || max_code > 7) return fail(RK_ERR_ARG, "max_code must be in 1..7");
  if (threshold < 1 || threshold > 127)
    return fail(RK_ERR_ARG, "pressure_threshold must be in [1, 127]");
  if (!(low >= 0.0f && low < high))
    return fail(RK_ERR_ARG, "bucket thresholds must satisfy 0 <= low < high");
  if (!(eps > 0.0f)) return fail(RK_ERR_ARG, "eps must be positive");
  if (K % 8 != 0) return fail(RK_ERR_UNSUPPORTED, "the fused update needs K %% 8 == 0");
  if (rms_mean && !row_rms) return fail(RK_ERR_ARG, "rms_mean needs row_rms");
  if (grad_out && (ld_grad_out < K || ld_grad_out % 8 != 0 || !aligned16(grad_out)))
    return fail(RK_ERR_ARG, "grad_out needs ld >= K, ld %% 8 == 0, 16-byte alignment");
  GradUpdateArgs u{};
  u.packed = packed;
  u.ldp = ldp;
  u.g_out = grad_out;
  u.ldgo = ld_grad_out;
  u.mc = max_code;
  u.T = threshold;
  u.low = low;
  u.high = high;
  u.eps = eps;
  u.rms_ema = rms_ema;
  u.beta1 = beta1;
  u.beta2 = beta2;
  u.counts = counts;
  u.row_rms = row_rms;
  u.nonfinite = nonfinite;
  u.vec_p = (reinterpret_cast<uintptr_t>(packed) % 8) == 0 && (ldp % 8) == 0;
  const int kind = x_dtype == RK_I8 ? GW_X_Q8 : (x_dtype == RK_BF16 ? GW_X_BF16 : GW_X_F32);
  return grad_weight_launch(g, g_dtype, ldg, x, kind, ldx, s, M, N, K, workspace, nsplit,
                            nullptr, 0, stream, &u, counters, rms_mean);
}

extern "C" int64_t rk_grad_weight_update_counters(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 1;
  const int64_t feat = gw_big_tiles(N, K) ? GwBig::FEAT : GwSmall::FEAT;
  return (N + feat - 1) / feat + 1;
}
