// The 32x32x32 int8 MFMA step shared by the int8 GEMM kernels: fragment layout, the LDS
// tile layouts it reads and one 64-byte k-step of v_mfma_i32_32x32x32_i8 over them.
#pragma once

#include "rk_common.h"

namespace rk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two fp32 values -> packed bf16 pair (low half = lo), round-to-nearest-even.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// ---------------------------------------------------------------------------
// The 32x32x32 form issues half as many MFMAs per MAC as 16x16x64 and sustained
// 4.3-4.5 POP/s in register-resident MFMA chains on MI355X (16x16x64: at most ~3.4).
// Fragment layout: lane l holds row (l & 31), k bytes 16 (l >> 5) .. +15 of a 32-byte
// k half. LDS rows are 64 bytes with the 16-byte segment XOR-swizzled by
// (row >> 2) & 3, which keeps these 32-row fragment reads free of bank conflicts.
// Operands are swapped (B rows feed the MFMA's first operand) so the accumulator gives
// each lane 4 consecutive output columns n for one row m:
//   acc[e], e = 0..15: n = 8 (e / 4) + 4 (l >> 5) + (e % 4), m = l & 31.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swz32(int row) { return (row >> 2) & 3; }

// B_PACKED_T tiles are staged as they lie in memory, [64 k rows][BN n bytes] at a
// BN + 32 byte pitch (eight consecutive rows then cover all 64 banks), and the fragments
// (16 consecutive k of one column n per lane) come from gfx950's transposing LDS read
// ds_read_b64_tr_b8: within each 16-lane group, source lane s points at row s >> 1,
// bytes 8 (s & 1) .. +7, and lane l receives byte column l of the eight rows, in row
// order (checked on the device).
typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i_t* lds_v2i_ptr;

template <bool BT, int MI, int NJ, int BTP>
__device__ __forceinline__ void mfma32_step(v16i (&acc)[MI][NJ], const uint8_t* at,
                                            const uint8_t* bt, int arow0, int brow0, int lane) {
  const int r32 = lane & 31, h = lane >> 5;
  // one 32-byte k half at a time: MI + NJ fragments live, MI * NJ MFMAs each
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
      if constexpr (BT) {
        const int sl = lane & 15;
        const int col = brow0 + j * 32 + 16 * ((lane >> 4) & 1) + 8 * (sl & 1);
        const int r0 = 16 * (h + 2 * kh) + (sl >> 1);
        const v2i_t lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (lds_v2i_ptr)(bt + r0 * BTP + col));
        const v2i_t hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (lds_v2i_ptr)(bt + (r0 + 8) * BTP + col));
        fb[j] = v4i{lo.x, lo.y, hi.x, hi.y};
      } else {
        const int rb = brow0 + j * 32 + r32;
        fb[j] = *reinterpret_cast<const v4i*>(bt + rb * 64 + 16 * ((h + 2 * kh) ^ swz32(rb)));
      }
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[j], fa[i], acc[i][j], 0, 0, 0);
  }
}

}  // namespace rk
