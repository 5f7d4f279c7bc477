// Transposed bf16 MFMA fragments from LDS (gfx950 ds_read_b64_tr_b16), shared by the kernels
// whose contraction runs along the rows of a staged tile (grad_weight: tokens; the lm_head's
// bf16 grad_input: vocabulary rows of the decoded weight).
#pragma once

#include "rk_common.h"

namespace rk {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s* lds_v4s_ptr;

// Fragment of 8 consecutive rows for column `col0 + lane % 32` (rows tok0 + 8 (lane / 32)
// .. +7: the v_mfma_*_32x32x16_bf16 operand layout) from a staged [row][column] bf16 tile of
// PITCH bytes per row. Within each 16-lane group, source lane s points at row (s >> 2),
// columns 4 (s & 3) .. +3, and lane l receives column l of the four rows.
template <int PITCH>
__device__ __forceinline__ v8bf tr16_fragment(const uint8_t* tile, int tok0, int col0, int lane) {
  const int grp = lane >> 4, sl = lane & 15;
  const int row = tok0 + 8 * (grp >> 1) + (sl >> 2);
  const int col = col0 + 16 * (grp & 1) + 4 * (sl & 3);
  const uint8_t* p = tile + row * PITCH + col * 2;
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)(p));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)(p + 4 * PITCH));
  const v4s both[2] = {lo, hi};
  v8bf f;
  __builtin_memcpy(&f, both, sizeof(f));
  return f;
}

}  // namespace rk
