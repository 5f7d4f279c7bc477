// HBM streaming probe: how many bytes per second a plain hand-written kernel moves on this
// device. It is the measured ceiling the bandwidth-bound kernels of the path (quant, update,
// decode GEMV) are compared against, next to the 8 TB/s published peak.
//
// Each thread streams 16-byte vectors in a grid-stride loop, U loads in flight before the
// first is consumed. Read mode folds every vector into a running XOR that is stored only
// under a condition the host never sets (so the loads stay live); copy mode writes each
// vector back out.
#include "rk_common.h"

namespace rk {

typedef unsigned int vec4u __attribute__((ext_vector_type(4)));

template <int U, bool COPY>
__global__ __launch_bounds__(256) void hbm_stream_kernel(const vec4u* __restrict__ src,
                                                         vec4u* __restrict__ dst, int64_t n16,
                                                         uint32_t never) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  uint32_t acc = 0;
  int64_t i = t0;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    vec4u v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (COPY) {
        dst[i + u * stride] = v[u];
      } else {
        acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
      }
    }
  }
  for (; i < n16; i += stride) {
    const vec4u v = __builtin_nontemporal_load(src + i);
    if constexpr (COPY) dst[i] = v;
    else acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if constexpr (!COPY) {
    if (acc == never && never != 0u) reinterpret_cast<uint32_t*>(dst)[t0] = acc;
  }
}

template <bool COPY>
static void launch_stream(int unroll, const vec4u* src, vec4u* dst, int64_t n16, unsigned blocks,
                          uint32_t never, hipStream_t st) {
  switch (unroll) {
    case 1: hbm_stream_kernel<1, COPY><<<blocks, 256, 0, st>>>(src, dst, n16, never); break;
    case 2: hbm_stream_kernel<2, COPY><<<blocks, 256, 0, st>>>(src, dst, n16, never); break;
    case 4: hbm_stream_kernel<4, COPY><<<blocks, 256, 0, st>>>(src, dst, n16, never); break;
    default: hbm_stream_kernel<8, COPY><<<blocks, 256, 0, st>>>(src, dst, n16, never); break;
  }
}

}  // namespace rk

using namespace rk;

extern "C" int rk_hbm_stream(const void* src, void* dst, int64_t bytes, int copy, int unroll,
                             int blocks, void* stream) {
  clear_error();
  if (!src || !dst) return fail(RK_ERR_ARG, "null pointer");
  if (bytes < 0 || bytes % 16 != 0) return fail(RK_ERR_ARG, "bytes must be a multiple of 16");
  if (!aligned16(src) || !aligned16(dst)) return fail(RK_ERR_ARG, "buffers must be 16-byte aligned");
  if (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8)
    return fail(RK_ERR_ARG, "unroll must be 1, 2, 4 or 8");
  if (blocks < 1 || blocks > 65536) return fail(RK_ERR_ARG, "blocks must be in 1..65536");
  const int64_t n16 = bytes / 16;
  if (n16 == 0) return RK_OK;
  const vec4u* s = static_cast<const vec4u*>(src);
  vec4u* d = static_cast<vec4u*>(dst);
  // read mode writes nothing (`never` is 0); dst must still hold blocks * 256 words
  if (copy) launch_stream<true>(unroll, s, d, n16, static_cast<unsigned>(blocks), 0u, as_stream(stream));
  else launch_stream<false>(unroll, s, d, n16, static_cast<unsigned>(blocks), 0u, as_stream(stream));
  return launch_status("hbm_stream");
}
