// Token cross-entropy of the training step, F.cross_entropy(logits, targets) with mean
// reduction and ignore_index (model.py:249, inside the autocast region of train.py:258-259),
// as the two kernels of its forward and the one of its backward.
//
// The arithmetic is torch's log_softmax + nll_loss restated per row of V logits x:
//   m = max_j x_j,  s = sum_j exp(x_j - m),  logsum = log(s),
//   out_j = (x_j - m) - logsum                      (the log-probabilities, never stored)
//   loss_row = -out_t                                (t = the row's target)
//   loss = (sum of loss_row over rows with t != ignore_index) / count
// and for the backward, with g_t = -(grad_loss / count) the nll gradient at the target:
//   grad_j = [j == t] g_t - exp(out_j) * g_t         (log_softmax backward, sum of the
//                                                     row's nll gradient = g_t)
// Rows whose target is ignore_index contribute nothing and get a zero gradient; a target
// outside [0, V) gives a NaN loss (torch raises a device assertion there).
//
//   xent_rows_kernel    one workgroup per row: max, sum of exponentials and the row's
//                       loss; writes (m, logsum, loss_row). Rows of up to 256 * kXentRes
//                       16-byte vectors stay in registers between the two passes.
//   xent_reduce_kernel  one workgroup: the mean over the valid rows in a fixed order.
//   xent_grad_kernel    one workgroup per row: the gradient from (m, logsum), written in
//                       the gradient's dtype (bfloat16 for bfloat16 logits).
//
// Each sum has a fixed association order (per thread in vector order, then the xor
// butterfly of the wavefront, then the four wavefront partials in order), so results repeat
// from run to run. Bytes: the forward reads the logits once, the backward reads them once
// and writes the gradient once; neither writes the [M, V] log-probabilities.
#include "rk_common.h"

#include <math.h>

namespace rk {

constexpr int kXentThreads = 256;
constexpr int kXentRes = 8;  // 16-byte vectors per thread held in registers

struct XentArgs {
  const void* logits;
  int64_t ldl;
  const int64_t* targets;
  int64_t M, V, ignore;
  float* stats;  // [3, M]: row max, log of the row's sum, row loss
};

template <int DT>
__device__ __forceinline__ void widen16(const uint4& raw, float* out) {
  if constexpr (DT == RK_F32) {
    out[0] = __uint_as_float(raw.x);
    out[1] = __uint_as_float(raw.y);
    out[2] = __uint_as_float(raw.z);
    out[3] = __uint_as_float(raw.w);
  } else {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
}

// Block-wide max / sum over the 4 wavefronts of a 256-thread workgroup (every thread gets
// the result). `red` holds 4 floats.
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum_butterfly(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

template <int DT>
__global__ __launch_bounds__(kXentThreads) void xent_rows_kernel(XentArgs a) {
  constexpr int EPV = Vec<DT>::N;            // elements per 16-byte vector
  constexpr int ES = DT == RK_F32 ? 4 : 2;
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const char* x = static_cast<const char*>(a.logits) + row * a.ldl * ES;
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  const int64_t nvec = a.V / EPV;
  const int tid = threadIdx.x;
  const bool resident = nvec <= int64_t{kXentThreads} * kXentRes;

  // pass 1: the row max (registers keep the first kXentRes vectors of each thread)
  uint4 keep[kXentRes];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kXentRes; ++i) {
    const int64_t c = tid + int64_t{kXentThreads} * i;
    keep[i] = c < nvec ? xv[c] : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int i = 0; i < kXentRes; ++i) {
    if (tid + int64_t{kXentThreads} * i < nvec) {
      float e[EPV];
      widen16<DT>(keep[i], e);
#pragma unroll
      for (int j = 0; j < EPV; ++j) m = fmaxf(m, e[j]);
    }
  }
  if (!resident) {
    for (int64_t c = tid + int64_t{kXentThreads} * kXentRes; c < nvec; c += kXentThreads) {
      float e[EPV];
      widen16<DT>(xv[c], e);
#pragma unroll
      for (int j = 0; j < EPV; ++j) m = fmaxf(m, e[j]);
    }
  }
  m = block_max(m, red);

  // pass 2: sum of exp(x - m), in vector order per thread
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < kXentRes; ++i) {
    const int64_t c = tid + int64_t{kXentThreads} * i;
    if (c < nvec) {
      float e[EPV];
      widen16<DT>(keep[i], e);
#pragma unroll
      for (int j = 0; j < EPV; ++j) s = s + expf(e[j] - m);
    }
  }
  if (!resident) {
    for (int64_t c = tid + int64_t{kXentThreads} * kXentRes; c < nvec; c += kXentThreads) {
      float e[EPV];
      widen16<DT>(xv[c], e);
#pragma unroll
      for (int j = 0; j < EPV; ++j) s = s + expf(e[j] - m);
    }
  }
  s = block_sum(s, red);
  if (tid == 0) {
    const float logsum = logf(s);
    const int64_t t = a.targets[row];
    float loss = 0.0f;
    if (t != a.ignore) {
      if (t < 0 || t >= a.V) {
        loss = NAN;
      } else {
        const float xt = DT == RK_F32 ? reinterpret_cast<const float*>(x)[t]
                                      : bf16_to_f32(reinterpret_cast<const uint16_t*>(x)[t]);
        loss = -((xt - m) - logsum);
      }
    }
    a.stats[row] = m;
    a.stats[a.M + row] = logsum;
    a.stats[2 * a.M + row] = loss;
  }
}

// The mean over the rows whose target is not ignore_index: each thread adds its rows
// (tid, tid + 1024, ...) in order, then the xor butterfly per wavefront, then the 16
// wavefront partials in order. out[0] = loss, out[1] = count (as float, torch's
// total_weight).
__global__ __launch_bounds__(1024) void xent_reduce_kernel(XentArgs a, float* loss_out,
                                                           float* count_out) {
  __shared__ float part[16];
  __shared__ int cnt[16];
  const int tid = threadIdx.x;
  float sum = 0.0f;
  int n = 0;
  for (int64_t r = tid; r < a.M; r += 1024) {
    if (a.targets[r] != a.ignore) {
      sum = sum + a.stats[2 * a.M + r];
      ++n;
    }
  }
  sum = wave_sum_butterfly(sum);
  n = wave_sum_int(n);
  if ((tid & 63) == 0) {
    part[tid >> 6] = sum;
    cnt[tid >> 6] = n;
  }
  __syncthreads();
  if (tid == 0) {
    float total = part[0];
    int64_t count = cnt[0];
    for (int w = 1; w < 16; ++w) {
      total = total + part[w];
      count += cnt[w];
    }
    const float c = static_cast<float>(count);
    *loss_out = total / c;
    *count_out = c;
  }
}

struct XentGradArgs {
  XentArgs x;
  const float* grad_loss;  // device scalar
  const float* count;      // device scalar (the forward's count)
  void* grad;
  int64_t ldg;
};

template <int DT, int GDT>
__global__ __launch_bounds__(kXentThreads) void xent_grad_kernel(XentGradArgs g) {
  constexpr int EPV = Vec<DT>::N;
  constexpr int ES = DT == RK_F32 ? 4 : 2;
  constexpr int GES = GDT == RK_F32 ? 4 : 2;
  const XentArgs& a = g.x;
  const int64_t row = blockIdx.x;
  const char* x = static_cast<const char*>(a.logits) + row * a.ldl * ES;
  char* out = static_cast<char*>(g.grad) + row * g.ldg * GES;
  const int64_t nvec = a.V / EPV;
  const int64_t t = a.targets[row];
  const float m = a.stats[row];
  const float logsum = a.stats[a.M + row];
  // nll_loss's gradient at the target (mean reduction), and the row's sum of it
  float gt = 0.0f;
  if (t != a.ignore) gt = (t < 0 || t >= a.V) ? NAN : -(*g.grad_loss / *g.count);
  // four vectors per thread in flight before the first is used
  constexpr int U = 4;
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  for (int64_t c0 = threadIdx.x; c0 < nvec; c0 += int64_t{kXentThreads} * U) {
    uint4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + int64_t{kXentThreads} * u;
      raw[u] = c < nvec ? xv[c] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + int64_t{kXentThreads} * u;
      if (c >= nvec) break;
      float e[EPV];
      widen16<DT>(raw[u], e);
      float r[EPV];
#pragma unroll
      for (int j = 0; j < EPV; ++j) {
        const float p = expf((e[j] - m) - logsum);
        const float go = (c * EPV + j == t) ? gt : 0.0f;
        r[j] = go - p * gt;
      }
      if constexpr (GDT == RK_F32) {
#pragma unroll
        for (int j = 0; j < EPV; j += 4)
          *reinterpret_cast<float4*>(out + (c * EPV + j) * 4) =
              make_float4(r[j], r[j + 1], r[j + 2], r[j + 3]);
      } else if constexpr (EPV == 8) {
        uint4 w;
        w.x = f32_to_bf16(r[0]) | (static_cast<uint32_t>(f32_to_bf16(r[1])) << 16);
        w.y = f32_to_bf16(r[2]) | (static_cast<uint32_t>(f32_to_bf16(r[3])) << 16);
        w.z = f32_to_bf16(r[4]) | (static_cast<uint32_t>(f32_to_bf16(r[5])) << 16);
        w.w = f32_to_bf16(r[6]) | (static_cast<uint32_t>(f32_to_bf16(r[7])) << 16);
        *reinterpret_cast<uint4*>(out + c * EPV * 2) = w;
      } else {
        uint2 w;
        w.x = f32_to_bf16(r[0]) | (static_cast<uint32_t>(f32_to_bf16(r[1])) << 16);
        w.y = f32_to_bf16(r[2]) | (static_cast<uint32_t>(f32_to_bf16(r[3])) << 16);
        *reinterpret_cast<uint2*>(out + c * EPV * 2) = w;
      }
    }
  }
}

static int check_xent(const void* logits, int dtype, int64_t ldl, const int64_t* targets,
                      int64_t M, int64_t V, const float* stats) {
  if (M < 0 || V < 0) return fail(RK_ERR_ARG, "negative size");
  if (dtype != RK_F32 && dtype != RK_BF16) return fail(RK_ERR_ARG, "logits must be float32 or bfloat16");
  if (M > 0x7fffffff) return fail(RK_ERR_ARG, "more than 2^31 - 1 rows");
  if (M == 0) return RK_OK;
  if (!logits || !targets || !stats) return fail(RK_ERR_ARG, "null pointer");
  const int epv = dtype == RK_F32 ? 4 : 8;
  if (V == 0 || V % epv != 0)
    return fail(RK_ERR_UNSUPPORTED, "the class count must be a positive multiple of %d", epv);
  if (ldl < V || (ldl % epv) != 0 || !aligned16(logits))
    return fail(RK_ERR_UNSUPPORTED, "logit rows must be 16-byte aligned and at least V wide");
  return RK_OK;
}

}  // namespace rk

using namespace rk;

extern "C" int rk_cross_entropy_forward(const void* logits, int dtype, int64_t ldl,
                                        const int64_t* targets, int64_t M, int64_t V,
                                        int64_t ignore_index, float* stats, float* loss,
                                        float* count, void* stream) {
  clear_error();
  if (int e = check_xent(logits, dtype, ldl, targets, M, V, stats)) return e;
  if (!loss || !count) return fail(RK_ERR_ARG, "null pointer");
  XentArgs a{logits, ldl, targets, M, V, ignore_index, stats};
  hipStream_t st = as_stream(stream);
  if (M > 0) {
    if (dtype == RK_F32) xent_rows_kernel<RK_F32><<<static_cast<unsigned>(M), kXentThreads, 0, st>>>(a);
    else xent_rows_kernel<RK_BF16><<<static_cast<unsigned>(M), kXentThreads, 0, st>>>(a);
    if (int e = launch_status("cross_entropy rows")) return e;
  }
  xent_reduce_kernel<<<1, 1024, 0, st>>>(a, loss, count);
  return launch_status("cross_entropy reduce");
}

extern "C" int rk_cross_entropy_backward(const void* logits, int dtype, int64_t ldl,
                                         const int64_t* targets, int64_t M, int64_t V,
                                         int64_t ignore_index, const float* stats,
                                         const float* count, const float* grad_loss, void* grad,
                                         int grad_dtype, int64_t ldg, void* stream) {
  clear_error();
  if (int e = check_xent(logits, dtype, ldl, targets, M, V, stats)) return e;
  if (grad_dtype != RK_F32 && grad_dtype != RK_BF16)
    return fail(RK_ERR_ARG, "grad must be float32 or bfloat16");
  if (M == 0) return RK_OK;
  if (!count || !grad_loss || !grad) return fail(RK_ERR_ARG, "null pointer");
  const int gpv = grad_dtype == RK_F32 ? 4 : 8;  // gradient elements per 16 bytes
  if (ldg < V || (ldg % gpv) != 0 || !aligned16(grad))
    return fail(RK_ERR_UNSUPPORTED, "gradient rows must be 16-byte aligned");
  XentGradArgs g{{logits, ldl, targets, M, V, ignore_index, const_cast<float*>(stats)},
                 grad_loss, count, grad, ldg};
  const dim3 grid(static_cast<unsigned>(M));
  hipStream_t st = as_stream(stream);
  if (dtype == RK_F32) {
    if (grad_dtype == RK_F32) xent_grad_kernel<RK_F32, RK_F32><<<grid, kXentThreads, 0, st>>>(g);
    else xent_grad_kernel<RK_F32, RK_BF16><<<grid, kXentThreads, 0, st>>>(g);
  } else {
    if (grad_dtype == RK_F32) xent_grad_kernel<RK_BF16, RK_F32><<<grid, kXentThreads, 0, st>>>(g);
    else xent_grad_kernel<RK_BF16, RK_BF16><<<grid, kXentThreads, 0, st>>>(g);
  }
  return launch_status("cross_entropy backward");
}
