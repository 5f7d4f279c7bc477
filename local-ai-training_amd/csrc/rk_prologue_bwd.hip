// Backward of the fused int8 prologues (RMSNorm+quant and tanh-GELU+quant).
//
// rmsnorm_backward, int8_backward.py:7-51, per row of x[M, K] and grad_y[M, K]:
//   variance = sum(x * x) / K;           rsqrt = 1 / sqrt(variance + eps)
//   dx_hat   = grad_y * w;               dvar  = sum(dx_hat * x) * -0.5 * rsqrt^3
//   dx       = dx_hat * rsqrt + dvar * 2 * x / K   -> rounded to bf16, stored in x's dtype
// and grad_w[k] = sum over rows of grad_y * x * rsqrt (float32).
//
// gelu_backward, int8_backward.py:53-89, elementwise:
//   t  = tanh(sqrt(2/pi) * (x + 0.044715 * x * x^2))
//   dx = grad_y * (0.5 * (1 + t) + 0.5 * x * (1 - t^2) * sqrt(2/pi) * (1 + 0.134145 * x^2))
//   -> rounded to bf16, stored in x's dtype. tanh is evaluated as 1 - 2 / (exp(2u) + 1) from
//   the hardware exp2 and reciprocal (absolute error < 3e-7, see tanh_fast).
//
// Both are HBM-bound streams. The RMSNorm kernel keeps a whole row in registers (one
// wavefront per row up to 1024 columns, 2 or 4 wavefronts per row up to 4096; 4 columns
// per lane per 256-column chunk), so x and grad_y are read once, dx is written once, and
// grad_w is accumulated per lane over the block's rows. Each block writes its grad_w partial; a second kernel sums the
// partials in block order, so grad_w is reproducible run to run (no float atomics).
#include "rk_common.h"

namespace rk {
namespace {

constexpr int kBwdV = 4;                   // columns per lane per chunk
constexpr int kBwdSpan = kWave * kBwdV;    // 256 columns per chunk
constexpr int kBwdMaxChunks = 16;          // K <= 4096 on the register-resident path
constexpr int kBwdTargetBlocks = 1024;     // grid size the row split aims for
constexpr int kGeluG = 8;                  // GELU backward: columns per thread

// Valid columns (0..4) of the 4-column group starting at e0 in a row of K.
__device__ __forceinline__ int quad_valid(int64_t K, int64_t e0) {
  const int64_t n = K - e0;
  return n <= 0 ? 0 : (n >= kBwdV ? kBwdV : static_cast<int>(n));
}

// Loads n (0..4) elements at base[idx..], zero-filling the rest; VEC: n == 4 and the
// address is 4-element aligned, so one 16-byte (f32) or 8-byte (bf16) load is used.
template <int DT>
__device__ __forceinline__ void load4(const void* base, int64_t idx, int n, bool vec,
                                      float* v) {
  if (vec && n == 4) {
    if constexpr (DT == RK_F32) {
      const float4 r = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
      v[0] = r.x; v[1] = r.y; v[2] = r.z; v[3] = r.w;
    } else {
      const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + idx);
      v[0] = __uint_as_float(r.x << 16);
      v[1] = __uint_as_float(r.x & 0xffff0000u);
      v[2] = __uint_as_float(r.y << 16);
      v[3] = __uint_as_float(r.y & 0xffff0000u);
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = i < n ? load_elem<DT>(base, idx + i) : 0.0f;
}

// Stores n (0..4) values rounded to bf16, in dtype DT (an f32 destination holds the
// bf16 value widened, as `dx.to(bfloat16)` stored into a float32 buffer).
template <int DT>
__device__ __forceinline__ void store4_bf16(void* base, int64_t idx, int n, bool vec,
                                            const float* v) {
  uint16_t h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) h[i] = f32_to_bf16(v[i]);
  if constexpr (DT == RK_F32) {
    float* p = static_cast<float*>(base) + idx;
    if (vec && n == 4) {
      *reinterpret_cast<float4*>(p) =
          make_float4(bf16_to_f32(h[0]), bf16_to_f32(h[1]), bf16_to_f32(h[2]), bf16_to_f32(h[3]));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < n) p[i] = bf16_to_f32(h[i]);
    }
  } else {
    uint16_t* p = static_cast<uint16_t*>(base) + idx;
    if (vec && n == 4) {
      *reinterpret_cast<uint2*>(p) = make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16),
                                                h[2] | (static_cast<uint32_t>(h[3]) << 16));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < n) p[i] = h[i];
    }
  }
}

struct NormBwdArgs {
  const void* gy;
  int64_t ldg;
  const void* x;
  int64_t ldx;
  const float* w;
  float eps;
  int64_t M, K;
  void* gx;
  int64_t ldgx;
  float* part;             // [gridDim.x][K] grad_w partial of each block
  int64_t rows_per_block;  // a multiple of 4
  int vec;                 // 4-element vector access is legal for x, grad_y, grad_x and w
  const float* add;        // float32 x only: grad_x = float32(bf16(dx)) + add (may be grad_x)
  int64_t lda;
};

// One row's x, grad_y and (float32 x with a residual gradient) the residual gradient from
// column c0 on, all requested before any is used.
template <int GDT, int XDT, int NC>
__device__ __forceinline__ void norm_load_row(const NormBwdArgs& a, int64_t row, int lane,
                                              int64_t c0, float (&xv)[NC][kBwdV],
                                              float (&gv)[NC][kBwdV], float (&av)[NC][kBwdV]) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t e0 = c0 + c * kBwdSpan + lane * kBwdV;
    const int n = quad_valid(a.K, e0);
    load4<XDT>(a.x, row * a.ldx + e0, n, a.vec, xv[c]);
    load4<GDT>(a.gy, row * a.ldg + e0, n, a.vec, gv[c]);
    if constexpr (XDT == RK_F32) {
      if (a.add) load4<RK_F32>(a.add, row * a.lda + e0, n, a.vec, av[c]);
    }
  }
}

// One block = 4 wavefronts over rows [blockIdx.x * rows_per_block, +rows_per_block). P
// wavefronts share a row (P = 1, 2 or 4), each holding NC 256-column chunks of it: wave w
// takes column slice w % P of rows w / P, w / P + 4 / P, ... With P > 1 the slices' sums of
// squares and of grad_y * w * x meet in LDS (one barrier per row step; the slices are added
// in slice order) and every slice finishes its own columns. Long rows so keep NC <= 4: the
// next row's loads are issued before the current row's reductions (PREFETCH) without
// lowering the occupancy, and there are enough rows in flight per CU to stream HBM.
template <int GDT, int XDT, int NC, bool PREFETCH, int P>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(NormBwdArgs a) {
  constexpr int G = 4 / P;                 // rows per block step
  constexpr int COLS = P * NC * kBwdSpan;  // columns one row step covers
  __shared__ __attribute__((aligned(16))) float red[G][COLS];
  __shared__ float sums[2][4][2];          // [step parity][wave] (sum x*x, sum g*w*x)
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int slice = wave % P, grp = wave / P;
  const int64_t c0 = static_cast<int64_t>(slice) * NC * kBwdSpan;  // the slice's first column
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * a.rows_per_block;
  const int64_t r1 = r0 + a.rows_per_block < a.M ? r0 + a.rows_per_block : a.M;
  const float kf = static_cast<float>(a.K);

  float wv[NC][kBwdV], gw[NC][kBwdV];
  int nv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t e0 = c0 + c * kBwdSpan + lane * kBwdV;
    nv[c] = quad_valid(a.K, e0);
    load4<RK_F32>(a.w, e0, nv[c], a.vec, wv[c]);
#pragma unroll
    for (int i = 0; i < kBwdV; ++i) gw[c][i] = 0.0f;
  }

  // the same step count in every wavefront of the block (the LDS exchange has a barrier)
  const int steps = static_cast<int>((r1 - r0 + G - 1) / G);
  int64_t row = r0 + grp;
  float xv[NC][kBwdV], gv[NC][kBwdV], av[NC][kBwdV];
  if (row < r1) norm_load_row<GDT, XDT, NC>(a, row, lane, c0, xv, gv, av);
  for (int st = 0; st < steps; ++st) {
    const bool valid = row < r1;  // uniform in the wavefront
    const int64_t next = row + G;
    float xn[NC][kBwdV], gn[NC][kBwdV], an[NC][kBwdV];
    if constexpr (PREFETCH) {
      if (next < r1) norm_load_row<GDT, XDT, NC>(a, next, lane, c0, xn, gn, an);
    }
    float sxx = 0.0f, sgx = 0.0f;
    if (valid) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int i = 0; i < kBwdV; ++i) {
          sxx = sxx + xv[c][i] * xv[c][i];
          sgx = sgx + (gv[c][i] * wv[c][i]) * xv[c][i];
        }
    }
    sxx = wave_sum_butterfly(sxx);
    sgx = wave_sum_butterfly(sgx);
    if constexpr (P > 1) {
      // two parity buffers: a slot is rewritten two steps later, after the next step's
      // barrier, which every wavefront reaches only once it has read this step's sums
      if (lane == 0) {
        sums[st & 1][wave][0] = sxx;
        sums[st & 1][wave][1] = sgx;
      }
      __syncthreads();
      sxx = sums[st & 1][grp * P][0];
      sgx = sums[st & 1][grp * P][1];
#pragma unroll
      for (int q = 1; q < P; ++q) {
        sxx = sxx + sums[st & 1][grp * P + q][0];
        sgx = sgx + sums[st & 1][grp * P + q][1];
      }
    }
    if (valid) {
      const float rs = 1.0f / sqrtf(sxx / kf + a.eps);
      const float dvar = sgx * -0.5f * (rs * rs * rs);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float dx[kBwdV];
#pragma unroll
        for (int i = 0; i < kBwdV; ++i) {
          dx[i] = (gv[c][i] * wv[c][i]) * rs + dvar * 2.0f * xv[c][i] / kf;
          gw[c][i] = gw[c][i] + gv[c][i] * xv[c][i] * rs;
        }
        const int64_t e0 = c0 + c * kBwdSpan + lane * kBwdV;
        if constexpr (XDT == RK_F32) {
          if (a.add && nv[c] > 0) {
            // the residual stream's gradient joins here: one float32 add of the two
            // contributions, the add autograd performs where x feeds both paths
#pragma unroll
            for (int i = 0; i < kBwdV; ++i) dx[i] = round_bf16(dx[i]) + av[c][i];
            float* p = static_cast<float*>(a.gx) + row * a.ldgx + e0;
            if (a.vec && nv[c] == 4) {
              *reinterpret_cast<float4*>(p) = make_float4(dx[0], dx[1], dx[2], dx[3]);
            } else {
#pragma unroll
              for (int i = 0; i < kBwdV; ++i)
                if (i < nv[c]) p[i] = dx[i];
            }
            continue;
          }
        }
        if (nv[c] > 0) store4_bf16<XDT>(a.gx, row * a.ldgx + e0, nv[c], a.vec, dx);
      }
    }
    if constexpr (PREFETCH) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int i = 0; i < kBwdV; ++i) {
          xv[c][i] = xn[c][i];
          gv[c][i] = gn[c][i];
          av[c][i] = an[c][i];
        }
    } else {
      if (next < r1) norm_load_row<GDT, XDT, NC>(a, next, lane, c0, xv, gv, av);
    }
    row = next;
  }

  // Block partial: the row groups' column sums, added in group order.
#pragma unroll
  for (int c = 0; c < NC; ++c)
    *reinterpret_cast<float4*>(&red[grp][c0 + c * kBwdSpan + lane * kBwdV]) =
        make_float4(gw[c][0], gw[c][1], gw[c][2], gw[c][3]);
  __syncthreads();
  float* out = a.part + static_cast<int64_t>(blockIdx.x) * a.K;
  for (int64_t col = threadIdx.x; col < a.K; col += 256) {
    float t = red[0][col];
#pragma unroll
    for (int q = 1; q < G; ++q) t = t + red[q][col];
    out[col] = t;
  }
}

// grad_w[k] = sum of part[p][k] over p: 16 columns x 16 part-groups per block; group g
// sums parts g, g + 16, ... and the 16 group sums are then added in group order.
__global__ __launch_bounds__(256) void rmsnorm_gw_reduce_kernel(const float* part,
                                                                int64_t nparts, int64_t K,
                                                                float* gw) {
  __shared__ float s[16][17];
  const int cl = threadIdx.x & 15, g = threadIdx.x >> 4;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 16 + cl;
  float acc = 0.0f;
  if (col < K) {
#pragma unroll 8
    for (int64_t p = g; p < nparts; p += 16) acc = acc + part[p * K + col];
  }
  s[g][cl] = acc;
  __syncthreads();
  if (threadIdx.x < 16 && col < K) {
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t = t + s[i][threadIdx.x];
    gw[col] = t;
  }
}

struct GeluBwdArgs {
  const void* gy;
  int64_t ldg;
  const void* x;
  int64_t ldx;
  void* gx;
  int64_t ldgx;
  int64_t M, K;
  int64_t groups;  // ceil(K / kGeluG) column groups per row
  int vec;         // 4-element vector access is legal for x, grad_y and grad_x
  int vec8;        // ... and every 8-column group starts 16-byte aligned
};

// 8 elements at a 16-byte aligned address, widened to float32.
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t idx, float* v) {
  if constexpr (DT == RK_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + idx);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
}

// The derivative of the tanh-GELU, evaluated in the operation order of
// int8_backward.py:65-72. It uses t only through 0.5 (1 + t) and 1 - t^2, where tanh_fast's
// absolute error is below a millionth of the result, far under the bf16 rounding of dx.
__device__ __forceinline__ float gelu_tanh_grad(float x) {
  const float k = 0.7978845608028654f;
  const float x_sq = x * x;
  const float inner = k * (x + 0.044715f * x * x_sq);
  const float t = tanh_fast(inner);
  const float term1 = 0.5f * (1.0f + t);
  const float term2 = 0.5f * x * (1.0f - t * t) * k * (1.0f + 0.134145f * x_sq);
  return term1 + term2;
}

// One thread = kGeluG consecutive columns of one row (two 4-column groups: 16-byte bf16 or
// 2 x 16-byte float32 accesses); grid-stride over M * groups.
template <int GDT, int XDT>
__global__ __launch_bounds__(256) void gelu_bwd_kernel(GeluBwdArgs a) {
  const int64_t total = a.M * a.groups;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += stride) {
    const int64_t row = u / a.groups;
    const int64_t e0 = (u - row * a.groups) * kGeluG;
    if (a.vec8) {
      float xv[kGeluG], gv[kGeluG], dx[kGeluG];
      load8<XDT>(a.x, row * a.ldx + e0, xv);
      load8<GDT>(a.gy, row * a.ldg + e0, gv);
#pragma unroll
      for (int i = 0; i < kGeluG; ++i) dx[i] = gv[i] * gelu_tanh_grad(xv[i]);
      store4_bf16<XDT>(a.gx, row * a.ldgx + e0, kBwdV, true, dx);
      store4_bf16<XDT>(a.gx, row * a.ldgx + e0 + kBwdV, kBwdV, true, dx + kBwdV);
      continue;
    }
    float xv[2][kBwdV], gv[2][kBwdV];
    int n[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      n[h] = quad_valid(a.K, e0 + h * kBwdV);
      load4<XDT>(a.x, row * a.ldx + e0 + h * kBwdV, n[h], a.vec, xv[h]);
      load4<GDT>(a.gy, row * a.ldg + e0 + h * kBwdV, n[h], a.vec, gv[h]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float dx[kBwdV];
#pragma unroll
      for (int i = 0; i < kBwdV; ++i) dx[i] = gv[h][i] * gelu_tanh_grad(xv[h][i]);
      if (n[h] > 0) store4_bf16<XDT>(a.gx, row * a.ldgx + e0 + h * kBwdV, n[h], a.vec, dx);
    }
  }
}

bool vec4_ok(const void* p, int dt, int64_t ld, int64_t K) {
  const uintptr_t align = static_cast<uintptr_t>(dtype_size(dt)) * 4;
  return (reinterpret_cast<uintptr_t>(p) % align) == 0 && ld % 4 == 0 && K % 4 == 0;
}

// Rows of up to 512 columns: one wavefront per row; longer rows: 2 or 4 wavefronts per row
// with at most 2 chunks each up to 2048 columns, 4 beyond. (K = 2048 with one wavefront per
// row and 8 chunks held 253 VGPRs, so no prefetch and one wavefront per SIMD: 80 us for
// 8192 rows of float32 x, grad_y and residual gradient, 3.4 TB/s.)
template <int GDT, int XDT>
int launch_norm(const NormBwdArgs& a, dim3 grid, hipStream_t st) {
  const int64_t nc = (a.K + kBwdSpan - 1) / kBwdSpan;
  if (nc <= 1) rmsnorm_bwd_kernel<GDT, XDT, 1, true, 1><<<grid, dim3(256), 0, st>>>(a);
  else if (nc <= 2) rmsnorm_bwd_kernel<GDT, XDT, 2, true, 1><<<grid, dim3(256), 0, st>>>(a);
  else if (nc <= 4) rmsnorm_bwd_kernel<GDT, XDT, 2, true, 2><<<grid, dim3(256), 0, st>>>(a);
  else if (nc <= 8) rmsnorm_bwd_kernel<GDT, XDT, 2, true, 4><<<grid, dim3(256), 0, st>>>(a);
  else rmsnorm_bwd_kernel<GDT, XDT, 4, true, 4><<<grid, dim3(256), 0, st>>>(a);
  return launch_status("rmsnorm_backward");
}

int64_t norm_rows_per_block(int64_t M) {
  const int64_t per = (M + kBwdTargetBlocks - 1) / kBwdTargetBlocks;
  return ((per + 3) / 4) * 4;
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" int rk_rmsnorm_backward_parts(int64_t M) {
  if (M <= 0) return 0;
  const int64_t rpb = norm_rows_per_block(M);
  return static_cast<int>((M + rpb - 1) / rpb);  // <= kBwdTargetBlocks
}

static int rmsnorm_backward_entry(const void* grad_y, int gy_dtype, int64_t ldg, const void* x,
                                  int x_dtype, int64_t ldx, const float* w, float eps, int64_t M,
                                  int64_t K, const float* add, int64_t lda, void* grad_x,
                                  int64_t ldgx, float* grad_w, float* workspace,
                                  int64_t workspace_floats, void* stream) {
  clear_error();
  if (M < 0 || K < 0) return fail(RK_ERR_ARG, "negative size M=%lld K=%lld", (long long)M,
                                  (long long)K);
  if (dtype_size(gy_dtype) == 0 || dtype_size(x_dtype) == 0)
    return fail(RK_ERR_ARG, "grad_y/x dtype must be RK_F32 or RK_BF16");
  if (K > static_cast<int64_t>(kBwdMaxChunks) * kBwdSpan)
    return fail(RK_ERR_UNSUPPORTED, "rmsnorm_backward supports K <= %d (got %lld)",
                kBwdMaxChunks * kBwdSpan, (long long)K);
  if (K == 0) return RK_OK;
  if (!grad_w || !w) return fail(RK_ERR_ARG, "null w or grad_w");
  hipStream_t st = as_stream(stream);
  const dim3 reduce_grid(static_cast<unsigned>((K + 15) / 16));
  if (M == 0) {  // grad_w = 0: the reduce over zero partials writes zeros
    rmsnorm_gw_reduce_kernel<<<reduce_grid, dim3(256), 0, st>>>(nullptr, 0, K, grad_w);
    return launch_status("rmsnorm_backward_reduce");
  }
  if (!grad_y || !x || !grad_x || !workspace) return fail(RK_ERR_ARG, "null pointer");
  if (ldg < K || ldx < K || ldgx < K) return fail(RK_ERR_ARG, "leading dimension below K");
  const int64_t nparts = rk_rmsnorm_backward_parts(M);
  if (workspace_floats < nparts * K)
    return fail(RK_ERR_ARG, "workspace holds %lld floats, needs %lld",
                (long long)workspace_floats, (long long)(nparts * K));
  if (add && lda < K) return fail(RK_ERR_ARG, "leading dimension below K");
  NormBwdArgs a{};
  a.gy = grad_y; a.ldg = ldg; a.x = x; a.ldx = ldx; a.w = w; a.eps = eps;
  a.M = M; a.K = K; a.gx = grad_x; a.ldgx = ldgx; a.part = workspace;
  a.add = add; a.lda = lda;
  a.rows_per_block = norm_rows_per_block(M);
  a.vec = vec4_ok(grad_y, gy_dtype, ldg, K) && vec4_ok(x, x_dtype, ldx, K) &&
          vec4_ok(grad_x, x_dtype, ldgx, K) && vec4_ok(w, RK_F32, K, K) &&
          (!add || vec4_ok(add, RK_F32, lda, K));
  const dim3 grid(static_cast<unsigned>(nparts));
  int e;
  if (gy_dtype == RK_F32) {
    e = x_dtype == RK_F32 ? launch_norm<RK_F32, RK_F32>(a, grid, st)
                          : launch_norm<RK_F32, RK_BF16>(a, grid, st);
  } else {
    e = x_dtype == RK_F32 ? launch_norm<RK_BF16, RK_F32>(a, grid, st)
                          : launch_norm<RK_BF16, RK_BF16>(a, grid, st);
  }
  if (e) return e;
  rmsnorm_gw_reduce_kernel<<<reduce_grid, dim3(256), 0, st>>>(workspace, nparts, K, grad_w);
  return launch_status("rmsnorm_backward_reduce");
}

extern "C" int rk_rmsnorm_backward(const void* grad_y, int gy_dtype, int64_t ldg, const void* x,
                                   int x_dtype, int64_t ldx, const float* w, float eps, int64_t M,
                                   int64_t K, void* grad_x, int64_t ldgx, float* grad_w,
                                   float* workspace, int64_t workspace_floats, void* stream) {
  return rmsnorm_backward_entry(grad_y, gy_dtype, ldg, x, x_dtype, ldx, w, eps, M, K, nullptr, 0,
                                grad_x, ldgx, grad_w, workspace, workspace_floats, stream);
}

extern "C" int rk_rmsnorm_backward_residual(const void* grad_y, int gy_dtype, int64_t ldg,
                                            const float* x, int64_t ldx, const float* w, float eps,
                                            int64_t M, int64_t K, const float* residual_grad,
                                            int64_t ldr, float* grad_x, int64_t ldgx,
                                            float* grad_w, float* workspace,
                                            int64_t workspace_floats, void* stream) {
  if (M > 0 && K > 0 && !residual_grad) {
    clear_error();
    return fail(RK_ERR_ARG, "null residual gradient");
  }
  if (residual_grad && residual_grad != grad_x) {
    // any overlap other than the same rows in place would let one row's store reach
    // another row's unread residual gradient
    const char* r0 = reinterpret_cast<const char*>(residual_grad);
    const char* r1 = r0 + ((M > 0 ? M - 1 : 0) * ldr + K) * 4;
    const char* g0 = reinterpret_cast<const char*>(grad_x);
    const char* g1 = g0 + ((M > 0 ? M - 1 : 0) * ldgx + K) * 4;
    if (M > 0 && K > 0 && r0 < g1 && g0 < r1) {
      clear_error();
      return fail(RK_ERR_ARG, "residual gradient partly overlaps grad_x");
    }
  } else if (residual_grad && ldr != ldgx) {
    clear_error();
    return fail(RK_ERR_ARG, "in place needs the same row stride");
  }
  return rmsnorm_backward_entry(grad_y, gy_dtype, ldg, x, RK_F32, ldx, w, eps, M, K,
                                residual_grad, ldr, grad_x, ldgx, grad_w, workspace,
                                workspace_floats, stream);
}

extern "C" int rk_gelu_backward(const void* grad_y, int gy_dtype, int64_t ldg, const void* x,
                                int x_dtype, int64_t ldx, int64_t M, int64_t K, void* grad_x,
                                int64_t ldgx, void* stream) {
  clear_error();
  if (M < 0 || K < 0) return fail(RK_ERR_ARG, "negative size M=%lld K=%lld", (long long)M,
                                  (long long)K);
  if (dtype_size(gy_dtype) == 0 || dtype_size(x_dtype) == 0)
    return fail(RK_ERR_ARG, "grad_y/x dtype must be RK_F32 or RK_BF16");
  if (M == 0 || K == 0) return RK_OK;
  if (!grad_y || !x || !grad_x) return fail(RK_ERR_ARG, "null pointer");
  if (ldg < K || ldx < K || ldgx < K) return fail(RK_ERR_ARG, "leading dimension below K");
  GeluBwdArgs a{};
  a.gy = grad_y; a.ldg = ldg; a.x = x; a.ldx = ldx; a.gx = grad_x; a.ldgx = ldgx;
  a.M = M; a.K = K; a.groups = (K + kGeluG - 1) / kGeluG;
  a.vec = vec4_ok(grad_y, gy_dtype, ldg, K) && vec4_ok(x, x_dtype, ldx, K) &&
          vec4_ok(grad_x, x_dtype, ldgx, K);
  a.vec8 = a.vec && K % kGeluG == 0 && ldg % kGeluG == 0 && ldx % kGeluG == 0 &&
           ldgx % kGeluG == 0 && aligned16(grad_y) && aligned16(x) && aligned16(grad_x);
  const int64_t total = M * a.groups;
  const int64_t want = (total + 255) / 256;
  const int64_t blocks = want < (int64_t{1} << 20) ? want : (int64_t{1} << 20);
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  hipStream_t st = as_stream(stream);
  if (gy_dtype == RK_F32) {
    if (x_dtype == RK_F32) gelu_bwd_kernel<RK_F32, RK_F32><<<grid, block, 0, st>>>(a);
    else gelu_bwd_kernel<RK_F32, RK_BF16><<<grid, block, 0, st>>>(a);
  } else {
    if (x_dtype == RK_F32) gelu_bwd_kernel<RK_BF16, RK_F32><<<grid, block, 0, st>>>(a);
    else gelu_bwd_kernel<RK_BF16, RK_BF16><<<grid, block, 0, st>>>(a);
  }
  return launch_status("gelu_backward");
}
