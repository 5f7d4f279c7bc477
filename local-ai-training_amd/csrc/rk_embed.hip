// Token-embedding weight gradient, the backward of the model's lookup
// `self.token_embedding(tokens)` (model.py:237, an nn.Embedding per model.py:219):
// grad_weight[v, :] = sum over the tokens t with ids[t] == v of grad[t, :], in float32, in a
// fixed order that does not depend on the launch.
//
// Order: tokens are cut into chunks of kEmbChunk consecutive positions. Within a chunk the
// rows of one id are summed in token order; the per-chunk sums of an id are then summed in
// chunk order. (torch's embedding_dense_backward sorts the ids with a device radix sort
// whose temporary state is cleared by a memset; inside a captured HIP graph that clear is a
// memset node. These kernels clear with a kernel and need no global sort.)
//
//   embed_clear_kernel   sets the [V, chunks] slot table to "absent" (0xff bytes);
//   embed_chunk_kernel   one wavefront per (chunk, 256-column slice): ranks the chunk's ids
//                        (id, then position) with lane shuffles and streams the chunk's
//                        gradient rows in sorted order into one partial row per distinct id,
//                        stored at the id's first sorted slot j; the table gets slot[v][c] = j;
//   embed_gather_kernel  one wavefront per (vocabulary row, 256-column block): lane c reads
//                        slot[v][c] (a coalesced row of bytes), and the present chunks'
//                        partial rows are added in chunk (lane) order, 16 rows' loads in
//                        flight.
//
// Bytes: the gradient is read once, the partial rows (at most one per token) are written
// once and read once, the [V, D] result is written once, and the V x chunks byte table is
// cleared, written sparsely and read once.
#include "rk_common.h"

namespace rk {

constexpr int kEmbChunk = 64;            // tokens per chunk (one lane each)
constexpr int kEmbCols = kWave * 4;      // columns per wavefront pass (4 per lane)
constexpr int kEmbMaxBlocks = 16;        // D <= 4096 (256-column blocks)
constexpr int32_t kNoId = 0x7fffffff;    // sorts after every valid id

struct EmbedArgs {
  const void* grad;
  int64_t ldg;
  const void* ids;
  int64_t T, V, D;
  float* partial;     // [chunks * kEmbChunk, D]
  uint8_t* slot;      // [V, ldslot]: slot of id v's partial row in chunk c, 0xff if absent
  int64_t chunks, ldslot;
  float* out;
  int64_t ldo;
};

template <int GDT>
__device__ __forceinline__ float4 load4(const void* base, int64_t idx) {
  if constexpr (GDT == RK_F32) {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
  } else {
    const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + idx);
    return make_float4(__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                       __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u));
  }
}

__device__ __forceinline__ void add4(float4& a, const float4& b) {
  a.x = a.x + b.x;
  a.y = a.y + b.y;
  a.z = a.z + b.z;
  a.w = a.w + b.w;
}

template <int GDT, bool I64>
__global__ __launch_bounds__(64) void embed_chunk_kernel(EmbedArgs a) {
  __shared__ int32_t s_id[kEmbChunk];
  __shared__ int32_t s_tok[kEmbChunk];
  const int lane = threadIdx.x;
  const int64_t c = blockIdx.x;
  const int64_t t = c * kEmbChunk + lane;
  int32_t id = kNoId;
  if (t < a.T) {
    const int64_t raw = I64 ? static_cast<const int64_t*>(a.ids)[t]
                            : static_cast<const int32_t*>(a.ids)[t];
    if (raw >= 0 && raw < a.V) id = static_cast<int32_t>(raw);
  }
  // rank by (id, position): a stable sort of the chunk's 64 ids
  int rank = 0;
#pragma unroll 8
  for (int k = 0; k < kEmbChunk; ++k) {
    const int32_t o = __shfl(id, k, kWave);
    rank += (o < id || (o == id && k < lane)) ? 1 : 0;
  }
  s_id[rank] = id;
  s_tok[rank] = static_cast<int32_t>(t);
  __syncthreads();
  const int valid = __popcll(__ballot(id != kNoId));  // sorted slots 0..valid-1 hold ids
  if (blockIdx.y == 0 && lane < valid && (lane == 0 || s_id[lane - 1] != s_id[lane]))
    a.slot[static_cast<int64_t>(s_id[lane]) * a.ldslot + c] = static_cast<uint8_t>(lane);
  const int64_t col = static_cast<int64_t>(blockIdx.y) * kEmbCols + lane * 4;
  if (col >= a.D) return;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  int start = 0;
  for (int j0 = 0; j0 < valid; j0 += 8) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (j0 + u < valid) v[u] = load4<GDT>(a.grad, s_tok[j0 + u] * a.ldg + col);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u;
      if (j < valid) {
        add4(acc, v[u]);
        if (j + 1 == valid || s_id[j + 1] != s_id[j]) {
          *reinterpret_cast<float4*>(a.partial + (c * kEmbChunk + start) * a.D + col) = acc;
          acc = make_float4(0.f, 0.f, 0.f, 0.f);
          start = j + 1;
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void embed_clear_kernel(uint4* p, int64_t n16) {
  const uint4 ff = make_uint4(0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n16;
       i += static_cast<int64_t>(gridDim.x) * 256)
    p[i] = ff;
}

// One wavefront per (vocabulary row, 256-column block). A frequent id has a partial row in
// nearly every chunk, so its wavefront walks up to `chunks` rows in order: the loads of
// kEmbBatch of them are issued before the first is added, in chunk order.
constexpr int kEmbBatch = 16;

__global__ __launch_bounds__(256) void embed_gather_kernel(EmbedArgs a, int nb) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t v = w / nb;
  if (v >= a.V) return;
  const int64_t col = static_cast<int64_t>(w - v * nb) * kEmbCols + lane * 4;
  const bool colok = col < a.D;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const uint8_t* srow = a.slot + v * a.ldslot;
  for (int64_t g = 0; g < a.chunks; g += kWave) {
    const int64_t c = g + lane;
    const int j = c < a.chunks ? srow[c] : 0xff;
    uint64_t hits = __ballot(j != 0xff);
    const int64_t row = c * kEmbChunk + j;
    while (hits) {
      int64_t rr[kEmbBatch];
#pragma unroll
      for (int u = 0; u < kEmbBatch; ++u) {
        rr[u] = -1;
        if (hits) {
          const int k = __ffsll(static_cast<unsigned long long>(hits)) - 1;
          hits &= hits - 1;
          rr[u] = __shfl(row, k, kWave);
        }
      }
      float4 x[kEmbBatch];
#pragma unroll
      for (int u = 0; u < kEmbBatch; ++u)
        x[u] = (rr[u] >= 0 && colok)
                   ? *reinterpret_cast<const float4*>(a.partial + rr[u] * a.D + col)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int u = 0; u < kEmbBatch; ++u)
        if (rr[u] >= 0) add4(acc, x[u]);
    }
  }
  if (colok) *reinterpret_cast<float4*>(a.out + v * a.ldo + col) = acc;
}

static int64_t embed_chunks(int64_t T) { return (T + kEmbChunk - 1) / kEmbChunk; }

}  // namespace rk

using namespace rk;

// slot-table row: one byte per chunk, padded to 16 bytes
static int64_t embed_ldslot(int64_t T) { return (embed_chunks(T) + 15) / 16 * 16; }

extern "C" int64_t rk_embedding_backward_workspace(int64_t T, int64_t V, int64_t D) {
  if (T < 0 || V < 0 || D < 0) return -1;
  const int64_t slots = embed_chunks(T) * kEmbChunk;
  return slots * D * 4 + V * embed_ldslot(T);
}

extern "C" int rk_embedding_backward(const void* grad, int grad_dtype, int64_t ldg,
                                     const void* ids, int ids_int64, int64_t T, int64_t V,
                                     int64_t D, float* out, int64_t ldo, void* work,
                                     int64_t work_bytes, void* stream) {
  clear_error();
  if (T < 0 || V < 0 || D < 0) return fail(RK_ERR_ARG, "negative size");
  if (V > 0x7ffffffe) return fail(RK_ERR_ARG, "vocabulary of %lld rows exceeds 2^31 - 2",
                                  static_cast<long long>(V));
  if (grad_dtype != RK_F32 && grad_dtype != RK_BF16)
    return fail(RK_ERR_ARG, "grad must be float32 or bfloat16");
  if (D % 4 != 0 || D > static_cast<int64_t>(kEmbCols) * kEmbMaxBlocks)
    return fail(RK_ERR_UNSUPPORTED, "embedding width %lld must be a multiple of 4 and at most %d",
                static_cast<long long>(D), kEmbCols * kEmbMaxBlocks);
  if (V == 0 || D == 0) return RK_OK;
  if (!out || (T > 0 && (!grad || !ids || !work))) return fail(RK_ERR_ARG, "null pointer");
  if (ldo < D || (T > 0 && ldg < D)) return fail(RK_ERR_ARG, "row stride below the width");
  if (ldg % 4 != 0 || ldo % 4 != 0) return fail(RK_ERR_ARG, "row strides must be multiples of 4");
  const int gsz = dtype_size(grad_dtype);
  if ((reinterpret_cast<uintptr_t>(grad) % (4 * gsz)) != 0 || !aligned16(out) || !aligned16(work))
    return fail(RK_ERR_ARG, "grad, out and work must be aligned to 4 elements / 16 bytes");
  const int64_t need = rk_embedding_backward_workspace(T, V, D);
  if (work_bytes < need)
    return fail(RK_ERR_ARG, "workspace of %lld bytes below the %lld needed",
                static_cast<long long>(work_bytes), static_cast<long long>(need));
  EmbedArgs a{};
  a.grad = grad;
  a.ldg = ldg;
  a.ids = ids;
  a.T = T;
  a.V = V;
  a.D = D;
  a.chunks = embed_chunks(T);
  a.partial = static_cast<float*>(work);
  a.slot = static_cast<uint8_t*>(work) + a.chunks * kEmbChunk * D * 4;
  a.ldslot = embed_ldslot(T);
  a.out = out;
  a.ldo = ldo;
  hipStream_t st = as_stream(stream);
  if (a.chunks > 0) {
    const int64_t n16 = V * a.ldslot / 16;
    const int64_t cb = (n16 + 255) / 256;
    embed_clear_kernel<<<static_cast<unsigned>(cb < 2048 ? cb : 2048), 256, 0, st>>>(
        reinterpret_cast<uint4*>(a.slot), n16);
    if (int e = launch_status("embedding_backward clear")) return e;
    const dim3 grid(static_cast<unsigned>(a.chunks),
                    static_cast<unsigned>((D + kEmbCols - 1) / kEmbCols));
    if (grad_dtype == RK_F32) {
      if (ids_int64) embed_chunk_kernel<RK_F32, true><<<grid, 64, 0, st>>>(a);
      else embed_chunk_kernel<RK_F32, false><<<grid, 64, 0, st>>>(a);
    } else {
      if (ids_int64) embed_chunk_kernel<RK_BF16, true><<<grid, 64, 0, st>>>(a);
      else embed_chunk_kernel<RK_BF16, false><<<grid, 64, 0, st>>>(a);
    }
    const int rc = launch_status("embedding_backward chunks");
    if (rc != RK_OK) return rc;
  }
  const int nb = static_cast<int>((D + kEmbCols - 1) / kEmbCols);
  const int64_t waves = V * nb;
  embed_gather_kernel<<<static_cast<unsigned>((waves + 3) / 4), 256, 0, st>>>(a, nb);
  return launch_status("embedding_backward gather");
}
