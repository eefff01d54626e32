// Greedy next-token selection on the device (gfx950): the index of each
// row's largest logit.
//
// Replaces greedy_argmax_token (model/flashinfer/sampling.py:8-15), i.e.
// torch.argmax(logits, dim=-1), with its tie and NaN rules: among equal
// maxima the first index wins, and a NaN counts as larger than any number
// (the first NaN wins).  The kernel can also write the index into the
// decode step's input-token buffer, so the next step reads it without a
// separate copy.
//
// Two launches, no atomics: argmax_partial_kernel splits each row over
// `slices` workgroups (256 threads, 8 chunks of 16 bytes per thread in
// flight) that write their best (value, index) to a caller workspace;
// argmax_final_kernel folds a row's slices in index order and writes the
// token.  A row then occupies many CUs instead of one (151,936 bf16 logits:
// 25 us on one CU per row).
#include "pl_common.h"

namespace pl {
namespace sampling {

constexpr int kThreads = 256;
constexpr int kBatch = 8;                        // 16-byte chunks per thread in flight
constexpr int kSliceChunks = kThreads * kBatch;  // chunks per slice
constexpr int kMaxSlices = 4096;

struct Best {
  float v;
  int i;
};

// a better than b: NaN first, then the larger value, then the smaller index
__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an != bn) return an;
  if (!an && av != bv) return av > bv;
  return ai < bi;
}

__device__ __forceinline__ void take(Best& b, float v, int i) {
  if (better(v, i, b.v, b.i)) {
    b.v = v;
    b.i = i;
  }
}

template <typename T> __device__ __forceinline__ void chunk_to_f32(const uint4& w, float (&f)[8]);
template <> __device__ __forceinline__ void chunk_to_f32<bf16_t>(const uint4& w, float (&f)[8]) {
  unpack2<bf16_t>(w.x, f[0], f[1]);
  unpack2<bf16_t>(w.y, f[2], f[3]);
  unpack2<bf16_t>(w.z, f[4], f[5]);
  unpack2<bf16_t>(w.w, f[6], f[7]);
}
template <> __device__ __forceinline__ void chunk_to_f32<f16_t>(const uint4& w, float (&f)[8]) {
  unpack2<f16_t>(w.x, f[0], f[1]);
  unpack2<f16_t>(w.y, f[2], f[3]);
  unpack2<f16_t>(w.z, f[4], f[5]);
  unpack2<f16_t>(w.w, f[6], f[7]);
}

// CE: elements per 16-byte chunk (8 for 16-bit types, 4 for fp32).  Slice
// z of a row covers chunks [z * kSliceChunks, (z+1) * kSliceChunks); the last
// slice also takes the elements past the last whole chunk.
template <typename T, int CE>
__global__ __launch_bounds__(kThreads) void argmax_partial_kernel(const T* __restrict__ logits, int64_t ld, int vocab,
                                                                  int slices, Best* __restrict__ part) {
  __shared__ float s_v[kThreads / 64];
  __shared__ int s_i[kThreads / 64];
  const int row = blockIdx.y, z = blockIdx.x;
  const T* p = logits + (int64_t)row * ld;
  Best best{-INFINITY, 0x7fffffff};
  const int chunks = vocab / CE;  // whole 16-byte chunks
  const int c0 = z * kSliceChunks;
  if (c0 < chunks) {
    uint4 w[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      // past the end: re-read the last chunk (in bounds), ignored below
      const int c = min(c0 + k * kThreads + (int)threadIdx.x, chunks - 1);
      w[k] = *reinterpret_cast<const uint4*>(p + (int64_t)c * CE);
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int c = c0 + k * kThreads + (int)threadIdx.x;
      if (c < chunks) {
        float f[8];
        if constexpr (CE == 8) {
          chunk_to_f32<T>(w[k], f);
        } else {
          f[0] = __uint_as_float(w[k].x); f[1] = __uint_as_float(w[k].y);
          f[2] = __uint_as_float(w[k].z); f[3] = __uint_as_float(w[k].w);
        }
#pragma unroll
        for (int e = 0; e < CE; ++e) take(best, f[e], c * CE + e);
      }
    }
  }
  if (z == slices - 1)
    for (int j = chunks * CE + (int)threadIdx.x; j < vocab; j += kThreads) take(best, to_float<T>(p[j]), j);
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float ov = __shfl_xor(best.v, off);
    const int oi = __shfl_xor(best.i, off);
    take(best, ov, oi);
  }
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  if (lane == 0) {
    s_v[wave] = best.v;
    s_i[wave] = best.i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w) take(best, s_v[w], s_i[w]);
    part[(int64_t)row * slices + z] = best;
  }
}

// One wave per row folds the row's slices (each lane a strided subset, then
// the wave; `take` keeps the first index among equals, so the order of the
// fold does not matter).
__global__ __launch_bounds__(64) void argmax_final_kernel(const Best* __restrict__ part, int slices,
                                                          int64_t* __restrict__ next_tokens,
                                                          int64_t* __restrict__ tokens_out) {
  const int row = blockIdx.x;
  Best best{-INFINITY, 0x7fffffff};
  for (int z = threadIdx.x; z < slices; z += 64) {
    const Best b = part[(int64_t)row * slices + z];
    take(best, b.v, b.i);
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float ov = __shfl_xor(best.v, off);
    const int oi = __shfl_xor(best.i, off);
    take(best, ov, oi);
  }
  if (threadIdx.x == 0) {
    next_tokens[row] = best.i;
    if (tokens_out != nullptr) tokens_out[row] = best.i;
  }
}

}  // namespace sampling
}  // namespace pl

using namespace pl;

static int argmax_slices(int vocab, int dtype) {
  const int ce = dtype == PL_DTYPE_F32 ? 4 : 8;
  const int chunks = vocab / ce;
  const int slices = (chunks + sampling::kSliceChunks - 1) / sampling::kSliceChunks;
  return slices < 1 ? 1 : slices;
}

extern "C" size_t pl_greedy_argmax_workspace_size(int rows, int vocab, int dtype) {
  if (rows <= 0 || vocab <= 0) return 0;
  return (size_t)rows * argmax_slices(vocab, dtype) * sizeof(sampling::Best);
}

extern "C" int pl_greedy_argmax(const void* logits, int64_t ld, int rows, int vocab, int dtype, int64_t* next_tokens,
                                int64_t* tokens_out, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || vocab <= 0) return fail(PL_ERR_INVALID, "rows must be >= 0 and vocab > 0");
  if (rows == 0) return ok();
  if (!logits || !next_tokens || !workspace) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ld < vocab) return fail(PL_ERR_INVALID, "ld %lld < vocab %d", (long long)ld, vocab);
  if (dtype != PL_DTYPE_F32 && dtype != PL_DTYPE_F16 && dtype != PL_DTYPE_BF16)
    return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
  const int eb = dtype_bytes(dtype);
  if ((uintptr_t)logits % 16 || (ld * eb) % 16)
    return fail(PL_ERR_INVALID, "logits rows must start 16-byte aligned");
  const int slices = argmax_slices(vocab, dtype);
  if (slices > sampling::kMaxSlices) return fail(PL_ERR_UNSUPPORTED, "vocab %d too large", vocab);
  if ((uintptr_t)workspace % alignof(sampling::Best)) return fail(PL_ERR_INVALID, "workspace must be 8-byte aligned");
  if (workspace_bytes < pl_greedy_argmax_workspace_size(rows, vocab, dtype))
    return fail(PL_ERR_WORKSPACE, "workspace of %zu bytes < %zu needed", workspace_bytes,
                pl_greedy_argmax_workspace_size(rows, vocab, dtype));
  hipStream_t s = (hipStream_t)stream;
  auto* part = (sampling::Best*)workspace;
  const dim3 grid(slices, rows);
  switch (dtype) {
    case PL_DTYPE_BF16:
      hipLaunchKernelGGL((sampling::argmax_partial_kernel<bf16_t, 8>), grid, dim3(sampling::kThreads), 0, s,
                         (const bf16_t*)logits, ld, vocab, slices, part);
      break;
    case PL_DTYPE_F16:
      hipLaunchKernelGGL((sampling::argmax_partial_kernel<f16_t, 8>), grid, dim3(sampling::kThreads), 0, s,
                         (const f16_t*)logits, ld, vocab, slices, part);
      break;
    default:
      hipLaunchKernelGGL((sampling::argmax_partial_kernel<float, 4>), grid, dim3(sampling::kThreads), 0, s,
                         (const float*)logits, ld, vocab, slices, part);
      break;
  }
  PL_LAUNCH_CHECK("argmax_partial_kernel");
  hipLaunchKernelGGL(sampling::argmax_final_kernel, dim3(rows), dim3(64), 0, s, (const sampling::Best*)part, slices,
                     next_tokens, tokens_out);
  PL_LAUNCH_CHECK("argmax_final_kernel");
  return ok();
}
