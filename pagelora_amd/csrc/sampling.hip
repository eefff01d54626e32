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
// One workgroup per row; each thread scans 16-byte chunks of the row with
// kBatch loads in flight, keeps its best (value, index), and the workgroup
// combines them with xor shuffles and LDS.
#include "pl_common.h"

namespace pl {
namespace sampling {

constexpr int kThreads = 1024;
constexpr int kBatch = 8;  // 16-byte chunks per thread in flight

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

// CE: elements per 16-byte chunk (8 for 16-bit types, 4 for fp32)
template <typename T, int CE>
__global__ __launch_bounds__(kThreads) void argmax_kernel(const T* __restrict__ logits, int64_t ld, int vocab,
                                                          int64_t* __restrict__ next_tokens,
                                                          int64_t* __restrict__ tokens_out) {
  __shared__ float s_v[kThreads / 64];
  __shared__ int s_i[kThreads / 64];
  const int row = blockIdx.x;
  const T* p = logits + (int64_t)row * ld;
  Best best{-INFINITY, 0x7fffffff};
  const int chunks = vocab / CE;  // whole 16-byte chunks
  for (int c0 = 0; c0 < chunks; c0 += kThreads * kBatch) {
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
  for (int j = chunks * CE + (int)threadIdx.x; j < vocab; j += kThreads) take(best, to_float<T>(p[j]), j);
  // combine: within the wave, then across the waves
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
    next_tokens[row] = best.i;
    if (tokens_out != nullptr) tokens_out[row] = best.i;
  }
}

}  // namespace sampling
}  // namespace pl

using namespace pl;

extern "C" int pl_greedy_argmax(const void* logits, int64_t ld, int rows, int vocab, int dtype, int64_t* next_tokens,
                                int64_t* tokens_out, void* stream) {
  if (rows < 0 || vocab <= 0) return fail(PL_ERR_INVALID, "rows must be >= 0 and vocab > 0");
  if (rows == 0) return ok();
  if (!logits || !next_tokens) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ld < vocab) return fail(PL_ERR_INVALID, "ld %lld < vocab %d", (long long)ld, vocab);
  if (dtype != PL_DTYPE_F32 && dtype != PL_DTYPE_F16 && dtype != PL_DTYPE_BF16)
    return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
  const int eb = dtype_bytes(dtype);
  if ((uintptr_t)logits % 16 || (ld * eb) % 16)
    return fail(PL_ERR_INVALID, "logits rows must start 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case PL_DTYPE_BF16:
      hipLaunchKernelGGL((sampling::argmax_kernel<bf16_t, 8>), dim3(rows), dim3(sampling::kThreads), 0, s,
                         (const bf16_t*)logits, ld, vocab, next_tokens, tokens_out);
      break;
    case PL_DTYPE_F16:
      hipLaunchKernelGGL((sampling::argmax_kernel<f16_t, 8>), dim3(rows), dim3(sampling::kThreads), 0, s,
                         (const f16_t*)logits, ld, vocab, next_tokens, tokens_out);
      break;
    default:
      hipLaunchKernelGGL((sampling::argmax_kernel<float, 4>), dim3(rows), dim3(sampling::kThreads), 0, s,
                         (const float*)logits, ld, vocab, next_tokens, tokens_out);
      break;
  }
  PL_LAUNCH_CHECK("argmax_kernel");
  return ok();
}
