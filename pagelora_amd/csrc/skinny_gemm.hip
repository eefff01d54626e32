// Decode-sized GEMM on pre-shuffled weights (gfx950):  out = x . W^T (+ bias)
// for few tokens (T <= 64) with W [N, K] streamed once from HBM.
//
// Weight layout.  MFMA 16x16x32's B operand gives lane l the 8 k-values
// (l / 16) * 8 .. +8 of column l % 16, so a wave reading a row-major W
// touches 16 rows x 64 bytes per instruction.  pl_weight_shuffle stores W
// once, at load time, as 1 KiB blocks in exactly that lane order:
//   block (nb, ks) = rows nb*16 .. +16, k = ks*32 .. +32;
//   element e of lane l at  ((nb * K/32 + ks) * 64 + l) * 8 + e
//                        =  W[nb*16 + l%16][ks*32 + (l/16)*8 + e]
// (rows past N are zero).  Every wave load is then one contiguous,
// fully coalesced 1 KiB read that lands directly in MFMA registers; a
// wave's k-range of a row block is contiguous in memory.
//
// shuffled_gemm_kernel  one workgroup of 16 waves per 16 output columns
//                       (x one 16-token tile); the waves split K, each
//                       streams its contiguous run of blocks four at a time
//                       (non-temporal loads) against x rows read from L2,
//                       and the 16 partial tiles are summed through LDS.
//                       Eight at a time measured slower at every decode
//                       shape (74 VGPRs: one workgroup per CU instead of two).
//
// Reference: the base F.linear of project_qkv_packed / project_gate_up_packed
// / project_linear (model/flashinfer/packed_ops.py:143, 179, 251-265) and
// LoRALinear.forward (multilora/linear.py:226-231) at decode batch sizes.
#include <algorithm>

#include "pl_common.h"

namespace pl {
namespace sgemm {

constexpr int kWave = 64;
constexpr int kWaves = 16;
constexpr int kThreads = kWave * kWaves;
constexpr int kUnroll = 4;
constexpr int kBlockElems = 512;  // 16 rows x 32 k

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T> __device__ __forceinline__ f32x4 mfma32(u32x4 a, u32x4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma32<bf16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma32<f16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

// One thread per 16-byte piece of the shuffled buffer (N_pad x K elements).
__global__ void shuffle_kernel(const uint16_t* __restrict__ W, int64_t ldw, int N, int K, uint16_t* __restrict__ Ws,
                               int64_t pieces) {
  const int ksteps = K / 32;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t blk = i / 64;
    const int l = (int)(i % 64);
    const int ks = (int)(blk % ksteps);
    const int64_t n = (blk / ksteps) * 16 + l % 16;
    const int k = ks * 32 + (l / 16) * 8;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (n < N) v = *reinterpret_cast<const uint4*>(W + n * ldw + k);
    *reinterpret_cast<uint4*>(Ws + i * 8) = v;
  }
}

// The inverse of shuffle_kernel: one thread per 16-byte piece, rows < N
// written back to the row-major W (row stride ldw).
__global__ void unshuffle_kernel(const uint16_t* __restrict__ Ws, int N, int K, uint16_t* __restrict__ W,
                                 int64_t ldw, int64_t pieces) {
  const int ksteps = K / 32;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t blk = i / 64;
    const int l = (int)(i % 64);
    const int ks = (int)(blk % ksteps);
    const int64_t n = (blk / ksteps) * 16 + l % 16;
    const int k = ks * 32 + (l / 16) * 8;
    if (n < N) *reinterpret_cast<uint4*>(W + n * ldw + k) = *reinterpret_cast<const uint4*>(Ws + i * 8);
  }
}

// PARTIAL: split-K over gridDim.z workgroups per row block; workgroup z sums
// k-steps [z*K/32/splits, ..) and writes its fp32 tile to plane z of
// `partial` (row t at t * ldp, planes plane_stride apart) instead of `out`.
// SIDE: row blocks below main_tiles are computed whole into `out`; the
// blocks from main_tiles on (the LoRA A rows stacked under W) are split-K
// over side_splits small workgroups each, appended to the grid, into fp32
// planes of `partial` (column n - 16 * main_tiles).  A row-block count that
// is a multiple of the CU count then stays one: one more whole block costs a
// CU two blocks' time (o_proj, 4 tokens: 4096 rows 7.6 us, 4112 rows 10.1).
template <typename T, bool PARTIAL, bool SIDE = false>
__global__ __launch_bounds__(kThreads) void shuffled_gemm_kernel(const T* __restrict__ x, int64_t ldx, int tokens,
                                                                 int K, const T* __restrict__ Ws, int N,
                                                                 const T* __restrict__ bias, T* __restrict__ out,
                                                                 int64_t ldo, float* __restrict__ partial,
                                                                 int64_t ldp, int64_t plane_stride,
                                                                 int main_tiles = 0, int side_splits = 1) {
  __shared__ float s_red[kWaves][256];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int lr = lane % 16, kq = (lane / 16) * 8;
  const bool side = SIDE && (int)blockIdx.x >= main_tiles;
  const int se_idx = (int)blockIdx.x - main_tiles;
  const int nb = side ? main_tiles + se_idx / side_splits : (int)blockIdx.x, t0 = blockIdx.y * 16;
  const int zs = SIDE ? (side ? se_idx % side_splits : 0) : (int)blockIdx.z;
  const int nz = SIDE ? (side ? side_splits : 1) : (int)gridDim.z;
  const int t = t0 + lr;
  const bool t_ok = t < tokens;
  const int ksteps = K / 32;
  const int chunk = (ksteps + nz - 1) / nz;
  const int kb0 = min(ksteps, zs * chunk), ke0 = min(ksteps, kb0 + chunk);
  const int per = (ke0 - kb0 + kWaves - 1) / kWaves;
  const int sb = min(ke0, kb0 + wave * per), se = min(ke0, sb + per);
  const u32x4* wb = reinterpret_cast<const u32x4*>(Ws + (int64_t)nb * ksteps * kBlockElems) + lane;
  const T* xr = x + (int64_t)(t_ok ? t : 0) * ldx + kq;

  // A rows of tokens >= `tokens` read token 0's row (xr is clamped): row i of
  // the MFMA result depends only on row i of A, and those rows are never
  // written, so the loads need no condition (a condition here becomes a
  // branch around each load, and a wait before the next batch).
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int s = sb;
  for (; s + kUnroll <= se; s += kUnroll) {
    u32x4 b[kUnroll], a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) b[u] = __builtin_nontemporal_load(wb + (s + u) * kWave);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = *reinterpret_cast<const u32x4*>(xr + (s + u) * 32);
    // all of a batch's loads before its first MFMA (measured: lm_head at 4
    // tokens 180.9 -> 175.6 us, down_proj split 3 20.0 -> 19.7 us)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc = mfma32<T>(a[u], b[u], acc);
  }
  for (; s < se; ++s) {
    const u32x4 b = __builtin_nontemporal_load(wb + s * kWave);
    const u32x4 a = *reinterpret_cast<const u32x4*>(xr + s * 32);
    acc = mfma32<T>(a, b, acc);
  }
  // D: rows = tokens 4*(lane/16)+i of the tile, column = lr
#pragma unroll
  for (int i = 0; i < 4; ++i) s_red[wave][((lane / 16) * 4 + i) * 16 + lr] = acc[i];
  __syncthreads();
  if (wave == 0) {
    const int n = nb * 16 + lr;
    const float bv = (!PARTIAL && !side && bias != nullptr && n < N) ? to_float<T>(bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cell = ((lane / 16) * 4 + i) * 16 + lr;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) sum += s_red[w][cell];
      const int tr = t0 + (lane / 16) * 4 + i;
      if (n < N && tr < tokens) {
        if (PARTIAL)
          partial[(int64_t)blockIdx.z * plane_stride + (int64_t)tr * ldp + n] = sum;
        else if (side)
          partial[(int64_t)zs * plane_stride + (int64_t)tr * ldp + (n - main_tiles * 16)] = sum;
        else
          out[(int64_t)tr * ldo + n] = from_float<T>(sum + bv);
      }
    }
  }
}

}  // namespace sgemm
}  // namespace pl

using namespace pl;
using namespace pl::sgemm;

extern "C" size_t pl_weight_shuffled_bytes(int out_features, int in_features) {
  if (out_features <= 0 || in_features <= 0 || in_features % 32) return 0;
  return (size_t)((out_features + 15) / 16) * 16 * in_features * 2;
}

extern "C" int pl_weight_shuffle(const void* weight, int64_t ldw, int out_features, int in_features, void* shuffled,
                                 size_t shuffled_bytes, int dtype, void* stream) {
  if (out_features <= 0 || in_features <= 0 || in_features % 32)
    return fail(PL_ERR_INVALID, "out_features > 0 and in_features a positive multiple of 32 required");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "shuffled weights are F16 or BF16 (got %d)", dtype);
  if (!weight || !shuffled) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldw < in_features || ldw % 8 || (uintptr_t)weight % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "weight rows and the shuffled buffer must be 16-byte aligned");
  const size_t need = pl_weight_shuffled_bytes(out_features, in_features);
  if (shuffled_bytes < need)
    return fail(PL_ERR_WORKSPACE, "shuffled buffer of %zu bytes < %zu needed", shuffled_bytes, need);
  const int64_t pieces = (int64_t)need / 16;
  const int64_t blocks = std::min<int64_t>((pieces + 255) / 256, 65536);
  hipLaunchKernelGGL(shuffle_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)weight, ldw, out_features, in_features, (uint16_t*)shuffled, pieces);
  PL_LAUNCH_CHECK("shuffle_kernel");
  return ok();
}

extern "C" int pl_weight_unshuffle(const void* shuffled, size_t shuffled_bytes, int out_features, int in_features,
                                   void* weight, int64_t ldw, int dtype, void* stream) {
  if (out_features <= 0 || in_features <= 0 || in_features % 32)
    return fail(PL_ERR_INVALID, "out_features > 0 and in_features a positive multiple of 32 required");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "shuffled weights are F16 or BF16 (got %d)", dtype);
  if (!weight || !shuffled) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldw < in_features || ldw % 8 || (uintptr_t)weight % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "weight rows and the shuffled buffer must be 16-byte aligned");
  const size_t need = pl_weight_shuffled_bytes(out_features, in_features);
  if (shuffled_bytes < need)
    return fail(PL_ERR_WORKSPACE, "shuffled buffer of %zu bytes < %zu needed", shuffled_bytes, need);
  const int64_t pieces = (int64_t)need / 16;
  const int64_t blocks = std::min<int64_t>((pieces + 255) / 256, 65536);
  hipLaunchKernelGGL(unshuffle_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)shuffled, out_features, in_features, (uint16_t*)weight, ldw, pieces);
  PL_LAUNCH_CHECK("unshuffle_kernel");
  return ok();
}

extern "C" int pl_linear_shuffled(const void* x, int64_t ldx, int num_tokens, int in_features, const void* shuffled,
                                  int out_features, const void* bias, void* out, int64_t ldo, int dtype,
                                  void* stream) {
  if (num_tokens < 0 || num_tokens > PL_LINEAR_MAX_TOKENS)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", PL_LINEAR_MAX_TOKENS, num_tokens);
  if (num_tokens == 0) return ok();
  if (in_features <= 0 || in_features % 32 || out_features <= 0)
    return fail(PL_ERR_INVALID, "in_features must be a positive multiple of 32 and out_features > 0");
  if (!x || !shuffled || !out) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx < in_features || ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "x rows and the shuffled weight must be 16-byte aligned");
  if (ldo < out_features) return fail(PL_ERR_INVALID, "ldo < out_features");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_linear_shuffled dtype must be F16 or BF16 (got %d)", dtype);
  const dim3 grid((out_features + 15) / 16, (num_tokens + 15) / 16);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PL_DTYPE_BF16)
    hipLaunchKernelGGL((shuffled_gemm_kernel<bf16_t, false>), grid, dim3(kThreads), 0, s, (const bf16_t*)x, ldx,
                       num_tokens, in_features, (const bf16_t*)shuffled, out_features, (const bf16_t*)bias,
                       (bf16_t*)out, ldo, nullptr, 0, 0);
  else
    hipLaunchKernelGGL((shuffled_gemm_kernel<f16_t, false>), grid, dim3(kThreads), 0, s, (const f16_t*)x, ldx,
                       num_tokens, in_features, (const f16_t*)shuffled, out_features, (const f16_t*)bias,
                       (f16_t*)out, ldo, nullptr, 0, 0);
  PL_LAUNCH_CHECK("shuffled_gemm_kernel");
  return ok();
}

extern "C" int pl_linear_shuffled_split(const void* x, int64_t ldx, int num_tokens, int in_features,
                                        const void* shuffled, int out_features, int splits, float* partials,
                                        int64_t ld, int64_t plane_stride, int dtype, void* stream) {
  if (num_tokens < 0 || num_tokens > PL_LINEAR_MAX_TOKENS)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", PL_LINEAR_MAX_TOKENS, num_tokens);
  if (num_tokens == 0) return ok();
  if (in_features <= 0 || in_features % 32 || out_features <= 0)
    return fail(PL_ERR_INVALID, "in_features must be a positive multiple of 32 and out_features > 0");
  if (splits < 1 || splits > 16 || splits > in_features / 32)
    return fail(PL_ERR_INVALID, "splits must be 1..min(16, in_features/32) (got %d)", splits);
  if (!x || !shuffled || !partials) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx < in_features || ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "x rows and the shuffled weight must be 16-byte aligned");
  if (ld < out_features || plane_stride < ld * num_tokens)
    return fail(PL_ERR_INVALID, "partial planes overlap (ld %lld, plane_stride %lld)", (long long)ld,
                (long long)plane_stride);
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_linear_shuffled_split dtype must be F16 or BF16 (got %d)", dtype);
  const dim3 grid((out_features + 15) / 16, (num_tokens + 15) / 16, splits);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PL_DTYPE_BF16)
    hipLaunchKernelGGL((shuffled_gemm_kernel<bf16_t, true>), grid, dim3(kThreads), 0, s, (const bf16_t*)x, ldx,
                       num_tokens, in_features, (const bf16_t*)shuffled, out_features, nullptr, nullptr, 0,
                       partials, ld, plane_stride);
  else
    hipLaunchKernelGGL((shuffled_gemm_kernel<f16_t, true>), grid, dim3(kThreads), 0, s, (const f16_t*)x, ldx,
                       num_tokens, in_features, (const f16_t*)shuffled, out_features, nullptr, nullptr, 0,
                       partials, ld, plane_stride);
  PL_LAUNCH_CHECK("shuffled_gemm_kernel");
  return ok();
}

extern "C" int pl_linear_shuffled_side(const void* x, int64_t ldx, int num_tokens, int in_features,
                                       const void* shuffled, int out_features, int main_features, void* out,
                                       int64_t ldo, int side_splits, float* side_partials, int64_t ld_side,
                                       int64_t side_plane_stride, int dtype, void* stream) {
  if (num_tokens < 0 || num_tokens > PL_LINEAR_MAX_TOKENS)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", PL_LINEAR_MAX_TOKENS, num_tokens);
  if (num_tokens == 0) return ok();
  if (in_features <= 0 || in_features % 32 || out_features <= 0)
    return fail(PL_ERR_INVALID, "in_features must be a positive multiple of 32 and out_features > 0");
  if (main_features <= 0 || main_features % 16 || main_features >= out_features)
    return fail(PL_ERR_INVALID, "main_features must be a positive multiple of 16 below out_features (got %d of %d)",
                main_features, out_features);
  if (side_splits < 1 || side_splits > 64 || side_splits > in_features / 32)
    return fail(PL_ERR_INVALID, "side_splits must be 1..min(64, in_features/32) (got %d)", side_splits);
  if (!x || !shuffled || !out || !side_partials) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx < in_features || ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "x rows and the shuffled weight must be 16-byte aligned");
  if (ldo < main_features) return fail(PL_ERR_INVALID, "ldo < main_features");
  const int side_features = out_features - main_features;
  if (ld_side < side_features || side_plane_stride < ld_side * num_tokens)
    return fail(PL_ERR_INVALID, "side planes overlap (ld %lld, plane_stride %lld)", (long long)ld_side,
                (long long)side_plane_stride);
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_linear_shuffled_side dtype must be F16 or BF16 (got %d)", dtype);
  const int main_tiles = main_features / 16;
  const int side_tiles = (out_features + 15) / 16 - main_tiles;
  const dim3 grid(main_tiles + side_tiles * side_splits, (num_tokens + 15) / 16, 1);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PL_DTYPE_BF16)
    hipLaunchKernelGGL((shuffled_gemm_kernel<bf16_t, false, true>), grid, dim3(kThreads), 0, s, (const bf16_t*)x,
                       ldx, num_tokens, in_features, (const bf16_t*)shuffled, out_features, nullptr, (bf16_t*)out,
                       ldo, side_partials, ld_side, side_plane_stride, main_tiles, side_splits);
  else
    hipLaunchKernelGGL((shuffled_gemm_kernel<f16_t, false, true>), grid, dim3(kThreads), 0, s, (const f16_t*)x,
                       ldx, num_tokens, in_features, (const f16_t*)shuffled, out_features, nullptr, (f16_t*)out,
                       ldo, side_partials, ld_side, side_plane_stride, main_tiles, side_splits);
  PL_LAUNCH_CHECK("shuffled_gemm_kernel");
  return ok();
}
