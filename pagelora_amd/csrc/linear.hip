// Decode-sized linear layer for gfx950:  out = x . W^T (+ bias)
//                                               (+ the no-merge LoRA delta)
// for few tokens (M <= 64) and weights W [N, K] streamed once from HBM.
//
// skinny_linear_kernel  one workgroup of kWaves waves per 16 output columns
//                       (x one 16-token tile).  The waves split K; each
//                       runs MFMA 16x16x32 with W rows as the B operand
//                       (16-byte non-temporal loads, eight steps in flight)
//                       and x as the A operand; the wave tiles are summed
//                       in LDS.  Optional epilogue: the LoRA expand of the
//                       no-merge path -- the workgroup folds the shrink's
//                       fp32 partials for its tokens into the rank-r
//                       intermediate (rounded to the input dtype, as the
//                       reference's F.linear returns it) and adds
//                       scale * y . B^T for its 16 columns, one MFMA per
//                       adapter present in the token tile.  The sum is
//                       rounded once into out.
//
// Reference: the base F.linear of project_qkv_packed / project_gate_up_packed
// / project_linear (model/flashinfer/packed_ops.py:143, 179, 251-265) plus the
// delta of _packed_lora_delta / LoRALinear.forward (packed_ops.py:314-325,
// multilora/linear.py:226-231).
#include "pl_common.h"

namespace pl {
namespace linear {

constexpr int kWave = 64;
constexpr int kWaves = 8;
constexpr int kThreads = kWave * kWaves;
constexpr int kUnroll = 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T> __device__ __forceinline__ f32x4 mfma32(u32x4 a, u32x4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma32<bf16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma32<f16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

// LoRA epilogue description (module column ranges inside [0, N)).
struct LoraMod {
  const void* B;      // [n_adapters, out_features, rank]
  int out_offset, out_features, rank, rank_offset;
  float scale;
};
struct LoraEpi {
  LoraMod m[PL_LORA_MAX_MODULES];
  int n;               // modules; 0 = no LoRA
  int r_total, r_pad;  // concatenated ranks, padded to 32
  int n_adapters;
  int ksplit;          // shrink k-slices to fold
  const float* part;   // [ksplit][tokens][r_pad]
  const int32_t* ids;  // [tokens]
};

template <typename T>
__global__ __launch_bounds__(kThreads) void skinny_linear_kernel(
    const T* __restrict__ x, int64_t ldx, int tokens, int K, const T* __restrict__ W, int64_t ldw, int N,
    const T* __restrict__ bias, T* __restrict__ out, int64_t ldo, LoraEpi lora) {
  __shared__ float s_red[kWaves][256];
  __shared__ __align__(16) uint16_t s_y[16][128 + 8];
  __shared__ int s_ids[16];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int lr = lane % 16;
  const int kq = (lane / 16) * 8;
  const int n0 = blockIdx.x * 16;
  const int t0 = blockIdx.y * 16;
  const int n = n0 + lr, t = t0 + lr;
  const bool n_ok = n < N, t_ok = t < tokens;

  // this wave's k range, whole 32-wide steps
  const int steps = (K + 31) / 32;
  const int per = (steps + kWaves - 1) / kWaves;
  const int k_begin = wave * per * 32;
  const int k_end = min(K, k_begin + per * 32);
  const T* wrow = W + (int64_t)(n_ok ? n : 0) * ldw;
  const T* xrow = x + (int64_t)(t_ok ? t : 0) * ldx;

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // Both loops step k0 uniformly over the wave (the MFMA needs every lane);
  // lane group kq covers k0 + kq .. + 8.  The unrolled loop runs only while
  // every group of every step is in range; in the tail a group past k_end
  // loads zeros (K % 8 == 0, so a group is wholly in or out of range).
  int k0 = k_begin;
  for (; k0 + kUnroll * 32 <= k_end; k0 += kUnroll * 32) {
    const int k = k0 + kq;
    u32x4 bw[kUnroll], ax[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      bw[u] = n_ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + k + u * 32)) : zero4();
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      ax[u] = t_ok ? *reinterpret_cast<const u32x4*>(xrow + k + u * 32) : zero4();
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc = mfma32<T>(ax[u], bw[u], acc);
  }
  for (; k0 < k_end; k0 += 32) {
    const int k = k0 + kq;
    const bool k_ok = k < k_end;
    const u32x4 bw = (n_ok & k_ok) ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + k)) : zero4();
    const u32x4 ax = (t_ok & k_ok) ? *reinterpret_cast<const u32x4*>(xrow + k) : zero4();
    acc = mfma32<T>(ax, bw, acc);
  }
  // D rows = tokens 4*(lane/16)+i of the tile, column = lr
#pragma unroll
  for (int i = 0; i < 4; ++i) s_red[wave][((lane / 16) * 4 + i) * 16 + lr] = acc[i];

  if (lora.n > 0) {
    // fold the shrink partials of this token tile into the rounded intermediate
    if (threadIdx.x < 16) s_ids[threadIdx.x] = (t0 + (int)threadIdx.x < tokens) ? lora.ids[t0 + threadIdx.x] : -1;
    for (int c = threadIdx.x; c < 16 * lora.r_pad; c += kThreads) {
      const int i = c / lora.r_pad, kk = c - i * lora.r_pad;
      float sum = 0.f;
      if (t0 + i < tokens && kk < lora.r_total) {
        const float* pp = lora.part + (int64_t)(t0 + i) * lora.r_pad + kk;
        const int64_t stride = (int64_t)tokens * lora.r_pad;
        int q = 0;
        for (; q + 8 <= lora.ksplit; q += 8) {
          float v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = pp[(q + u) * stride];
#pragma unroll
          for (int u = 0; u < 8; ++u) sum += v[u];
        }
        for (; q < lora.ksplit; ++q) sum += pp[q * stride];
      }
      s_y[i][kk] = __builtin_bit_cast(uint16_t, from_float<T>(sum));
    }
  }
  __syncthreads();

  if (wave == 0) {
    // sum the waves' tiles: lane holds rows 4*(lane/16)+i, column lr
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cell = ((lane / 16) * 4 + i) * 16 + lr;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += s_red[w][cell];
      v[i] = s;
    }
    if (lora.n > 0) {  // uniform: the MFMAs below run with every lane active
      int mi = -1;
#pragma unroll
      for (int m = 0; m < PL_LORA_MAX_MODULES; ++m)
        if (n_ok && m < lora.n && n >= lora.m[m].out_offset && n < lora.m[m].out_offset + lora.m[m].out_features)
          mi = m;
      // one MFMA pass per adapter present in the tile; rows of other tokens masked
      for (int j = 0; j < 16; ++j) {
        const int a = s_ids[j];
        if (a < 0 || a >= lora.n_adapters) continue;
        bool seen = false;
        for (int jj = 0; jj < j; ++jj) seen |= (s_ids[jj] == a);
        if (seen) continue;
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
        for (int kt = 0; kt * 32 < lora.r_pad; ++kt) {
          u32x4 bop = zero4();
          if (mi >= 0) {
            const LoraMod& m = lora.m[mi];
            const int j0 = kt * 32 + kq - m.rank_offset;
            const T* brow = (const T*)m.B + ((int64_t)a * m.out_features + (n - m.out_offset)) * m.rank;
            if (m.rank % 8 == 0 && j0 >= 0 && j0 + 8 <= m.rank) {
              bop = *reinterpret_cast<const u32x4*>(brow + j0);
            } else {
              uint32_t e[8];
#pragma unroll
              for (int q = 0; q < 8; ++q) {
                const int jl = j0 + q;
                e[q] = (jl >= 0 && jl < m.rank) ? (uint32_t)__builtin_bit_cast(uint16_t, brow[jl]) : 0u;
              }
              bop = u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
            }
          }
          const bool row_is_a = s_ids[lr] == a;
          const u32x4 av = row_is_a ? *reinterpret_cast<const u32x4*>(&s_y[lr][kt * 32 + kq]) : zero4();
          d = mfma32<T>(av, bop, d);
        }
        if (mi >= 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] += lora.m[mi].scale * d[i];
        }
      }
    }
    if (n_ok) {
      const float b = bias != nullptr ? to_float<T>(bias[n]) : 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tr = t0 + (lane / 16) * 4 + i;
        if (tr < tokens) out[(int64_t)tr * ldo + n] = from_float<T>(v[i] + b);
      }
    }
  }
}

}  // namespace linear
}  // namespace pl

using namespace pl;
using namespace pl::linear;

extern "C" int pl_linear(const void* x, int64_t ldx, int num_tokens, int in_features, const void* weight,
                         int64_t ldw, int out_features, const void* bias, void* out, int64_t ldo,
                         const pl_linear_lora* lora_h, int num_lora, const int32_t* adapter_ids,
                         int num_adapters, const void* lora_workspace, size_t lora_workspace_bytes,
                         int dtype, void* stream) {
  if (num_tokens < 0 || num_tokens > PL_LINEAR_MAX_TOKENS)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", PL_LINEAR_MAX_TOKENS, num_tokens);
  if (num_tokens == 0) return ok();
  if (in_features <= 0 || in_features % 8 || out_features <= 0)
    return fail(PL_ERR_INVALID, "in_features must be a positive multiple of 8 and out_features > 0");
  if (!x || !weight || !out) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx % 8 || ldw % 8 || (uintptr_t)x % 16 || (uintptr_t)weight % 16)
    return fail(PL_ERR_INVALID, "x and weight rows must be 16-byte aligned");
  if (ldw < in_features || ldx < in_features || ldo < out_features) return fail(PL_ERR_INVALID, "bad leading dimension");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_linear dtype must be F16 or BF16 (got %d)", dtype);
  LoraEpi epi{};
  epi.n = 0;
  if (num_lora > 0) {
    if (num_lora > PL_LORA_MAX_MODULES) return fail(PL_ERR_INVALID, "at most %d LoRA modules", PL_LORA_MAX_MODULES);
    if (!lora_h || !adapter_ids || !lora_workspace) return fail(PL_ERR_INVALID, "LoRA arguments are null");
    if (num_adapters < 1) return fail(PL_ERR_INVALID, "num_adapters must be >= 1");
    int r = 0;
    for (int i = 0; i < num_lora; ++i) {
      const pl_linear_lora& m = lora_h[i];
      if (!m.B || m.rank <= 0 || m.out_features <= 0) return fail(PL_ERR_INVALID, "LoRA module %d is invalid", i);
      if (m.col_offset < 0 || (int64_t)m.col_offset + m.out_features > out_features)
        return fail(PL_ERR_INVALID, "LoRA module %d columns [%d, +%d) exceed out_features", i, m.col_offset,
                    m.out_features);
      epi.m[i].B = m.B;
      epi.m[i].out_offset = m.col_offset;
      epi.m[i].out_features = m.out_features;
      epi.m[i].rank = m.rank;
      epi.m[i].rank_offset = r;
      epi.m[i].scale = m.scale;
      r += m.rank;
    }
    epi.n = num_lora;
    epi.r_total = r;
    epi.r_pad = (r + 31) / 32 * 32;
    if (epi.r_pad > 128) return fail(PL_ERR_UNSUPPORTED, "sum of ranks %d > 128", r);
    epi.n_adapters = num_adapters;
    epi.ksplit = lora_ksplit(num_tokens, in_features);
    const size_t need = (size_t)epi.ksplit * num_tokens * epi.r_pad * sizeof(float);
    if (need > lora_workspace_bytes)
      return fail(PL_ERR_WORKSPACE, "LoRA workspace of %zu bytes < %zu needed", lora_workspace_bytes, need);
    epi.part = (const float*)lora_workspace;
    epi.ids = adapter_ids;
  }
  dim3 grid((out_features + 15) / 16, (num_tokens + 15) / 16);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PL_DTYPE_BF16)
    hipLaunchKernelGGL(skinny_linear_kernel<bf16_t>, grid, dim3(kThreads), 0, s, (const bf16_t*)x, ldx, num_tokens,
                       in_features, (const bf16_t*)weight, ldw, out_features, (const bf16_t*)bias, (bf16_t*)out, ldo,
                       epi);
  else
    hipLaunchKernelGGL(skinny_linear_kernel<f16_t>, grid, dim3(kThreads), 0, s, (const f16_t*)x, ldx, num_tokens,
                       in_features, (const f16_t*)weight, ldw, out_features, (const f16_t*)bias, (f16_t*)out, ldo, epi);
  PL_LAUNCH_CHECK("skinny_linear_kernel");
  return ok();
}
