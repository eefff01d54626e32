// Fused element-wise kernels of the decode layer (gfx950):
//
//   rmsnorm_kernel           out = bf16(x * rsqrt(mean(x^2) + eps) * w)
//   add_rmsnorm_kernel       r = r + x (rounded to the storage type), then
//                            out = rmsnorm(r): the residual add of the
//                            previous block fused with the next block's norm
//   silu_mul_kernel          out = silu(gate) * up, one rounding
//   qk_norm_rope_append      per decode token: q/k per-head RMSNorm, rotate-
//                            half RoPE at the token's position, q written
//                            out, k and v written straight into their page
//
// Reference: norm.py:15-65 (FlashInfer rmsnorm / fused_add_rmsnorm, fp32
// statistics, one rounding), packed_ops.py:230-239 (silu_and_mul),
// projection.py:155-190, 248-260 (apply_rope_pos_ids non-interleaved, head
// norm) and layer_runner.py:399-412 (the page append the fused kernel
// replaces).  All arithmetic is fp32; each output is rounded once.
#include "pl_common.h"

namespace pl {
namespace fused {

constexpr int kThreads = 256;
constexpr int kWave = 64;

template <typename T> __device__ __forceinline__ void load_row8(const T* p, float (&f)[8]);
template <> __device__ __forceinline__ void load_row8<float>(const float* p, float (&f)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
template <typename T> __device__ __forceinline__ void load_row8_16(const T* p, float (&f)[8]) {
  const uint4 a = *reinterpret_cast<const uint4*>(p);
  unpack2<T>(a.x, f[0], f[1]);
  unpack2<T>(a.y, f[2], f[3]);
  unpack2<T>(a.z, f[4], f[5]);
  unpack2<T>(a.w, f[6], f[7]);
}
template <> __device__ __forceinline__ void load_row8<f16_t>(const f16_t* p, float (&f)[8]) { load_row8_16(p, f); }
template <> __device__ __forceinline__ void load_row8<bf16_t>(const bf16_t* p, float (&f)[8]) { load_row8_16(p, f); }

template <typename T> __device__ __forceinline__ void store_row8(T* p, const float (&f)[8]);
template <> __device__ __forceinline__ void store_row8<float>(float* p, const float (&f)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(f[4], f[5], f[6], f[7]);
}
template <typename T> __device__ __forceinline__ void store_row8_16(T* p, const float (&f)[8]) {
  uint4 a;
  a.x = pack2<T>(f[0], f[1]);
  a.y = pack2<T>(f[2], f[3]);
  a.z = pack2<T>(f[4], f[5]);
  a.w = pack2<T>(f[6], f[7]);
  *reinterpret_cast<uint4*>(p) = a;
}
template <> __device__ __forceinline__ void store_row8<f16_t>(f16_t* p, const float (&f)[8]) { store_row8_16(p, f); }
template <> __device__ __forceinline__ void store_row8<bf16_t>(bf16_t* p, const float (&f)[8]) { store_row8_16(p, f); }

// Round a float through the storage type T (what a store + reload would give).
template <typename T> __device__ __forceinline__ float through(float v) { return to_float<T>(from_float<T>(v)); }

__device__ __forceinline__ float block_sum(float v, float* s_red) {
  v = wave_sum(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < kThreads / kWave; ++i) t += s_red[i];
  __syncthreads();
  return t;
}

// One workgroup per row; each thread owns 8-element chunks (hidden % 8 == 0).
// ADD: residual r (in/out) += x first (the sum is stored rounded, as a
// separate bf16 add would leave it) and the norm reads the stored sum.
template <typename T, bool ADD>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(
    T* __restrict__ r, int64_t ldr, const T* __restrict__ x, int64_t ldx, const T* __restrict__ w,
    T* __restrict__ out, int64_t ldo, int hidden, float eps) {
  __shared__ float s_red[kThreads / kWave];
  constexpr int kMaxChunks = 8;  // hidden <= 8 * 8 * 256 = 16384
  const int row = blockIdx.x;
  const int chunks = hidden / 8;
  float v[kMaxChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int idx = (threadIdx.x + c * kThreads) * 8;
    if (threadIdx.x + c * kThreads < chunks) {
      if (ADD) {
        float a[8];
        load_row8<T>(r + row * ldr + idx, v[c]);
        load_row8<T>(x + row * ldx + idx, a);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] = through<T>(v[c][i] + a[i]);
        store_row8<T>(r + row * ldr + idx, v[c]);
      } else {
        load_row8<T>(x + row * ldx + idx, v[c]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(v[c][i], v[c][i], ss);
    }
  }
  ss = block_sum(ss, s_red);
  const float rstd = rsqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int idx = (threadIdx.x + c * kThreads) * 8;
    if (threadIdx.x + c * kThreads < chunks) {
      float wf[8];
      load_row8<T>(w + idx, wf);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = v[c][i] * rstd * wf[i];
      store_row8<T>(out + row * ldo + idx, v[c]);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const T* __restrict__ gu, int64_t ldg,
                                                            T* __restrict__ out, int64_t ldo,
                                                            int inter) {
  const int row = blockIdx.y;
  const int chunk = blockIdx.x * kThreads + threadIdx.x;
  if (chunk * 8 >= inter) return;
  float g[8], u[8], o[8];
  load_row8<T>(gu + row * ldg + chunk * 8, g);
  load_row8<T>(gu + row * ldg + inter + chunk * 8, u);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = g[i] / (1.f + expf(-g[i])) * u[i];
  store_row8<T>(out + row * ldo + chunk * 8, o);
}

// Grid (token, group of 4 heads); a wave takes one head; lane l holds dims l
// and l + D/2 (the rotate-half pair), i.e. D/128 pairs per lane.
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_append_kernel(
    const T* __restrict__ qkv, int64_t ld_qkv, const T* __restrict__ q_norm_w,
    const T* __restrict__ k_norm_w, const int64_t* __restrict__ positions,
    const int64_t* __restrict__ page_id, const int64_t* __restrict__ offset, T* __restrict__ q_out,
    T* __restrict__ k_cache, T* __restrict__ v_cache, int64_t page_stride, int64_t token_stride,
    int64_t head_stride, int64_t num_pages, int page_size, int hq, int hkv,
    const float* __restrict__ inv_freq, float eps) {
  constexpr int kPairs = D / 2;
  constexpr int kPPL = (kPairs + kWave - 1) / kWave;  // pairs per lane
  const int b = blockIdx.x;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const float pos = (float)positions[b];
  // rotation of pair i: angle = pos * inv_freq[i], the fp32 product the
  // reference forms (inv_freq is the caller's table, scaling folded in)
  float cs[kPPL], sn[kPPL];
#pragma unroll
  for (int j = 0; j < kPPL; ++j) {
    const int i = lane + j * kWave;
    sincosf(pos * (i < kPairs ? inv_freq[i] : 0.f), &sn[j], &cs[j]);
  }
  const int64_t p = page_id[b], off = offset[b];
  const bool slot_ok = p >= 0 && p < num_pages && off >= 0 && off < page_size;
  const T* row = qkv + b * ld_qkv;
  const int heads = hq + 2 * hkv;
  // grid.y spreads the heads: this wave's heads are h = blockIdx.y * 4 + wave (+ stride)
  for (int h = blockIdx.y * (kThreads / kWave) + wave; h < heads; h += gridDim.y * (kThreads / kWave)) {
    const bool is_q = h < hq, is_k = !is_q && h < hq + hkv;
    const T* src = row + (int64_t)h * D;
    float lo[kPPL], hi[kPPL];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kPPL; ++j) {
      const int i = lane + j * kWave;
      lo[j] = i < kPairs ? to_float<T>(src[i]) : 0.f;
      hi[j] = i < kPairs ? to_float<T>(src[i + kPairs]) : 0.f;
      ss += lo[j] * lo[j] + hi[j] * hi[j];
    }
    T* dst;
    if (is_q) {
      dst = q_out + ((int64_t)b * hq + h) * D;
    } else {
      if (!slot_ok) continue;  // a slot outside the pool is skipped, never written
      const int kvh = is_k ? h - hq : h - hq - hkv;
      dst = (is_k ? k_cache : v_cache) + p * page_stride + off * token_stride + (int64_t)kvh * head_stride;
    }
    if (is_q || is_k) {
      const T* nw = is_q ? q_norm_w : k_norm_w;
      if (nw != nullptr) {
        ss = wave_sum(ss);
        const float rstd = rsqrtf(ss / (float)D + eps);
#pragma unroll
        for (int j = 0; j < kPPL; ++j) {
          const int i = lane + j * kWave;
          if (i < kPairs) {
            lo[j] *= rstd * to_float<T>(nw[i]);
            hi[j] *= rstd * to_float<T>(nw[i + kPairs]);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kPPL; ++j) {
        const float a = lo[j], c = hi[j];
        lo[j] = a * cs[j] - c * sn[j];
        hi[j] = c * cs[j] + a * sn[j];
      }
    }
#pragma unroll
    for (int j = 0; j < kPPL; ++j) {
      const int i = lane + j * kWave;
      if (i < kPairs) {
        dst[i] = from_float<T>(lo[j]);
        dst[i + kPairs] = from_float<T>(hi[j]);
      }
    }
  }
}

}  // namespace fused
}  // namespace pl

using namespace pl;
using namespace pl::fused;

template <typename T>
static void launch_norm(bool add, void* r, int64_t ldr, const void* x, int64_t ldx, const void* w, void* out,
                        int64_t ldo, int rows, int hidden, float eps, hipStream_t s) {
  if (add)
    hipLaunchKernelGGL((rmsnorm_kernel<T, true>), dim3(rows), dim3(kThreads), 0, s, (T*)r, ldr, (const T*)x, ldx,
                       (const T*)w, (T*)out, ldo, hidden, eps);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<T, false>), dim3(rows), dim3(kThreads), 0, s, (T*)r, ldr, (const T*)x, ldx,
                       (const T*)w, (T*)out, ldo, hidden, eps);
}

static int norm_common(bool add, void* r, int64_t ldr, const void* x, int64_t ldx, const void* w, void* out,
                       int64_t ldo, int rows, int hidden, float eps, int dtype, void* stream) {
  if (rows < 0 || hidden <= 0 || hidden % 8 || hidden > 16384)
    return fail(PL_ERR_INVALID, "hidden must be a positive multiple of 8 up to 16384 (got %d)", hidden);
  if (rows == 0) return ok();
  if (!x || !w || !out || (add && !r)) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx % 8 || ldo % 8 || (add && ldr % 8)) return fail(PL_ERR_INVALID, "row strides must be multiples of 8");
  const void* ptrs[] = {x, w, out, add ? r : x};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return fail(PL_ERR_INVALID, "pointers must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case PL_DTYPE_F32: launch_norm<float>(add, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, s); break;
    case PL_DTYPE_F16: launch_norm<f16_t>(add, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, s); break;
    case PL_DTYPE_BF16: launch_norm<bf16_t>(add, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, s); break;
    default: return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
  }
  PL_LAUNCH_CHECK("rmsnorm_kernel");
  return ok();
}

extern "C" int pl_rmsnorm(const void* x, int64_t ldx, const void* weight, void* out, int64_t ldo, int rows,
                          int hidden, float eps, int dtype, void* stream) {
  return norm_common(false, nullptr, 0, x, ldx, weight, out, ldo, rows, hidden, eps, dtype, stream);
}

extern "C" int pl_add_rmsnorm(void* residual, int64_t ldr, const void* x, int64_t ldx, const void* weight,
                              void* out, int64_t ldo, int rows, int hidden, float eps, int dtype, void* stream) {
  return norm_common(true, residual, ldr, x, ldx, weight, out, ldo, rows, hidden, eps, dtype, stream);
}

extern "C" int pl_silu_mul(const void* gate_up, int64_t ldg, void* out, int64_t ldo, int rows, int inter,
                           int dtype, void* stream) {
  if (rows < 0 || inter <= 0 || inter % 8) return fail(PL_ERR_INVALID, "inter must be a positive multiple of 8");
  if (rows == 0) return ok();
  if (!gate_up || !out) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldg % 8 || ldo % 8 || (uintptr_t)gate_up % 16 || (uintptr_t)out % 16)
    return fail(PL_ERR_INVALID, "16-byte aligned rows required");
  dim3 grid((inter / 8 + kThreads - 1) / kThreads, rows);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case PL_DTYPE_F32:
      hipLaunchKernelGGL(silu_mul_kernel<float>, grid, dim3(kThreads), 0, s, (const float*)gate_up, ldg, (float*)out, ldo, inter);
      break;
    case PL_DTYPE_F16:
      hipLaunchKernelGGL(silu_mul_kernel<f16_t>, grid, dim3(kThreads), 0, s, (const f16_t*)gate_up, ldg, (f16_t*)out, ldo, inter);
      break;
    case PL_DTYPE_BF16:
      hipLaunchKernelGGL(silu_mul_kernel<bf16_t>, grid, dim3(kThreads), 0, s, (const bf16_t*)gate_up, ldg, (bf16_t*)out, ldo, inter);
      break;
    default:
      return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
  }
  PL_LAUNCH_CHECK("silu_mul_kernel");
  return ok();
}

template <typename T, int D>
static void launch_qkr(const void* qkv, int64_t ld, const void* qn, const void* kn, const int64_t* pos,
                       const int64_t* pid, const int64_t* off, void* q_out, void* kc, void* vc, int64_t ps_,
                       int64_t ts, int64_t hs, int64_t np, int page_size, int batch, int hq, int hkv,
                       const float* invf, float eps, hipStream_t s) {
  const int head_groups = (hq + 2 * hkv + kThreads / kWave - 1) / (kThreads / kWave);
  hipLaunchKernelGGL((qk_norm_rope_append_kernel<T, D>), dim3(batch, head_groups), dim3(kThreads), 0, s, (const T*)qkv, ld,
                     (const T*)qn, (const T*)kn, pos, pid, off, (T*)q_out, (T*)kc, (T*)vc, ps_, ts, hs, np,
                     page_size, hq, hkv, invf, eps);
}

template <typename T>
static int qkr_by_dim(int d, const void* qkv, int64_t ld, const void* qn, const void* kn, const int64_t* pos,
                      const int64_t* pid, const int64_t* off, void* q_out, void* kc, void* vc, int64_t ps_,
                      int64_t ts, int64_t hs, int64_t np, int page_size, int batch, int hq, int hkv,
                      const float* invf, float eps, hipStream_t s) {
  switch (d) {
    case 64: launch_qkr<T, 64>(qkv, ld, qn, kn, pos, pid, off, q_out, kc, vc, ps_, ts, hs, np, page_size, batch, hq, hkv, invf, eps, s); break;
    case 128: launch_qkr<T, 128>(qkv, ld, qn, kn, pos, pid, off, q_out, kc, vc, ps_, ts, hs, np, page_size, batch, hq, hkv, invf, eps, s); break;
    case 256: launch_qkr<T, 256>(qkv, ld, qn, kn, pos, pid, off, q_out, kc, vc, ps_, ts, hs, np, page_size, batch, hq, hkv, invf, eps, s); break;
    default: return fail(PL_ERR_UNSUPPORTED, "head_dim %d not built (64, 128, 256)", d);
  }
  PL_LAUNCH_CHECK("qk_norm_rope_append_kernel");
  return ok();
}

extern "C" int pl_qk_norm_rope_append(const void* qkv, int64_t ld_qkv, const void* q_norm_weight,
                                      const void* k_norm_weight, const int64_t* positions,
                                      const int64_t* page_id, const int64_t* offset, void* q_out,
                                      void* k_cache, void* v_cache, int64_t page_stride, int64_t token_stride,
                                      int64_t head_stride, int64_t num_pages, int page_size, int batch,
                                      int num_qo_heads, int num_kv_heads, int head_dim,
                                      const float* inv_freq, float eps, int dtype, void* stream) {
  if (batch < 0 || num_qo_heads <= 0 || num_kv_heads <= 0) return fail(PL_ERR_INVALID, "bad shape");
  if (batch == 0) return ok();
  if (!qkv || !positions || !page_id || !offset || !q_out || !k_cache || !v_cache || !inv_freq)
    return fail(PL_ERR_INVALID, "null pointer argument");
  if (num_pages <= 0 || page_size <= 0) return fail(PL_ERR_INVALID, "num_pages and page_size must be > 0");
  if (ld_qkv < (int64_t)(num_qo_heads + 2 * num_kv_heads) * head_dim)
    return fail(PL_ERR_INVALID, "ld_qkv is shorter than the q|k|v row");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case PL_DTYPE_F32:
      return qkr_by_dim<float>(head_dim, qkv, ld_qkv, q_norm_weight, k_norm_weight, positions, page_id, offset, q_out,
                               k_cache, v_cache, page_stride, token_stride, head_stride, num_pages, page_size, batch,
                               num_qo_heads, num_kv_heads, inv_freq, eps, s);
    case PL_DTYPE_F16:
      return qkr_by_dim<f16_t>(head_dim, qkv, ld_qkv, q_norm_weight, k_norm_weight, positions, page_id, offset, q_out,
                               k_cache, v_cache, page_stride, token_stride, head_stride, num_pages, page_size, batch,
                               num_qo_heads, num_kv_heads, inv_freq, eps, s);
    case PL_DTYPE_BF16:
      return qkr_by_dim<bf16_t>(head_dim, qkv, ld_qkv, q_norm_weight, k_norm_weight, positions, page_id, offset, q_out,
                                k_cache, v_cache, page_stride, token_stride, head_stride, num_pages, page_size, batch,
                                num_qo_heads, num_kv_heads, inv_freq, eps, s);
  }
  return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
}
