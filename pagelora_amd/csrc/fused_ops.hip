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
// Each kernel can also apply the up-projection of the no-merge LoRA delta
// to the columns it reads ("_lora" entry points): the producer GEMM ran on
// [W; A] stacked, so its extra columns hold y = x . A^T (rounded to the
// storage type, as the reference's F.linear(x, A) returns it); the kernel
// stages the token's y in LDS and forms
//   value[c] = round(base[c] + scale * sum_j y[j] * B[adapter][c][j])
// before its own arithmetic -- the module output the reference's
// LoRALinear.forward / _packed_lora_delta produce (multilora/linear.py:226-231,
// packed_ops.py:314-325), without a separate expand kernel.
//
// Reference: norm.py:15-65 (FlashInfer rmsnorm / fused_add_rmsnorm, fp32
// statistics, one rounding), packed_ops.py:230-239 (silu_and_mul),
// projection.py:155-190, 248-260 (apply_rope_pos_ids non-interleaved, head
// norm) and layer_runner.py:399-412 (the page append the fused kernel
// replaces).  All arithmetic is fp32; each output is rounded once.
#include <type_traits>

#include "pl_common.h"
#include "lora_up.h"

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

// A GEMM output given as split-K partial planes: element (t, c) is the fp32
// sum over planes s = 0, 1, .. of p[s * plane + t * ld + c], rounded through
// the storage type (what the GEMM's own output would hold).  splits == 0:
// not in use.
struct SplitIn {
  const float* p;
  int splits;
  int64_t ld, plane;
};

// Planes are read kPlaneBatch at a time with every load of a batch issued
// before the first add (an index past the last plane re-reads the last one
// and is not added), so a split row costs one memory round trip, not one per
// plane.  The sum still runs over planes 0, 1, .. in order.
constexpr int kPlaneBatch = 4;

// 8 consecutive elements (c % 8 == 0; ld, plane multiples of 8, p 16-byte aligned).
template <typename T>
__device__ __forceinline__ void load8_split(const SplitIn& sp, int64_t t, int c, float (&f)[8]) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int z0 = 0; z0 < sp.splits; z0 += kPlaneBatch) {
    float4 a[kPlaneBatch], b[kPlaneBatch];
#pragma unroll
    for (int k = 0; k < kPlaneBatch; ++k) {
      const float* q = sp.p + min(z0 + k, sp.splits - 1) * sp.plane + t * sp.ld + c;
      a[k] = *reinterpret_cast<const float4*>(q);
      b[k] = *reinterpret_cast<const float4*>(q + 4);
    }
#pragma unroll
    for (int k = 0; k < kPlaneBatch; ++k) {
      if (z0 + k < sp.splits) {
        acc[0] += a[k].x; acc[1] += a[k].y; acc[2] += a[k].z; acc[3] += a[k].w;
        acc[4] += b[k].x; acc[5] += b[k].y; acc[6] += b[k].z; acc[7] += b[k].w;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = through<T>(acc[i]);
}

template <typename T>
__device__ __forceinline__ float load1_split(const SplitIn& sp, int64_t t, int c) {
  float acc = 0.f;
  for (int z0 = 0; z0 < sp.splits; z0 += kPlaneBatch) {
    float v[kPlaneBatch];
#pragma unroll
    for (int k = 0; k < kPlaneBatch; ++k) v[k] = sp.p[min(z0 + k, sp.splits - 1) * sp.plane + t * sp.ld + c];
#pragma unroll
    for (int k = 0; k < kPlaneBatch; ++k)
      if (z0 + k < sp.splits) acc += v[k];
  }
  return through<T>(acc);
}

// y[t, a, :] of module m read from the partial planes (columns y_offset + a*R ..).
template <typename T, int R>
__device__ __forceinline__ void load_y_split(const SplitIn& sp, const LoraUp& m, int64_t t, int a, LoraRow<R>& y) {
#pragma unroll
  for (int v = 0; v < R / 8; ++v) {
    float f[8];
    load8_split<T>(sp, t, m.y_offset + a * R + v * 8, f);
    y.v[v] = make_uint4(pack2<T>(f[0], f[1]), pack2<T>(f[2], f[3]), pack2<T>(f[4], f[5]), pack2<T>(f[6], f[7]));
  }
}


template <int THREADS>
__device__ __forceinline__ float block_sum(float v, float* s_red) {
  v = wave_sum(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < THREADS / kWave; ++i) t += s_red[i];
  return t;
}

// One workgroup per row; each thread owns 8-element chunks (hidden % 8 == 0).
// ADD: residual r (in/out) += x first (the sum is stored rounded, as a
// separate bf16 add would leave it) and the norm reads the stored sum.
// R > 0 (with ADD): x is the base output of a LoRA module of rank R and gets
// its up-projection first, rounded as the module output (the reference's
// o_proj / down_proj output followed by `hidden + out`).
// Every global load a thread needs is issued before the first use.
template <typename T, bool ADD, int R, int THREADS>
__global__ __launch_bounds__(THREADS) void rmsnorm_kernel(
    T* __restrict__ r, int64_t ldr, const T* __restrict__ x, int64_t ldx, const T* __restrict__ w,
    T* __restrict__ out, int64_t ldo, int hidden, float eps, LoraUp lora, const int32_t* __restrict__ ids,
    int n_adapters, SplitIn xs) {
  __shared__ float s_red[THREADS / kWave];
  constexpr int kMaxChunks = 16384 / 8 / THREADS;
  const int row = blockIdx.x;
  const int chunks = hidden / 8;
  float v[kMaxChunks][8], xa[kMaxChunks][8], wf[kMaxChunks][8];
  // The adapter id first: the y and B loads depend on it, and with it in
  // hand they are issued together with the row's own loads.
  const int a_raw = R > 0 ? (lora.adapter >= 0 ? lora.adapter : ids[row]) : -1;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int idx = (threadIdx.x + c * THREADS) * 8;
    if (threadIdx.x + c * THREADS < chunks) {
      if (xs.splits > 0)
        load8_split<T>(xs, row, idx, xa[c]);
      else
        load_row8<T>(x + row * ldx + idx, xa[c]);
      if (ADD) load_row8<T>(r + row * ldr + idx, v[c]);
      load_row8<T>(w + idx, wf[c]);
    }
  }
  if constexpr (R > 0) {
    // No branch on the id before the loads: an id outside [0, n_adapters)
    // reads adapter 0 (n_adapters >= 1) and its delta is not applied.
    const bool a_ok = a_raw >= 0 && a_raw < n_adapters;
    const int a = a_ok ? a_raw : 0;
    LoraRow<R> y;
    if (xs.splits > 0)
      load_y_split<T, R>(xs, lora, row, a, y);
    else
      load_y<T, R>(lora, row, a, y);
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      const int idx = (threadIdx.x + c * THREADS) * 8;
      if (threadIdx.x + c * THREADS < chunks) {
        float d[8];
        lora_delta8<T, R>(lora, a, idx, y, d);
#pragma unroll
        for (int i = 0; i < 8; ++i) xa[c][i] = a_ok ? through<T>(xa[c][i] + d[i]) : xa[c][i];
      }
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int idx = (threadIdx.x + c * THREADS) * 8;
    if (threadIdx.x + c * THREADS < chunks) {
      if (ADD) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] = through<T>(v[c][i] + xa[c][i]);
        store_row8<T>(r + row * ldr + idx, v[c]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] = xa[c][i];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(v[c][i], v[c][i], ss);
    }
  }
  ss = block_sum<THREADS>(ss, s_red);
  const float rstd = rsqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int idx = (threadIdx.x + c * THREADS) * 8;
    if (threadIdx.x + c * THREADS < chunks) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = v[c][i] * rstd * wf[c][i];
      store_row8<T>(out + row * ldo + idx, v[c]);
    }
  }
}

// The decode-sized add + RMSNorm: one workgroup per row and exactly one
// 8-column chunk per thread (blockDim = hidden / 8 rounded up to whole
// waves, hidden <= 8192, 16-bit T).  Every load is issued before the first
// wait: the row's own loads together with the adapter id, then (needing only
// the id) the B rows and y, so the kernel costs two memory round trips.
// P = 0: x is a T row; P = 1..4: x (and y) are exactly P split-K planes,
// summed over planes 0, 1, .. in order.  Same arithmetic and roundings as
// rmsnorm_kernel<T, true, R>.
template <typename T, int P>
__device__ __forceinline__ void load8_planes(const SplitIn& sp, int64_t t, int c, float (&f)[8]) {
  float4 a[P], b[P];
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const float* q = sp.p + k * sp.plane + t * sp.ld + c;
    a[k] = *reinterpret_cast<const float4*>(q);
    b[k] = *reinterpret_cast<const float4*>(q + 4);
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < P; ++k) {
    acc[0] += a[k].x; acc[1] += a[k].y; acc[2] += a[k].z; acc[3] += a[k].w;
    acc[4] += b[k].x; acc[5] += b[k].y; acc[6] += b[k].z; acc[7] += b[k].w;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = through<T>(acc[i]);
}

constexpr int kRowNormMaxHidden = 8192;

// YS: the module's y comes from ys.splits fp32 side planes (the LoRA A rows
// of pl_linear_shuffled_side, column y_offset + a*R of each plane): thread
// r < R adds rank r over the planes in order (SplitOutput.sum's order), the
// sum is shared through LDS and rounded to T.
template <typename T, int R, int P, bool YS = false>
__global__ __launch_bounds__(1024) void add_rmsnorm_row_kernel(
    T* __restrict__ r, int64_t ldr, const T* __restrict__ x, int64_t ldx, const T* __restrict__ w,
    T* __restrict__ out, int64_t ldo, int hidden, float eps, LoraUp lora, const int32_t* __restrict__ ids,
    int n_adapters, SplitIn xs, SplitIn ys) {
  __shared__ float s_red[1024 / kWave];
  __shared__ float s_y[YS ? (R > 0 ? R : 1) : 1];
  const int row = blockIdx.x;
  const int a_raw = R > 0 ? (lora.adapter >= 0 ? lora.adapter : ids[row]) : -1;
  const bool live = (int)threadIdx.x * 8 < hidden;
  const int idx = live ? threadIdx.x * 8 : hidden - 8;  // idle threads re-read the last chunk
  float v[8], xa[8], wf[8];
  if constexpr (P > 0)
    load8_planes<T, P>(xs, row, idx, xa);
  else
    load_row8<T>(x + row * ldx + idx, xa);
  load_row8<T>(r + row * ldr + idx, v);
  load_row8<T>(w + idx, wf);
  if constexpr (R > 0) {
    // no branch on the id before the loads: an id outside [0, n_adapters)
    // reads adapter 0 (n_adapters >= 1) and its delta is not applied
    const bool a_ok = a_raw >= 0 && a_raw < n_adapters;
    const int a = a_ok ? a_raw : 0;
    float d[8];
    if constexpr (R <= 16) {
      // B rows first (they need only the id), then y, then the dots
      uint4 b[8][R / 8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int k = 0; k < R / 8; ++k) b[i][k] = *lora_b_piece<T, R>(lora, a, idx, i, k);
      // keep the scheduler from moving y's loads (and the wait for them)
      // in front of the B loads: both depend only on the id
      __builtin_amdgcn_sched_barrier(0);
      LoraRow<R> y;
      if constexpr (YS) {
        // thread r < R adds rank r's planes in plane order, 16 loads in
        // flight at a time (one memory round trip for up to 16 planes)
        if ((int)threadIdx.x < R) {
          const float* src = ys.p + (int64_t)row * ys.ld + lora.y_offset + (int64_t)a * R + threadIdx.x;
          float tot = 0.f;
          for (int p0 = 0; p0 < ys.splits; p0 += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = src[(int64_t)min(p0 + u, ys.splits - 1) * ys.plane];
#pragma unroll
            for (int u = 0; u < 16; ++u) tot += p0 + u < ys.splits ? v[u] : 0.f;
          }
          s_y[threadIdx.x] = tot;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < R / 8; ++k)
          y.v[k] = make_uint4(pack2<T>(s_y[k * 8 + 0], s_y[k * 8 + 1]), pack2<T>(s_y[k * 8 + 2], s_y[k * 8 + 3]),
                              pack2<T>(s_y[k * 8 + 4], s_y[k * 8 + 5]), pack2<T>(s_y[k * 8 + 6], s_y[k * 8 + 7]));
      } else if constexpr (P > 0) {
#pragma unroll
        for (int k = 0; k < R / 8; ++k) {
          float f[8];
          load8_planes<T, P>(xs, row, lora.y_offset + a * R + k * 8, f);
          y.v[k] = make_uint4(pack2<T>(f[0], f[1]), pack2<T>(f[2], f[3]), pack2<T>(f[4], f[5]),
                              pack2<T>(f[6], f[7]));
        }
      } else {
        load_y<T, R>(lora, row, a, y);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < R / 8; ++k) acc = dot8<T>(y.v[k], b[i][k], acc);
        d[i] = acc * lora.scale;
      }
    } else {
      LoraRow<R> y;
      if constexpr (P > 0) {
#pragma unroll
        for (int k = 0; k < R / 8; ++k) {
          float f[8];
          load8_planes<T, P>(xs, row, lora.y_offset + a * R + k * 8, f);
          y.v[k] = make_uint4(pack2<T>(f[0], f[1]), pack2<T>(f[2], f[3]), pack2<T>(f[4], f[5]),
                              pack2<T>(f[6], f[7]));
        }
      } else {
        load_y<T, R>(lora, row, a, y);
      }
      lora_delta8<T, R>(lora, a, idx, y, d);
    }
    // x + -0.f == x exactly and xa already holds a T value, so a row without
    // an adapter keeps its bits; the delta's loads stay unconditional.
#pragma unroll
    for (int i = 0; i < 8; ++i) xa[i] = through<T>(xa[i] + (a_ok ? d[i] : -0.f));
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = through<T>(v[i] + xa[i]);
    ss = fmaf(v[i], v[i], ss);
  }
  if (live) store_row8<T>(r + row * ldr + idx, v);
  ss = live ? ss : 0.f;
  // block sum over the launched waves
  ss = wave_sum(ss);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) s_red[wave] = ss;
  __syncthreads();
  float tot = 0.f;
  const int nw = blockDim.x / kWave;
  for (int i = 0; i < nw; ++i) tot += s_red[i];
  const float rstd = rsqrtf(tot / (float)hidden + eps);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = v[i] * rstd * wf[i];
  if (live) store_row8<T>(out + row * ldo + idx, v);
}

// One 8-column chunk per thread.  R > 0: lg / lu are the gate and up
// modules' up-projections (rank R), added to gate / up first.
template <typename T, int R>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const T* __restrict__ gu, int64_t ldg, T* __restrict__ out, int64_t ldo, int inter,
                                LoraUp lg, LoraUp lu, const int32_t* __restrict__ ids, int n_adapters) {
  const int row = blockIdx.y;
  const int chunk = blockIdx.x * blockDim.x + threadIdx.x;
  if (chunk * 8 >= inter) return;
  // The adapter first (its id load is the only branch); then the row's
  // values and the LoRA rows are loaded in one block, so every load is in
  // flight before the first wait.  No adapter: adapter 0's rows are read and
  // -0 is added instead of the delta.
  int a_ld = 0;
  bool a_ok = false;
  if constexpr (R > 0) {
    const int a = lg.adapter >= 0 ? lg.adapter : ids[row];
    a_ok = a >= 0 && a < n_adapters;
    a_ld = a_ok ? a : 0;
  }
  float g[8], u[8], o[8];
  load_row8<T>(gu + row * ldg + chunk * 8, g);
  load_row8<T>(gu + row * ldg + inter + chunk * 8, u);
  if constexpr (R > 0) {
    LoraRow<R> yg, yu;
    load_y<T, R>(lg, row, a_ld, yg);
    load_y<T, R>(lu, row, a_ld, yu);
    float dg[8], du[8];
    if constexpr (R <= 16) {
      lora_delta8_pair<T, R>(lg, lu, a_ld, chunk * 8, yg, yu, dg, du);
    } else {
      lora_delta8<T, R>(lg, a_ld, chunk * 8, yg, dg);
      lora_delta8<T, R>(lu, a_ld, chunk * 8, yu, du);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      g[i] = through<T>(g[i] + (a_ok ? dg[i] : -0.f));
      u[i] = through<T>(u[i] + (a_ok ? du[i] : -0.f));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = g[i] / (1.f + expf(-g[i])) * u[i];
  store_row8<T>(out + row * ldo + chunk * 8, o);
}

// SiLU*up with gate / up's LoRA rank-R up-projection (one wave per
// workgroup, 4 columns per lane: 256 per wave, twice the waves of the 8-column
// silu_mul_kernel, which at decode sizes is one wave per CU) that also forms
// down_proj's LoRA shrink: the product of the stored output (the down
// projection's input) with the same columns of the row's adapter's down A
// rows, read from the shuffled [W_down; A_down] weight (adapter a's rank r is
// row a_row0 + a * OR + r), summed over the wave's 256 columns in a fixed
// order and written as one partial per workgroup:
// part[row * ldp + blockIdx.x * OR + r].  An adapter outside [0,
// n_adapters) gives adapter 0's products (the consumer does not apply them).
constexpr int kShrinkCols = 4;  // columns per lane
struct DownShrink {
  const void* A;
  int ksteps;  // inter / 32
  int a_row0;
  float* part;
  int64_t ldp;
};

template <typename T, int R, int OR>
__global__ __launch_bounds__(kWave) void silu_mul_shrink_kernel(const T* __restrict__ gu, int64_t ldg,
                                                                T* __restrict__ out, int64_t ldo, int inter, LoraUp lg,
                                                                LoraUp lu, const int32_t* __restrict__ ids,
                                                                int n_adapters, DownShrink ds) {
  static_assert(R > 0 && R <= 16 && (OR == 8 || OR == 16), "gate / up rank up to 16, down rank 8 or 16");
  constexpr int C = kShrinkCols;
  const int row = blockIdx.y;
  const int lane = threadIdx.x;
  const int chunk_raw = blockIdx.x * kWave + lane;
  const bool live = chunk_raw * C < inter;
  const int c0 = (live ? chunk_raw : inter / C - 1) * C;  // idle lanes redo the last columns, contributing nothing
  const int a = lg.adapter >= 0 ? lg.adapter : ids[row];
  const bool a_ok = a >= 0 && a < n_adapters;
  const int a_ld = a_ok ? a : 0;
  float g[C], u[C], o[C];
  const uint2 gw = *reinterpret_cast<const uint2*>(gu + row * ldg + c0);
  const uint2 uw = *reinterpret_cast<const uint2*>(gu + row * ldg + inter + c0);
  LoraRow<R> yg, yu;
  load_y<T, R>(lg, row, a_ld, yg);
  load_y<T, R>(lu, row, a_ld, yu);
  __builtin_amdgcn_sched_barrier(0);  // y (scalar loads) out before the B and A pieces
  // gate's and up's B pieces of the lane's 4 columns: one base per module
  // (the 8-column group's, moved to its second half for c0 % 8 == 4) and
  // the uniform steps of the columns and rank pieces
  constexpr int KB = R >= 16 ? 2 : 1;
  uint4 bg[C][KB], bu[C][KB];
  {
    const int half = c0 & 7;
    const T* gb = lora_b_base<T, R>(lg, a_ld, c0 - half) + (half ? lora_b_step<R>(lg, half, 0) : 0);
    const T* ub = lora_b_base<T, R>(lu, a_ld, c0 - half) + (half ? lora_b_step<R>(lu, half, 0) : 0);
#pragma unroll
    for (int i = 0; i < C; ++i)
#pragma unroll
      for (int k = 0; k < KB; ++k) {
        bg[i][k] = *reinterpret_cast<const uint4*>(gb + lora_b_step<R>(lg, i, k));
        bu[i][k] = *reinterpret_cast<const uint4*>(ub + lora_b_step<R>(lu, i, k));
      }
  }
  // the down A half-pieces: ranks 0 .. OR-1 of columns c0 .. c0+3 (8 bytes of
  // the 16-byte piece that holds 8 consecutive columns of a rank)
  uint2 ap[OR];
  {
#pragma unroll
    for (int r = 0; r < OR; ++r) {
      const int64_t n = (int64_t)ds.a_row0 + (int64_t)a_ld * OR + r;
      const int64_t e = (((n / 16) * ds.ksteps + c0 / 32) * 64 + ((c0 % 32) / 8) * 16 + n % 16) * 8 + (c0 % 8);
      ap[r] = *reinterpret_cast<const uint2*>((const T*)ds.A + e);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  unpack2<T>(gw.x, g[0], g[1]);
  unpack2<T>(gw.y, g[2], g[3]);
  unpack2<T>(uw.x, u[0], u[1]);
  unpack2<T>(uw.y, u[2], u[3]);
#pragma unroll
  for (int i = 0; i < C; ++i) {
    float dg = 0.f, du = 0.f;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      dg = dot8<T>(yg.v[k], bg[i][k], dg);
      du = dot8<T>(yu.v[k], bu[i][k], du);
    }
    g[i] = through<T>(g[i] + (a_ok ? dg * lg.scale : -0.f));
    u[i] = through<T>(u[i] + (a_ok ? du * lu.scale : -0.f));
  }
#pragma unroll
  for (int i = 0; i < C; ++i) o[i] = g[i] / (1.f + expf(-g[i])) * u[i];
  // the stored values' 16-bit pairs (idle lanes zero) against the A pieces
  // on v_dot2
  uint2 ov = make_uint2(pack2_hw<T>(o[0], o[1]), pack2_hw<T>(o[2], o[3]));
  // every lane stores (an idle lane rewrites the last 4 columns with the
  // bits their own lane stores): under a test, the compiler sinks the
  // gate / up loads into it, behind every B and A load
  *reinterpret_cast<uint2*>(out + row * ldo + c0) = ov;
  if (!live) ov = make_uint2(0u, 0u);
  float p[OR];
#pragma unroll
  for (int r = 0; r < OR; ++r) p[r] = dot2<T>(ov.y, ap[r].y, dot2<T>(ov.x, ap[r].x, 0.f));
  // Transposed reduction: each step pairs lanes with DPP and halves the
  // values a lane holds (it keeps one of each pair and adds its partner's),
  // until lane i of every 16-lane row holds rank rank_of(i) summed over the
  // row; then the rows are summed.
  const int lr = lane % 16;
  float x;
  {
    float w8[OR / 2];
    const bool s3 = lr & 8;
#pragma unroll
    for (int k = 0; k < OR / 2; ++k)
      w8[k] = (s3 ? p[2 * k + 1] : p[2 * k]) + dpp_mov<0x128>(s3 ? p[2 * k] : p[2 * k + 1]);  // row_ror:8: lane ^ 8
    float w4[OR / 4];
    const bool s2 = lr & 4;
#pragma unroll
    for (int k = 0; k < OR / 4; ++k)  // row_half_mirror: lane ^ 7 (the same bit 3)
      w4[k] = (s2 ? w8[2 * k + 1] : w8[2 * k]) + dpp_mov<0x141>(s2 ? w8[2 * k] : w8[2 * k + 1]);
    float w2[OR / 8];
    const bool s1 = lr & 2;
#pragma unroll
    for (int k = 0; k < OR / 8; ++k)  // quad_perm [2,3,0,1]: lane ^ 2
      w2[k] = (s1 ? w4[2 * k + 1] : w4[2 * k]) + dpp_mov<0x4e>(s1 ? w4[2 * k] : w4[2 * k + 1]);
    const bool s0 = lr & 1;
    if constexpr (OR == 16)  // quad_perm [1,0,3,2]: lane ^ 1
      x = (s0 ? w2[1] : w2[0]) + dpp_mov<0xb1>(s0 ? w2[0] : w2[1]);
    else
      x = w2[0] + dpp_mov<0xb1>(w2[0]);
  }
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  // lane i of row 0 holds rank 8 (i&1) + 4 ((i>>1)&1) + 2 ((i>>2)&1) + (i>>3)
  // (OR == 8: 4 ((i>>1)&1) + 2 ((i>>2)&1) + (i>>3), lanes i and i ^ 1 alike)
  const int rk = OR == 16 ? 8 * (lr & 1) + 4 * ((lr >> 1) & 1) + 2 * ((lr >> 2) & 1) + (lr >> 3)
                          : 4 * ((lr >> 1) & 1) + 2 * ((lr >> 2) & 1) + (lr >> 3);
  if (lane < 16 && (OR == 16 || (lane & 1) == 0))
    ds.part[(int64_t)row * ds.ldp + (int64_t)blockIdx.x * OR + rk] = x;
}

// R > 0: the q, k and v modules' up-projections (rank R); their columns are
// head-major within each module.
struct QkvLora {
  LoraUp m[3];
};

// Grid (token, group of 4 heads); a wave takes one head; lane l holds dims l
// and l + D/2 (the rotate-half pair), i.e. D/128 pairs per lane.
template <typename T, int D, int R, bool SPLIT>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_append_kernel(
    const T* __restrict__ qkv, int64_t ld_qkv, const T* __restrict__ q_norm_w,
    const T* __restrict__ k_norm_w, const int64_t* __restrict__ positions,
    const int64_t* __restrict__ page_id, const int64_t* __restrict__ offset, T* __restrict__ q_out,
    T* __restrict__ k_cache, T* __restrict__ v_cache, int64_t page_stride, int64_t token_stride,
    int64_t head_stride, int64_t num_pages, int page_size, int hq, int hkv,
    const float* __restrict__ inv_freq, float eps, QkvLora lora, const int32_t* __restrict__ ids, int n_adapters,
    SplitIn xs) {
  constexpr int kPairs = D / 2;
  constexpr int kPPL = (kPairs + kWave - 1) / kWave;  // pairs per lane
  constexpr int RR = R > 0 ? R : 8;
  const int b = blockIdx.x;
  // the wave's head: the grid has ceil(heads / 4) groups of 4 waves, so each
  // wave has at most one; it is wave-uniform, and so is its LoRA module,
  // whose descriptor then comes from scalar loads
  const int lane = threadIdx.x % kWave, wave = uniform(threadIdx.x / kWave);
  const int heads = hq + 2 * hkv;
  const int h = blockIdx.y * (kThreads / kWave) + wave;
  if (h >= heads) return;
  const bool is_q = h < hq, is_k = !is_q && h < hq + hkv;
  const T* src = qkv + b * ld_qkv + (int64_t)h * D;

  // ---- every load first: the row's values, the norm weights, the LoRA
  // rows, the position and the append slot, all in one round trip
  float lo[kPPL], hi[kPPL];
#pragma unroll
  for (int j = 0; j < kPPL; ++j) {
    const int i = lane + j * kWave;
    if constexpr (SPLIT) {
      lo[j] = i < kPairs ? load1_split<T>(xs, b, h * D + i) : 0.f;
      hi[j] = i < kPairs ? load1_split<T>(xs, b, h * D + i + kPairs) : 0.f;
    } else {
      lo[j] = i < kPairs ? to_float<T>(src[i]) : 0.f;
      hi[j] = i < kPairs ? to_float<T>(src[i + kPairs]) : 0.f;
    }
  }
  // norm weights: loaded unconditionally (from the head's own input when the
  // head has none) and blended in with bit operations, so the loads are not
  // moved under a branch behind the sum of squares.  That fallback must be
  // readable memory of at least D elements: the head's T row, or with split-K
  // input (no T row exists; qkv is then only a placeholder) the head's fp32
  // values in plane 0, whose D floats hold 2D T-sized elements.
  const T* nw = is_q ? q_norm_w : (is_k ? k_norm_w : nullptr);
  const bool do_norm = nw != nullptr;
  const T* own = SPLIT ? reinterpret_cast<const T*>(xs.p + (int64_t)b * xs.ld + (int64_t)h * D) : src;
  const T* nwp = do_norm ? nw : own;
  const uint32_t keep = do_norm ? 0xffffffffu : 0u;
  float wlo[kPPL], whi[kPPL];
#pragma unroll
  for (int j = 0; j < kPPL; ++j) {
    const int i = lane + j * kWave;
    const float a0 = i < kPairs ? to_float<T>(nwp[i]) : 0.f;
    const float a1 = i < kPairs ? to_float<T>(nwp[i + kPairs]) : 0.f;
    wlo[j] = __uint_as_float((__float_as_uint(a0) & keep) | (0x3f800000u & ~keep));
    whi[j] = __uint_as_float((__float_as_uint(a1) & keep) | (0x3f800000u & ~keep));
  }
  // LoRA: the rows are read whether or not the token has an adapter (adapter
  // 0's when it has none, and a -0 added instead of the delta)
  if constexpr (R > 0) {
    const int a = lora.m[0].adapter >= 0 ? lora.m[0].adapter : ids[b];
    const bool a_ok = a >= 0 && a < n_adapters;
    const int a_ld = a_ok ? a : 0;
    const int mod = is_q ? 0 : (is_k ? 1 : 2);
    const int mcol = (h - (is_q ? 0 : (is_k ? hq : hq + hkv))) * D;  // first column in its module
    LoraRow<RR> ym;
    if constexpr (SPLIT)
      load_y_split<T, R>(xs, lora.m[mod], b, a_ld, ym);
    else
      load_y<T, R>(lora.m[mod], b, a_ld, ym);
#pragma unroll
    for (int j = 0; j < kPPL; ++j) {
      const int i = lane + j * kWave;
      if (i < kPairs) {
        const float dl = lora_delta1<T, R>(lora.m[mod], a_ld, mcol + i, ym);
        const float dh = lora_delta1<T, R>(lora.m[mod], a_ld, mcol + i + kPairs, ym);
        // no adapter: + (-0) and a rounding that leaves the T value as it is
        lo[j] = through<T>(lo[j] + (a_ok ? dl : -0.f));
        hi[j] = through<T>(hi[j] + (a_ok ? dh : -0.f));
      }
    }
  }
  const float pos = (float)positions[b];
  const int64_t p = page_id[b], off = offset[b];

  // ---- q/k: per-head RMSNorm, then the rotation.  Computed for every head
  // and kept for q/k only by a bit blend: under a q/k branch the compiler
  // moves the weight and position loads into it, behind the LoRA round trip.
  {
    const uint32_t qk = (is_q || is_k) ? 0xffffffffu : 0u;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kPPL; ++j) ss += lo[j] * lo[j] + hi[j] * hi[j];
    ss = wave_sum(ss);
    const float rstd = do_norm ? rsqrtf(ss / (float)D + eps) : 1.f;
#pragma unroll
    for (int j = 0; j < kPPL; ++j) {
      const int i = lane + j * kWave;
      // rotation of pair i: angle = pos * inv_freq[i], the fp32 product the
      // reference forms (inv_freq is the caller's table, scaling folded in)
      float sn, cs;
      sincosf(pos * (i < kPairs ? inv_freq[i] : 0.f), &sn, &cs);
      const float a0 = lo[j] * (rstd * wlo[j]), c = hi[j] * (rstd * whi[j]);
      const float rl = a0 * cs - c * sn, rh = c * cs + a0 * sn;
      lo[j] = __uint_as_float((__float_as_uint(rl) & qk) | (__float_as_uint(lo[j]) & ~qk));
      hi[j] = __uint_as_float((__float_as_uint(rh) & qk) | (__float_as_uint(hi[j]) & ~qk));
    }
  }

  // ---- store: q to q_out, k and v into their page slot
  T* dst;
  if (is_q) {
    dst = q_out + ((int64_t)b * hq + h) * D;
  } else {
    const bool slot_ok = p >= 0 && p < num_pages && off >= 0 && off < page_size;
    if (!slot_ok) return;  // a slot outside the pool is skipped, never written
    const int kvh = is_k ? h - hq : h - hq - hkv;
    dst = (is_k ? k_cache : v_cache) + p * page_stride + off * token_stride + (int64_t)kvh * head_stride;
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

}  // namespace fused
}  // namespace pl

using namespace pl;
using namespace pl::fused;

// Host copy of a pl_lora_up into the device struct, with its checks.
// With `split`, y is read from the split-K planes (h->y may be NULL) and its
// columns y_offset + n_adapters*rank must fit the planes' row.
// adapter ids: per token (ids required) or one bound adapter for all tokens
static int adapter_check(const pl_lora_up* mods, int n, const int32_t* ids, int n_adapters, const char* what) {
  if (n_adapters < 1) return fail(PL_ERR_INVALID, "%s: n_adapters must be >= 1", what);
  for (int m = 0; m < n; ++m) {
    if (mods[m].adapter != mods[0].adapter)
      return fail(PL_ERR_INVALID, "%s: every module of a call must bind the same adapter", what);
  }
  const int a = mods[0].adapter;
  if (a < -1 || a >= n_adapters) return fail(PL_ERR_INVALID, "%s: adapter %d outside [-1, %d)", what, a, n_adapters);
  if (a < 0 && !ids) return fail(PL_ERR_INVALID, "%s: per-token adapters need adapter_ids", what);
  return ok();
}

static int b_layout_check(const pl_lora_up* h, const char* what) {
  if (h->b_layout == PL_LORA_B_ROWS) return ok();
  if (h->b_layout != PL_LORA_B_CHUNK8) return fail(PL_ERR_INVALID, "%s: unknown b_layout %d", what, h->b_layout);
  if (h->out_features % 8) return fail(PL_ERR_INVALID, "%s: PL_LORA_B_CHUNK8 needs out_features %% 8 == 0", what);
  return ok();
}

static int lora_up_from(const pl_lora_up* h, int need_out, LoraUp* d, const char* what,
                        const SplitIn* split = nullptr, int n_adapters = 0) {
  if (split != nullptr) {
    if (!h->B) return fail(PL_ERR_INVALID, "%s: null B", what);
    if (h->rank != 8 && h->rank != 16 && h->rank != 32 && h->rank != 64)
      return fail(PL_ERR_UNSUPPORTED, "%s: rank %d not built (8, 16, 32, 64)", what, h->rank);
    if (h->out_features < need_out)
      return fail(PL_ERR_INVALID, "%s: B has %d output features, %d needed", what, h->out_features, need_out);
    if (h->y_offset < 0 || h->y_offset % 8 || (int64_t)h->y_offset + (int64_t)n_adapters * h->rank > split->ld)
      return fail(PL_ERR_INVALID, "%s: y columns outside the split planes' rows", what);
    if ((uintptr_t)h->B % 16) return fail(PL_ERR_INVALID, "%s: B must be 16-byte aligned", what);
    if (const int st = b_layout_check(h, what)) return st;
    *d = LoraUp{nullptr, 0, h->y_offset, h->B, h->out_features, h->rank, h->scale, h->b_layout, h->adapter};
    return ok();
  }
  if (!h->y || !h->B) return fail(PL_ERR_INVALID, "%s: null y or B", what);
  if (h->rank != 8 && h->rank != 16 && h->rank != 32 && h->rank != 64)
    return fail(PL_ERR_UNSUPPORTED, "%s: rank %d not built (8, 16, 32, 64)", what, h->rank);
  if (h->out_features < need_out)
    return fail(PL_ERR_INVALID, "%s: B has %d output features, %d needed", what, h->out_features, need_out);
  if (h->y_offset < 0 || h->ldy <= 0 || h->y_offset % 8 || h->ldy % 8 || (uintptr_t)h->y % 16)
    return fail(PL_ERR_INVALID, "%s: y must be 16-byte aligned with ldy and y_offset multiples of 8", what);
  if ((uintptr_t)h->B % 16) return fail(PL_ERR_INVALID, "%s: B must be 16-byte aligned", what);
  if (const int st = b_layout_check(h, what)) return st;
  *d = LoraUp{h->y, h->ldy, h->y_offset, h->B, h->out_features, h->rank, h->scale, h->b_layout, h->adapter};
  return ok();
}

namespace pl {
int lora_up_checked(const pl_lora_up* h, int need_out, LoraUp* d, const char* what) {
  return lora_up_from(h, need_out, d, what);
}
int lora_adapters_checked(const pl_lora_up* mods, int n, const int32_t* ids, int n_adapters, const char* what) {
  return adapter_check(mods, n, ids, n_adapters, what);
}
}  // namespace pl

// Host copy of a pl_split_out with its checks (need_cols: columns read per row).
static int split_from(const pl_split_out* h, int need_cols, SplitIn* d, const char* what) {
  if (!h->partials) return fail(PL_ERR_INVALID, "%s: null partials", what);
  if (h->splits < 1 || h->splits > 16) return fail(PL_ERR_INVALID, "%s: splits must be 1..16", what);
  if (h->ld < need_cols || h->ld % 8 || h->plane_stride % 8 || (uintptr_t)h->partials % 16)
    return fail(PL_ERR_INVALID, "%s: partial planes need ld >= %d, ld and plane stride multiples of 8, "
                "16-byte alignment", what, need_cols);
  *d = SplitIn{h->partials, h->splits, h->ld, h->plane_stride};
  return ok();
}

constexpr int kNormThreads = 512;

template <typename T, bool ADD, int R>
static void launch_norm_t(void* r, int64_t ldr, const void* x, int64_t ldx, const void* w, void* out, int64_t ldo,
                          int rows, int hidden, float eps, const LoraUp& lu, const int32_t* ids, int na,
                          const SplitIn& xs, hipStream_t s) {
  hipLaunchKernelGGL((rmsnorm_kernel<T, ADD, R, kNormThreads>), dim3(rows), dim3(kNormThreads), 0, s, (T*)r, ldr,
                     (const T*)x, ldx, (const T*)w, (T*)out, ldo, hidden, eps, lu, ids, na, xs);
}

template <typename T, int R, int P>
static void launch_row_norm_t(void* r, int64_t ldr, const void* x, int64_t ldx, const void* w, void* out,
                              int64_t ldo, int rows, int hidden, float eps, const LoraUp& lu, const int32_t* ids,
                              int na, const SplitIn& xs, hipStream_t s) {
  const int threads = (hidden / 8 + kWave - 1) / kWave * kWave;
  hipLaunchKernelGGL((add_rmsnorm_row_kernel<T, R, P>), dim3(rows), dim3(threads), 0, s, (T*)r, ldr, (const T*)x,
                     ldx, (const T*)w, (T*)out, ldo, hidden, eps, lu, ids, na, xs, SplitIn{nullptr, 0, 0, 0});
}

template <typename T, int P>
static void launch_row_norm_p(int rank, void* r, int64_t ldr, const void* x, int64_t ldx, const void* w, void* out,
                              int64_t ldo, int rows, int hidden, float eps, const LoraUp& lu, const int32_t* ids,
                              int na, const SplitIn& xs, hipStream_t s) {
  switch (rank) {
    case 0: launch_row_norm_t<T, 0, P>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
    case 8: launch_row_norm_t<T, 8, P>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
    case 16: launch_row_norm_t<T, 16, P>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
    case 32: launch_row_norm_t<T, 32, P>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
    case 64: launch_row_norm_t<T, 64, P>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
  }
}

template <typename T>
static int launch_norm(bool add, int rank, void* r, int64_t ldr, const void* x, int64_t ldx, const void* w,
                       void* out, int64_t ldo, int rows, int hidden, float eps, const LoraUp& lu,
                       const int32_t* ids, int na, const SplitIn& xs, hipStream_t s) {
  if constexpr (sizeof(T) == 2) {
    // decode-sized rows: the single-chunk kernel (two memory round trips)
    if (add && hidden <= kRowNormMaxHidden && xs.splits <= 4) {
      switch (xs.splits) {
        case 0: launch_row_norm_p<T, 0>(rank, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
        case 1: launch_row_norm_p<T, 1>(rank, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
        case 2: launch_row_norm_p<T, 2>(rank, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
        case 3: launch_row_norm_p<T, 3>(rank, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
        default: launch_row_norm_p<T, 4>(rank, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
      }
      PL_LAUNCH_CHECK("add_rmsnorm_row_kernel");
      return ok();
    }
  }
  if (rank == 0) {
    if (add)
      launch_norm_t<T, true, 0>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s);
    else
      launch_norm_t<T, false, 0>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s);
  } else if constexpr (sizeof(T) == 2) {
    switch (rank) {
      case 8: launch_norm_t<T, true, 8>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
      case 16: launch_norm_t<T, true, 16>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
      case 32: launch_norm_t<T, true, 32>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
      case 64: launch_norm_t<T, true, 64>(r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, na, xs, s); break;
    }
  } else {
    return fail(PL_ERR_UNSUPPORTED, "LoRA prologue needs F16 or BF16");
  }
  PL_LAUNCH_CHECK("rmsnorm_kernel");
  return ok();
}

static int norm_common(bool add, void* r, int64_t ldr, const void* x, int64_t ldx, const void* w, void* out,
                       int64_t ldo, int rows, int hidden, float eps, int dtype, void* stream,
                       const pl_lora_up* lora = nullptr, const int32_t* ids = nullptr, int n_adapters = 0,
                       const pl_split_out* x_split = nullptr) {
  if (rows < 0 || hidden <= 0 || hidden % 8 || hidden > 16384)
    return fail(PL_ERR_INVALID, "hidden must be a positive multiple of 8 up to 16384 (got %d)", hidden);
  if (rows == 0) return ok();
  SplitIn xs{nullptr, 0, 0, 0};
  if (x_split) {
    if (const int st = split_from(x_split, hidden, &xs, "add_rmsnorm input")) return st;
    x = w;  // unused: the input comes from the partial planes
    ldx = 0;
  }
  if (!x || !w || !out || (add && !r)) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx % 8 || ldo % 8 || (add && ldr % 8)) return fail(PL_ERR_INVALID, "row strides must be multiples of 8");
  const void* ptrs[] = {x, w, out, add ? r : x};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return fail(PL_ERR_INVALID, "pointers must be 16-byte aligned");
  LoraUp lu{};
  int rank = 0;
  if (lora) {
    if (const int st = adapter_check(lora, 1, ids, n_adapters, "add_rmsnorm LoRA")) return st;
    if (const int st = lora_up_from(lora, hidden, &lu, "add_rmsnorm LoRA", x_split ? &xs : nullptr, n_adapters))
      return st;
    rank = lu.rank;
  }
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case PL_DTYPE_F32: return launch_norm<float>(add, rank, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, n_adapters, xs, s);
    case PL_DTYPE_F16: return launch_norm<f16_t>(add, rank, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, n_adapters, xs, s);
    case PL_DTYPE_BF16: return launch_norm<bf16_t>(add, rank, r, ldr, x, ldx, w, out, ldo, rows, hidden, eps, lu, ids, n_adapters, xs, s);
  }
  return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
}

extern "C" int pl_rmsnorm(const void* x, int64_t ldx, const void* weight, void* out, int64_t ldo, int rows,
                          int hidden, float eps, int dtype, void* stream) {
  return norm_common(false, nullptr, 0, x, ldx, weight, out, ldo, rows, hidden, eps, dtype, stream);
}

extern "C" int pl_add_rmsnorm(void* residual, int64_t ldr, const void* x, int64_t ldx, const void* weight,
                              void* out, int64_t ldo, int rows, int hidden, float eps, int dtype, void* stream) {
  return norm_common(true, residual, ldr, x, ldx, weight, out, ldo, rows, hidden, eps, dtype, stream);
}

extern "C" int pl_add_rmsnorm_lora(void* residual, int64_t ldr, const void* x, int64_t ldx,
                                   const pl_split_out* x_split_h, const pl_lora_up* lora_h,
                                   const int32_t* adapter_ids, int num_adapters, const void* weight, void* out,
                                   int64_t ldo, int rows, int hidden, float eps, int dtype, void* stream) {
  if (!lora_h) return fail(PL_ERR_INVALID, "lora_h must not be null (use pl_add_rmsnorm)");
  return norm_common(true, residual, ldr, x, ldx, weight, out, ldo, rows, hidden, eps, dtype, stream, lora_h,
                     adapter_ids, num_adapters, x_split_h);
}

extern "C" int pl_add_rmsnorm_lora_side(void* residual, int64_t ldr, const void* x, int64_t ldx,
                                        const pl_split_out* y_side_h, const pl_lora_up* lora_h,
                                        const int32_t* adapter_ids, int num_adapters, const void* weight,
                                        void* out, int64_t ldo, int rows, int hidden, float eps, int dtype,
                                        void* stream) {
  if (!lora_h || !y_side_h) return fail(PL_ERR_INVALID, "lora_h and y_side_h must not be null");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_add_rmsnorm_lora_side dtype must be F16 or BF16 (got %d)", dtype);
  if (rows < 0 || hidden <= 0 || hidden % 8 || hidden > kRowNormMaxHidden)
    return fail(PL_ERR_INVALID, "hidden must be a positive multiple of 8 up to %d (got %d)", kRowNormMaxHidden,
                hidden);
  if (rows == 0) return ok();
  if (!x || !weight || !out || !residual) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx % 8 || ldo % 8 || ldr % 8) return fail(PL_ERR_INVALID, "row strides must be multiples of 8");
  const void* ptrs[] = {x, weight, out, residual};
  for (const void* q : ptrs)
    if ((uintptr_t)q % 16) return fail(PL_ERR_INVALID, "pointers must be 16-byte aligned");
  const pl_split_out& ysh = *y_side_h;
  if (!ysh.partials || ysh.splits < 1 || ysh.splits > 64 || ysh.ld <= 0 || ysh.plane_stride < ysh.ld * rows)
    return fail(PL_ERR_INVALID, "y side planes: 1..64 planes of rows x ld floats, non-overlapping");
  const SplitIn ys{ysh.partials, ysh.splits, ysh.ld, ysh.plane_stride};
  if (const int st = adapter_check(lora_h, 1, adapter_ids, num_adapters, "add_rmsnorm LoRA")) return st;
  LoraUp lu{};
  if (const int st = lora_up_from(lora_h, hidden, &lu, "add_rmsnorm LoRA", &ys, num_adapters)) return st;
  if (lu.rank != 8 && lu.rank != 16) return fail(PL_ERR_UNSUPPORTED, "side-plane y: rank 8 or 16 (got %d)", lu.rank);
  const int threads = (hidden / 8 + kWave - 1) / kWave * kWave;
  const SplitIn none{nullptr, 0, 0, 0};
  hipStream_t s = (hipStream_t)stream;
  auto go = [&](auto tag, auto rank) {
    using T = decltype(tag);
    constexpr int R = decltype(rank)::value;
    hipLaunchKernelGGL((add_rmsnorm_row_kernel<T, R, 0, true>), dim3(rows), dim3(threads), 0, s, (T*)residual, ldr,
                       (const T*)x, ldx, (const T*)weight, (T*)out, ldo, hidden, eps, lu, adapter_ids, num_adapters,
                       none, ys);
  };
  if (dtype == PL_DTYPE_BF16) {
    if (lu.rank == 8) go(bf16_t{}, std::integral_constant<int, 8>{});
    else go(bf16_t{}, std::integral_constant<int, 16>{});
  } else {
    if (lu.rank == 8) go(f16_t{}, std::integral_constant<int, 8>{});
    else go(f16_t{}, std::integral_constant<int, 16>{});
  }
  PL_LAUNCH_CHECK("add_rmsnorm_row_kernel");
  return ok();
}

// Plain SiLU*up: 256 threads per workgroup; with the LoRA prologue every
// thread also streams 8 B rows per module, so workgroups shrink to 64
// threads to spread those reads over more CUs.
template <typename T, int R>
static void launch_silu_t(hipStream_t s, const void* gu, int64_t ldg, void* out, int64_t ldo, int rows, int inter,
                          const LoraUp& lg, const LoraUp& lu, const int32_t* ids, int na) {
  const int threads = R > 0 ? 64 : kThreads;
  dim3 grid((inter / 8 + threads - 1) / threads, rows);
  hipLaunchKernelGGL((silu_mul_kernel<T, R>), grid, dim3(threads), 0, s, (const T*)gu, ldg, (T*)out, ldo, inter, lg,
                     lu, ids, na);
}

template <typename T>
static int launch_silu(int rank, hipStream_t s, const void* gu, int64_t ldg, void* out, int64_t ldo, int rows,
                       int inter, const LoraUp& lg, const LoraUp& lu, const int32_t* ids, int na) {
  if (rank == 0) {
    launch_silu_t<T, 0>(s, gu, ldg, out, ldo, rows, inter, lg, lu, ids, na);
  } else if constexpr (sizeof(T) == 2) {
    switch (rank) {
      case 8: launch_silu_t<T, 8>(s, gu, ldg, out, ldo, rows, inter, lg, lu, ids, na); break;
      case 16: launch_silu_t<T, 16>(s, gu, ldg, out, ldo, rows, inter, lg, lu, ids, na); break;
      case 32: launch_silu_t<T, 32>(s, gu, ldg, out, ldo, rows, inter, lg, lu, ids, na); break;
      case 64: launch_silu_t<T, 64>(s, gu, ldg, out, ldo, rows, inter, lg, lu, ids, na); break;
    }
  } else {
    return fail(PL_ERR_UNSUPPORTED, "LoRA prologue needs F16 or BF16");
  }
  PL_LAUNCH_CHECK("silu_mul_kernel");
  return ok();
}

static int silu_common(const void* gate_up, int64_t ldg, void* out, int64_t ldo, int rows, int inter, int dtype,
                       void* stream, const pl_lora_up* lora, const int32_t* ids, int n_adapters) {
  if (rows < 0 || inter <= 0 || inter % 8) return fail(PL_ERR_INVALID, "inter must be a positive multiple of 8");
  if (rows == 0) return ok();
  if (!gate_up || !out) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldg % 8 || ldo % 8 || (uintptr_t)gate_up % 16 || (uintptr_t)out % 16)
    return fail(PL_ERR_INVALID, "16-byte aligned rows required");
  LoraUp lg{}, lu{};
  int rank = 0;
  if (lora) {
    if (const int st = adapter_check(lora, 2, ids, n_adapters, "silu_mul LoRA")) return st;
    if (const int st = lora_up_from(&lora[0], inter, &lg, "silu_mul gate LoRA")) return st;
    if (const int st = lora_up_from(&lora[1], inter, &lu, "silu_mul up LoRA")) return st;
    if (lg.rank != lu.rank) return fail(PL_ERR_UNSUPPORTED, "gate and up LoRA ranks differ (%d, %d)", lg.rank, lu.rank);
    rank = lg.rank;
  }
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case PL_DTYPE_F32: return launch_silu<float>(rank, s, gate_up, ldg, out, ldo, rows, inter, lg, lu, ids, n_adapters);
    case PL_DTYPE_F16: return launch_silu<f16_t>(rank, s, gate_up, ldg, out, ldo, rows, inter, lg, lu, ids, n_adapters);
    case PL_DTYPE_BF16: return launch_silu<bf16_t>(rank, s, gate_up, ldg, out, ldo, rows, inter, lg, lu, ids, n_adapters);
  }
  return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
}

extern "C" int pl_silu_mul(const void* gate_up, int64_t ldg, void* out, int64_t ldo, int rows, int inter,
                           int dtype, void* stream) {
  return silu_common(gate_up, ldg, out, ldo, rows, inter, dtype, stream, nullptr, nullptr, 0);
}

extern "C" int pl_silu_mul_lora_shrink(const void* gate_up, int64_t ldg, const pl_lora_up* lora_gate_up_h,
                                       const int32_t* adapter_ids, int num_adapters, void* out, int64_t ldo, int rows,
                                       int inter, const pl_lora_a_rows* down_lora_a,
                                       const pl_lora_partials* down_lora_y, int dtype, void* stream) {
  if (rows < 0 || inter <= 0 || inter % 32) return fail(PL_ERR_INVALID, "inter must be a positive multiple of 32");
  if (rows == 0) return ok();
  if (!gate_up || !out || !lora_gate_up_h || !down_lora_a || !down_lora_y)
    return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldg % 8 || ldo % 8 || (uintptr_t)gate_up % 16 || (uintptr_t)out % 16)
    return fail(PL_ERR_INVALID, "16-byte aligned rows required");
  if (dtype != PL_DTYPE_F16 && dtype != PL_DTYPE_BF16)
    return fail(PL_ERR_UNSUPPORTED, "pl_silu_mul_lora_shrink dtype must be F16 or BF16 (got %d)", dtype);
  if (const int st = adapter_check(lora_gate_up_h, 2, adapter_ids, num_adapters, "silu_mul LoRA")) return st;
  LoraUp lg{}, lu{};
  if (const int st = lora_up_from(&lora_gate_up_h[0], inter, &lg, "silu_mul gate LoRA")) return st;
  if (const int st = lora_up_from(&lora_gate_up_h[1], inter, &lu, "silu_mul up LoRA")) return st;
  if (lg.rank != lu.rank || lg.rank > 16)
    return fail(PL_ERR_UNSUPPORTED, "gate and up LoRA: one rank up to 16 (got %d, %d)", lg.rank, lu.rank);
  const pl_lora_a_rows& da = *down_lora_a;
  const pl_lora_partials& dy = *down_lora_y;
  if (da.rank != 8 && da.rank != 16) return fail(PL_ERR_UNSUPPORTED, "down_proj shrink rank %d not built (8, 16)", da.rank);
  if (da.adapter != lora_gate_up_h[0].adapter)
    return fail(PL_ERR_INVALID, "down_proj's A rows must bind the gate / up modules' adapter");
  if (!da.shuffled || (uintptr_t)da.shuffled % 16 || da.in_features != inter || da.a_row0 < 0 ||
      (int64_t)da.a_row0 + (int64_t)num_adapters * da.rank > da.out_features)
    return fail(PL_ERR_INVALID, "down_proj A rows: a 16-byte aligned shuffled weight %d wide (got %d) whose %d rows "
                "hold rows a_row0 (%d) .. + %d adapters x rank %d", inter, da.in_features, da.out_features, da.a_row0,
                num_adapters, da.rank);
  const int parts = (inter / kShrinkCols + kWave - 1) / kWave;
  if (!dy.partials || (uintptr_t)dy.partials % 16 || dy.rank != da.rank || dy.parts != parts ||
      dy.ld < (int64_t)parts * dy.rank || dy.ld % 4)
    return fail(PL_ERR_INVALID, "down_proj partials: rank %d, %d parts per row (one per 256 columns), ld >= %d and a "
                "multiple of 4, 16-byte aligned", da.rank, parts, parts * da.rank);
  const DownShrink dsh{da.shuffled, inter / 32, da.a_row0, dy.partials, dy.ld};
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(parts, rows);
  auto go = [&](auto t, auto r, auto orr) {
    using T = decltype(t);
    constexpr int R = decltype(r)::value, OR = decltype(orr)::value;
    hipLaunchKernelGGL((silu_mul_shrink_kernel<T, R, OR>), grid, dim3(kWave), 0, s, (const T*)gate_up, ldg, (T*)out,
                       ldo, inter, lg, lu, adapter_ids, num_adapters, dsh);
  };
  auto by_or = [&](auto t, auto r) {
    if (da.rank == 8) go(t, r, std::integral_constant<int, 8>{});
    else go(t, r, std::integral_constant<int, 16>{});
  };
  auto by_r = [&](auto t) {
    if (lg.rank == 8) by_or(t, std::integral_constant<int, 8>{});
    else by_or(t, std::integral_constant<int, 16>{});
  };
  if (dtype == PL_DTYPE_BF16) by_r(bf16_t{});
  else by_r(f16_t{});
  PL_LAUNCH_CHECK("silu_mul_shrink_kernel");
  return ok();
}

extern "C" int pl_silu_mul_lora(const void* gate_up, int64_t ldg, const pl_lora_up* lora_gate_up_h,
                                const int32_t* adapter_ids, int num_adapters, void* out, int64_t ldo, int rows,
                                int inter, int dtype, void* stream) {
  if (!lora_gate_up_h) return fail(PL_ERR_INVALID, "lora_gate_up_h must not be null (use pl_silu_mul)");
  return silu_common(gate_up, ldg, out, ldo, rows, inter, dtype, stream, lora_gate_up_h, adapter_ids, num_adapters);
}

struct QkrArgs {
  const void *qkv, *qn, *kn;
  int64_t ld;
  const int64_t *pos, *pid, *off;
  void *q_out, *kc, *vc;
  int64_t ps_, ts, hs, np;
  int page_size, batch, hq, hkv;
  const float* invf;
  float eps;
  QkvLora lora;
  const int32_t* ids;
  int na;
  SplitIn xs;
};

template <typename T, int D, int R>
static void launch_qkr(const QkrArgs& a, hipStream_t s) {
  const int head_groups = (a.hq + 2 * a.hkv + kThreads / kWave - 1) / (kThreads / kWave);
  auto kern = a.xs.splits > 0 ? qk_norm_rope_append_kernel<T, D, R, true> : qk_norm_rope_append_kernel<T, D, R, false>;
  hipLaunchKernelGGL(kern, dim3(a.batch, head_groups), dim3(kThreads), 0, s,
                     (const T*)a.qkv, a.ld, (const T*)a.qn, (const T*)a.kn, a.pos, a.pid, a.off, (T*)a.q_out,
                     (T*)a.kc, (T*)a.vc, a.ps_, a.ts, a.hs, a.np, a.page_size, a.hq, a.hkv, a.invf, a.eps, a.lora,
                     a.ids, a.na, a.xs);
}

template <typename T, int R>
static int qkr_by_dim(int d, const QkrArgs& a, hipStream_t s) {
  switch (d) {
    case 64: launch_qkr<T, 64, R>(a, s); break;
    case 128: launch_qkr<T, 128, R>(a, s); break;
    case 256: launch_qkr<T, 256, R>(a, s); break;
    default: return fail(PL_ERR_UNSUPPORTED, "head_dim %d not built (64, 128, 256)", d);
  }
  PL_LAUNCH_CHECK("qk_norm_rope_append_kernel");
  return ok();
}

template <typename T>
static int qkr_by_rank(int rank, int d, const QkrArgs& a, hipStream_t s) {
  if (rank == 0) return qkr_by_dim<T, 0>(d, a, s);
  if constexpr (sizeof(T) == 2) {
    switch (rank) {
      case 8: return qkr_by_dim<T, 8>(d, a, s);
      case 16: return qkr_by_dim<T, 16>(d, a, s);
      case 32: return qkr_by_dim<T, 32>(d, a, s);
      case 64: return qkr_by_dim<T, 64>(d, a, s);
    }
    return fail(PL_ERR_UNSUPPORTED, "rank %d", rank);
  } else {
    return fail(PL_ERR_UNSUPPORTED, "LoRA prologue needs F16 or BF16");
  }
}

static int qkr_by_dtype(int dtype, int rank, int d, const QkrArgs& a, hipStream_t s) {
  switch (dtype) {
    case PL_DTYPE_F32: return qkr_by_rank<float>(rank, d, a, s);
    case PL_DTYPE_F16: return qkr_by_rank<f16_t>(rank, d, a, s);
    case PL_DTYPE_BF16: return qkr_by_rank<bf16_t>(rank, d, a, s);
  }
  return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
}

static int qkr_common(const void* qkv, int64_t ld_qkv, const void* q_norm_weight, const void* k_norm_weight,
                      const int64_t* positions, const int64_t* page_id, const int64_t* offset, void* q_out,
                      void* k_cache, void* v_cache, int64_t page_stride, int64_t token_stride, int64_t head_stride,
                      int64_t num_pages, int page_size, int batch, int num_qo_heads, int num_kv_heads, int head_dim,
                      const float* inv_freq, float eps, int dtype, void* stream, const pl_lora_up* lora,
                      const int32_t* ids, int n_adapters, const pl_split_out* qkv_split = nullptr) {
  if (batch < 0 || num_qo_heads <= 0 || num_kv_heads <= 0) return fail(PL_ERR_INVALID, "bad shape");
  if (batch == 0) return ok();
  const int row_cols = (num_qo_heads + 2 * num_kv_heads) * head_dim;
  SplitIn xs{nullptr, 0, 0, 0};
  if (qkv_split) {
    if (const int st = split_from(qkv_split, row_cols, &xs, "qkv input")) return st;
    // The row comes from the partial planes: the kernel never dereferences
    // qkv in this mode (it must only be non-null for the checks below).
    qkv = inv_freq;
    ld_qkv = row_cols;
  }
  if (!qkv || !positions || !page_id || !offset || !q_out || !k_cache || !v_cache || !inv_freq)
    return fail(PL_ERR_INVALID, "null pointer argument");
  if (num_pages <= 0 || page_size <= 0) return fail(PL_ERR_INVALID, "num_pages and page_size must be > 0");
  if (ld_qkv < (int64_t)row_cols) return fail(PL_ERR_INVALID, "ld_qkv is shorter than the q|k|v row");
  QkrArgs a{qkv, q_norm_weight, k_norm_weight, ld_qkv, positions, page_id, offset, q_out, k_cache, v_cache,
            page_stride, token_stride, head_stride, num_pages, page_size, batch, num_qo_heads, num_kv_heads,
            inv_freq, eps, QkvLora{}, ids, n_adapters, xs};
  if (lora) {
    if (const int st = adapter_check(lora, 3, ids, n_adapters, "qk_norm_rope_append LoRA")) return st;
    const int need[3] = {num_qo_heads * head_dim, num_kv_heads * head_dim, num_kv_heads * head_dim};
    const char* names[3] = {"q LoRA", "k LoRA", "v LoRA"};
    for (int m = 0; m < 3; ++m)
      if (const int st = lora_up_from(&lora[m], need[m], &a.lora.m[m], names[m], qkv_split ? &xs : nullptr,
                                      n_adapters))
        return st;
    if (a.lora.m[1].rank != a.lora.m[0].rank || a.lora.m[2].rank != a.lora.m[0].rank)
      return fail(PL_ERR_UNSUPPORTED, "q, k and v LoRA ranks differ");
    return qkr_by_dtype(dtype, a.lora.m[0].rank, head_dim, a, (hipStream_t)stream);
  }
  return qkr_by_dtype(dtype, 0, head_dim, a, (hipStream_t)stream);
}

extern "C" int pl_qk_norm_rope_append(const void* qkv, int64_t ld_qkv, const void* q_norm_weight,
                                      const void* k_norm_weight, const int64_t* positions,
                                      const int64_t* page_id, const int64_t* offset, void* q_out,
                                      void* k_cache, void* v_cache, int64_t page_stride, int64_t token_stride,
                                      int64_t head_stride, int64_t num_pages, int page_size, int batch,
                                      int num_qo_heads, int num_kv_heads, int head_dim,
                                      const float* inv_freq, float eps, int dtype, void* stream) {
  return qkr_common(qkv, ld_qkv, q_norm_weight, k_norm_weight, positions, page_id, offset, q_out, k_cache, v_cache,
                    page_stride, token_stride, head_stride, num_pages, page_size, batch, num_qo_heads, num_kv_heads,
                    head_dim, inv_freq, eps, dtype, stream, nullptr, nullptr, 0);
}

extern "C" int pl_qk_norm_rope_append_lora(const void* qkv, int64_t ld_qkv, const pl_split_out* qkv_split_h,
                                           const pl_lora_up* lora_qkv_h,
                                           const int32_t* adapter_ids, int num_adapters, const void* q_norm_weight,
                                           const void* k_norm_weight, const int64_t* positions,
                                           const int64_t* page_id, const int64_t* offset, void* q_out,
                                           void* k_cache, void* v_cache, int64_t page_stride,
                                           int64_t token_stride, int64_t head_stride, int64_t num_pages,
                                           int page_size, int batch, int num_qo_heads, int num_kv_heads,
                                           int head_dim, const float* inv_freq, float eps, int dtype,
                                           void* stream) {
  if (!lora_qkv_h) return fail(PL_ERR_INVALID, "lora_qkv_h must not be null (use pl_qk_norm_rope_append)");
  return qkr_common(qkv, ld_qkv, q_norm_weight, k_norm_weight, positions, page_id, offset, q_out, k_cache, v_cache,
                    page_stride, token_stride, head_stride, num_pages, page_size, batch, num_qo_heads, num_kv_heads,
                    head_dim, inv_freq, eps, dtype, stream, lora_qkv_h, adapter_ids, num_adapters, qkv_split_h);
}

// cos and sin of positions[b] * inv_freq[i] for every row and rotation pair:
// the angles of one decode step, shared by all its layers (the same fp32
// product and sincosf as qk_norm_rope_append_kernel).
__global__ __launch_bounds__(64) void rope_cos_sin_kernel(const int64_t* __restrict__ positions,
                                                          const float* __restrict__ inv_freq, int half,
                                                          float* __restrict__ out) {
  const int b = blockIdx.x;
  const float pos = (float)positions[b];
  for (int i = threadIdx.x; i < half; i += 64) {
    float sn, cs;
    sincosf(pos * inv_freq[i], &sn, &cs);
    *reinterpret_cast<float2*>(out + ((int64_t)b * half + i) * 2) = make_float2(cs, sn);
  }
}

extern "C" int pl_rope_cos_sin(const int64_t* positions, int batch, const float* inv_freq, int half_dim, float* out,
                               void* stream) {
  if (batch < 0 || half_dim <= 0) return fail(PL_ERR_INVALID, "batch must be >= 0 and half_dim > 0");
  if (batch == 0) return ok();
  if (!positions || !inv_freq || !out) return fail(PL_ERR_INVALID, "null pointer argument");
  if ((uintptr_t)out % 8) return fail(PL_ERR_INVALID, "out must be 8-byte aligned");
  hipLaunchKernelGGL(rope_cos_sin_kernel, dim3(batch), dim3(64), 0, (hipStream_t)stream, positions, inv_freq,
                     half_dim, out);
  PL_LAUNCH_CHECK("rope_cos_sin_kernel");
  return ok();
}
