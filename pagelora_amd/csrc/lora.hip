// No-merge multi-adapter LoRA delta for gfx950:
//   out_m[t] += scale_m * B_m[a_t] . (A_m[a_t] . x[t])
// for the modules m of a group that share their input x (q/k/v, gate/up, or a
// lone o_proj / down_proj) and per-token adapter ids a_t.
//
//   shrink_kernel  grid (k-slice, 16 rank rows, adapter).  Gathers the
//                  tokens of its adapter (LDS list), multiplies their x
//                  slice by the adapter's concatenated A rows on MFMA
//                  16x16x32 tiles and writes fp32 partial sums per slice.
//   expand_kernel  grid (16-column tiles x 4, adapter).  Folds the slices
//                  into the rank-r intermediate rounded to the input dtype
//                  (as the reference's F.linear returns it), multiplies it
//                  by B^T on MFMA 16x16x32 tiles and accumulates
//                  scale * result into the outputs in place.
//                  The contraction runs over the group's concatenated ranks,
//                  with the B operand zero outside the column's own module,
//                  i.e. the block-diagonal product of the reference without
//                  storing its zeros.
//
// Reference semantics: packed_ops.py:314-384 (packed A_cat / block-diagonal
// B with the scale folded in), packed_ops.py:534-553 and
// multilora/linear.py:226-231 (per-module F.linear(F.linear(x, A), B) * s).
#include "pl_common.h"

namespace pl {
namespace lora {

constexpr int kWave = 64;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxTokens = 4096; // tokens per call (LDS token list)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Mod {
  const void* A;
  const void* B;
  void* out;
  int64_t ldo;
  int out_features, rank, out_offset, rank_offset;
  float scale;
};

struct Group {
  Mod m[PL_LORA_MAX_MODULES];
  int n;          // modules
  int r_total;    // sum of ranks
  int r_pad;      // r_total rounded up to 32
  int out_total;  // sum of out_features
};

template <typename T> __device__ __forceinline__ f32x4 mfma32(uint4 a, uint4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma32<bf16_t>(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma32<f16_t>(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}



// Gather the tokens of adapter `a` into LDS; returns their count (all threads).
__device__ __forceinline__ int gather_tokens(const int32_t* __restrict__ ids, int tokens, int a,
                                             int* s_list, int* s_count, int nthreads) {
  if (threadIdx.x == 0) *s_count = 0;
  __syncthreads();
  for (int t = threadIdx.x; t < tokens; t += nthreads) {
    if (ids[t] == a) {
      const int slot = atomicAdd(s_count, 1);
      s_list[slot] = t;
    }
  }
  __syncthreads();
  return *s_count;
}

// Load 8 consecutive 16-bit elements as one 16-byte word, or zeros.
__device__ __forceinline__ uint4 load8(const void* p, bool ok) {
  if (!ok) return make_uint4(0, 0, 0, 0);
  return *reinterpret_cast<const uint4*>(p);
}

// Shrink: split-K.  Workgroup (k-slice, 16 rank rows, adapter) multiplies the
// adapter's tokens (up to four 16-token tiles per pass) by 16 rows of its
// concatenated A over one k-slice on MFMA 16x16x32; its four waves split the
// slice and are summed in LDS; the fp32 partial goes to part[slice][token][j].
// The slice count grows as the token count shrinks (decode: many slices,
// so the A rows stream from many CUs at once).
constexpr int kShrinkWaves = 4;
constexpr int kShrinkThreads = kShrinkWaves * kWave;
constexpr int kTilesPerPass = 4;

inline int ksplit_for(int tokens, int in_features) { return lora_ksplit(tokens, in_features); }
inline int kslice_for(int in_features, int ksplit) {  // multiple of 32 * waves
  const int step = 32 * kShrinkWaves;
  return ((in_features + ksplit - 1) / ksplit + step - 1) / step * step;
}

template <typename T>
__global__ __launch_bounds__(kShrinkThreads) void shrink_kernel(
    const T* __restrict__ x, int64_t ldx, int tokens, int in_features, Group g,
    const int32_t* __restrict__ ids, int kslice, float* __restrict__ part) {
  __shared__ int s_list[kMaxTokens];
  __shared__ int s_count;
  __shared__ float s_red[kShrinkWaves][kTilesPerPass][256];
  const int ks = blockIdx.x;
  const int jt = blockIdx.y;
  const int a = blockIdx.z;
  const int n_a = gather_tokens(ids, tokens, a, s_list, &s_count, kShrinkThreads);
  if (n_a == 0) return;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int lr = lane % 16;       // MFMA row (token) / column (rank row)
  const int kq = (lane / 16) * 8; // this lane's 8-element k group
  const int sub = kslice / kShrinkWaves;
  const int k_begin = ks * kslice + wave * sub;
  const int k_end = min(in_features, k_begin + sub);

  // rank row j -> module, local row
  const int j = jt * 16 + lr;
  const T* arow = x;  // placeholder address; never dereferenced unless a_ok
  bool a_ok = false;
  if (j < g.r_total) {
#pragma unroll
    for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
      if (m < g.n && j >= g.m[m].rank_offset && j < g.m[m].rank_offset + g.m[m].rank) {
        arow = (const T*)g.m[m].A + ((int64_t)a * g.m[m].rank + (j - g.m[m].rank_offset)) * in_features;
        a_ok = true;
      }
    }
  }

  const int n_tt = (n_a + 15) / 16;
  for (int tt0 = 0; tt0 < n_tt; tt0 += kTilesPerPass) {
    f32x4 acc[kTilesPerPass];
    const T* xrow[kTilesPerPass];
    bool tok_ok[kTilesPerPass];
#pragma unroll
    for (int u = 0; u < kTilesPerPass; ++u) {
      acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int ti = (tt0 + u) * 16 + lr;
      tok_ok[u] = ti < n_a;
      xrow[u] = x + (int64_t)(tok_ok[u] ? s_list[ti] : 0) * ldx;
    }
    // The k loop is uniform over the wave (every lane runs the same steps,
    // as the MFMA needs); a lane whose 8-element group lies past k_end loads
    // zeros.  in_features % 8 == 0, so a group is wholly in or out of range.
    for (int k0 = k_begin; k0 < k_end; k0 += 32) {
      const int k = k0 + kq;
      const bool k_ok = k < k_end;
      const uint4 bv = load8(arow + k, a_ok & k_ok);
#pragma unroll
      for (int u = 0; u < kTilesPerPass; ++u) {
        if (tt0 + u < n_tt) acc[u] = mfma32<T>(load8(xrow[u] + k, tok_ok[u] & k_ok), bv, acc[u]);
      }
    }
    // D rows = tokens 4*(lane/16)+i of the tile, column = rank row lr.
#pragma unroll
    for (int u = 0; u < kTilesPerPass; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_red[wave][u][((lane / 16) * 4 + i) * 16 + lr] = acc[u][i];
    __syncthreads();
    for (int c = threadIdx.x; c < kTilesPerPass * 256; c += kShrinkThreads) {
      const int u = c / 256, cell = c % 256;
      const int tr = (tt0 + u) * 16 + cell / 16;
      if (tt0 + u < n_tt && tr < n_a) {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kShrinkWaves; ++w) sum += s_red[w][u][cell];
        part[((int64_t)ks * tokens + s_list[tr]) * g.r_pad + jt * 16 + cell % 16] = sum;
      }
    }
    __syncthreads();
  }
}

template <typename OT> __device__ __forceinline__ void accumulate(OT* p, float v);
template <> __device__ __forceinline__ void accumulate<float>(float* p, float v) { *p += v; }
template <> __device__ __forceinline__ void accumulate<f16_t>(f16_t* p, float v) {
  *p = (f16_t)((float)*p + v);
}
template <> __device__ __forceinline__ void accumulate<bf16_t>(bf16_t* p, float v) {
  *p = from_float<bf16_t>(to_float<bf16_t>(*p) + v);
}

// Expand: workgroup (64 output columns, adapter).  Per 16-token tile the
// workgroup first folds the shrink's k-slice partials into the rounded
// rank-r intermediate (an LDS tile, the dtype of x), then each wave runs
// MFMA 16x16x32 over the concatenated ranks for its 16 columns and adds
// scale * result into the outputs.
template <typename T, typename OT>
__global__ __launch_bounds__(kThreads) void expand_kernel(
    int tokens, Group g, const int32_t* __restrict__ ids, int ksplit, const float* __restrict__ part) {
  __shared__ int s_list[kMaxTokens];
  __shared__ int s_count;
  __shared__ __align__(16) uint16_t s_y[16][128 + 8];  // r_pad <= 128; +8 keeps rows 16-byte aligned
  const int a = blockIdx.y;
  const int n_a = gather_tokens(ids, tokens, a, s_list, &s_count, kThreads);
  if (n_a == 0) return;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int lr = lane % 16;
  const int kq = (lane / 16) * 8;
  const int tile = blockIdx.x * kWaves + wave;
  const int o = tile * 16 + lr;  // this lane's output column (concatenated space)
  const bool tile_ok = tile * 16 < g.out_total;

  int mi = -1;
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m)
    if (m < g.n && o >= g.m[m].out_offset && o < g.m[m].out_offset + g.m[m].out_features) mi = m;

  // B operand for every 32-wide k tile: B_m[a][o_local][j - rank_offset] for
  // j inside the column's module, zero elsewhere.
  constexpr int kMaxKt = 4;  // r_pad <= 128
  uint4 bop[kMaxKt];
  const int n_kt = g.r_pad / 32;
  float scale = 0.f;
  OT* out_col = nullptr;
  int64_t ldo = 0;
  if (mi >= 0) {
    const Mod& m = g.m[mi];
    scale = m.scale;
    ldo = m.ldo;
    out_col = (OT*)m.out + (o - m.out_offset);
  }
#pragma unroll
  for (int kt = 0; kt < kMaxKt; ++kt) {
    bop[kt] = make_uint4(0, 0, 0, 0);
    if (kt >= n_kt || mi < 0) continue;
    const Mod& m = g.m[mi];
    const int j0 = kt * 32 + kq - m.rank_offset;  // local rank index of element 0
    const T* brow = (const T*)m.B + ((int64_t)a * m.out_features + (o - m.out_offset)) * m.rank;
    if (m.rank % 8 == 0 && j0 >= 0 && j0 + 8 <= m.rank) {
      bop[kt] = *reinterpret_cast<const uint4*>(brow + j0);
    } else {
      uint16_t e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int jl = j0 + i;
        e[i] = (jl >= 0 && jl < m.rank) ? __builtin_bit_cast(uint16_t, brow[jl]) : (uint16_t)0;
      }
      bop[kt] = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                           e[6] | (e[7] << 16));
    }
  }

  for (int tt = 0; tt * 16 < n_a; ++tt) {
    // fold the partials of this token tile into the rounded intermediate:
    // one thread per (valid token, rank) cell, eight independent loads in
    // flight per step; rows of absent tokens are zero
    const int valid = min(16, n_a - tt * 16);
    for (int c = threadIdx.x; c < 16 * g.r_pad; c += kThreads) {
      const int i = c / g.r_pad, k = c - i * g.r_pad;
      float sum = 0.f;
      if (i < valid && k < g.r_total) {
        const float* pp = part + (int64_t)s_list[tt * 16 + i] * g.r_pad + k;
        const int64_t stride = (int64_t)tokens * g.r_pad;
        int q = 0;
        for (; q + 8 <= ksplit; q += 8) {
          float v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = pp[(q + u) * stride];
#pragma unroll
          for (int u = 0; u < 8; ++u) sum += v[u];
        }
        for (; q < ksplit; ++q) sum += pp[q * stride];
      }
      s_y[i][k] = __builtin_bit_cast(uint16_t, from_float<T>(sum));
    }
    __syncthreads();
    if (tile_ok) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < kMaxKt; ++kt) {  // static indices keep bop[] in registers
        if (kt < n_kt) {
          const uint4 av = *reinterpret_cast<const uint4*>(&s_y[lr][kt * 32 + kq]);
          acc = mfma32<T>(av, bop[kt], acc);
        }
      }
      if (out_col != nullptr) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tr = tt * 16 + (lane / 16) * 4 + i;
          if (tr < n_a) accumulate<OT>(out_col + (int64_t)s_list[tr] * ldo, scale * acc[i]);
        }
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------ host side ---
int make_group(const pl_lora_module* mods, int n, int in_features, Group* g) {
  if (n < 1 || n > PL_LORA_MAX_MODULES)
    return fail(PL_ERR_INVALID, "num_modules must be 1..%d (got %d)", PL_LORA_MAX_MODULES, n);
  if (mods == nullptr) return fail(PL_ERR_INVALID, "modules is null");
  if (in_features <= 0 || in_features % 8)
    return fail(PL_ERR_INVALID, "in_features must be a positive multiple of 8 (got %d)", in_features);
  int r = 0, o = 0;
  for (int i = 0; i < n; ++i) {
    const pl_lora_module& m = mods[i];
    if (!m.A || !m.B || !m.out) return fail(PL_ERR_INVALID, "module %d has a null pointer", i);
    if (m.rank <= 0 || m.out_features <= 0)
      return fail(PL_ERR_INVALID, "module %d: rank and out_features must be > 0", i);
    if (m.ldo < m.out_features) return fail(PL_ERR_INVALID, "module %d: ldo < out_features", i);
    if ((uintptr_t)m.A % 16) return fail(PL_ERR_INVALID, "module %d: A must be 16-byte aligned", i);
    g->m[i].A = m.A;
    g->m[i].B = m.B;
    g->m[i].out = m.out;
    g->m[i].ldo = m.ldo;
    g->m[i].out_features = m.out_features;
    g->m[i].rank = m.rank;
    g->m[i].out_offset = o;
    g->m[i].rank_offset = r;
    g->m[i].scale = m.scale;
    r += m.rank;
    o += m.out_features;
  }
  for (int i = n; i < PL_LORA_MAX_MODULES; ++i) g->m[i] = Mod{};
  g->n = n;
  g->r_total = r;
  g->r_pad = (r + 31) / 32 * 32;
  g->out_total = o;
  if (g->r_pad > 128) return fail(PL_ERR_UNSUPPORTED, "sum of ranks %d > 128", r);
  return PL_OK;
}

int check_common(const void* x, int64_t ldx, int tokens, int n_adapters, const int32_t* ids,
                 int dtype) {
  if (tokens < 0 || tokens > kMaxTokens)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", kMaxTokens, tokens);
  if (n_adapters < 1 || n_adapters > 65535)
    return fail(PL_ERR_INVALID, "num_adapters must be 1..65535");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "LoRA dtype must be F16 or BF16 (got %d)", dtype);
  if (tokens > 0 && (!x || !ids)) return fail(PL_ERR_INVALID, "x and adapter_ids must be non-null");
  if ((uintptr_t)x % 16 || ldx % 8) return fail(PL_ERR_INVALID, "x must be 16-byte aligned, ldx % 8 == 0");
  return PL_OK;
}

}  // namespace lora
}  // namespace pl

using namespace pl;
using namespace pl::lora;

// Workspace: the shrink's fp32 partials [ksplit][T][r_pad].
static size_t ws_bytes_needed(int tokens, int in_features, int r_pad) {
  return align_up((size_t)ksplit_for(tokens, in_features) * tokens * r_pad * sizeof(float), 256);
}

extern "C" size_t pl_lora_workspace_size(int num_tokens, int in_features,
                                         const pl_lora_module* modules_h, int num_modules) {
  Group g;
  if (make_group(modules_h, num_modules, in_features, &g) != PL_OK || num_tokens < 0) return 0;
  return ws_bytes_needed(num_tokens, in_features, g.r_pad);
}

static int lora_shrink_impl(const void* x, int64_t ldx, int tokens, int in_features,
                            const Group& g, const int32_t* ids, int n_adapters, int dtype,
                            void* ws, size_t ws_bytes, hipStream_t stream) {
  const size_t need = ws_bytes_needed(tokens, in_features, g.r_pad);
  if (need > ws_bytes)
    return fail(PL_ERR_WORKSPACE, "LoRA workspace of %zu bytes < %zu needed", ws_bytes, need);
  if (ws == nullptr || (uintptr_t)ws % 256) return fail(PL_ERR_INVALID, "workspace must be 256-byte aligned");
  if (n_adapters > 65535) return fail(PL_ERR_UNSUPPORTED, "num_adapters %d > 65535", n_adapters);
  const int ksplit = ksplit_for(tokens, in_features);
  const int kslice = kslice_for(in_features, ksplit);
  dim3 grid(ksplit, g.r_pad / 16, n_adapters);
  if (dtype == PL_DTYPE_BF16)
    hipLaunchKernelGGL(shrink_kernel<bf16_t>, grid, dim3(kShrinkThreads), 0, stream, (const bf16_t*)x,
                       ldx, tokens, in_features, g, ids, kslice, (float*)ws);
  else
    hipLaunchKernelGGL(shrink_kernel<f16_t>, grid, dim3(kShrinkThreads), 0, stream, (const f16_t*)x,
                       ldx, tokens, in_features, g, ids, kslice, (float*)ws);
  PL_LAUNCH_CHECK("lora shrink_kernel");
  return PL_OK;
}

template <typename T>
static int launch_expand(int tokens, int in_features, const Group& g, const int32_t* ids, int n_adapters,
                         int out_dtype, const float* part, hipStream_t stream) {
  dim3 grid((g.out_total + 16 * kWaves - 1) / (16 * kWaves), n_adapters);
  const int ksplit = ksplit_for(tokens, in_features);
  switch (out_dtype) {
    case PL_DTYPE_F32:
      hipLaunchKernelGGL((expand_kernel<T, float>), grid, dim3(kThreads), 0, stream, tokens, g, ids, ksplit, part);
      break;
    case PL_DTYPE_F16:
      hipLaunchKernelGGL((expand_kernel<T, f16_t>), grid, dim3(kThreads), 0, stream, tokens, g, ids, ksplit, part);
      break;
    case PL_DTYPE_BF16:
      hipLaunchKernelGGL((expand_kernel<T, bf16_t>), grid, dim3(kThreads), 0, stream, tokens, g, ids, ksplit, part);
      break;
    default:
      return fail(PL_ERR_UNSUPPORTED, "out_dtype %d", out_dtype);
  }
  PL_LAUNCH_CHECK("lora expand_kernel");
  return PL_OK;
}

static int lora_expand_impl(int tokens, int in_features, const Group& g, const int32_t* ids,
                            int n_adapters, int dtype, int out_dtype, const void* ws,
                            size_t ws_bytes, hipStream_t stream) {
  const size_t need = ws_bytes_needed(tokens, in_features, g.r_pad);
  if (need > ws_bytes)
    return fail(PL_ERR_WORKSPACE, "LoRA workspace of %zu bytes < %zu needed", ws_bytes, need);
  if (n_adapters > 65535) return fail(PL_ERR_UNSUPPORTED, "num_adapters %d > 65535", n_adapters);
  const float* part = (const float*)ws;
  return dtype == PL_DTYPE_BF16 ? launch_expand<bf16_t>(tokens, in_features, g, ids, n_adapters, out_dtype, part, stream)
                                : launch_expand<f16_t>(tokens, in_features, g, ids, n_adapters, out_dtype, part, stream);
}

extern "C" int pl_lora_shrink(const void* x, int64_t ldx, int num_tokens, int in_features,
                              const pl_lora_module* modules_h, int num_modules,
                              const int32_t* adapter_ids, int num_adapters, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_common(x, ldx, num_tokens, num_adapters, adapter_ids, dtype);
  if (st) return st;
  Group g;
  if ((st = make_group(modules_h, num_modules, in_features, &g))) return st;
  if (num_tokens == 0) return ok();
  if ((st = lora_shrink_impl(x, ldx, num_tokens, in_features, g, adapter_ids, num_adapters, dtype,
                             workspace, workspace_bytes, (hipStream_t)stream)))
    return st;
  return ok();
}

extern "C" int pl_lora_expand(int num_tokens, int in_features, const pl_lora_module* modules_h,
                              int num_modules, const int32_t* adapter_ids, int num_adapters,
                              int dtype, int out_dtype, const void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (num_tokens < 0 || num_tokens > kMaxTokens)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", kMaxTokens, num_tokens);
  if (num_adapters < 1) return fail(PL_ERR_INVALID, "num_adapters must be >= 1");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "LoRA dtype must be F16 or BF16 (got %d)", dtype);
  if (num_tokens > 0 && (adapter_ids == nullptr || workspace == nullptr))
    return fail(PL_ERR_INVALID, "adapter_ids and workspace must be non-null");
  int st;
  Group g;
  if ((st = make_group(modules_h, num_modules, in_features, &g))) return st;
  if (num_tokens == 0) return ok();
  if ((st = lora_expand_impl(num_tokens, in_features, g, adapter_ids, num_adapters, dtype,
                             out_dtype, workspace, workspace_bytes, (hipStream_t)stream)))
    return st;
  return ok();
}

extern "C" int pl_lora_delta(const void* x, int64_t ldx, int num_tokens, int in_features,
                             const pl_lora_module* modules_h, int num_modules,
                             const int32_t* adapter_ids, int num_adapters, int dtype,
                             int out_dtype, void* workspace, size_t workspace_bytes,
                             void* stream) {
  int st = check_common(x, ldx, num_tokens, num_adapters, adapter_ids, dtype);
  if (st) return st;
  Group g;
  if ((st = make_group(modules_h, num_modules, in_features, &g))) return st;
  if (num_tokens == 0) return ok();
  if ((st = lora_shrink_impl(x, ldx, num_tokens, in_features, g, adapter_ids, num_adapters, dtype,
                             workspace, workspace_bytes, (hipStream_t)stream)))
    return st;
  if ((st = lora_expand_impl(num_tokens, in_features, g, adapter_ids, num_adapters, dtype,
                             out_dtype, workspace, workspace_bytes, (hipStream_t)stream)))
    return st;
  return ok();
}
