// No-merge multi-adapter LoRA delta for gfx950:
//   out_m[t] += scale_m * B_m[a_t] . (A_m[a_t] . x[t])
// for the modules m of a group that share their input x (q/k/v, gate/up, or a
// lone o_proj / down_proj) and per-token adapter ids a_t.
//
//   shrink_kernel  grid (k-slice, adapter).  Gathers the tokens of its adapter
//                  (LDS list), multiplies their x slice by the adapter's
//                  concatenated A rows on MFMA 16x16x32 tiles, writes fp32
//                  partial sums; the last workgroup of each adapter (atomic
//                  ticket) reduces the partials and rounds the rank-r
//                  intermediate to the input dtype.
//   expand_kernel  grid (16-column tiles x 4, adapter).  Multiplies the
//                  rounded intermediate by B^T on MFMA 16x16x32 tiles and
//                  accumulates scale * result into the outputs in place.
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
constexpr int kSlice = 256;      // k elements per shrink workgroup
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

// Workspace layout: per-adapter tickets, fp32 partials [ksplit][T][r_pad],
// rounded intermediate [T][r_pad] of the input dtype.
struct WsLayout {
  size_t tickets, part, y, total;
};
inline int ksplit_for(int in_features) { return (in_features + kSlice - 1) / kSlice; }
inline WsLayout ws_layout(int tokens, int in_features, int r_pad, int n_adapters) {
  WsLayout L;
  L.tickets = 0;
  L.part = align_up((size_t)(n_adapters > 0 ? n_adapters : 1) * sizeof(int), 256);
  L.y = align_up(L.part + (size_t)ksplit_for(in_features) * tokens * r_pad * sizeof(float), 256);
  L.total = align_up(L.y + (size_t)tokens * r_pad * 2, 256);
  return L;
}

// Gather the tokens of adapter `a` into LDS; returns their count (all threads).
__device__ __forceinline__ int gather_tokens(const int32_t* __restrict__ ids, int tokens, int a,
                                             int* s_list, int* s_count) {
  if (threadIdx.x == 0) *s_count = 0;
  __syncthreads();
  for (int t = threadIdx.x; t < tokens; t += kThreads) {
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

template <typename T>
__global__ __launch_bounds__(kThreads) void shrink_kernel(
    const T* __restrict__ x, int64_t ldx, int tokens, int in_features, Group g,
    const int32_t* __restrict__ ids, int ksplit, int* __restrict__ tickets,
    float* __restrict__ part, uint16_t* __restrict__ y) {
  __shared__ int s_list[kMaxTokens];
  __shared__ int s_count, s_last;
  const int ks = blockIdx.x;
  const int a = blockIdx.y;
  const int n_a = gather_tokens(ids, tokens, a, s_list, &s_count);
  if (n_a == 0) return;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int lr = lane % 16;       // MFMA row (token) / column (rank row)
  const int kq = (lane / 16) * 8; // this lane's 8-element k group
  const int k0 = ks * kSlice;
  const int n_tt = (n_a + 15) / 16;
  const int n_jt = g.r_pad / 16;

  for (int pair = wave; pair < n_tt * n_jt; pair += kWaves) {
    const int tt = pair / n_jt, jt = pair - tt * n_jt;
    const int ti = tt * 16 + lr;
    const bool tok_ok = ti < n_a;
    const T* xrow = x + (int64_t)(tok_ok ? s_list[ti] : 0) * ldx;
    // rank row j -> module, local row
    const int j = jt * 16 + lr;
    const T* arow = x;  // placeholder address; never dereferenced unless a_ok
    bool a_ok = false;
    if (j < g.r_total) {
#pragma unroll
      for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
        if (m < g.n && j >= g.m[m].rank_offset && j < g.m[m].rank_offset + g.m[m].rank) {
          const int jr = j - g.m[m].rank_offset;
          arow = (const T*)g.m[m].A + ((int64_t)a * g.m[m].rank + jr) * in_features;
          a_ok = true;
        }
      }
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int kk = 0; kk < kSlice; kk += 32) {
      const int k = k0 + kk + kq;
      const bool k_ok = k < in_features;  // in_features % 8 == 0: a group is all in or all out
      const uint4 av = load8(xrow + k, tok_ok && k_ok);
      const uint4 bv = load8(arow + k, a_ok && k_ok);
      acc = mfma32<T>(av, bv, acc);
    }
    // D rows = tokens 4*(lane/16)+i, column = rank row jt*16 + lr.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tr = tt * 16 + (lane / 16) * 4 + i;
      if (tr < n_a)
        part[((int64_t)ks * tokens + s_list[tr]) * g.r_pad + jt * 16 + lr] = acc[i];
    }
  }

  // Ticket: the last workgroup of this adapter reduces the k-slices.  Every
  // thread publishes its partial stores at agent scope before the barrier.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&tickets[a], 1, __ATOMIC_ACQ_REL,
                                            __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == ksplit - 1;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();  // acquire: the other slices' partials are visible from here on
  const int cells = n_a * g.r_pad;
  for (int c = threadIdx.x; c < cells; c += kThreads) {
    const int ti = c / g.r_pad, jj = c - ti * g.r_pad;
    const int t = s_list[ti];
    float s = 0.f;
    if (jj < g.r_total)
      for (int q = 0; q < ksplit; ++q)
        s += part[((int64_t)q * tokens + t) * g.r_pad + jj];
    const T v = from_float<T>(s);
    y[(int64_t)t * g.r_pad + jj] = __builtin_bit_cast(uint16_t, v);
  }
  if (threadIdx.x == 0) tickets[a] = 0;  // ready for the next call
}

template <typename OT> __device__ __forceinline__ void accumulate(OT* p, float v);
template <> __device__ __forceinline__ void accumulate<float>(float* p, float v) { *p += v; }
template <> __device__ __forceinline__ void accumulate<f16_t>(f16_t* p, float v) {
  *p = (f16_t)((float)*p + v);
}
template <> __device__ __forceinline__ void accumulate<bf16_t>(bf16_t* p, float v) {
  *p = from_float<bf16_t>(to_float<bf16_t>(*p) + v);
}

template <typename T, typename OT>
__global__ __launch_bounds__(kThreads) void expand_kernel(
    int tokens, Group g, const int32_t* __restrict__ ids, const uint16_t* __restrict__ y) {
  __shared__ int s_list[kMaxTokens];
  __shared__ int s_count;
  const int a = blockIdx.y;
  const int n_a = gather_tokens(ids, tokens, a, s_list, &s_count);
  if (n_a == 0) return;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int lr = lane % 16;
  const int kq = (lane / 16) * 8;
  const int tile = blockIdx.x * kWaves + wave;
  const int o = tile * 16 + lr;  // this lane's output column (concatenated space)
  if (tile * 16 >= g.out_total) return;

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
    const int ti = tt * 16 + lr;
    const bool tok_ok = ti < n_a;
    const uint16_t* yrow = y + (int64_t)(tok_ok ? s_list[ti] : 0) * g.r_pad;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int kt = 0; kt < n_kt; ++kt) {
      const uint4 av = load8(yrow + kt * 32 + kq, tok_ok);
      acc = mfma32<T>(av, bop[kt], acc);
    }
    if (out_col != nullptr) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tr = tt * 16 + (lane / 16) * 4 + i;
        if (tr < n_a) accumulate<OT>(out_col + (int64_t)s_list[tr] * ldo, scale * acc[i]);
      }
    }
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

extern "C" size_t pl_lora_workspace_size(int num_tokens, int in_features,
                                         const pl_lora_module* modules_h, int num_modules) {
  Group g;
  if (make_group(modules_h, num_modules, in_features, &g) != PL_OK || num_tokens < 0) return 0;
  // Ticket slots for up to 65535 adapters would be wasteful; the layout is
  // sized for the adapters actually passed at call time, so report the
  // size for 256 adapter slots, the largest a single call accepts cheaply.
  return ws_layout(num_tokens, in_features, g.r_pad, 256).total;
}

static int lora_shrink_impl(const void* x, int64_t ldx, int tokens, int in_features,
                            const Group& g, const int32_t* ids, int n_adapters, int dtype,
                            void* ws, size_t ws_bytes, hipStream_t stream) {
  const WsLayout L = ws_layout(tokens, in_features, g.r_pad, n_adapters);
  if (n_adapters > 256) return fail(PL_ERR_UNSUPPORTED, "num_adapters %d > 256", n_adapters);
  if (L.total > ws_bytes)
    return fail(PL_ERR_WORKSPACE, "LoRA workspace of %zu bytes < %zu needed", ws_bytes, L.total);
  if (ws == nullptr || (uintptr_t)ws % 256) return fail(PL_ERR_INVALID, "workspace must be 256-byte aligned");
  char* w = (char*)ws;
  const int ksplit = ksplit_for(in_features);
  dim3 grid(ksplit, n_adapters);
  if (dtype == PL_DTYPE_BF16)
    hipLaunchKernelGGL(shrink_kernel<bf16_t>, grid, dim3(kThreads), 0, stream, (const bf16_t*)x,
                       ldx, tokens, in_features, g, ids, ksplit, (int*)(w + L.tickets),
                       (float*)(w + L.part), (uint16_t*)(w + L.y));
  else
    hipLaunchKernelGGL(shrink_kernel<f16_t>, grid, dim3(kThreads), 0, stream, (const f16_t*)x,
                       ldx, tokens, in_features, g, ids, ksplit, (int*)(w + L.tickets),
                       (float*)(w + L.part), (uint16_t*)(w + L.y));
  PL_LAUNCH_CHECK("lora shrink_kernel");
  return PL_OK;
}

template <typename T>
static int launch_expand(int tokens, const Group& g, const int32_t* ids, int n_adapters,
                         int out_dtype, const uint16_t* y, hipStream_t stream) {
  dim3 grid((g.out_total + 16 * kWaves - 1) / (16 * kWaves), n_adapters);
  switch (out_dtype) {
    case PL_DTYPE_F32:
      hipLaunchKernelGGL((expand_kernel<T, float>), grid, dim3(kThreads), 0, stream, tokens, g, ids, y);
      break;
    case PL_DTYPE_F16:
      hipLaunchKernelGGL((expand_kernel<T, f16_t>), grid, dim3(kThreads), 0, stream, tokens, g, ids, y);
      break;
    case PL_DTYPE_BF16:
      hipLaunchKernelGGL((expand_kernel<T, bf16_t>), grid, dim3(kThreads), 0, stream, tokens, g, ids, y);
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
  const WsLayout L = ws_layout(tokens, in_features, g.r_pad, n_adapters);
  if (n_adapters > 256) return fail(PL_ERR_UNSUPPORTED, "num_adapters %d > 256", n_adapters);
  if (L.total > ws_bytes)
    return fail(PL_ERR_WORKSPACE, "LoRA workspace of %zu bytes < %zu needed", ws_bytes, L.total);
  const uint16_t* y = (const uint16_t*)((const char*)ws + L.y);
  return dtype == PL_DTYPE_BF16 ? launch_expand<bf16_t>(tokens, g, ids, n_adapters, out_dtype, y, stream)
                                : launch_expand<f16_t>(tokens, g, ids, n_adapters, out_dtype, y, stream);
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
