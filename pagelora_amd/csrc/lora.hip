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
// Decode-sized calls (<= 64 tokens, <= 64 adapters) of pl_lora_delta and
// pl_lora_delta_groups take a two-launch path built for latency, for up to
// four groups with their own inputs in the same two launches:
//
//   fast_shrink_kernel  grid (group, 256-element k-slice, 16 rank rows,
//                  adapter): every load of the workgroup (ids, x of all
//                  tokens, the A rows) issued at once, one MFMA chain per
//                  token tile, the adapter's tokens' results added into a
//                  64-bit fixed-point accumulator (order-independent, so
//                  deterministic).
//   fast_expand_kernel  grid (group, 64 output columns): the intermediate
//                  (rounded to the input dtype into LDS), ids, B rows and
//                  outputs in one round trip, MFMA per adapter over the
//                  token tiles, out += scale * result; the group's last
//                  workgroup clears the accumulator for the next call.
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

// load8 without a branch: p must be readable whether or not ok holds (the
// caller clamps it), the value is zeroed afterwards.  Branches around loads
// make the compiler re-read kernel arguments inside each one.
__device__ __forceinline__ uint4 load8_sel(const void* p, bool ok) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  return ok ? v : make_uint4(0, 0, 0, 0);
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

// ------------------------------------------------------ decode-size path ---
constexpr int kFastMaxTokens = 64;    // one 16-token tile per wave of a shrink workgroup
constexpr int kFastMaxAdapters = 64;
constexpr int kFastKSlice = 256;      // k elements per shrink workgroup: 8 MFMA steps
constexpr int kFastKSteps = kFastKSlice / 32;
constexpr int kFastMaxSlices = 64;    // in_features <= 64 * kFastKSlice on this path
constexpr int kExpandWaves = 4;  // 8 (128 columns) measured no faster: 30.2 vs 30.3 us per layer, per-group calls 60.9 vs 57.2
constexpr int kExpandThreads = kExpandWaves * 64;
constexpr int kFastCols = 16 * kExpandWaves;  // output columns per expand workgroup (16 per wave)
constexpr int kFastAChunk = 4;        // adapters whose B rows an expand wave holds at once
constexpr int kFastTt = kFastMaxTokens / 16;
// The shrink's slices meet in a signed 64-bit fixed-point accumulator with
// 26 fraction bits: integer adds are associative, so the sum (and the
// rounded intermediate) does not depend on the order the slices arrive in.
// Each partial is clamped to +-2^31 first, so 64 slices cannot overflow.
constexpr float kFixScale = 67108864.f;          // 2^26
constexpr double kFixInv = 1.0 / 67108864.0;
constexpr float kFixClamp = 2147483648.f;        // 2^31
// Workspace of pl_lora_delta(_groups): per group a parity word, then per
// group two fixed-size accumulator slots, then the general path's shrink
// partials (disjoint regions, so a general-path call never disturbs the
// decode path's state).  A call's shrink adds into slot `parity` and clears
// the other slot whole (the one the previous call's expand read); the expand
// reads the sum of both slots and flips the parity.  Starting from an
// all-zero workspace, the slot a shrink adds into is therefore always zero,
// with no wait inside either kernel: the kernel boundaries order the clear
// against the reads.
constexpr size_t kParityBytes = 256;
constexpr size_t kAccSlotBytes = (size_t)kFastMaxTokens * 128 * sizeof(long long);
constexpr size_t kAccSlotPairs = kAccSlotBytes / 16;
constexpr size_t kGeneralOffset = kParityBytes + 2 * PL_LORA_MAX_GROUPS * kAccSlotBytes;

struct FastGroup {
  Group g;
  const void* x;
  int64_t ldx;
  int in_features;
  int ksplit;        // k-slices of kFastKSlice
  int n_rt;          // rank tiles of 16 rows holding real ranks
  int shrink_begin;  // first shrink workgroup of the group
  int expand_begin;  // first expand workgroup of the group
  int n_expand;      // expand workgroups of the group
  long long* acc;    // two slots of [tokens][r_pad] fixed point (kAccSlotBytes apart)
  int* parity;       // the slot this call's shrink adds into
};

struct FastArgs {
  FastGroup grp[PL_LORA_MAX_GROUPS];
  int n_groups, tokens, n_adapters;
  const int32_t* ids;
};

// Which group a flattened workgroup index belongs to (groups in order).
template <bool SHRINK>
__device__ __forceinline__ int group_of(const FastArgs& fa, int wg) {
  int gi = 0;
#pragma unroll
  for (int i = 1; i < PL_LORA_MAX_GROUPS; ++i)
    if (i < fa.n_groups && wg >= (SHRINK ? fa.grp[i].shrink_begin : fa.grp[i].expand_begin)) gi = i;
  return gi;
}

__device__ __forceinline__ long long to_fixed(float v) {
  return (long long)__builtin_rintf(fminf(fmaxf(v, -kFixClamp), kFixClamp) * kFixScale);
}

// Shrink: workgroup (group, k-slice, 16 rank rows, adapter), one 16-token
// tile per wave.  All loads of the workgroup (ids, x of every token, the A
// rows) go out at once, the wave runs one MFMA chain over its slice, and the
// results of the adapter's tokens are added into the fixed-point
// accumulator (device-scope atomics, nothing waits on them).
template <typename T>
__global__ __launch_bounds__(kShrinkThreads) void fast_shrink_kernel(FastArgs fa) {
  const int gi = group_of<true>(fa, blockIdx.x);
  const FastGroup& G = fa.grp[gi];
  int local = blockIdx.x - G.shrink_begin;
  const int a = local % fa.n_adapters;
  local /= fa.n_adapters;
  const int rt = local % G.n_rt;
  const int ks = local / G.n_rt;
  const int T_ = fa.tokens;
  const int r_pad = G.g.r_pad;
  const int par = *G.parity & 1;
  long long* acc = G.acc + (par ? kAccSlotBytes / sizeof(long long) : 0);
  long long* other = G.acc + (par ? 0 : kAccSlotBytes / sizeof(long long));

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;   // token tile
  const int lr = lane % 16;
  const int kq = (lane / 16) * 8;
  const int t = wave * 16 + lr;           // the token of this lane's x row
  const bool t_ok = t < T_;
  const int id_raw = fa.ids[t_ok ? t : 0];
  const int id = t_ok ? id_raw : -1;

  // rank row j -> its module's A row of adapter a (blended with bit masks,
  // not branches, so the module fields come in a few batched scalar loads)
  const int j = rt * 16 + lr;
  const T* arow = (const T*)G.x;  // placeholder address; never dereferenced unless a_ok
  bool a_ok = false;
  uint64_t row_bits = 0;
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
    const Mod& M = G.g.m[m];
    const bool in = (m < G.g.n) & (j >= M.rank_offset) & (j < M.rank_offset + M.rank);
    const T* row = (const T*)M.A + ((int64_t)a * M.rank + (j - M.rank_offset)) * G.in_features;
    row_bits |= (uint64_t)(uintptr_t)row & (0 - (uint64_t)in);
    a_ok |= in;
  }
  if (a_ok) arow = (const T*)(uintptr_t)row_bits;
  const T* xrow = (const T*)G.x + (int64_t)(t_ok ? t : 0) * G.ldx;
  const int k0 = ks * kFastKSlice;
  // every load before the first MFMA; the k steps are uniform over the wave
  // and a lane's 8-element group lies wholly inside or outside in_features
  // (in_features % 8 == 0); out-of-range groups re-read the row's first
  uint4 xv[kFastKSteps], av[kFastKSteps];
#pragma unroll
  for (int s = 0; s < kFastKSteps; ++s) {
    const int k = k0 + s * 32 + kq;
    const bool k_ok = k < G.in_features;
    const int kc = k_ok ? k : 0;
    xv[s] = load8_sel(xrow + kc, t_ok & k_ok);
    av[s] = load8_sel(arow + kc, a_ok & k_ok);
  }
  __builtin_amdgcn_sched_barrier(0);
  f32x4 part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kFastKSteps; ++s) part = mfma32<T>(xv[s], av[s], part);
  // D rows = tokens wave*16 + 4*(lane/16) + i, column = rank row j (ranks
  // past r_total have zero A rows and add zero)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (lane / 16) * 4 + i;
    const int tr = wave * 16 + r;
    const int id_tr = __shfl(id, r);
    if (tr < T_ && id_tr == a && j < r_pad)
      __hip_atomic_fetch_add(acc + (int64_t)tr * r_pad + j, to_fixed(part[i]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
  // this workgroup's share of clearing the other slot (all of it: an earlier
  // call may have used it with another layout)
  const int n_wg = G.ksplit * G.n_rt * fa.n_adapters;
  const int per = (int)((kAccSlotPairs + n_wg - 1) / n_wg);
  const int c_end = min((int)kAccSlotPairs, (blockIdx.x - G.shrink_begin + 1) * per);
  for (int c = (blockIdx.x - G.shrink_begin) * per + threadIdx.x; c < c_end; c += kShrinkThreads)
    *reinterpret_cast<longlong2*>(other + 2 * (int64_t)c) = longlong2{0, 0};
}

// Expand: workgroup (group, 64 output columns), every adapter; NKT: the
// largest r_pad / 32 of the launch's groups.  One round trip for all of its loads:
// the fixed-point intermediate of every token, the ids and outputs of the
// wave's rows, the B rows of the first adapters.  The intermediate is
// rounded to the input dtype into LDS (as the reference's F.linear returns
// it); per adapter an MFMA over the token tiles, the result kept for the
// rows of that adapter; out = out + scale * delta for every row with an
// adapter.  The group's last workgroup to arrive clears the accumulator for
// the next call (every workgroup has read it by then).
template <typename T, typename OT, int NKT>
__global__ __launch_bounds__(kExpandThreads) void fast_expand_kernel(FastArgs fa) {
  constexpr int RP = NKT * 32;                         // the largest r_pad
  constexpr int kStage = kFastMaxTokens * RP / 2 / kExpandThreads;  // 16-byte accumulator loads per thread
  __shared__ __align__(16) uint16_t s_y[kFastMaxTokens][RP + 8];  // +8 keeps rows 16-byte aligned
  const int gi = group_of<false>(fa, blockIdx.x);
  const FastGroup& G = fa.grp[gi];
  const int ct = blockIdx.x - G.expand_begin;
  const int T_ = fa.tokens;
  const int n_tt = (T_ + 15) / 16;
  const int n_ad = fa.n_adapters;
  const int r_pad = G.g.r_pad;
  const int n_kt = r_pad / 32;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int lr = lane % 16;
  const int kq = (lane / 16) * 8;
  const int tile = ct * kExpandWaves + wave;
  const int o = tile * 16 + lr;  // this lane's output column (concatenated space)
  const long long* accp = G.acc;

  // the accumulator loads go out first (they gate the barrier): both slots,
  // one of which the shrink cleared
  const int n_pairs = T_ * r_pad / 2;
  constexpr int64_t kSlot = kAccSlotBytes / sizeof(long long);
  longlong2 av2[kStage], bv2[kStage];
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int c = u * kExpandThreads + threadIdx.x;
    const int64_t off = 2 * (int64_t)(c < n_pairs ? c : 0);
    av2[u] = *reinterpret_cast<const longlong2*>(accp + off);
    bv2[u] = *reinterpret_cast<const longlong2*>(accp + kSlot + off);
  }
  // ids of the lane's rows (4*(lane/16) + i of each tile)
  int idr[kFastTt][4];
#pragma unroll
  for (int tt = 0; tt < kFastTt; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tr = tt * 16 + (lane / 16) * 4 + i;
      const int v = fa.ids[tr < T_ ? tr : 0];
      idr[tt][i] = tr < T_ ? v : -1;
    }

  // The lane's module, blended from the four (uniform) module descriptors
  // with bit masks: a per-lane index into them would read the kernel
  // arguments with dependent vector loads, and a select lets the compiler
  // sink each field's load into a branch of its own (one wait apiece).
  // Pointers are blended as byte offsets from module 0's, so they stay
  // global-memory pointers to the compiler (no flat accesses).
  const Mod& M0 = G.g.m[0];
  bool has_mod = false;
  uint64_t b_off = 0, o_off = 0, ldo_bits = 0;
  uint32_t scale_bits = 0;
  int m_rank = 0, m_roff = 0, m_out = 0, m_ooff = 0;
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
    const Mod& M = G.g.m[m];
    const bool in = (m < G.g.n) & (o >= M.out_offset) & (o < M.out_offset + M.out_features);
    const uint64_t mask = 0 - (uint64_t)in;
    has_mod |= in;
    b_off |= ((uint64_t)(uintptr_t)M.B - (uint64_t)(uintptr_t)M0.B) & mask;
    o_off |= ((uint64_t)(uintptr_t)M.out - (uint64_t)(uintptr_t)M0.out) & mask;
    ldo_bits |= (uint64_t)M.ldo & mask;
    scale_bits |= __float_as_uint(M.scale) & (uint32_t)mask;
    m_rank |= M.rank & (int)mask;
    m_roff |= M.rank_offset & (int)mask;
    m_out |= M.out_features & (int)mask;
    m_ooff |= M.out_offset & (int)mask;
  }
  const T* bbase = (const T*)((const char*)M0.B + (int64_t)b_off);
  // (a lane past the group's columns points at module 0's first output, which it never writes)
  OT* out_col = (OT*)((char*)M0.out + (int64_t)o_off) + (has_mod ? o - m_ooff : 0);
  const int64_t ldo = (int64_t)ldo_bits;
  const float scale = __uint_as_float(scale_bits);

  // B operand of adapter a for every 32-wide k tile: B_m[a][o_local][j -
  // rank_offset] for j inside the column's module, zero elsewhere.  Ranks
  // and rank offsets are multiples of 8 on this path, so a lane's 8 ranks
  // lie wholly inside or outside its module.
  auto load_b = [&](int a, uint4 (&bop)[NKT]) {
    const bool a_ok = a < n_ad;
    const T* brow = bbase + ((int64_t)(a_ok ? a : 0) * m_out + (has_mod ? o - m_ooff : 0)) * m_rank;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      const int j0 = kt * 32 + kq - m_roff;  // local rank index of element 0
      const bool ok = (j0 >= 0) & (j0 < m_rank) & has_mod & a_ok;
      bop[kt] = load8_sel(brow + (ok ? j0 : 0), ok);
    }
  };
  uint4 bop[kFastAChunk][NKT];
#pragma unroll
  for (int u = 0; u < kFastAChunk; ++u) load_b(u, bop[u]);
  // the wave's outputs of every token; rows that do not exist re-read a
  // valid output whose value goes unused (no select on the loaded value: it
  // would put each load in a branch)
  OT cur[kFastTt][4];
#pragma unroll
  for (int tt = 0; tt < kFastTt; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tr = tt * 16 + (lane / 16) * 4 + i;
      cur[tt][i] = out_col[(has_mod & (tr < T_)) ? (int64_t)tr * ldo : 0];
    }
  __builtin_amdgcn_sched_barrier(0);  // every load of the workgroup in flight

  // the intermediate into LDS: one rounding to T per value
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int c = u * kExpandThreads + threadIdx.x;
    if (c < n_pairs) {
      const int tk = c / (r_pad / 2), j2 = 2 * (c % (r_pad / 2));
      const long long x0 = av2[u].x + bv2[u].x, x1 = av2[u].y + bv2[u].y;
      const uint16_t lo = __builtin_bit_cast(uint16_t, from_float<T>((float)((double)x0 * kFixInv)));
      const uint16_t hi = __builtin_bit_cast(uint16_t, from_float<T>((float)((double)x1 * kFixInv)));
      *reinterpret_cast<uint32_t*>(&s_y[tk][j2]) = lo | ((uint32_t)hi << 16);
    }
  }
  __syncthreads();
  // the next call's shrink adds into the other slot (no expand workgroup
  // reads the parity, so the flip can go out at any time)
  if (ct == 0 && threadIdx.x == 0) *G.parity ^= 1;

  float delta[kFastTt][4];
#pragma unroll
  for (int tt = 0; tt < kFastTt; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) delta[tt][i] = 0.f;
  for (int a0 = 0; a0 < n_ad; a0 += kFastAChunk) {
    if (a0 > 0) {
#pragma unroll
      for (int u = 0; u < kFastAChunk; ++u) load_b(a0 + u, bop[u]);
    }
#pragma unroll
    for (int u = 0; u < kFastAChunk; ++u) {
#pragma unroll
      for (int tt = 0; tt < kFastTt; ++tt) {
        if (tt >= n_tt) break;
        f32x4 r4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
          if (kt >= n_kt) break;  // the group's own rank tiles (uniform)
          const uint4 yv = *reinterpret_cast<const uint4*>(&s_y[tt * 16 + lr][kt * 32 + kq]);
          r4 = mfma32<T>(yv, bop[u][kt], r4);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) delta[tt][i] = idr[tt][i] == a0 + u ? scale * r4[i] : delta[tt][i];
      }
    }
  }
#pragma unroll
  for (int tt = 0; tt < kFastTt; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool mine = has_mod & (idr[tt][i] >= 0) & (idr[tt][i] < n_ad);
      if (mine)
        out_col[(int64_t)(tt * 16 + (lane / 16) * 4 + i) * ldo] =
            from_float<OT>(to_float<OT>(cur[tt][i]) + delta[tt][i]);
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

// ---------------------------------------------- pl_lora_delta(_groups) ---
// Workspace: [parities][accumulator slot pairs][general partials] (see
// kGeneralOffset).
struct DeltaPlan {
  bool fast;
  FastArgs fa;
  Group g[PL_LORA_MAX_GROUPS];  // general path
  size_t need;
  int shrink_total, expand_total;
};

static int plan_delta(const pl_lora_group* groups, int n_groups, int tokens, int n_adapters, int dtype,
                      char* ws, DeltaPlan* P) {
  if (n_groups < 1 || n_groups > PL_LORA_MAX_GROUPS)
    return fail(PL_ERR_INVALID, "num_groups must be 1..%d (got %d)", PL_LORA_MAX_GROUPS, n_groups);
  if (groups == nullptr) return fail(PL_ERR_INVALID, "groups is null");
  if (tokens < 0 || tokens > kMaxTokens)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", kMaxTokens, tokens);
  if (n_adapters < 1 || n_adapters > 65535) return fail(PL_ERR_INVALID, "num_adapters must be 1..65535");
  // the decode path: decode sizes, ranks of a multiple of 8, 16-byte aligned B
  P->fast = tokens <= kFastMaxTokens && n_adapters <= kFastMaxAdapters;
  for (int i = 0; i < n_groups && groups != nullptr; ++i) {
    P->fast = P->fast && groups[i].in_features <= kFastMaxSlices * kFastKSlice;
    for (int m = 0; m < groups[i].num_modules && groups[i].modules != nullptr; ++m)
      P->fast = P->fast && groups[i].modules[m].rank % 8 == 0 && (uintptr_t)groups[i].modules[m].B % 16 == 0;
  }
  size_t general = 0;
  int sb = 0, eb = 0;
  for (int i = 0; i < n_groups; ++i) {
    const pl_lora_group& gr = groups[i];
    int st = make_group(gr.modules, gr.num_modules, gr.in_features, &P->g[i]);
    if (st) return st;
    if (tokens > 0 && gr.x == nullptr) return fail(PL_ERR_INVALID, "group %d: x is null", i);
    if ((uintptr_t)gr.x % 16 || gr.ldx % 8 || gr.ldx < gr.in_features)
      return fail(PL_ERR_INVALID, "group %d: x must be 16-byte aligned with ldx %% 8 == 0 and ldx >= in_features", i);
    general = general > ws_bytes_needed(tokens, gr.in_features, P->g[i].r_pad)
                  ? general : ws_bytes_needed(tokens, gr.in_features, P->g[i].r_pad);
    FastGroup& F = P->fa.grp[i];
    F.g = P->g[i];
    F.x = gr.x;
    F.ldx = gr.ldx;
    F.in_features = gr.in_features;
    F.ksplit = (gr.in_features + kFastKSlice - 1) / kFastKSlice;
    F.n_rt = (F.g.r_total + 15) / 16;
    F.shrink_begin = sb;
    F.expand_begin = eb;
    F.n_expand = (F.g.out_total + kFastCols - 1) / kFastCols;
    sb += F.ksplit * F.n_rt * n_adapters;
    eb += F.n_expand;
    F.parity = (int*)(ws + (size_t)i * sizeof(int));
    F.acc = (long long*)(ws + kParityBytes + (size_t)i * 2 * kAccSlotBytes);
  }
  P->fa.n_groups = n_groups;
  P->fa.tokens = tokens;
  P->fa.n_adapters = n_adapters;
  P->shrink_total = sb;
  P->expand_total = eb;
  P->need = P->fast ? kParityBytes + (size_t)n_groups * 2 * kAccSlotBytes : kGeneralOffset + general;
  (void)dtype;
  return PL_OK;
}

extern "C" size_t pl_lora_delta_workspace_size(const pl_lora_group* groups_h, int num_groups, int num_tokens,
                                               int num_adapters) {
  DeltaPlan P;
  if (plan_delta(groups_h, num_groups, num_tokens, num_adapters, PL_DTYPE_BF16, nullptr, &P) != PL_OK) return 0;
  return P.need;
}

template <typename T, int NKT>
static int launch_expand_fast(const DeltaPlan& P, int out_dtype, hipStream_t stream) {
  const dim3 grid(P.expand_total);
  switch (out_dtype) {
    case PL_DTYPE_F32:
      hipLaunchKernelGGL((fast_expand_kernel<T, float, NKT>), grid, dim3(kExpandThreads), 0, stream, P.fa);
      break;
    case PL_DTYPE_F16:
      hipLaunchKernelGGL((fast_expand_kernel<T, f16_t, NKT>), grid, dim3(kExpandThreads), 0, stream, P.fa);
      break;
    case PL_DTYPE_BF16:
      hipLaunchKernelGGL((fast_expand_kernel<T, bf16_t, NKT>), grid, dim3(kExpandThreads), 0, stream, P.fa);
      break;
    default:
      return fail(PL_ERR_UNSUPPORTED, "out_dtype %d", out_dtype);
  }
  PL_LAUNCH_CHECK("lora fast_expand_kernel");
  return PL_OK;
}

template <typename T>
static int launch_fast(const DeltaPlan& P, int out_dtype, hipStream_t stream) {
  hipLaunchKernelGGL(fast_shrink_kernel<T>, dim3(P.shrink_total), dim3(kShrinkThreads), 0, stream, P.fa);
  PL_LAUNCH_CHECK("lora fast_shrink_kernel");
  int nkt = 1;
  for (int i = 0; i < P.fa.n_groups; ++i) nkt = nkt > P.fa.grp[i].g.r_pad / 32 ? nkt : P.fa.grp[i].g.r_pad / 32;
  switch (nkt) {
    case 1: return launch_expand_fast<T, 1>(P, out_dtype, stream);
    case 2: return launch_expand_fast<T, 2>(P, out_dtype, stream);
    case 3: return launch_expand_fast<T, 3>(P, out_dtype, stream);
    case 4: return launch_expand_fast<T, 4>(P, out_dtype, stream);
  }
  return fail(PL_ERR_UNSUPPORTED, "r_pad %d", nkt * 32);
}

static int delta_groups_impl(const pl_lora_group* groups_h, int num_groups, int num_tokens,
                             const int32_t* adapter_ids, int num_adapters, int dtype, int out_dtype,
                             void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "LoRA dtype must be F16 or BF16 (got %d)", dtype);
  if (out_dtype != PL_DTYPE_F32 && out_dtype != PL_DTYPE_F16 && out_dtype != PL_DTYPE_BF16)
    return fail(PL_ERR_UNSUPPORTED, "out_dtype %d", out_dtype);
  if (num_tokens > 0 && adapter_ids == nullptr) return fail(PL_ERR_INVALID, "adapter_ids is null");
  if (workspace == nullptr || (uintptr_t)workspace % 256)
    return fail(PL_ERR_INVALID, "workspace must be non-null and 256-byte aligned");
  DeltaPlan P;
  int st = plan_delta(groups_h, num_groups, num_tokens, num_adapters, dtype, (char*)workspace, &P);
  if (st) return st;
  if (P.need > workspace_bytes)
    return fail(PL_ERR_WORKSPACE, "LoRA workspace of %zu bytes < %zu needed", workspace_bytes, P.need);
  if (num_tokens == 0) return ok();
  if (P.fast) {
    P.fa.ids = adapter_ids;
    st = dtype == PL_DTYPE_BF16 ? launch_fast<bf16_t>(P, out_dtype, stream) : launch_fast<f16_t>(P, out_dtype, stream);
    return st ? st : ok();
  }
  void* body = (char*)workspace + kGeneralOffset;
  const size_t body_bytes = workspace_bytes - kGeneralOffset;
  for (int i = 0; i < num_groups; ++i) {
    const pl_lora_group& gr = groups_h[i];
    if ((st = lora_shrink_impl(gr.x, gr.ldx, num_tokens, gr.in_features, P.g[i], adapter_ids, num_adapters, dtype,
                               body, body_bytes, stream)))
      return st;
    if ((st = lora_expand_impl(num_tokens, gr.in_features, P.g[i], adapter_ids, num_adapters, dtype, out_dtype,
                               body, body_bytes, stream)))
      return st;
  }
  return ok();
}

extern "C" int pl_lora_delta_groups(const pl_lora_group* groups_h, int num_groups, int num_tokens,
                                    const int32_t* adapter_ids, int num_adapters, int dtype, int out_dtype,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  return delta_groups_impl(groups_h, num_groups, num_tokens, adapter_ids, num_adapters, dtype, out_dtype,
                           workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int pl_lora_delta(const void* x, int64_t ldx, int num_tokens, int in_features,
                             const pl_lora_module* modules_h, int num_modules,
                             const int32_t* adapter_ids, int num_adapters, int dtype,
                             int out_dtype, void* workspace, size_t workspace_bytes,
                             void* stream) {
  const pl_lora_group g = {x, ldx, in_features, num_modules, modules_h};
  return delta_groups_impl(&g, 1, num_tokens, adapter_ids, num_adapters, dtype, out_dtype, workspace,
                           workspace_bytes, (hipStream_t)stream);
}
