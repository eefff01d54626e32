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
//   fast_shrink_kernel  grid (group, 256-element k-slice, 16 rank rows):
//                  each wave loads its 16 tokens' x slice once, the
//                  workgroup stages every adapter's A tile once in LDS (in
//                  the MFMA operand order), one MFMA chain per adapter keeps
//                  the rows of the tokens that use it, and each (token,
//                  rank) sum is added into a 64-bit fixed-point accumulator
//                  (order-independent, so deterministic).
//   fast_expand_kernel  grid (group, 256 output columns): the 32-rank tiles
//                  of the intermediate its columns use (rounded to the input
//                  dtype into LDS), ids, B rows and outputs in one round
//                  trip, MFMA per adapter over the token tiles,
//                  out += scale * result.
//
// Reference semantics: packed_ops.py:314-384 (packed A_cat / block-diagonal
// B with the scale folded in), packed_ops.py:534-553 and
// multilora/linear.py:226-231 (per-module F.linear(F.linear(x, A), B) * s).
#include <algorithm>
#include <type_traits>

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
// caller clamps it), the value is zeroed afterwards with a mask (a select
// lets the compiler skip the load in a branch, and a load inside a branch
// makes every later wait on the load counter conservative).
__device__ __forceinline__ uint4 load8_sel(const void* p, bool ok) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  const uint32_t m = 0u - (uint32_t)ok;
  return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
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
  __shared__ int s_nf[kWaves];
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
    bool nonfinite = false;  // this thread rounded a NaN or an infinity into the tile
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
      const T yt = from_float<T>(sum);
      nonfinite |= !__builtin_isfinite(to_float<T>(yt));
      s_y[i][k] = __builtin_bit_cast(uint16_t, yt);
    }
    const uint64_t nf_ballot = __ballot(nonfinite);
    if (lane == 0) s_nf[wave] = nf_ballot != 0;
    __syncthreads();
    bool any_nonfinite = false;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) any_nonfinite |= s_nf[w] != 0;
    if (tile_ok) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if (!any_nonfinite) {
#pragma unroll
        for (int kt = 0; kt < kMaxKt; ++kt) {  // static indices keep bop[] in registers
          if (kt < n_kt) {
            const uint4 av = *reinterpret_cast<const uint4*>(&s_y[lr][kt * 32 + kq]);
            acc = mfma32<T>(av, bop[kt], acc);
          }
        }
      } else if (mi >= 0) {
        // a NaN or an infinity in the tile: the contraction over the
        // concatenated ranks would carry it into the other modules' columns
        // through B's zeros (0 * inf = NaN), so each output is the column
        // module's own dot product, as F.linear(F.linear(x, A_m), B_m) gives
        const Mod& m = g.m[mi];
        const T* brow = (const T*)m.B + ((int64_t)a * m.out_features + (o - m.out_offset)) * m.rank;
#pragma unroll 1
        for (int i = 0; i < 4; ++i) {
          const int row = (lane / 16) * 4 + i;
          float sum = 0.f;
#pragma unroll 1
          for (int jl = 0; jl < m.rank; ++jl)
            sum += to_float<T>(__builtin_bit_cast(T, s_y[row][m.rank_offset + jl])) * to_float<T>(brow[jl]);
          acc[i] = sum;
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
constexpr int kShrinkAChunk = 4;      // adapters whose A tiles a shrink workgroup holds in LDS at once
// Expand workgroups: 8 waves (128 columns) when a call needs at most one
// workgroup per CU that way, else 16 waves (256 columns).  More workgroups
// than CUs put two on some CUs, and those finish last: a decoder layer's
// 38912 output columns in 304 128-column workgroups took as long as in 152
// 256-column ones, while one group alone (16-96 workgroups) needs the narrow
// ones to spread over the chip.
constexpr int kExpandCUs = 256;
constexpr int kFastAChunk = 4;        // adapters whose B rows an expand wave holds at once
constexpr int kFastTt = kFastMaxTokens / 16;
constexpr int kFastMaxRank = 128;     // r_pad limit (make_group)
// The shrink's slices meet in a signed 64-bit fixed-point accumulator with
// 26 fraction bits: integer adds are associative, so the sum (and the
// rounded intermediate) does not depend on the order the slices arrive in.
// Each finite partial is clamped to +-2^31 first, so 64 slices cannot
// overflow.  A non-finite partial is not added: it sets a flag bit of its
// (token, rank) instead (kFlagNaN, kFlagPosInf, kFlagNegInf, ORed over the
// slices) and the slot's any-flag word, and the expand turns a flagged value
// into what a float sum of the partials gives: NaN when a NaN or both
// infinities were seen, else the infinity.  The expand then computes the
// outputs of a call with non-finite intermediates per module (below).
constexpr float kFixScale = 67108864.f;          // 2^26
constexpr double kFixInv = 1.0 / 67108864.0;
constexpr float kFixClamp = 2147483648.f;        // 2^31
constexpr int kFlagNaN = 1, kFlagPosInf = 2, kFlagNegInf = 4;
// Workspace of pl_lora_delta(_groups): per group a parity word, then per
// group two fixed-size accumulator slots, then the general path's shrink
// partials (disjoint regions, so a general-path call never disturbs the
// decode path's state).  A call's shrink adds into slot `parity` and clears
// the other slot whole (the one the previous call's expand read); the expand
// reads the sum of both slots and flips the parity.  Starting from an
// all-zero workspace, the slot a shrink adds into is therefore always zero,
// with no wait inside either kernel: the kernel boundaries order the clear
// against the reads.  A slot is the accumulator [tokens][r_pad] (int64),
// the non-finite flags [tokens][r_pad] (int32) and the any-flag word.
constexpr size_t kParityBytes = 256;
constexpr size_t kAccBytes = (size_t)kFastMaxTokens * kFastMaxRank * sizeof(long long);
constexpr size_t kFlagBytes = (size_t)kFastMaxTokens * kFastMaxRank * sizeof(int);
constexpr size_t kAccSlotBytes = kAccBytes + kFlagBytes + 256;
constexpr size_t kAccSlotPairs = kAccSlotBytes / 16;
static_assert(kAccSlotBytes % 256 == 0, "slots stay 256-byte aligned");
constexpr size_t kGeneralOffset = kParityBytes + 2 * PL_LORA_MAX_GROUPS * kAccSlotBytes;

struct FastGroup {
  Group g;
  const void* x;
  int64_t ldx;
  int in_features;
  int ksplit;        // k-slices of kFastKSlice
  int n_rt;          // rank tiles of 16 rows holding real ranks
  int n_expand;      // expand workgroups of the group
  int expand_begin;  // its first workgroup in the (flat) expand grid
  long long* acc;    // two slots of [tokens][r_pad] fixed point (kAccSlotBytes apart)
  int* parity;       // the slot this call's shrink adds into
};

struct FastArgs {
  FastGroup grp[PL_LORA_MAX_GROUPS];
  int n_groups, tokens, n_adapters;
  const int32_t* ids;
};

// In an SGPR from here on and opaque to the compiler: every argument field
// pinned at a kernel's top is loaded in one batch with one wait (otherwise
// each is loaded next to its first use, a dependent round trip apiece), and
// is never re-read from the argument segment later.
template <typename V>
__device__ __forceinline__ V pin(V v) {
  if constexpr (sizeof(V) == 8) {
    uint64_t u = __builtin_bit_cast(uint64_t, v);
    asm volatile("" : "+s"(u));
    return __builtin_bit_cast(V, u);
  } else {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    asm volatile("" : "+s"(u));
    return __builtin_bit_cast(V, u);
  }
}

__device__ __forceinline__ long long to_fixed(float v) {
  return (long long)__builtin_rintf(fminf(fmaxf(v, -kFixClamp), kFixClamp) * kFixScale);
}

// The flag bit of a non-finite partial.
__device__ __forceinline__ int nonfinite_flag(float v) {
  return __builtin_isnan(v) ? kFlagNaN : (v > 0.f ? kFlagPosInf : kFlagNegInf);
}

// Row j of the group's concatenated A (adapter 0) as a byte offset from
// module 0's A, plus the element stride between adapters; blended from the
// module descriptors with bit masks (no per-lane indexing into them).
struct ARow {
  uint64_t off;    // bytes from m[0].A to A_m[0][j - rank_offset][0]
  int64_t stride;  // elements between adapters a and a + 1 (rank_m * in_features)
  bool ok;         // j is a real rank row
};

// The shrink's view of a group's modules (pinned argument fields).
struct ShrinkMods {
  const void* A[PL_LORA_MAX_MODULES];
  int rank[PL_LORA_MAX_MODULES], roff[PL_LORA_MAX_MODULES];
  int n;
};

template <typename T>
__device__ __forceinline__ ARow a_row(const ShrinkMods& g, int j, int in_features) {
  ARow r{0, 0, false};
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
    const bool in = (m < g.n) & (j >= g.roff[m]) & (j < g.roff[m] + g.rank[m]);
    const uint64_t mask = 0 - (uint64_t)in;
    const uint64_t row = (uint64_t)(uintptr_t)((const T*)g.A[m] + (int64_t)(j - g.roff[m]) * in_features);
    r.off |= (row - (uint64_t)(uintptr_t)g.A[0]) & mask;
    r.stride |= ((int64_t)g.rank[m] * in_features) & (int64_t)mask;
    r.ok |= in;
  }
  return r;
}

// Shrink: workgroup (group, k-slice, 16 rank rows), one 16-token tile per
// wave, every adapter.  The wave loads its tokens' x slice once; the
// workgroup stages each adapter's 16 x kFastKSlice A tile once, in the MFMA
// B-operand order, in LDS (kShrinkAChunk adapters at a time, the first
// chunk's loads issued with x); per adapter the wave runs one MFMA chain and
// keeps the rows of its tokens that use that adapter.  Each (token, rank)
// result is then added into the fixed-point accumulator with one
// device-scope atomic (nothing waits on it).
template <typename T>
__global__ __launch_bounds__(kShrinkThreads) void fast_shrink_kernel(FastArgs fa) {
  __shared__ __align__(16) uint4 s_a[kShrinkAChunk][kFastKSteps][kWave];
  // grid (most workgroups of a group, groups): a flat grid without the
  // padding workgroups measured slower (cfg4 layer 16.90 vs 16.82 us), its
  // group lookup putting a dependent argument load before the others
  const FastGroup& G = fa.grp[blockIdx.y];
  // every argument field before the first address: loaded in one batch,
  // then held in SGPRs (one asm statement takes them all, so there is one
  // wait, and the compiler cannot re-read them from the argument segment)
  ShrinkMods sm;
  uint64_t a_ptr[PL_LORA_MAX_MODULES];
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
    a_ptr[m] = (uint64_t)(uintptr_t)G.g.m[m].A;
    sm.rank[m] = G.g.m[m].rank;
    sm.roff[m] = G.g.m[m].rank_offset;
  }
  sm.n = G.g.n;
  int n_rt = G.n_rt, ksplit = G.ksplit, in_f = G.in_features, r_pad = G.g.r_pad, r_total = G.g.r_total;
  int T_ = fa.tokens, n_ad = fa.n_adapters;
  uint64_t gx_u = (uint64_t)(uintptr_t)G.x, acc_u = (uint64_t)(uintptr_t)G.acc;
  uint64_t par_u = (uint64_t)(uintptr_t)G.parity, ids_u = (uint64_t)(uintptr_t)fa.ids;
  int64_t ldx = G.ldx;
  asm volatile(""
               : "+s"(a_ptr[0]), "+s"(a_ptr[1]), "+s"(a_ptr[2]), "+s"(a_ptr[3]), "+s"(sm.rank[0]),
                 "+s"(sm.rank[1]), "+s"(sm.rank[2]), "+s"(sm.rank[3]), "+s"(sm.roff[0]), "+s"(sm.roff[1]),
                 "+s"(sm.roff[2]), "+s"(sm.roff[3]), "+s"(sm.n), "+s"(n_rt), "+s"(ksplit), "+s"(in_f),
                 "+s"(r_pad), "+s"(r_total), "+s"(T_), "+s"(n_ad), "+s"(gx_u), "+s"(acc_u), "+s"(par_u),
                 "+s"(ids_u), "+s"(ldx));
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) sm.A[m] = gptr<const char*>(a_ptr[m]);
  const void* gx = gptr<const char*>(gx_u);
  long long* const gacc = gptr<long long*>(acc_u);
  const int* const gpar = gptr<const int*>(par_u);
  const int32_t* const ids = gptr<const int32_t*>(ids_u);
  const int local = blockIdx.x;
  if (local >= ksplit * n_rt) return;  // past the group's count (after the one argument batch)
  const int rt = local % n_rt;
  const int ks = local / n_rt;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;   // token tile
  const int lr = lane % 16;
  const int kq = (lane / 16) * 8;
  const int t = wave * 16 + lr;           // the token of this lane's x row
  const bool t_ok = t < T_;
  const int k0 = ks * kFastKSlice;

  // staging role: pieces p = threadIdx.x + u * kShrinkThreads of an A tile,
  // p -> rank row p / 32 of the tile, k elements (p % 32) * 8 .. +8; in LDS
  // at k-step (p % 32) / 4, lane ((p % 32) % 4) * 16 + row
  constexpr int kPieces = 16 * kFastKSlice / 8 / kShrinkThreads;  // 2
  const T* a0p = (const T*)sm.A[0];
  const T* arow[kPieces];
  int64_t astride[kPieces];
  bool aok[kPieces];
  int lds_s[kPieces], lds_l[kPieces];
#pragma unroll
  for (int u = 0; u < kPieces; ++u) {
    const int p = threadIdx.x + u * kShrinkThreads;
    const int row = p / 32, kp = p % 32;
    const int k = k0 + kp * 8;
    const ARow ar = a_row<T>(sm, rt * 16 + row, in_f);
    const bool ok = ar.ok & (k < in_f);
    arow[u] = (const T*)((const char*)a0p + (ok ? ar.off : 0)) + (ok ? k : 0);
    astride[u] = ok ? ar.stride : 0;
    aok[u] = ok;
    lds_s[u] = kp / 4;
    lds_l[u] = (kp % 4) * 16 + row;
  }
  auto load_chunk = [&](int a_first, uint4 (&av)[kShrinkAChunk][kPieces]) {
#pragma unroll
    for (int c = 0; c < kShrinkAChunk; ++c)
#pragma unroll
      for (int u = 0; u < kPieces; ++u) {
        const bool ok = aok[u] & (a_first + c < n_ad);
        av[c][u] = load8_sel(arow[u] + (ok ? (int64_t)(a_first + c) * astride[u] : 0), ok);
      }
  };
  // the first A chunk, then x of the wave's tokens (a lane's 8-element
  // group lies wholly inside or outside in_features, in_features % 8 == 0;
  // out-of-range groups re-read the row's first and are zeroed), then the ids
  uint4 av[kShrinkAChunk][kPieces];
  load_chunk(0, av);
  const T* xrow = (const T*)gx + (int64_t)(t_ok ? t : 0) * ldx;
  uint4 xv[kFastKSteps];
#pragma unroll
  for (int s = 0; s < kFastKSteps; ++s) {
    const int k = k0 + s * 32 + kq;
    const bool k_ok = k < in_f;
    xv[s] = load8_sel(xrow + (k_ok ? k : 0), t_ok & k_ok);
  }
  const int id_raw = ids[t_ok ? t : 0];
  const int id = t_ok ? id_raw : -1;
  __builtin_amdgcn_sched_barrier(0);  // the first A chunk, x and ids in flight together
  const int par = *gpar & 1;
  long long* acc = gacc + (par ? kAccSlotBytes / sizeof(long long) : 0);
  long long* other = gacc + (par ? 0 : kAccSlotBytes / sizeof(long long));

  int id_tr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) id_tr[i] = __shfl(id, (lane / 16) * 4 + i);
  f32x4 res = {0.f, 0.f, 0.f, 0.f};
  for (int a0 = 0; a0 < n_ad; a0 += kShrinkAChunk) {
    if (a0 > 0) {
      load_chunk(a0, av);
      __syncthreads();  // every wave is done with the previous chunk's tiles
    }
#pragma unroll
    for (int c = 0; c < kShrinkAChunk; ++c)
#pragma unroll
      for (int u = 0; u < kPieces; ++u) s_a[c][lds_s[u]][lds_l[u]] = av[c][u];
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kShrinkAChunk; ++c) {
      const int a = a0 + c;
      if (a >= n_ad) break;
      f32x4 part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kFastKSteps; ++s) part = mfma32<T>(xv[s], s_a[c][s][lane], part);
#pragma unroll
      for (int i = 0; i < 4; ++i) res[i] = id_tr[i] == a ? part[i] : res[i];
    }
  }
  // D rows = tokens wave*16 + 4*(lane/16) + i, column = rank row j
  const int j = rt * 16 + lr;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tr = wave * 16 + (lane / 16) * 4 + i;
    if (tr < T_ && id_tr[i] >= 0 && id_tr[i] < n_ad && j < r_total) {
      const int64_t e = (int64_t)tr * r_pad + j;
      if (__builtin_isfinite(res[i])) {
        __hip_atomic_fetch_add(acc + e, to_fixed(res[i]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {  // flagged instead (the expand reads the flags when the slot's any-flag is set)
        int* flags = reinterpret_cast<int*>(reinterpret_cast<char*>(acc) + kAccBytes);
        __hip_atomic_fetch_or(flags + e, nonfinite_flag(res[i]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_or(flags + kFlagBytes / sizeof(int), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // this workgroup's share of clearing the other slot (all of it: an earlier
  // call may have used it with another layout)
  const int n_wg = ksplit * n_rt;
  const int per = (int)((kAccSlotPairs + n_wg - 1) / n_wg);
  const int c_end = min((int)kAccSlotPairs, (local + 1) * per);
  for (int c = local * per + threadIdx.x; c < c_end; c += kShrinkThreads)
    *reinterpret_cast<longlong2*>(other + 2 * (int64_t)c) = longlong2{0, 0};
}

// The 32-rank tiles [lo, hi] that the modules of columns c_first .. c_last
// (inside the group's columns) use; modules are ordered by both column and
// rank offset, so the first and last columns' modules bound the range.
// The expand's view of a group's modules (pinned argument fields).
struct ExpandMods {
  uint64_t B[PL_LORA_MAX_MODULES], out[PL_LORA_MAX_MODULES];
  int64_t ldo[PL_LORA_MAX_MODULES];
  uint32_t scale[PL_LORA_MAX_MODULES];  // float bits
  int rank[PL_LORA_MAX_MODULES], roff[PL_LORA_MAX_MODULES], outf[PL_LORA_MAX_MODULES], ooff[PL_LORA_MAX_MODULES];
  int n;
};

__device__ __forceinline__ void rank_tiles(const ExpandMods& g, int c_first, int c_last, int& lo, int& hi) {
  lo = 0;
  hi = 0;
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
    const bool f = (m < g.n) & (c_first >= g.ooff[m]) & (c_first < g.ooff[m] + g.outf[m]);
    const bool l = (m < g.n) & (c_last >= g.ooff[m]) & (c_last < g.ooff[m] + g.outf[m]);
    lo |= (g.roff[m] / 32) & -(int)f;
    hi |= ((g.roff[m] + g.rank[m] - 1) / 32) & -(int)l;
  }
}

// Expand: workgroup (group, 256 output columns), every adapter; NKT: the
// most 32-rank tiles any wave's 16 columns use (1 when every module's ranks
// sit in one tile).  The workgroup stages only the tiles its columns use:
// the fixed-point intermediate of every token (both slots, one of which the
// shrink cleared), rounded to the input dtype into LDS as the reference's
// F.linear returns it.  Those loads, the ids, the B rows of the first
// adapters and the outputs go out together (one round trip).  Per token
// tile and adapter an MFMA over the wave's tiles gives scale * y . B^T for
// the wave's 16 columns, kept for the rows of that adapter; the deltas meet
// in LDS, and each thread then adds them into two 8-column chunks of one
// output row (16-byte loads and stores; the host routes outputs that are not
// 16-byte aligned in 8-column chunks to the general path).
template <typename OT>
struct OutChunk {  // 8 consecutive outputs
  static constexpr int kWords = 8 * sizeof(OT) / 16;
  uint4 w[kWords];
};

// The value a float sum of partials gives whose non-finite ones set `flags`
// (nonzero): NaN when a NaN or both infinities were seen, else the infinity.
__device__ __forceinline__ float flagged_value(int flags) {
  const bool nan = (flags & kFlagNaN) | ((flags & (kFlagPosInf | kFlagNegInf)) == (kFlagPosInf | kFlagNegInf));
  return nan ? __builtin_nanf("") : ((flags & kFlagPosInf) ? __builtin_inff() : -__builtin_inff());
}

// A call whose rounded intermediate holds a NaN or an infinity: the MFMA's
// contraction over the group's concatenated ranks multiplies it by the zeros
// of B outside its module (0 * inf = NaN), so the outputs of the
// decode-size expand are computed here instead, per module as
// F.linear(F.linear(x, A_m), B_m) * scale does:
//   d[e] = scale * sum_j y[j] * B[c + e][j],  j over the columns' module,
// in fp32 with IEEE semantics, y read from the LDS tile (the values rounded
// to T) and B from memory.  Slow, and taken only by such calls.
template <typename T>
__device__ __forceinline__ void module_dot(const ExpandMods& em, const uint16_t* y_row, int c, int a,
                                           float (&d)[8]) {
  uint64_t b_off = 0;
  uint32_t scale_bits = 0;
  int roff = 0, rank = 0, outf = 0, ooff = 0;
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {  // blended with masks (an index would move em to scratch)
    const bool in = (m < em.n) & (c >= em.ooff[m]) & (c < em.ooff[m] + em.outf[m]);
    const uint64_t mask = 0 - (uint64_t)in;
    b_off |= (em.B[m] - em.B[0]) & mask;
    scale_bits |= em.scale[m] & (uint32_t)mask;
    roff |= em.roff[m] & (int)mask;
    rank |= em.rank[m] & (int)mask;
    outf |= em.outf[m] & (int)mask;
    ooff |= em.ooff[m] & (int)mask;
  }
  const T* B = (const T*)(gptr<const char*>(em.B[0]) + (int64_t)b_off) + ((int64_t)a * outf + (c - ooff)) * rank;
#pragma unroll 1
  for (int e8 = 0; e8 < 8; ++e8) {
    float sum = 0.f;
#pragma unroll 1
    for (int jl = 0; jl < rank; ++jl)
      sum += to_float<T>(__builtin_bit_cast(T, y_row[roff + jl])) * to_float<T>(B[(int64_t)e8 * rank + jl]);
    d[e8] = __uint_as_float(scale_bits) * sum;
  }
}

template <typename T, typename OT, int NKT, bool MANY, int EW>
__global__ __launch_bounds__(EW * 64) void fast_expand_kernel(FastArgs fa) {
  constexpr int kExpandWaves = EW;
  constexpr int kExpandThreads = EW * 64;
  constexpr int kFastCols = 16 * EW;  // output columns per workgroup (16 per wave)
  // 16-byte accumulator pairs one thread stages per slot and 32-rank tile
  constexpr int kStagePairs = kFastMaxTokens * 32 / 2 / kExpandThreads;
  static_assert(kStagePairs * kExpandThreads * 2 == kFastMaxTokens * 32, "staging covers one 32-rank tile");
  __shared__ __align__(16) uint16_t s_y[kFastMaxTokens][kFastMaxRank + 8];  // +8 keeps rows 16-byte aligned
  __shared__ __align__(16) float s_d[kFastMaxTokens][kFastCols + 4];        // +4: rows start on other banks
  __shared__ int s_nf[EW];
  // flat grid, groups in order (a 2-D grid pads every group to the largest:
  // the idle workgroups slow the dispatch of the rest)
  int gi = 0;
#pragma unroll
  for (int i = 1; i < PL_LORA_MAX_GROUPS; ++i)
    if (i < fa.n_groups && (int)blockIdx.x >= fa.grp[i].expand_begin) gi = i;
  const FastGroup& G = fa.grp[gi];
  // every argument field before the first address: loaded in one batch,
  // then held in SGPRs (the first asm statement waits for every load issued
  // before it, and the compiler cannot re-read them from the argument segment)
  ExpandMods em;
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
    const Mod& M = G.g.m[m];
    em.B[m] = (uint64_t)(uintptr_t)M.B;
    em.out[m] = (uint64_t)(uintptr_t)M.out;
    em.ldo[m] = M.ldo;
    em.scale[m] = __float_as_uint(M.scale);
    em.rank[m] = M.rank;
    em.roff[m] = M.rank_offset;
    em.outf[m] = M.out_features;
    em.ooff[m] = M.out_offset;
  }
  em.n = G.g.n;
  int e_begin = G.expand_begin, r_pad = G.g.r_pad, out_total = G.g.out_total, T_ = fa.tokens, n_ad = fa.n_adapters;
  uint64_t acc_u = (uint64_t)(uintptr_t)G.acc, par_u = (uint64_t)(uintptr_t)G.parity;
  uint64_t ids_u = (uint64_t)(uintptr_t)fa.ids;
  asm volatile(""
               : "+s"(em.B[0]), "+s"(em.B[1]), "+s"(em.B[2]), "+s"(em.B[3]), "+s"(em.out[0]), "+s"(em.out[1]),
                 "+s"(em.out[2]), "+s"(em.out[3]), "+s"(em.ldo[0]), "+s"(em.ldo[1]), "+s"(em.ldo[2]),
                 "+s"(em.ldo[3]), "+s"(em.scale[0]), "+s"(em.scale[1]), "+s"(em.scale[2]), "+s"(em.scale[3]),
                 "+s"(em.rank[0]), "+s"(em.rank[1]), "+s"(em.rank[2]), "+s"(em.rank[3]));
  asm volatile(""
               : "+s"(em.roff[0]), "+s"(em.roff[1]), "+s"(em.roff[2]), "+s"(em.roff[3]), "+s"(em.outf[0]),
                 "+s"(em.outf[1]), "+s"(em.outf[2]), "+s"(em.outf[3]), "+s"(em.ooff[0]), "+s"(em.ooff[1]),
                 "+s"(em.ooff[2]), "+s"(em.ooff[3]), "+s"(em.n), "+s"(e_begin), "+s"(r_pad), "+s"(out_total),
                 "+s"(T_), "+s"(n_ad), "+s"(acc_u), "+s"(par_u), "+s"(ids_u));
  const int32_t* const ids = gptr<const int32_t*>(ids_u);
  const int ct = blockIdx.x - e_begin;
  const int n_tt = (T_ + 15) / 16;
  const int c0 = ct * kFastCols;

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform: scalar loop bounds
  const int lr = lane % 16;
  const int kq = (lane / 16) * 8;
  const int tile = ct * kExpandWaves + wave;
  const int o = tile * 16 + lr;  // this lane's output column (concatenated space)
  const long long* accp = gptr<const long long*>(acc_u);
  constexpr int64_t kSlot = kAccSlotBytes / sizeof(long long);

  // the workgroup's tiles; the first one's accumulator loads go out first
  int kt_lo, kt_hi;
  rank_tiles(em, c0, min(c0 + kFastCols, out_total) - 1, kt_lo, kt_hi);
  auto stage_load = [&](int kt, longlong2 (&av)[kStagePairs], longlong2 (&bv)[kStagePairs]) {
#pragma unroll
    for (int u = 0; u < kStagePairs; ++u) {
      const int p = u * kExpandThreads + threadIdx.x;
      const int tk = p / 16, j2 = kt * 32 + 2 * (p % 16);
      const int64_t off = tk < T_ ? (int64_t)tk * r_pad + j2 : 0;
      av[u] = *reinterpret_cast<const longlong2*>(accp + off);
      bv[u] = *reinterpret_cast<const longlong2*>(accp + kSlot + off);
    }
  };
  // the slots' non-finite flags (read only when a shrink flagged a value)
  const int* const flg = reinterpret_cast<const int*>(reinterpret_cast<const char*>(accp) + kAccBytes);
  constexpr int64_t kFlagSlot = kAccSlotBytes / sizeof(int);
  bool nonfinite = false;  // this thread staged a NaN or an infinity
  auto stage_store = [&](int kt, const longlong2 (&av)[kStagePairs], const longlong2 (&bv)[kStagePairs],
                         bool flagged) {
#pragma unroll
    for (int u = 0; u < kStagePairs; ++u) {
      const int p = u * kExpandThreads + threadIdx.x;
      const int tk = p / 16, j2 = kt * 32 + 2 * (p % 16);
      if (tk < T_) {
        const long long x0 = av[u].x + bv[u].x, x1 = av[u].y + bv[u].y;
        float y0 = (float)((double)x0 * kFixInv), y1 = (float)((double)x1 * kFixInv);
        if (flagged) {  // uniform: a shrink of this call flagged a non-finite partial
          const int64_t e = (int64_t)tk * r_pad + j2;
          const int f0 = flg[e] | flg[kFlagSlot + e], f1 = flg[e + 1] | flg[kFlagSlot + e + 1];
          y0 = f0 ? flagged_value(f0) : y0;
          y1 = f1 ? flagged_value(f1) : y1;
        }
        const T t0 = from_float<T>(y0), t1 = from_float<T>(y1);
        // a NaN or an infinity, also from rounding a finite value past T's range
        nonfinite = nonfinite || !__builtin_isfinite(to_float<T>(t0)) || !__builtin_isfinite(to_float<T>(t1));
        *reinterpret_cast<uint32_t*>(&s_y[tk][j2]) =
            __builtin_bit_cast(uint16_t, t0) | ((uint32_t)__builtin_bit_cast(uint16_t, t1) << 16);
      }
    }
  };
  // lane l holds token l's adapter (tokens <= 64 = the wave); -1: none.
  // Issued first: the counter of outstanding loads drains in issue order,
  // so the staging's wait for the accumulator then covers the ids too.
  const int id_raw = ids[lane < T_ ? lane : 0];
  longlong2 av2[kStagePairs], bv2[kStagePairs];
  stage_load(kt_lo, av2, bv2);
  // the any-flag words of both slots (nonzero only after a non-finite
  // partial), loaded with the accumulator and read once every load is out
  const int any0 = flg[kFlagBytes / sizeof(int)], any1 = flg[kFlagSlot + kFlagBytes / sizeof(int)];
  __builtin_amdgcn_sched_barrier(0);  // these first: the staging then waits for them alone

  // the read-modify-write role: chunks q = threadIdx.x + u * kExpandThreads,
  // token row q / kRowChunks, columns c0 + (q % kRowChunks) * 8 .. +8, each
  // inside one module
  constexpr int kRowChunks = kFastCols / 8;
  constexpr int kChunks = kFastMaxTokens * kRowChunks / kExpandThreads;  // 2
  static_assert(kChunks * kExpandThreads == kFastMaxTokens * kRowChunks, "every chunk has a thread");
  OutChunk<OT> cur[kChunks];
  OT* cptr[kChunks];
  bool cok[kChunks];
#pragma unroll
  for (int u = 0; u < kChunks; ++u) {
    const int q = threadIdx.x + u * kExpandThreads;
    const int tk = q / kRowChunks, c = c0 + (q % kRowChunks) * 8;
    uint64_t off = 0, ld = 0;
    int ooff = 0;
    bool in_any = false;
#pragma unroll
    for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
      const bool in = (m < em.n) & (c >= em.ooff[m]) & (c < em.ooff[m] + em.outf[m]);
      const uint64_t mask = 0 - (uint64_t)in;
      off |= (em.out[m] - em.out[0]) & mask;
      ld |= (uint64_t)em.ldo[m] & mask;
      ooff |= em.ooff[m] & (int)mask;
      in_any |= in;
    }
    // the address needs no id (the id only decides the store)
    cok[u] = in_any & (tk < T_);
    cptr[u] = (OT*)(gptr<char*>(em.out[0]) + (cok[u] ? (int64_t)off : 0)) +
              (cok[u] ? (int64_t)tk * (int64_t)ld + (c - ooff) : 0);
#pragma unroll
    for (int w = 0; w < OutChunk<OT>::kWords; ++w) cur[u].w[w] = reinterpret_cast<const uint4*>(cptr[u])[w];
  }

  // The lane's module, blended from the four (uniform) module descriptors
  // with bit masks: a per-lane index into them would read the kernel
  // arguments with dependent vector loads, and a select lets the compiler
  // sink each field's load into a branch of its own (one wait apiece).
  // B is addressed as a byte offset from module 0's, so it stays a
  // global-memory pointer to the compiler (no flat accesses).
  bool has_mod = false;
  uint64_t b_off = 0;
  uint32_t scale_bits = 0;
  int m_rank = 0, m_roff = 0, m_out = 0, m_ooff = 0;
#pragma unroll
  for (int m = 0; m < PL_LORA_MAX_MODULES; ++m) {
    const bool in = (m < em.n) & (o >= em.ooff[m]) & (o < em.ooff[m] + em.outf[m]);
    const uint64_t mask = 0 - (uint64_t)in;
    has_mod |= in;
    b_off |= (em.B[m] - em.B[0]) & mask;
    scale_bits |= em.scale[m] & (uint32_t)mask;
    m_rank |= em.rank[m] & (int)mask;
    m_roff |= em.roff[m] & (int)mask;
    m_out |= em.outf[m] & (int)mask;
    m_ooff |= em.ooff[m] & (int)mask;
  }
  const float scale = __uint_as_float(scale_bits);
  // the wave's tiles: kw_lo .. kw_hi (at most NKT), none for a wave past the columns
  int kw_lo = 0, kw_hi = -1;
  if (tile * 16 < out_total) rank_tiles(em, tile * 16, min(tile * 16 + 16, out_total) - 1, kw_lo, kw_hi);

  // B operand of adapter a for the wave's tile kw_lo + k: B_m[a][o_local][j -
  // rank_offset] for j inside the column's module, zero elsewhere.  Ranks
  // and rank offsets are multiples of 8 on this path, so a lane's 8 ranks
  // lie wholly inside or outside its module.
  auto load_b = [&](int a, uint4 (&bop)[NKT]) {
    const bool a_ok = a < n_ad;
    const T* brow = (const T*)(gptr<const char*>(em.B[0]) + (int64_t)b_off) +
                    ((int64_t)(a_ok ? a : 0) * m_out + (has_mod ? o - m_ooff : 0)) * m_rank;
#pragma unroll
    for (int k = 0; k < NKT; ++k) {
      const int j0 = (kw_lo + k) * 32 + kq - m_roff;  // local rank index of element 0
      const bool ok = (j0 >= 0) & (j0 < m_rank) & has_mod & a_ok;
      bop[k] = load8_sel(brow + (ok ? j0 : 0), ok);
    }
  };
  uint4 bop[kFastAChunk][NKT];
#pragma unroll
  for (int u = 0; u < kFastAChunk; ++u) load_b(u, bop[u]);
  __builtin_amdgcn_sched_barrier(0);  // every load of the workgroup in flight
  const bool flagged = __builtin_amdgcn_readfirstlane(any0 | any1) != 0;

  // the intermediate into LDS: one rounding to T per value; further tiles
  // (a workgroup whose columns straddle modules of different tiles) one
  // round trip each
  stage_store(kt_lo, av2, bv2, flagged);
  for (int kt = kt_lo + 1; kt <= kt_hi; ++kt) {
    stage_load(kt, av2, bv2);
    stage_store(kt, av2, bv2, flagged);
  }
  // whether any wave staged a non-finite value (one word per wave, no
  // initialisation needed), read after the barrier
  const uint64_t nf_ballot = __ballot(nonfinite);
  if (lane == 0) s_nf[wave] = nf_ballot != 0;
  __syncthreads();
  bool any_nonfinite = false;
#pragma unroll
  for (int w = 0; w < kExpandWaves; ++w) any_nonfinite |= s_nf[w] != 0;
  // the next call's shrink adds into the other slot (no expand workgroup
  // reads the parity, so the flip can go out at any time)
  if (ct == 0 && threadIdx.x == 0) *gptr<int*>(par_u) ^= 1;
  if (any_nonfinite) {
    // a NaN or an infinity in the staged intermediate: each output of the
    // thread's chunks is its module's own dot product (module_dot), added to
    // the output read again; the MFMA part is skipped.  The values of the
    // main path are dead here, so this branch adds no registers to it.
#pragma unroll
    for (int u = 0; u < kChunks; ++u) {
      const int q = threadIdx.x + u * kExpandThreads;
      const int tk = q / kRowChunks;
      const int a = cok[u] ? ids[tk] : -1;
      if (a < 0 || a >= n_ad) continue;
      float d[8];
      module_dot<T>(em, &s_y[tk][0], c0 + (q % kRowChunks) * 8, a, d);
      OT* const op = cptr[u];
#pragma unroll 1
      for (int e = 0; e < 8; ++e) op[e] = from_float<OT>(to_float<OT>(op[e]) + d[e]);
    }
    return;
  }

  // the adapter of the lane's y row in each token tile (row tt*16 + lr: the
  // MFMA's A operand), and of its chunks' rows
  const int id_lane = (lane < T_ && id_raw >= 0 && id_raw < n_ad) ? id_raw : -1;
  int idr[kFastTt];
#pragma unroll
  for (int tt = 0; tt < kFastTt; ++tt) idr[tt] = __shfl(id_lane, tt * 16 + lr);
#pragma unroll
  for (int u = 0; u < kChunks; ++u)
    cok[u] = cok[u] & (__shfl(id_lane, ((int)threadIdx.x + u * kExpandThreads) / kRowChunks) >= 0);

  // Per token tile and adapter: the y rows of that adapter's tokens (the
  // others zeroed) times the adapter's B, every adapter accumulated into one
  // MFMA result.  A row gets its own adapter's product plus exact zeros, and
  // a row without an adapter stays zero.  Adapters outermost, so the token
  // tiles' accumulation chains interleave.
  f32x4 acc4[kFastTt];
#pragma unroll
  for (int tt = 0; tt < kFastTt; ++tt) acc4[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nk_w = kw_hi - kw_lo + 1;  // the wave's own tiles (uniform; 0 past the columns)
  uint4 yv[kFastTt][NKT];
#pragma unroll
  for (int tt = 0; tt < kFastTt; ++tt)
#pragma unroll
    for (int k = 0; k < NKT; ++k)
      yv[tt][k] = *reinterpret_cast<const uint4*>(&s_y[tt * 16 + lr][min(kw_lo + k, kFastMaxRank / 32 - 1) * 32 + kq]);
  auto apply_chunk = [&](int a0, const uint4 (&bc)[kFastAChunk][NKT]) {
#pragma unroll
    for (int u = 0; u < kFastAChunk; ++u) {
#pragma unroll
      for (int tt = 0; tt < kFastTt; ++tt) {
        if (tt >= n_tt) break;
        const uint32_t m = 0u - (uint32_t)(idr[tt] == a0 + u);
#pragma unroll
        for (int k = 0; k < NKT; ++k) {
          if (k >= nk_w) break;
          const uint4 ym = make_uint4(yv[tt][k].x & m, yv[tt][k].y & m, yv[tt][k].z & m, yv[tt][k].w & m);
          acc4[tt] = mfma32<T>(ym, bc[u][k], acc4[tt]);
        }
      }
    }
  };
  apply_chunk(0, bop);
  // MANY (more adapters than one chunk, a kernel of its own so the common
  // case keeps its registers): a round trip per further chunk, its B rows in
  // registers of their own
#pragma unroll 1
  for (int a0 = kFastAChunk; MANY && a0 < n_ad; a0 += kFastAChunk) {
    // opaque to the compiler each pass: otherwise it hoists per-(row,
    // adapter) comparisons out of the loop and keeps them all live
#pragma unroll
    for (int tt = 0; tt < kFastTt; ++tt) asm volatile("" : "+v"(idr[tt]));
    asm volatile("" : "+v"(b_off), "+v"(m_out), "+v"(m_rank), "+v"(m_roff), "+v"(m_ooff));
    uint4 bnext[kFastAChunk][NKT];
#pragma unroll
    for (int u = 0; u < kFastAChunk; ++u) load_b(a0 + u, bnext[u]);
    apply_chunk(a0, bnext);
  }
  // the deltas of the wave's columns into LDS, then each thread's chunks
#pragma unroll
  for (int tt = 0; tt < kFastTt; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_d[tt * 16 + (lane / 16) * 4 + i][wave * 16 + lr] = scale * acc4[tt][i];
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kChunks; ++u) {
    const int q = threadIdx.x + u * kExpandThreads;
    if (cok[u]) {
      const float4 d0 = *reinterpret_cast<const float4*>(&s_d[q / kRowChunks][(q % kRowChunks) * 8]);
      const float4 d1 = *reinterpret_cast<const float4*>(&s_d[q / kRowChunks][(q % kRowChunks) * 8 + 4]);
      const float d[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
      OutChunk<OT> r;
      const OT* cv = reinterpret_cast<const OT*>(cur[u].w);
      OT* rv = reinterpret_cast<OT*>(r.w);
#pragma unroll
      for (int e = 0; e < 8; ++e) rv[e] = from_float<OT>(to_float<OT>(cv[e]) + d[e]);
#pragma unroll
      for (int w = 0; w < OutChunk<OT>::kWords; ++w) reinterpret_cast<uint4*>(cptr[u])[w] = r.w[w];
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
  int shrink_x;  // shrink grid x: the most workgroups any group needs (y: groups)
  int expand_x;  // expand grid: every group's workgroups in order
  int expand_waves;
  int nkt;        // the most 32-rank tiles any expand wave's columns use
};

// The most 32-rank tiles the modules of any 16 consecutive output columns
// (one expand wave) use: a wave inside a module uses that module's tiles,
// and only the waves holding a module's first or last column can reach into
// a neighbour.
static int max_wave_tiles(const Group& g) {
  auto span = [&](int c_first, int c_last) {
    int lo = 0, hi = 0;
    for (int m = 0; m < g.n; ++m) {
      const Mod& M = g.m[m];
      if (c_first >= M.out_offset && c_first < M.out_offset + M.out_features) lo = M.rank_offset / 32;
      if (c_last >= M.out_offset && c_last < M.out_offset + M.out_features) hi = (M.rank_offset + M.rank - 1) / 32;
    }
    return hi - lo + 1;
  };
  int best = 1;
  for (int m = 0; m < g.n; ++m) {
    const Mod& M = g.m[m];
    best = std::max(best, span(M.out_offset, M.out_offset + M.out_features - 1));
    for (const int c : {M.out_offset, M.out_offset + M.out_features - 1}) {
      const int w0 = c / 16 * 16;
      best = std::max(best, span(w0, std::min(w0 + 15, g.out_total - 1)));
    }
  }
  return best;
}

static int plan_delta(const pl_lora_group* groups, int n_groups, int tokens, int n_adapters, int dtype,
                      char* ws, DeltaPlan* P) {
  if (n_groups < 1 || n_groups > PL_LORA_MAX_GROUPS)
    return fail(PL_ERR_INVALID, "num_groups must be 1..%d (got %d)", PL_LORA_MAX_GROUPS, n_groups);
  if (groups == nullptr) return fail(PL_ERR_INVALID, "groups is null");
  if (tokens < 0 || tokens > kMaxTokens)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", kMaxTokens, tokens);
  if (n_adapters < 1 || n_adapters > 65535) return fail(PL_ERR_INVALID, "num_adapters must be 1..65535");
  // the decode path: decode sizes, ranks of a multiple of 8, 16-byte aligned
  // B, outputs in 16-byte aligned 8-column chunks (out_features and ldo
  // multiples of 8)
  P->fast = tokens <= kFastMaxTokens && n_adapters <= kFastMaxAdapters;
  for (int i = 0; i < n_groups && groups != nullptr; ++i) {
    P->fast = P->fast && groups[i].in_features <= kFastMaxSlices * kFastKSlice;
    for (int m = 0; m < groups[i].num_modules && groups[i].modules != nullptr; ++m) {
      const pl_lora_module& md = groups[i].modules[m];
      P->fast = P->fast && md.rank % 8 == 0 && (uintptr_t)md.B % 16 == 0 && md.out_features % 8 == 0 &&
                md.ldo % 8 == 0 && (uintptr_t)md.out % 16 == 0;
    }
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
    F.n_expand = (F.g.out_total + 127) / 128;  // at 8 waves; recounted below for 16
    sb = std::max(sb, F.ksplit * F.n_rt);
    F.expand_begin = eb;
    eb += F.n_expand;
    F.parity = (int*)(ws + (size_t)i * sizeof(int));
    F.acc = (long long*)(ws + kParityBytes + (size_t)i * 2 * kAccSlotBytes);
  }
  P->fa.n_groups = n_groups;
  P->fa.tokens = tokens;
  P->fa.n_adapters = n_adapters;
  P->shrink_x = sb;
  P->nkt = 1;
  for (int i = 0; i < n_groups; ++i) P->nkt = std::max(P->nkt, max_wave_tiles(P->g[i]));
  // 16 waves of 1024 threads cap a kernel at 128 registers: waves spanning
  // more than two 32-rank tiles would spill there, and stay at 8
  P->expand_waves = eb > kExpandCUs && P->nkt <= 2 ? 16 : 8;
  if (P->expand_waves == 16) {
    eb = 0;
    for (int i = 0; i < n_groups; ++i) {
      FastGroup& F = P->fa.grp[i];
      F.n_expand = (F.g.out_total + 255) / 256;
      F.expand_begin = eb;
      eb += F.n_expand;
    }
  }
  P->expand_x = eb;
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

template <typename T, int NKT, bool MANY, int EW>
static int launch_expand_fast(const DeltaPlan& P, int out_dtype, hipStream_t stream) {
  const dim3 grid(P.expand_x), block(EW * 64);
  switch (out_dtype) {
    case PL_DTYPE_F32:
      hipLaunchKernelGGL((fast_expand_kernel<T, float, NKT, MANY, EW>), grid, block, 0, stream, P.fa);
      break;
    case PL_DTYPE_F16:
      hipLaunchKernelGGL((fast_expand_kernel<T, f16_t, NKT, MANY, EW>), grid, block, 0, stream, P.fa);
      break;
    case PL_DTYPE_BF16:
      hipLaunchKernelGGL((fast_expand_kernel<T, bf16_t, NKT, MANY, EW>), grid, block, 0, stream, P.fa);
      break;
    default:
      return fail(PL_ERR_UNSUPPORTED, "out_dtype %d", out_dtype);
  }
  PL_LAUNCH_CHECK("lora fast_expand_kernel");
  return PL_OK;
}

template <typename T, int NKT>
static int launch_expand_fast(const DeltaPlan& P, int out_dtype, hipStream_t stream) {
  const bool many = P.fa.n_adapters > kFastAChunk;
  if constexpr (NKT <= 2) {
    if (P.expand_waves == 16)
      return many ? launch_expand_fast<T, NKT, true, 16>(P, out_dtype, stream)
                  : launch_expand_fast<T, NKT, false, 16>(P, out_dtype, stream);
  }
  return many ? launch_expand_fast<T, NKT, true, 8>(P, out_dtype, stream)
              : launch_expand_fast<T, NKT, false, 8>(P, out_dtype, stream);
}

template <typename T>
static int launch_fast(const DeltaPlan& P, int out_dtype, hipStream_t stream) {
  hipLaunchKernelGGL(fast_shrink_kernel<T>, dim3(P.shrink_x, P.fa.n_groups), dim3(kShrinkThreads), 0, stream,
                     P.fa);
  PL_LAUNCH_CHECK("lora fast_shrink_kernel");
  // 3 tiles run as 4: a wave's loop stops at its own last tile
  switch (P.nkt) {
    case 1: return launch_expand_fast<T, 1>(P, out_dtype, stream);
    case 2: return launch_expand_fast<T, 2>(P, out_dtype, stream);
    case 3:
    case 4: return launch_expand_fast<T, 4>(P, out_dtype, stream);
  }
  return fail(PL_ERR_UNSUPPORTED, "r_pad %d", P.nkt * 32);
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
