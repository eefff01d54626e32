// The up-projection half of a no-merge LoRA module as the consuming kernels
// apply it: the device descriptor of pl_lora_up, the rank-space row y of a
// token and the products scale * y . B[a][c]^T, for 8 consecutive output
// columns (lora_delta8, lora_delta8_pair) or one (lora_delta1).  The module
// output is round(base + scale * y . B^T) (multilora/linear.py:226-231).
#pragma once
#include "pl_common.h"

namespace pl {

// Round a float through the storage type T (what a store + reload would give).
template <typename T> __device__ __forceinline__ float through(float v) { return to_float<T>(from_float<T>(v)); }

// Device copy of pl_lora_up: adapter a's y columns are y_offset + a*rank ..
struct LoraUp {
  const void* y;
  int64_t ldy;
  int y_offset;
  const void* B;  // b_chunk8 ? [n_adapters, ceil(out/512), 8, rank/8, 64, 8] : [n_adapters, out, rank]
  int out_features, rank;
  float scale;
  int b_chunk8;
  int adapter;  // >= 0: every token's adapter (no adapter-id load); -1: per-token ids
};

// The 16-byte piece kb (ranks 8kb .. 8kb+7) of B[a][c0 + i] (c0 % 8 == 0 in
// the chunked layout: chunk c0 / 8 is lane l of block j).  The layout flag
// is wave-uniform: the piece is a per-lane base (a select of the two
// layouts' addresses, shared by every piece of the same columns) plus a
// uniform step, so a lane's 8 x R/8 pieces cost one base and a scalar
// offset each.
template <typename T, int R>
__device__ __forceinline__ const T* lora_b_base(const LoraUp& m, int a, int c0) {
  const int64_t rows = ((int64_t)a * m.out_features + c0) * R;
  const int nblk = (m.out_features + 511) / 512, ch = c0 / 8;
  const int64_t chunk = ((((int64_t)a * nblk + (ch >> 6)) * 8 * (R / 8)) * 64 + (ch & 63)) * 8;
  return (const T*)m.B + (m.b_chunk8 ? chunk : rows);
}
template <int R>
__device__ __forceinline__ int lora_b_step(const LoraUp& m, int i, int kb) {
  return m.b_chunk8 ? (i * (R / 8) + kb) * 512 : i * R + kb * 8;
}
template <typename T, int R>
__device__ __forceinline__ const uint4* lora_b_piece(const LoraUp& m, int a, int c0, int i, int kb) {
  return reinterpret_cast<const uint4*>(lora_b_base<T, R>(m, a, c0) + lora_b_step<R>(m, i, kb));
}

// One token's rank-space intermediate y[t, a, :], kept packed (R/8 x 16 B).
template <int R>
struct LoraRow {
  uint4 v[R / 8];
};

// Loads y[t, a, :] (16-byte aligned: y, ldy and y_offset are checked on the host).
template <typename T, int R>
__device__ __forceinline__ void load_y(const LoraUp& m, int64_t t, int a, LoraRow<R>& y) {
  const T* p = (const T*)m.y + t * m.ldy + m.y_offset + (int64_t)a * R;
#pragma unroll
  for (int v = 0; v < R / 8; ++v) y.v[v] = *reinterpret_cast<const uint4*>(p + v * 8);
}

template <typename T>
__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float acc) {
  acc = dot2<T>(a.x, b.x, acc);
  acc = dot2<T>(a.y, b.y, acc);
  acc = dot2<T>(a.z, b.z, acc);
  return dot2<T>(a.w, b.w, acc);
}

// d[i] = scale * y . B[a][c0 + i]^T for 8 consecutive output columns; the
// rows' loads are issued together, 16 ranks at a time.
template <typename T, int R>
__device__ __forceinline__ void lora_delta8(const LoraUp& m, int a, int c0, const LoraRow<R>& y, float (&d)[8]) {
  constexpr int KB = R >= 16 ? 2 : 1;  // 16-byte pieces of a B row per pass
#pragma unroll
  for (int i = 0; i < 8; ++i) d[i] = 0.f;
  // ranks above 16: one 16-rank pass in flight at a time (bounded registers)
  constexpr int kPassUnroll = R <= 16 ? R / 8 : 1;
#pragma unroll kPassUnroll
  for (int kb = 0; kb < R / 8; kb += KB) {
    uint4 b[8][KB];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int k = 0; k < KB; ++k) b[i][k] = *lora_b_piece<T, R>(m, a, c0, i, kb + k);
    // all of the pass's loads in flight before the first dot product (the
    // scheduler otherwise pairs each load with its use to save registers,
    // which turns one round trip into eight)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int k = 0; k < KB; ++k) d[i] = dot8<T>(y.v[kb + k], b[i][k], d[i]);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) d[i] *= m.scale;
}

// The B pieces of 8 consecutive output columns at rank R <= 16, loaded by
// load_cols8 and applied by dot_cols8: lora_delta8 split in two, for callers
// that issue the loads well before the products.
template <int R>
struct LoraCols8 {
  static_assert(R > 0 && R <= 16, "one pass of at most 16 ranks");
  uint4 b[8][R / 8];
};

template <typename T, int R>
__device__ __forceinline__ void load_cols8(const LoraUp& m, int a, int c0, LoraCols8<R>& p) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int k = 0; k < R / 8; ++k) p.b[i][k] = *lora_b_piece<T, R>(m, a, c0, i, k);
}

template <typename T, int R>
__device__ __forceinline__ void dot_cols8(const LoraUp& m, const LoraCols8<R>& p, const LoraRow<R>& y,
                                          float (&d)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < R / 8; ++k) acc = dot8<T>(y.v[k], p.b[i][k], acc);
    d[i] = acc * m.scale;
  }
}

// lora_delta8 for two modules at once (rank <= 16): both modules' B rows in
// flight together, then the dot products.  For consumers that add two
// modules' deltas (SiLU.up): one memory round trip instead of two.
template <typename T, int R>
__device__ __forceinline__ void lora_delta8_pair(const LoraUp& m0, const LoraUp& m1, int a, int c0,
                                                 const LoraRow<R>& y0, const LoraRow<R>& y1, float (&d0)[8],
                                                 float (&d1)[8]) {
  static_assert(R > 0 && R <= 16, "pairs are for ranks up to 16");
  constexpr int KB = R / 8;
  uint4 b0[8][KB], b1[8][KB];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      b0[i][k] = *lora_b_piece<T, R>(m0, a, c0, i, k);
      b1[i][k] = *lora_b_piece<T, R>(m1, a, c0, i, k);
    }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    d0[i] = 0.f;
    d1[i] = 0.f;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      d0[i] = dot8<T>(y0.v[k], b0[i][k], d0[i]);
      d1[i] = dot8<T>(y1.v[k], b1[i][k], d1[i]);
    }
    d0[i] *= m0.scale;
    d1[i] *= m1.scale;
  }
}

// scale * y . B[a][c]^T for one output column.
template <typename T, int R>
__device__ __forceinline__ float lora_delta1(const LoraUp& m, int a, int c, const LoraRow<R>& y) {
  uint4 b[R / 8];
#pragma unroll
  for (int v = 0; v < R / 8; ++v) b[v] = *lora_b_piece<T, R>(m, a, c & ~7, c & 7, v);
  float acc = 0.f;
#pragma unroll
  for (int v = 0; v < R / 8; ++v) acc = dot8<T>(y.v[v], b[v], acc);
  return acc * m.scale;
}

// Host side (defined in fused_ops.hip): the checked device copy of a
// pl_lora_up whose output has at least need_out columns, and the adapter
// binding check of a call's modules (every module binds the same adapter;
// per-token adapters need ids).
int lora_up_checked(const pl_lora_up* h, int need_out, LoraUp* d, const char* what);
int lora_adapters_checked(const pl_lora_up* mods, int n, const int32_t* ids, int n_adapters, const char* what);

}  // namespace pl
