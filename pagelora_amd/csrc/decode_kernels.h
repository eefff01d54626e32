// Device code of the batched paged decode attention for gfx950, shared by
// paged_decode.hip (pages of a multiple of 16 tokens, the plan kernel and the
// C ABI) and paged_decode_small.hip (every other page size), which compile in
// parallel.
#pragma once
#include <type_traits>

#include "pl_common.h"
#include "lora_up.h"

namespace pl {
namespace decode {

constexpr int kWave = 64;
constexpr int kBlockTokens = 16;   // tokens consumed per pipeline step
// Decode waves per workgroup (consecutive kv heads of one item).  Measured
// on the ragged batch-64 MHA fp16 step: 1 -> 0.794 of peak, 2 -> 0.834,
// 4 -> 0.827, 8 -> 0.810; Qwen3 layer 1 x 2048 bf16 (caches evicted):
// 10.8 / 11.2 / 12.9 / 18.3 us.  The kernel with the folded q/k/v epilogue
// keeps 4 (end to end at 1 x 32K tokens: 225.0 tok/s with 4, 222.8 with 2;
// equal with 4 rows).
template <bool FUSED>
constexpr int waves_per_wg() { return FUSED ? 4 : 2; }

struct Item {   // one split-KV work item; lives in the workspace
  int row;      // batch row, -1 = unused slot
  int page_begin;  // absolute index into `indices`
  int page_end;
  int flags;    // bit0: row has a single item (write o directly)
                // bit1: item holds the row's last (possibly partial) page
                // bits 2..: the item's slot (index of its partial output)
};
static_assert(sizeof(Item) == 16, "the decode kernel reads an item as one 16-byte load");

struct Layout {
  size_t header, items, row_info, lse, partial_o, total;
};

inline Layout layout(int batch, int max_items, int hq, int d) {
  Layout L;
  L.header = 0;
  L.items = 256;
  L.row_info = align_up(L.items + (size_t)max_items * sizeof(Item), 256);
  L.lse = align_up(L.row_info + (size_t)batch * 2 * sizeof(int), 256);
  L.partial_o = align_up(L.lse + (size_t)max_items * hq * sizeof(float), 256);
  L.total = align_up(L.partial_o + (size_t)max_items * hq * d * sizeof(float), 256);
  return L;
}

// Stamp written into header[2..3] by the plan and checked by the decode and
// merge kernels, so a run on an unplanned or differently planned workspace
// does no work instead of reading stale item ranges.
__host__ __device__ inline int plan_stamp(int batch, int max_items) {
  return (int)(0x51A70000u ^ ((unsigned)batch * 2654435761u) ^ (unsigned)max_items);
}

// ------------------------------------------------------- direct items ---
// Batches of up to kDirectMaxBatch rows skip the plan kernel: every decode
// wave (and every merge workgroup) derives the split from indptr itself, one
// row per lane: the chunk size as the plan computes it, each row's chunk
// count, their scan, and from it the row and page range of an item (or the
// slot range of a row).  Items and slots are in row order.  Costs one load
// of indptr in place of the item load.
constexpr int kDirectMaxBatch = 16;

struct Direct {
  const int32_t* indptr;  // nullptr: the items come from the plan in the workspace
  int capacity;           // indices capacity: page ranges are clamped to it, as the plan does
  int target_items;
  int min_chunk;
  // Shared prefix (folded q/k/v kernel only): every row's first `shared`
  // page ids are the same pages.  They are split into prefix items of
  // `pchunk` pages, each attended for every row at once (prefix_wave); the
  // rows' own items cover their pages after the prefix.  Row b's partial
  // slots are its prefix chunks, then its own items.  0: no shared prefix.
  int shared;
  int pchunk;
};

struct DirectScan {
  int ip;     // this lane's clamped indptr[lane] (lanes < batch: the rows' starts)
  int ip1;    // and indptr[lane + 1] (the rows' ends)
  int n;      // own chunks of row `lane` (lanes < batch; 0 elsewhere)
  int incl;   // inclusive scan of n over lanes 0..15
  int chunk;  // pages per own chunk (uniform)
  int total;  // items of the batch, prefix items included (uniform)
  int n_pref; // prefix items (uniform; 0 without a shared prefix)
};

// a / b for 0 <= a < 2^23, 1 <= b: float quotient, then one correction step
__device__ __forceinline__ int small_div(int a, int b) {
  int q = (int)((float)a * __builtin_amdgcn_rcpf((float)b));
  const int r = a - q * b;
  q += r >= b ? 1 : 0;
  q -= r < 0 ? 1 : 0;
  return q;
}

__device__ __forceinline__ DirectScan direct_scan(const Direct& d, int batch) {
  const int lane = threadIdx.x % kWave;
  DirectScan r;
  // both ends of row `lane` in one round trip (batch <= 16, so lanes 0..15
  // cover every row)
  auto clampi = [&](int v) { return v < 0 ? 0 : (v > d.capacity ? d.capacity : v); };
  const int ip = clampi(d.indptr[lane < batch ? lane : batch]);
  const int ip1 = clampi(d.indptr[lane < batch ? lane + 1 : batch]);
  r.ip = ip;
  r.ip1 = ip1;
  const int ip0 = __builtin_amdgcn_readfirstlane(ip);
  const int ipb = __builtin_amdgcn_readlane(ip1, batch - 1);
  // the rows' own pages: past the shared prefix (every row holds more than it)
  const int sh = d.shared;
  const int total_pages = (ipb > ip0 ? ipb - ip0 : 0) - sh * batch;
  int c = (total_pages + d.target_items - 1) / d.target_items;  // uniform
  c = c > d.min_chunk ? c : d.min_chunk;
  r.chunk = c > 1 ? c : 1;
  const int pages = ip1 > ip + sh ? ip1 - ip - sh : 0;
  r.n = lane < batch ? (pages > 0 ? small_div(pages + r.chunk - 1, r.chunk) : 1) : 0;
  r.n_pref = sh > 0 ? (sh + d.pchunk - 1) / d.pchunk : 0;
  // inclusive scan over the 16 lanes of DPP row 0 (row_shr shifts in zeros)
  int x = r.n;
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  r.incl = x;
  r.total = __builtin_amdgcn_readlane(x, 15) + r.n_pref;
  return r;
}

// Row, page range and flags (single-slot row, holds the last page, slot) of
// own item `item` (items are numbered from the n_pref prefix items on);
// false past the batch's items.  Every lane of the wave calls it.
__device__ __forceinline__ bool direct_item_of(const DirectScan& s, const Direct& d, int item, int& b, int& pbeg,
                                               int& pend, int& flags) {
  if (item >= s.total) return false;
  const int lane = threadIdx.x % kWave;
  const int own = item - s.n_pref;
  b = __builtin_amdgcn_readfirstlane(__popcll(__builtin_amdgcn_ballot_w64((lane < 16) & (s.incl <= own))));
  const int n_b = __builtin_amdgcn_readlane(s.n, b);
  const int first = __builtin_amdgcn_readlane(s.incl, b) - n_b;
  const int row_beg = __builtin_amdgcn_readlane(s.ip, b) + d.shared;
  const int row_end = __builtin_amdgcn_readlane(s.ip1, b);
  pbeg = row_beg + (own - first) * s.chunk;
  pend = min(row_end > row_beg ? row_end : row_beg, pbeg + s.chunk);
  // row b's slots follow the earlier rows' (n_pref + own items each), its
  // prefix chunks first
  const int slot = (b + 1) * s.n_pref + own;
  flags = (slot << 2) | (s.n_pref + n_b == 1 ? 1 : 0) | (pend >= row_end ? 2 : 0);
  return true;
}

__device__ __forceinline__ bool direct_item(const Direct& d, int batch, int item, int& b, int& pbeg, int& pend,
                                            int& flags) {
  return direct_item_of(direct_scan(d, batch), d, item, b, pbeg, pend, flags);
}

// First slot and item count of row b.  Every lane of the wave calls it.
__device__ __forceinline__ void direct_row(const Direct& d, int batch, int b, int& first, int& n) {
  const DirectScan s = direct_scan(d, batch);
  const int n_own = __builtin_amdgcn_readlane(s.n, b);
  first = b * s.n_pref + __builtin_amdgcn_readlane(s.incl, b) - n_own;
  n = s.n_pref + n_own;
}

// ---------------------------------------------------------------- decode ---
// Per-type traits: how one lane's 8 elements of a token row are loaded and
// consumed.  16-bit types: one 16-byte load; fp32: two.
template <typename T> struct Lane8;

template <> struct Lane8<float> {
  static constexpr int kWords = 8;
  __device__ static void load(uint32_t (&w)[8], const float* p) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  }
  __device__ static float dot(const uint32_t (&q)[8], const uint32_t (&k)[8]) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = fmaf(__uint_as_float(q[i]), __uint_as_float(k[i]), acc);
    return acc;
  }
  __device__ static void to_f32(const uint32_t (&w)[8], float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = __uint_as_float(w[i]);
  }
  __device__ static void store(float* p, const float (&f)[8]) {
    *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(f[4], f[5], f[6], f[7]);
  }
};

// K/V rows are read exactly once per call: non-temporal loads keep them from
// displacing reusable lines in the L2 / infinity cache.
#ifndef PL_DECODE_NT_LOADS
#define PL_DECODE_NT_LOADS 1
#endif
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Lane8Half {
  static constexpr int kWords = 4;
  __device__ static void load(uint32_t (&w)[4], const T* p) {
#if PL_DECODE_NT_LOADS
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
#else
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
#endif
  }
  __device__ static float dot(const uint32_t (&q)[4], const uint32_t (&k)[4]) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = dot2<T>(q[i], k[i], acc);
    return acc;
  }
  __device__ static void to_f32(const uint32_t (&w)[4], float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) unpack2<T>(w[i], f[2 * i], f[2 * i + 1]);
  }
  __device__ static void store(T* p, const float (&f)[8]) {
    uint4 a;
    a.x = pack2<T>(f[0], f[1]);
    a.y = pack2<T>(f[2], f[3]);
    a.z = pack2<T>(f[4], f[5]);
    a.w = pack2<T>(f[6], f[7]);
    *reinterpret_cast<uint4*>(p) = a;
  }
};
template <> struct Lane8<f16_t> : Lane8Half<f16_t> {};
template <> struct Lane8<bf16_t> : Lane8Half<bf16_t> {};

// Sum across the LPT lanes that share one token row.
template <int LPT> __device__ __forceinline__ float row_sum(float x);
template <> __device__ __forceinline__ float row_sum<8>(float x) { return row8_sum(x); }
template <> __device__ __forceinline__ float row_sum<16>(float x) { return row16_sum(x); }
template <> __device__ __forceinline__ float row_sum<32>(float x) { return row32_sum(x); }

// Fold the lane rows of a wave's online-softmax states together (xor over
// the row bits of the lane id, LPT lanes per row); afterwards every lane
// holds the combined state for its 8 dims.
template <int G, int LPT>
__device__ __forceinline__ void merge_lane_rows(float (&m)[G], float (&l)[G], float (&acc)[G][8]) {
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int off = LPT; off < kWave; off <<= 1) {
      const float m_o = __shfl_xor(m[g], off);
      const float l_o = __shfl_xor(l[g], off);
      const float m_new = fmaxf(m[g], m_o);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float a_s = fast_exp2(m[g] - m_use);
      const float a_o = fast_exp2(m_o - m_use);
      l[g] = l[g] * a_s + l_o * a_o;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float o_o = __shfl_xor(acc[g][i], off);
        acc[g][i] = acc[g][i] * a_s + o_o * a_o;
      }
      m[g] = m_new;
    }
  }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// D += A . B on a 16x16x32 MFMA tile, A and B as 4 packed words per lane.
template <typename T>
__device__ __forceinline__ f32x4 mfma_16x16x32(const uint32_t (&a)[4], const uint32_t (&b)[4], f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma_16x16x32<bf16_t>(const uint32_t (&a)[4], const uint32_t (&b)[4], f32x4 c) {
  const u32x4 av = {a[0], a[1], a[2], a[3]}, bv = {b[0], b[1], b[2], b[3]};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), __builtin_bit_cast(bf16x8_t, bv),
                                                 c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_16x16x32<f16_t>(const uint32_t (&a)[4], const uint32_t (&b)[4], f32x4 c) {
  const u32x4 av = {a[0], a[1], a[2], a[3]}, bv = {b[0], b[1], b[2], b[3]};
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, av), __builtin_bit_cast(f16x8_t, bv), c,
                                                0, 0, 0);
}

template <typename T, int D, int G>
struct DecodeWave {
  static constexpr int LPT = D / 8;             // lanes per token row
  static constexpr int TPI = kWave / LPT;       // token rows per load instruction
  static constexpr int NS = kBlockTokens / TPI; // loads per lane per block
  static constexpr int W = Lane8<T>::kWords;
  static constexpr bool kMfmaScores = false;
  using L8 = Lane8<T>;

  uint32_t q[G][W];   // this lane's 8 dims of the g query heads
  float m[G], l[G];   // online-softmax state of this lane row (log2 domain)
  float acc[G][8];    // unnormalised output, this lane's 8 dims

  __device__ void init() {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = -INFINITY;
      l[g] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
    }
  }

  // Consume one block of 16 tokens already in registers.  `valid` = number
  // of tokens of the block that exist (16 for all blocks but the last).
  template <bool MASK>
  __device__ __forceinline__ void consume(const uint32_t (&kw)[NS][W], const uint32_t (&vw)[NS][W],
                                          float scale_log2, int row, int valid) {
    float sc[NS][G];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = L8::dot(q[g], kw[s]);
        d = row_sum<LPT>(d) * scale_log2;
        if (MASK) d = (row + s * TPI < valid) ? d : -INFINITY;
        sc[s][g] = d;
      }
    }
    float vf[NS][8];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      L8::to_f32(vw[s], vf[s]);
      if (MASK) {
        const bool ok = row + s * TPI < valid;
#pragma unroll
        for (int i = 0; i < 8; ++i) vf[s][i] = ok ? vf[s][i] : 0.f;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = sc[0][g];
#pragma unroll
      for (int s = 1; s < NS; ++s) mx = fmaxf(mx, sc[s][g]);
      const float m_new = fmaxf(m[g], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;  // all masked so far
      const float alpha = fast_exp2(m[g] - m_use);
      m[g] = m_new;
      float psum = 0.f;
      float p[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        p[s] = fast_exp2(sc[s][g] - m_use);
        psum += p[s];
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float a = acc[g][i] * alpha;
#pragma unroll
        for (int s = 0; s < NS; ++s) a = fmaf(p[s], vf[s][i], a);
        acc[g][i] = a;
      }
    }
  }

  // Fold the TPI lane rows together (xor over the row bits of the lane id).
  // Afterwards every lane holds the wave's combined state for its 8 dims.
  __device__ __forceinline__ void merge_rows() { merge_lane_rows<G, LPT>(m, l, acc); }
};

// The score-on-MFMA wave for GQA groups of 4 heads, head_dim 128, 16-bit
// types: per block of 16 tokens, S^T = K . Q^T is four
// v_mfma_f32_16x16x32 (A: the block's K, lane l holding 8 dims of token
// perm(l % 16); B: q, the group's 4 heads repeated over the 16 columns), in
// place of 64 dot2 and 64 DPP reductions.  The token permutation
// perm(m) = m / 4 + 4 * (m % 4) puts the scores of lane l's output rows
// 4*(l/16) + i on tokens l/16 + 4i: the tokens whose V rows the lane already
// holds in the VALU layout (row l/16, load s = i).  Lane l's scores are those
// of head l % 4; each lane runs the online softmax of that head for its lane
// row, and the quad's lanes (l & ~3 .. l | 3: heads 0..3 of the same tokens)
// exchange p and the rescale factors with quad-permute DPP, so P . V stays
// on VALU in registers as in DecodeWave.
template <typename T, int D, int G>
struct DecodeWaveMfma {
  static_assert(D == 128 && G == 4 && sizeof(T) == 2, "MFMA scores: GQA 4, head_dim 128, 16-bit");
  static constexpr int LPT = D / 8;             // V: lanes per token row
  static constexpr int TPI = kWave / LPT;       // V: token rows per load instruction
  static constexpr int NS = kBlockTokens / TPI; // loads per lane per block (K: one per 32 dims)
  static constexpr int W = 4;
  static constexpr bool kMfmaScores = true;
  using L8 = Lane8<T>;

  uint32_t qb[NS][W];  // B operand: head lane % 4, dims 32 j + 8 (lane / 16) ..
  float mo, lo;        // online-softmax state of head lane % 4, lane row lane / 16 (log2)
  float m[G], l[G];    // merge_rows: the state of every head
  float acc[G][8];     // unnormalised output, this lane's 8 dims (8 * (lane % 16))

  __device__ void init() {
    mo = -INFINITY;
    lo = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  }

  // Element offset of lane `lane`'s K piece for load j = 0 within a block:
  // token perm(lane % 16), dims 8 * (lane / 16); load j adds 32 dims.
  __device__ static int64_t k_lane_off(int lane, int64_t token_stride) {
    const int m16 = lane % 16;
    return (int64_t)(m16 / 4 + 4 * (m16 % 4)) * token_stride + 8 * (lane / 16);
  }
  // Lane of the block that holds token t's K (its 4 loads hold dims 32 j +
  // 8 * (lane / 16)): the lanes l with l % 16 == perm^-1(t).
  __device__ static int k_lane_of(int t) { return 4 * (t % 4) + t / 4; }

  template <int CTRL>
  __device__ static float quad_bcast(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
  }

  template <bool MASK>
  __device__ __forceinline__ void consume(const uint32_t (&kw)[NS][W], const uint32_t (&vw)[NS][W],
                                          float scale_log2, int row, int valid) {
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NS; ++j) sacc = mfma_16x16x32<T>(kw[j], qb[j], sacc);
    float sc[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      sc[i] = sacc[i] * scale_log2;
      if (MASK) sc[i] = (row + i * TPI < valid) ? sc[i] : -INFINITY;
    }
    float vf[NS][8];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      L8::to_f32(vw[s], vf[s]);
      if (MASK) {
        const bool ok = row + s * TPI < valid;
#pragma unroll
        for (int i = 0; i < 8; ++i) vf[s][i] = ok ? vf[s][i] : 0.f;
      }
    }
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < NS; ++i) mx = fmaxf(mx, sc[i]);
    const float m_new = fmaxf(mo, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;  // all masked so far
    const float alpha = fast_exp2(mo - m_use);
    mo = m_new;
    float p[NS], psum = 0.f;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      p[i] = fast_exp2(sc[i] - m_use);
      psum += p[i];
    }
    lo = lo * alpha + psum;
    // quad_perm:[g,g,g,g]: lane 4k + g of the quad holds head g
    float ag[G], pg[NS][G];
    ag[0] = quad_bcast<0x00>(alpha);
    ag[1] = quad_bcast<0x55>(alpha);
    ag[2] = quad_bcast<0xAA>(alpha);
    ag[3] = quad_bcast<0xFF>(alpha);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      pg[i][0] = quad_bcast<0x00>(p[i]);
      pg[i][1] = quad_bcast<0x55>(p[i]);
      pg[i][2] = quad_bcast<0xAA>(p[i]);
      pg[i][3] = quad_bcast<0xFF>(p[i]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        float a = acc[g][d] * ag[g];
#pragma unroll
        for (int i = 0; i < NS; ++i) a = fmaf(pg[i][g], vf[i][d], a);
        acc[g][d] = a;
      }
  }

  __device__ __forceinline__ void merge_rows() {
    m[0] = quad_bcast<0x00>(mo);
    m[1] = quad_bcast<0x55>(mo);
    m[2] = quad_bcast<0xAA>(mo);
    m[3] = quad_bcast<0xFF>(mo);
    l[0] = quad_bcast<0x00>(lo);
    l[1] = quad_bcast<0x55>(lo);
    l[2] = quad_bcast<0xAA>(lo);
    l[3] = quad_bcast<0xFF>(lo);
    merge_lane_rows<G, LPT>(m, l, acc);
  }
};

template <typename T, int D, int G>
using WaveFor = std::conditional_t<D == 128 && G == 4 && sizeof(T) == 2, DecodeWaveMfma<T, D, G>, DecodeWave<T, D, G>>;

// Stream blocks [blk0, blk1) of an item (16 tokens each, the item's first
// `ntok` tokens are real) through one wave's online-softmax state: each
// block's K and V rows are loaded one block ahead of their use (two blocks
// in flight per wave).
// Where a lane's K and V pieces of a block lie: element offsets from the
// block's first token row, and the step between the lane's loads.
struct KvLanes {
  int64_t k_off, k_step, v_off, v_step;
};

template <typename T, class WaveT>
__device__ __forceinline__ void stream_blocks(WaveT& st, const T* __restrict__ kc, const T* __restrict__ vc,
                                              int64_t page_stride, int64_t token_stride, const KvLanes& ln,
                                              const int32_t* __restrict__ indices, int pbeg, int page_size,
                                              int64_t num_pages, int ntok, int blk0, int blk1, float scale_log2,
                                              int row, int first_page, int second_page) {
  constexpr int NS = WaveT::NS, W = WaveT::W;
  using L8 = Lane8<T>;
  // first_page / second_page: the page ids of blocks blk0 and blk0 + 1
  // (clamped to the item, as page_of does), read by the caller in an earlier
  // round trip, so the loop's first loads wait on no scalar load
  const int last_page = (int)min(num_pages, (int64_t)INT32_MAX) - 1;  // 32-bit: scalar compares
  auto load_at = [&](int blk, int page, uint32_t (&kw)[NS][W], uint32_t (&vw)[NS][W]) {
    const int t0 = blk * kBlockTokens;
    const int tip = t0 - (t0 / page_size) * page_size;
    page = page < 0 ? 0 : min(page, last_page);  // stay inside the pool
    const int64_t base = (int64_t)page * page_stride + (int64_t)tip * token_stride;
    const T* kp = kc + base + ln.k_off;
    const T* vp = vc + base + ln.v_off;
#pragma unroll
    for (int s = 0; s < NS; ++s) L8::load(kw[s], kp + s * ln.k_step);
#pragma unroll
    for (int s = 0; s < NS; ++s) L8::load(vw[s], vp + s * ln.v_step);
  };
  // page id of block blk (blocks past the last re-read the last one)
  auto page_of = [&](int blk) -> int { return uniform(indices[pbeg + min(blk, blk1 - 1) * kBlockTokens / page_size]); };
  if (blk1 <= blk0) return;
  uint32_t ka[NS][W], va[NS][W], kb[NS][W], vb[NS][W];
  load_at(blk0, first_page, ka, va);
  // Page ids run one block ahead of the K/V loads: the id a block's loads
  // need was read an iteration earlier, so no scalar load stands between a
  // wave and its next K/V loads.  (Measured against reading the id in front
  // of the loads: headline 746.5 -> 743 us, 64 x 2K GQA-4 114.2 -> 113.2 us;
  // entering the loop with both buffers in flight instead was 1-10% slower.)
  int pid_next = second_page;
  auto consume = [&](int blk, uint32_t (&kw)[NS][W], uint32_t (&vw)[NS][W]) {
    if ((blk + 1) * kBlockTokens <= ntok)
      st.template consume<false>(kw, vw, scale_log2, row, kBlockTokens);
    else
      st.template consume<true>(kw, vw, scale_log2, row, ntok - blk * kBlockTokens);
  };
  // Pairs of blocks, then the odd last one.  The loop has one exit: a break
  // between the halves gives the compiler a path from the first half's
  // loads back to the loop head, where it then waits for every load in
  // flight before reusing their registers (one block in flight, not two).
  int i = blk0;
  for (; i + 1 < blk1; i += 2) {
    // Prefetch the next block before consuming this one.  The second load's
    // index is clamped instead of branched on so the load count is the same
    // on every path (a re-load of the last block hits in cache).
    const int p1 = pid_next;
    pid_next = page_of(i + 2);
    load_at(i + 1, p1, kb, vb);
    // keep the scheduler from pulling the consume (and its waits on this
    // block's data) above the prefetch
    __builtin_amdgcn_sched_barrier(0);
    consume(i, ka, va);
    const int p2 = pid_next;
    pid_next = page_of(i + 3);
    load_at(min(i + 2, blk1 - 1), p2, ka, va);
    __builtin_amdgcn_sched_barrier(0);
    consume(i + 1, kb, vb);
  }
  if (i < blk1) consume(i, ka, va);
}

// stream_blocks for pages whose size is not a multiple of 16 tokens (1, 2,
// 4, 8, 3, 24, ...): a 16-token block then spans several pages, so every
// lane looks up the page of each token row it loads.  The page ids of block
// i + 2 are loaded (vector loads, one per token row the lane holds) before
// the K/V loads of block i + 1 are issued, so a K/V load waits only on ids
// fetched a whole block earlier.  Tokens past the item's last are clamped to
// it (their scores are masked in consume).
// v_fix / k_fix: the lane's element offset inside a token row (kv head and
// dims); k_tok >= 0: the token of the block whose K the lane loads for every
// load (MFMA-score waves, K dims 32 apart), else K follows the V rows.
template <int NS, int NK>
struct SmallBlockIds {
  int vpg[NS], vtip[NS];  // page id and row in page of the lane's V token rows
  int kpg[NK], ktip[NK];  // the same for its K token (MFMA-score waves)
};

template <typename T, class WaveT>
__device__ __forceinline__ void stream_blocks_small(WaveT& st, const T* __restrict__ kc, const T* __restrict__ vc,
                                                    int64_t page_stride, int64_t token_stride, int64_t k_fix,
                                                    int64_t v_fix, int k_tok, const int32_t* __restrict__ indices,
                                                    int pbeg, int page_size, int64_t num_pages, int ntok, int nblk,
                                                    float scale_log2, int row) {
  constexpr int NS = WaveT::NS, W = WaveT::W, TPI = WaveT::TPI;
  constexpr bool KM = WaveT::kMfmaScores;
  using L8 = Lane8<T>;
  using Ids = SmallBlockIds<NS, 1>;  // one K token per lane on MFMA waves (unused otherwise)
  if (nblk <= 0) return;
  const float inv_ps = 1.f / (float)page_size;
  // token t of the item -> (page slot, row in page); t < 2^23, so the float
  // quotient is off by at most one and one correction step makes it exact
  auto split = [&](int t, int& slot, int& tip) {
    int q = (int)((float)t * inv_ps);
    int r = t - q * page_size;
    if (r < 0) { --q; r += page_size; }
    else if (r >= page_size) { ++q; r -= page_size; }
    slot = q;
    tip = r;
  };
  auto fetch_ids = [&](int blk, Ids& w) {
    const int t0 = blk * kBlockTokens;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      int slot, tip;
      split(min(t0 + row + s * TPI, ntok - 1), slot, tip);
      w.vpg[s] = indices[pbeg + slot];
      w.vtip[s] = tip;
    }
    if constexpr (KM) {
      int slot, tip;
      split(min(t0 + k_tok, ntok - 1), slot, tip);
      w.kpg[0] = indices[pbeg + slot];
      w.ktip[0] = tip;
    }
  };
  auto addr = [&](int pg, int tip) -> int64_t {
    const int64_t p = pg < 0 ? 0 : (pg >= num_pages ? num_pages - 1 : pg);  // stay inside the pool
    return p * page_stride + (int64_t)tip * token_stride;
  };
  auto load_at = [&](const Ids& w, uint32_t (&kw)[NS][W], uint32_t (&vw)[NS][W]) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if constexpr (KM) L8::load(kw[s], kc + addr(w.kpg[0], w.ktip[0]) + k_fix + 32 * s);
      else L8::load(kw[s], kc + addr(w.vpg[s], w.vtip[s]) + k_fix);
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) L8::load(vw[s], vc + addr(w.vpg[s], w.vtip[s]) + v_fix);
  };
  uint32_t ka[NS][W], va[NS][W], kb[NS][W], vb[NS][W];
  Ids wa, wb;
  fetch_ids(0, wa);
  fetch_ids(min(1, nblk - 1), wb);
  load_at(wa, ka, va);
  auto consume = [&](int blk, uint32_t (&kw)[NS][W], uint32_t (&vw)[NS][W]) {
    if ((blk + 1) * kBlockTokens <= ntok)
      st.template consume<false>(kw, vw, scale_log2, row, kBlockTokens);
    else
      st.template consume<true>(kw, vw, scale_log2, row, ntok - blk * kBlockTokens);
  };
  // pairs of blocks, then the odd last one: one loop exit, as in stream_blocks
  int i = 0;
  for (; i + 1 < nblk; i += 2) {
    fetch_ids(min(i + 2, nblk - 1), wa);  // block i's loads are issued: wa is free
    load_at(wb, kb, vb);                  // block i + 1
    __builtin_amdgcn_sched_barrier(0);
    consume(i, ka, va);
    fetch_ids(min(i + 3, nblk - 1), wb);
    load_at(wa, ka, va);  // block i + 2 (a re-load of the last block past the end)
    __builtin_amdgcn_sched_barrier(0);
    consume(i + 1, kb, vb);
  }
  if (i < nblk) consume(i, ka, va);
}

// The new token's K and V of a wave's kv head, as registers to splice into
// the block that holds it (blk: block index, s: load instruction, row: lane
// row; k / v: this lane's 8 dims, valid in the lanes of that row).
struct NewToken {
  int blk, pg, s, row;  // blk < 0: none; pg: the page the block must come from
  uint32_t k[4], v[4];
  int klane;            // MFMA-score waves: K sits in the lanes l % 16 == klane,
  uint32_t kq[4][4];    // load j holding dims 32 j + 8 (l / 16) ..
};

// stream_blocks for the folded q/k/v epilogue: `pre` issues loads ahead of
// the first block's, and `hook` runs once the first block's loads are in
// flight (it forms q, and for the item holding the
// row's last page the new token's k / v, filling `nt`), and the new token's
// K/V rows are taken from `nt` rather than from memory, so no load waits on
// the append's stores.
template <typename T, class WaveT, class Pre, class Hook>
__device__ __forceinline__ void stream_blocks_fused(WaveT& st, const T* __restrict__ kc, const T* __restrict__ vc,
                                                    int64_t page_stride, int64_t token_stride, const KvLanes& ln,
                                                    const int32_t* __restrict__ indices, int pbeg, int page_size,
                                                    int64_t num_pages, int ntok, int blk0, int blk1,
                                                    float scale_log2, int row, int first_page, int second_page,
                                                    Pre&& pre, Hook&& hook, const NewToken& nt) {
  constexpr int NS = WaveT::NS, W = WaveT::W;
  static_assert(W == 4, "16-bit types: 4 words per lane per token");
  using L8 = Lane8<T>;
  const int last_page = (int)min(num_pages, (int64_t)INT32_MAX) - 1;  // 32-bit: scalar compares
  auto load_at = [&](int blk, int page, uint32_t (&kw)[NS][W], uint32_t (&vw)[NS][W]) {
    const int t0 = blk * kBlockTokens;
    const int tip = t0 - (t0 / page_size) * page_size;
    page = page < 0 ? 0 : min(page, last_page);  // stay inside the pool
    const int64_t base = (int64_t)page * page_stride + (int64_t)tip * token_stride;
    const T* kp = kc + base + ln.k_off;
    const T* vp = vc + base + ln.v_off;
#pragma unroll
    for (int s = 0; s < NS; ++s) L8::load(kw[s], kp + s * ln.k_step);
#pragma unroll
    for (int s = 0; s < NS; ++s) L8::load(vw[s], vp + s * ln.v_step);
  };
  auto page_of = [&](int blk) -> int { return uniform(indices[pbeg + min(blk, blk1 - 1) * kBlockTokens / page_size]); };
  const int lane16 = threadIdx.x % 16;
  auto splice = [&](int blk, int page, uint32_t (&kw)[NS][W], uint32_t (&vw)[NS][W]) {
    if ((blk != nt.blk) | (page != nt.pg)) return;  // wave-uniform
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
      for (int w = 0; w < W; ++w) {
        if constexpr (WaveT::kMfmaScores)
          kw[s][w] = lane16 == nt.klane ? nt.kq[s][w] : kw[s][w];
        else
          kw[s][w] = ((s == nt.s) & (row == nt.row)) ? nt.k[w] : kw[s][w];
        vw[s][w] = ((s == nt.s) & (row == nt.row)) ? nt.v[w] : vw[s][w];
      }
    }
  };
  pre();
  if (blk1 <= blk0) {
    hook();
    return;
  }
  uint32_t ka[NS][W], va[NS][W], kb[NS][W], vb[NS][W];
  int pa = first_page, pb;
  load_at(blk0, pa, ka, va);
  int pid_next = second_page;
  hook();
  auto consume = [&](int blk, int page, uint32_t (&kw)[NS][W], uint32_t (&vw)[NS][W]) {
    splice(blk, page, kw, vw);
    if ((blk + 1) * kBlockTokens <= ntok)
      st.template consume<false>(kw, vw, scale_log2, row, kBlockTokens);
    else
      st.template consume<true>(kw, vw, scale_log2, row, ntok - blk * kBlockTokens);
  };
  // pairs of blocks, then the odd last one: one loop exit, as in stream_blocks
  int i = blk0;
  for (; i + 1 < blk1; i += 2) {
    pb = pid_next;
    pid_next = page_of(i + 2);
    load_at(i + 1, pb, kb, vb);
    __builtin_amdgcn_sched_barrier(0);
    consume(i, pa, ka, va);
    pa = pid_next;
    pid_next = page_of(i + 3);
    load_at(min(i + 2, blk1 - 1), pa, ka, va);
    __builtin_amdgcn_sched_barrier(0);
    consume(i + 1, pb, kb, vb);
  }
  if (i < blk1) consume(i, pa, ka, va);
}

// Inputs of the decode run with the q/k/v epilogue folded in
// (pl_decode_run_qkv): the packed projection rows instead of a finished q.
struct QkvIn {
  const void* qkv;           // [batch, ld]: q heads | k heads | v heads, head-major, D each
  int64_t ld;
  const void* q_norm_w;      // [D] or null
  const void* k_norm_w;      // [D] or null
  const float* rope;         // [batch, D/2, 2]: cos, sin of the row's position * inv_freq[i]
  const int64_t* page_id;    // the row's new token: its page and slot in the page
  const int64_t* page_off;
  float eps;
  LoraUp m[3];               // q, k, v up-projections (rank R > 0)
  const int32_t* ids;
  int n_adapters;
  int no_direct;             // 1: single-item rows publish a partial too (the merge writes them)
};

// One lane's 8 dims (8*col ..) of head `hh` of packed projection row b: the
// module output (base + LoRA delta, rounded through T), the head RMSNorm
// with weights w (none: w == nullptr) and the rotate-half RoPE (rot) -- the
// arithmetic of qk_norm_rope_append_kernel, with the sum of squares reduced
// over the lane's 16-lane row group and the rotation partner (the other half
// of the head) taken from lane col ^ 8 of the group.  In three phases, so the
// caller can issue each group of loads as soon as its addresses are known:
// head_base_load (the packed row, the norm weights, the step's cos / sin:
// needs only b), head_lora_load (y and the B pieces: needs the adapter) and
// head_finish.  Every load is issued unconditionally and optional terms are
// blended in, so none waits behind a test.
template <typename T, int R>
struct HeadIn {
  uint4 raw, wr;
  float4 r[4];  // (cos, sin) of pairs 8 * (col % 8) ..
  LoraRow<(R > 0 ? R : 8)> y;
  LoraCols8<(R > 0 ? R : 8)> bp;
};

template <typename T, int R>
__device__ __forceinline__ void head_base_load(const QkvIn& in, int b, int hh, int col, const T* w,
                                               HeadIn<T, R>& x) {
  constexpr int D = 128;
  const T* src = (const T*)in.qkv + (int64_t)b * in.ld + (int64_t)hh * D + col * 8;
  x.raw = *reinterpret_cast<const uint4*>(src);
  x.wr = *reinterpret_cast<const uint4*>(w != nullptr ? w + col * 8 : src);
  const float4* rp = reinterpret_cast<const float4*>(in.rope + ((int64_t)b * (D / 2) + (col * 8) % (D / 2)) * 2);
#pragma unroll
  for (int i = 0; i < 4; ++i) x.r[i] = rp[i];
}

template <typename T, int R>
__device__ __forceinline__ void head_lora_load(const QkvIn& in, int b, int mod, int mcol, int col, int a_ld,
                                               HeadIn<T, R>& x) {
  if constexpr (R > 0) {
    load_y<T, R>(in.m[mod], b, a_ld, x.y);
    load_cols8<T, R>(in.m[mod], a_ld, mcol + col * 8, x.bp);
  }
}

template <typename T, int R>
__device__ __forceinline__ void head_finish(const QkvIn& in, const HeadIn<T, R>& x, int mod, int col, bool has_w,
                                            bool rot, bool a_ok, float (&v)[8]) {
  constexpr int D = 128;
  unpack2<T>(x.raw.x, v[0], v[1]);
  unpack2<T>(x.raw.y, v[2], v[3]);
  unpack2<T>(x.raw.z, v[4], v[5]);
  unpack2<T>(x.raw.w, v[6], v[7]);
  if constexpr (R > 0) {
    float d[8];
    dot_cols8<T, R>(in.m[mod], x.bp, x.y, d);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = through<T>(v[e] + (a_ok ? d[e] : -0.f));
  }
  const uint32_t keep = has_w ? 0xffffffffu : 0u;
  float wf[8];
  unpack2<T>(x.wr.x, wf[0], wf[1]);
  unpack2<T>(x.wr.y, wf[2], wf[3]);
  unpack2<T>(x.wr.z, wf[4], wf[5]);
  unpack2<T>(x.wr.w, wf[6], wf[7]);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    wf[e] = __uint_as_float((__float_as_uint(wf[e]) & keep) | (0x3f800000u & ~keep));
    ss += v[e] * v[e];
  }
  ss = row16_sum(ss);
  const float rstd = has_w ? rsqrtf(ss / (float)D + in.eps) : 1.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] *= rstd * wf[e];
  const float cs[8] = {x.r[0].x, x.r[0].z, x.r[1].x, x.r[1].z, x.r[2].x, x.r[2].z, x.r[3].x, x.r[3].z};
  const float sn[8] = {x.r[0].y, x.r[0].w, x.r[1].y, x.r[1].w, x.r[2].y, x.r[2].w, x.r[3].y, x.r[3].w};
  const uint32_t rk = rot ? 0xffffffffu : 0u;
  const bool lo_half = col < 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float pe = dpp_mov<0x128>(v[e]);  // row_ror:8: lane col ^ 8 of the row group
    const float r = lo_half ? v[e] * cs[e] - pe * sn[e] : v[e] * cs[e] + pe * sn[e];
    v[e] = __uint_as_float((__float_as_uint(r) & rk) | (__float_as_uint(v[e]) & ~rk));
  }
}

// ------------------------------------------------------ shared prefix ---
// A prefix item: kPrefixTokens tokens of the pages every row shares, for one
// kv head h and every row of the batch at once (batch <= 4): the 16 MFMA
// columns are (row n / 4, query head 4h + n % 4).  The wave forms those
// rows' q as the folded epilogue does (one bound adapter), scores
// S^T = K . Q^T (a lane holds tokens 4*(l/16) + i of each 16-token block,
// column l % 16), runs the fp32 online softmax per column (its four lanes
// exchange max and sum), and forms O^T = V^T . P^T on MFMA: V is staged in
// LDS row-major and read as pairs of head dims (tile 2a: dims 32a + 2r,
// tile 2a+1: dims 32a + 2r + 1, r = l % 16) with byte permutes, P is split
// into a hi and a lo part of the 16-bit type (about 16 mantissa bits).  The
// normalised partial and its log2-sum-exp go to slot first_b + j of each
// row b, where the merge finds them with the row's own items.
constexpr int kPrefixTokens = 32;   // tokens per prefix item: one P.V step of 16x16x32 MFMAs
constexpr int kPrefixMaxRows = 4;   // 16 columns / GQA 4

template <typename T> __device__ __forceinline__ uint32_t pack_pv(float a, float b);
template <> __device__ __forceinline__ uint32_t pack_pv<bf16_t>(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
template <> __device__ __forceinline__ uint32_t pack_pv<f16_t>(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, half2_t));
}

template <typename T, int R>
__device__ __forceinline__ void prefix_wave(const DirectScan& sc, const Direct& dir, int batch, int j, int h,
                                            const T* __restrict__ kc, const T* __restrict__ vc,
                                            int64_t page_stride, int64_t token_stride, int64_t head_stride,
                                            const int32_t* __restrict__ indices, int page_size, int64_t num_pages,
                                            float scale_log2, const QkvIn& qin, int num_qo_heads,
                                            float* __restrict__ part_lse, float* __restrict__ part_o,
                                            uint32_t* __restrict__ s_v, uint4 (*s_q)[4][16]) {
  constexpr int D = 128, G = 4;
  const int lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  const int rg = lane / 16, col = lane % 16;  // q formation: row group (head 4h + rg), 8-dim slice
  const int nrows = min(batch, kPrefixMaxRows);
  const bool live = j < sc.n_pref;  // the workgroup's last chunk group may be partial
  // ---- wave w forms row w's q for the workgroup's kv head (the four waves
  // share them through LDS): loads first, with the item's page ids
  const int hq_form = h * G + rg;
  const int a_ld = R > 0 ? qin.m[0].adapter : 0;  // the bound adapter (the host requires one)
  const int qb_row = min(wv, nrows - 1);
  // the item's pages: tokens j*32 .. of row 0's list (every row's, up to the
  // prefix).  Issued before q's loads: loads complete in order, so the K
  // loads below then wait for the page ids alone.
  const int ip0 = __builtin_amdgcn_readfirstlane(sc.ip);
  const int tok0 = (live ? j : 0) * kPrefixTokens;
  const int last_idx = dir.capacity > 0 ? dir.capacity - 1 : 0;  // page reads stay inside the indices buffer
  const int psh = page_size == 16 ? 4 : 5;  // log2 of the page size (16 or 32 tokens)
  const int pid_a = indices[min(ip0 + (tok0 >> psh), last_idx)];
  const int pid_b = indices[min(ip0 + ((tok0 + 16) >> psh), last_idx)];
  __builtin_amdgcn_sched_barrier(0);
  HeadIn<T, R> x;
  head_base_load<T, R>(qin, qb_row, hq_form, col, (const T*)qin.q_norm_w, x);
  head_lora_load<T, R>(qin, qb_row, 0, hq_form * D, col, a_ld, x);
  __builtin_amdgcn_sched_barrier(0);
  const int pg_a = uniform(pid_a), pg_b = uniform(pid_b);
  // ---- K (A operand: token l % 16 of each block, dims 8 (l/16) + 32 jj) and
  // V (token rows l/16 + 4 s of the 32, dims 8 (l % 16) ..) of the 32 tokens,
  // issued before q is formed (a wave past the prefix reads chunk 0's)
  // the item's two 16-token halves (pages of 16 or 32 tokens here, and tok0
  // a multiple of 32): rows 0.. of page pg_a, then rows 0.. of page pg_b
  // (16-token pages) or rows 16.. of page pg_a (32-token pages).  Element
  // offset of row r of half hf, kv head h: uniform bases, one per half.
  auto page_off = [&](int pg) -> int64_t {
    const int64_t pc = pg < 0 ? 0 : (pg >= num_pages ? num_pages - 1 : pg);
    return pc * page_stride + (int64_t)h * head_stride;
  };
  const int64_t half0 = page_off(pg_a);
  const int64_t half1 = page_size == 16 ? page_off(pg_b) : half0 + 16 * token_stride;
  auto tok_addr = [&](int hf, int64_t row_off) -> int64_t { return (hf ? half1 : half0) + row_off; };
  uint32_t kw[2][4][4];
  const int64_t col_off = (int64_t)col * token_stride;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const T* kp = kc + tok_addr(blk, col_off) + 8 * rg;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const uint4 t = *reinterpret_cast<const uint4*>(kp + 32 * jj);
      kw[blk][jj][0] = t.x; kw[blk][jj][1] = t.y; kw[blk][jj][2] = t.z; kw[blk][jj][3] = t.w;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  {
    float v[8];
    head_finish<T, R>(qin, x, 0, col, qin.q_norm_w != nullptr, true, R > 0, v);
    if (wv < nrows)
      s_q[wv][rg][col] = make_uint4(pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]), pack2<T>(v[4], v[5]),
                                    pack2<T>(v[6], v[7]));
  }
  __syncthreads();
  if (!live) return;
  // B operand of S^T: column l % 16 = (row (l%16)/4, head l % 4), dims 32 jj + 8 (l / 16) ..
  uint32_t qb[4][4];
  {
    const int qrow = min(col / 4, nrows - 1);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const uint4 t = s_q[qrow][lane % 4][4 * jj + lane / 16];
      qb[jj][0] = t.x; qb[jj][1] = t.y; qb[jj][2] = t.z; qb[jj][3] = t.w;
    }
  }
  uint4 vr[8];
#pragma unroll
  for (int s2 = 0; s2 < 8; ++s2)
    vr[s2] = *reinterpret_cast<const uint4*>(vc + tok_addr(s2 >= 4, (int64_t)(rg + 4 * (s2 & 3)) * token_stride) + 8 * col);
  // ---- S^T and the softmax of each column over the 32 tokens
  f32x4 sacc[2];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    sacc[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) sacc[blk] = mfma_16x16x32<T>(kw[blk][jj], qb[jj], sacc[blk]);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sacc[blk][i] *= scale_log2;
      mx = fmaxf(mx, sacc[blk][i]);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  float pv[8], ps = 0.f;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pv[blk * 4 + i] = fast_exp2(sacc[blk][i] - mx);
      ps += pv[blk * 4 + i];
    }
  ps += __shfl_xor(ps, 16);
  ps += __shfl_xor(ps, 32);
  // ---- V into LDS (this wave's 8 KB: token row t at words 64 t ..), then O^T
#pragma unroll
  for (int s2 = 0; s2 < 8; ++s2)
    *reinterpret_cast<uint4*>(s_v + (rg + 4 * s2) * 64 + 4 * col) = vr[s2];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // P^T as the B operand: k = 8 (l/16) + e <-> token 4 (l/16) + e of block 0 (e < 4), of block 1 (e >= 4)
  u32x4 pb_hi, pb_lo;
  {
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hw[e] = pack_pv<T>(pv[2 * e], pv[2 * e + 1]);
      float h0, h1;
      unpack2<T>(hw[e], h0, h1);
      lw[e] = pack_pv<T>(pv[2 * e] - h0, pv[2 * e + 1] - h1);
    }
    pb_hi = u32x4{hw[0], hw[1], hw[2], hw[3]};
    pb_lo = u32x4{lw[0], lw[1], lw[2], lw[3]};
  }
  int trow[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) trow[e] = (e < 4 ? 4 * rg + e : 16 + 4 * rg + e - 4) * 64;
  f32x4 acc[8];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    uint32_t w[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = s_v[trow[e] + 16 * a + col];
    uint32_t alo[4], ahi[4];
    alo[0] = __builtin_amdgcn_perm(w[1], w[0], 0x05040100u);
    ahi[0] = __builtin_amdgcn_perm(w[1], w[0], 0x07060302u);
    alo[1] = __builtin_amdgcn_perm(w[3], w[2], 0x05040100u);
    ahi[1] = __builtin_amdgcn_perm(w[3], w[2], 0x07060302u);
    alo[2] = __builtin_amdgcn_perm(w[5], w[4], 0x05040100u);
    ahi[2] = __builtin_amdgcn_perm(w[5], w[4], 0x07060302u);
    alo[3] = __builtin_amdgcn_perm(w[7], w[6], 0x05040100u);
    ahi[3] = __builtin_amdgcn_perm(w[7], w[6], 0x07060302u);
    const uint32_t phi[4] = {pb_hi[0], pb_hi[1], pb_hi[2], pb_hi[3]};
    const uint32_t plo[4] = {pb_lo[0], pb_lo[1], pb_lo[2], pb_lo[3]};
    acc[2 * a] = mfma_16x16x32<T>(alo, phi, f32x4{0.f, 0.f, 0.f, 0.f});
    acc[2 * a + 1] = mfma_16x16x32<T>(ahi, phi, f32x4{0.f, 0.f, 0.f, 0.f});
    acc[2 * a] = mfma_16x16x32<T>(alo, plo, acc[2 * a]);
    acc[2 * a + 1] = mfma_16x16x32<T>(ahi, plo, acc[2 * a + 1]);
  }
  // ---- the partial of column col = lane % 16: row b, query head 4h + col % 4,
  // dims 32a + 8 (l/16) + 2i (tile 2a) and + 1 (tile 2a + 1)
  const int b = col / 4;
  if (b >= nrows) return;
  const int hq = h * G + col % 4;
  int first = 0;
  // row b's first slot: b * n_pref + the own items of the rows before it
#pragma unroll
  for (int bb = 0; bb < kPrefixMaxRows; ++bb) {
    const int incl_bb = __builtin_amdgcn_readlane(sc.incl, bb);
    const int n_bb = __builtin_amdgcn_readlane(sc.n, bb);
    first = (b == bb) ? bb * sc.n_pref + incl_bb - n_bb : first;
  }
  const int slot = first + j;
  const float inv = ps > 0.f ? 1.f / ps : 0.f;
  float* op = part_o + ((int64_t)slot * num_qo_heads + hq) * D + 8 * rg;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const float o8[8] = {acc[2 * a][0] * inv, acc[2 * a + 1][0] * inv, acc[2 * a][1] * inv,
                         acc[2 * a + 1][1] * inv, acc[2 * a][2] * inv, acc[2 * a + 1][2] * inv,
                         acc[2 * a][3] * inv, acc[2 * a + 1][3] * inv};
    Lane8<float>::store(op + 32 * a, o8);
  }
  if (rg == 0) part_lse[(int64_t)slot * num_qo_heads + hq] = ps > 0.f ? mx + __log2f(ps) : -INFINITY;
}

// SMALL: pages of a size that is not a multiple of 16 tokens (stream_blocks_small).
// kv_split: the kernel's kv heads are virtual, kv_split of them per real kv
// head, each serving G of that head's query heads (GQA groups above 8 run as
// several waves of at most 8 heads); 1 otherwise.
// PREFIX (FUSED): the launch has a shared prefix (prefix_wave items); its
// own instantiation, so the prefix code's registers do not cost the plain
// kernel occupancy.
template <typename T, int D, int G, bool FUSED = false, int R = 0, bool SMALL = false, bool PREFIX = false>
__global__ __launch_bounds__(kWave * waves_per_wg<FUSED>()) void decode_kernel(
    const T* __restrict__ q, int64_t q_sb, int64_t q_sh, const T* __restrict__ kc,
    const T* __restrict__ vc, int64_t page_stride, int64_t token_stride, int64_t head_stride,
    const int32_t* __restrict__ indices, const int32_t* __restrict__ last_page_len,
    T* __restrict__ o, int64_t o_sb, int64_t o_sh, float* __restrict__ lse, int num_qo_heads,
    int num_kv_heads, int page_size, int64_t num_pages, float scale_log2,
    const int* __restrict__ header, const Item* __restrict__ items, int batch, int max_items,
    float* __restrict__ part_lse, float* __restrict__ part_o, QkvIn qin, int kv_split, Direct dir) {
  static_assert(!(FUSED && SMALL), "the folded q/k/v epilogue is built for 16-token pages");
  using WaveT = WaveFor<T, D, G>;
  constexpr int LPT = WaveT::LPT;
  using L8 = Lane8<T>;

  static_assert(!PREFIX || FUSED, "prefix items are built into the folded q/k/v kernel");
  // One word of each cache line of the arguments, read first and dropped:
  // every line is then in the scalar cache before the code reads its fields
  // (otherwise each line first read later costs a round trip there).  In
  // the shared-prefix instantiation only: the plain folded kernel's register
  // allocation came out worse with it (1 x 32K -1.5%).
  if constexpr (PREFIX) {
    asm volatile("" ::"s"(q), "s"(indices), "s"(num_pages), "s"(qin.ld), "s"(qin.m[0].ldy),
                 "s"(qin.m[1].y_offset), "s"(qin.m[2].B), "s"(dir.capacity));
  }
  // the prefix workgroups' V tiles (one 8 KB tile per wave) and q (4 rows x 4 heads)
  __shared__ uint32_t s_pv[PREFIX ? waves_per_wg<FUSED>() : 1][PREFIX ? kPrefixTokens * 64 : 1];
  __shared__ uint4 s_q[PREFIX ? kPrefixMaxRows : 1][4][16];
  const int lane = threadIdx.x % kWave;
  int wave = uniform(blockIdx.x * waves_per_wg<FUSED>() + threadIdx.x / kWave);
  int b, pbeg, pend, flags;
  [[maybe_unused]] DirectScan sc;
  if constexpr (PREFIX) {
    // The first ceil(n_pref / 4) * kv-heads workgroups are prefix
    // workgroups: workgroup g takes kv head g % hkv and prefix chunks
    // 4 (g / hkv) + w in its waves w; the rest take the own items as usual.
    sc = direct_scan(dir, batch);
    const int pref_wgs = (sc.n_pref + 3) / 4 * num_kv_heads;
    if ((int)blockIdx.x < pref_wgs) {
      const int hh = blockIdx.x % num_kv_heads;
      const int jj = (blockIdx.x / num_kv_heads) * 4 + threadIdx.x / kWave;
      prefix_wave<T, R>(sc, dir, batch, jj, hh, kc, vc, page_stride, token_stride, head_stride, indices, page_size,
                        num_pages, scale_log2, qin, num_qo_heads, part_lse, part_o, s_pv[threadIdx.x / kWave], s_q);
      return;
    }
    wave = uniform((blockIdx.x - pref_wgs) * waves_per_wg<FUSED>() + threadIdx.x / kWave) +
           sc.n_pref * num_kv_heads;
  }
  const int item_idx = wave / num_kv_heads;
  const int h = wave - item_idx * num_kv_heads;
  const int hk = FUSED ? h : uniform(h / kv_split);  // the real kv head whose pages this wave reads
  if (item_idx >= max_items) return;
  if (dir.indptr != nullptr) {  // direct items (uniform)
    bool found;
    if constexpr (PREFIX)
      found = direct_item_of(sc, dir, item_idx, b, pbeg, pend, flags);
    else
      found = direct_item(dir, batch, item_idx, b, pbeg, pend, flags);
    if (!found) return;
  } else {
    // The item is read together with the plan stamp (item_idx < max_items
    // keeps the read inside the item table) and used only if the stamp
    // matches: one combined check needs both, so both loads issue together.
    const int stamp_batch = uniform(header[2]), stamp = uniform(header[3]);
    const int4 iv = *reinterpret_cast<const int4*>(items + item_idx);  // the whole item in one load
    b = uniform(iv.x), pbeg = uniform(iv.y), pend = uniform(iv.z), flags = uniform(iv.w);
    // (every field takes part in the check, so no part of the item load is
    // deferred past it)
    if (!((stamp_batch == batch) & (stamp == plan_stamp(batch, max_items)) & (b >= 0) & (b < batch) & (pbeg >= 0) &
          (pend >= pbeg) & (flags >= 0) & ((flags >> 2) < max_items)))
      return;
  }
  // Second round trip, all at once: the row's last-page fill, the page ids
  // of the item's first two blocks and q (below).  The item's pages lie
  // inside the indices buffer (the plan clamps them), so indices[pbeg] exists
  // when pend > pbeg; an empty item reads its own first word instead (unused:
  // it streams no block), so the loads need no branch.  Block 1 starts at
  // token 16: in page pbeg + 1 when pages hold 16 tokens and the item has a
  // second page, else in page pbeg (or it does not exist, and the stream
  // clamps it to block 0).
  const int last_raw = last_page_len[b];
  const int32_t* idx0 = pend > pbeg ? indices + pbeg : reinterpret_cast<const int32_t*>(items + item_idx);
  const int first_page = uniform(idx0[0]);
  const int second_page = uniform(idx0[((page_size == kBlockTokens) & (pend - pbeg >= 2)) ? 1 : 0]);

  const int row = lane / LPT;   // token row inside a load instruction
  const int col = lane % LPT;   // 8-element slice of the head dim

  WaveT st;
  st.init();
  // The folded epilogue's loads that need only b go out with this round
  // trip too: the adapter id, the new token's slot, and the packed rows,
  // norm weights and cos / sin of this wave's q head (row group r: head
  // h*G + r) and of its kv head's k (row group 0) and v (the other groups).
  [[maybe_unused]] int id_raw = -1;
  [[maybe_unused]] int64_t pg = -1, off = -1;
  [[maybe_unused]] HeadIn<T, R> hq_in, hkv_in;
  [[maybe_unused]] const bool is_k = row == 0;
  if constexpr (FUSED) {
    static_assert(G == 4 && D == 128 && sizeof(T) == 2, "the folded q/k/v epilogue is built for GQA 4, head_dim 128");
    // ids is always readable (the host points it at a dummy array for a
    // uniform adapter), so its load needs no test
    if constexpr (R > 0) id_raw = qin.ids[b];
    pg = qin.page_id[b];
    off = qin.page_off[b];
    head_base_load<T, R>(qin, b, h * G + row, col, (const T*)qin.q_norm_w, hq_in);
    head_base_load<T, R>(qin, b, (is_k ? num_qo_heads : num_qo_heads + num_kv_heads) + h, col,
                         is_k ? (const T*)qin.k_norm_w : nullptr, hkv_in);
  } else if constexpr (WaveT::kMfmaScores) {
    // the B operand: head lane % 4 of the group, dims 32 j + 8 (lane / 16)
    const T* qp = q + (int64_t)b * q_sb + (int64_t)(h * G + lane % 4) * q_sh + 8 * (lane / 16);
#pragma unroll
    for (int j = 0; j < WaveT::NS; ++j) L8::load(st.qb[j], qp + 32 * j);
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const T* qp = q + (int64_t)b * q_sb + (int64_t)(h * G + g) * q_sh + col * 8;
      L8::load(st.q[g], qp);
    }
  }

  // (no branch on pend > pbeg: a load whose only use sits in a branch is
  // moved into it, a round trip of its own; an empty item gives <= 0)
  const int last = last_raw < 1 ? 1 : (last_raw > page_size ? page_size : last_raw);
  const int ntok = uniform(max(0, (pend - pbeg) * page_size - ((flags & 2) ? page_size - last : 0)));
  const int nblk = (ntok + kBlockTokens - 1) / kBlockTokens;

  KvLanes ln;
  ln.v_off = (int64_t)row * token_stride + (int64_t)hk * head_stride + col * 8;
  ln.v_step = (int64_t)WaveT::TPI * token_stride;
  if constexpr (WaveT::kMfmaScores) {
    ln.k_off = WaveT::k_lane_off(lane, token_stride) + (int64_t)hk * head_stride;
    ln.k_step = 32;
  } else {
    ln.k_off = ln.v_off;
    ln.k_step = ln.v_step;
  }
  if constexpr (FUSED) {
    NewToken nt;
    nt.blk = -1;
    // Runs with the first block's loads in flight: q (row group r computes
    // q head h*G + r, dims 8*col .., rounded to T as the standalone epilogue
    // stores it; every lane then gathers the 4 heads) and, in the item
    // holding the row's last page, the new token's k (row group 0: + LoRA,
    // k-norm, RoPE) and v (row group 1: + LoRA) of this kv head, stored into
    // its slot and spliced into the block that holds it.
    // the adapter: blended with bit operations, so the id's load is not
    // moved under a test of the uniform adapter
    const uint32_t per_row = (uint32_t)(qin.m[0].adapter >> 31);  // all ones: per-row ids
    const int a_in = (int)(((uint32_t)qin.m[0].adapter & ~per_row) | ((uint32_t)id_raw & per_row));
    const bool a_ok = R > 0 && a_in >= 0 && a_in < qin.n_adapters;
    const int a_ld = a_ok ? a_in : 0;
    const int qh = h * G + row;
    // q's LoRA rows: without a shared prefix (long rows) they go out before
    // the first block's loads, so q's products wait for them alone (loads
    // complete in order), not for the block (1 x 32K +0.4%); in a
    // shared-prefix launch after them (4 rows -0.3% the other way)
    auto q_lora = [&]() { head_lora_load<T, R>(qin, b, 0, qh * D, col, a_ld, hq_in); };
    auto pre = [&]() {
      if constexpr (!PREFIX) q_lora();
    };
    auto hook = [&]() {
      const bool slot_ok = (pg >= 0) & (pg < num_pages) & (off >= 0) & (off < page_size);
      const int mod = is_k ? 1 : 2;
      auto form_q = [&]() {
        float v[8];
        head_finish<T, R>(qin, hq_in, 0, col, qin.q_norm_w != nullptr, true, a_ok, v);
        const uint32_t w4[4] = {pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]), pack2<T>(v[4], v[5]),
                                pack2<T>(v[6], v[7])};
        if constexpr (WaveT::kMfmaScores) {
          // B operand: head lane % 4, dims 32 j + 8 (lane / 16) .. = the
          // 8-dim slice 4 j + lane / 16 of row group lane % 4
#pragma unroll
          for (int j = 0; j < WaveT::NS; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k)
              st.qb[j][k] = (uint32_t)__shfl((int)w4[k], (lane % 4) * LPT + 4 * j + lane / 16);
        } else {
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int k = 0; k < 4; ++k) st.q[g][k] = (uint32_t)__shfl((int)w4[k], g * LPT + col);
        }
      };
      if constexpr (PREFIX) q_lora();
      if (!(flags & 2)) {
        __builtin_amdgcn_sched_barrier(0);
        form_q();
        return;
      }
      // The item holding the row's last page: the new token's k / v LoRA rows
      // go out right after q's (q's products wait only for the loads before
      // them), one round trip for both.
      head_lora_load<T, R>(qin, b, mod, h * D, col, a_ld, hkv_in);
      __builtin_amdgcn_sched_barrier(0);
      form_q();
      float v[8];
      head_finish<T, R>(qin, hkv_in, mod, col, is_k & (qin.k_norm_w != nullptr), is_k, a_ok,
                        v);  // rows 2, 3 compute v again; unused
      const uint32_t kv4[4] = {pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]), pack2<T>(v[4], v[5]),
                               pack2<T>(v[6], v[7])};
      if (row < 2 && slot_ok) {
        T* dst = const_cast<T*>(is_k ? kc : vc) + pg * page_stride + off * token_stride +
                 (int64_t)h * head_stride + col * 8;
        *reinterpret_cast<uint4*>(dst) = make_uint4(kv4[0], kv4[1], kv4[2], kv4[3]);
      }
      // A slot at the row's last token (where a decode step appends) is
      // the item's token ntok - 1: attend over the computed k / v there.
      // The store above is not waited for: nothing in this launch reads
      // the slot from memory then.
      const int lst = last_raw < 1 ? 1 : (last_raw > page_size ? page_size : last_raw);
      const int t = ntok - 1, tt = t - (t / kBlockTokens) * kBlockTokens;
      nt.blk = (slot_ok & (off == lst - 1) & (ntok > 0)) ? t / kBlockTokens : -1;
      nt.pg = (int)pg;  // the block must also come from the slot's page
      nt.s = tt / WaveT::TPI;
      nt.row = tt - nt.s * WaveT::TPI;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        nt.k[k] = (uint32_t)__shfl((int)kv4[k], col);        // row group 0
        nt.v[k] = (uint32_t)__shfl((int)kv4[k], LPT + col);  // row group 1
      }
      if constexpr (WaveT::kMfmaScores) {
        nt.klane = WaveT::k_lane_of(tt);
#pragma unroll
        for (int j = 0; j < WaveT::NS; ++j)
#pragma unroll
          for (int k = 0; k < 4; ++k) nt.kq[j][k] = (uint32_t)__shfl((int)kv4[k], 4 * j + lane / 16);
      }
    };
    stream_blocks_fused<T>(st, kc, vc, page_stride, token_stride, ln, indices, pbeg, page_size,
                                 num_pages, ntok, 0, nblk, scale_log2, row, first_page, second_page, pre, hook, nt);
  } else if constexpr (SMALL) {
    const int64_t v_fix = (int64_t)hk * head_stride + col * 8;
    int k_tok = -1;
    int64_t k_fix = v_fix;
    if constexpr (WaveT::kMfmaScores) {
      const int m16 = lane % 16;
      k_tok = m16 / 4 + 4 * (m16 % 4);
      k_fix = (int64_t)hk * head_stride + 8 * (lane / 16);
    }
    stream_blocks_small<T>(st, kc, vc, page_stride, token_stride, k_fix, v_fix, k_tok, indices, pbeg, page_size,
                           num_pages, ntok, nblk, scale_log2, row);
  } else {
    stream_blocks<T>(st, kc, vc, page_stride, token_stride, ln, indices, pbeg, page_size, num_pages,
                           ntok, 0, nblk, scale_log2, row, first_page, second_page);
  }

  st.merge_rows();

  constexpr float kLn2 = 0.69314718055994530942f;
  bool direct = flags & 1;  // the row is one item: write the output directly
  if constexpr (FUSED) direct = direct && !qin.no_direct;
  if (direct) {
    if (row != 0) return;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int hq = h * G + g;
      const float inv = st.l[g] > 0.f ? 1.f / st.l[g] : 0.f;
      float out[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) out[i] = st.acc[g][i] * inv;
      L8::store(o + (int64_t)b * o_sb + (int64_t)hq * o_sh + col * 8, out);
      if (lse != nullptr && col == 0)
        lse[(int64_t)b * num_qo_heads + hq] =
            st.l[g] > 0.f ? (st.m[g] + __log2f(st.l[g])) * kLn2 : -INFINITY;
    }
    return;
  }

  // Split row: publish this item's normalised partial and its log2-sum-exp at
  // the item's slot; merge_kernel combines them after this kernel has finished.
  if (row != 0) return;
  const int slot = flags >> 2;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int hq = h * G + g;
    const float inv = st.l[g] > 0.f ? 1.f / st.l[g] : 0.f;
    float out[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = st.acc[g][i] * inv;
    Lane8<float>::store(part_o + ((int64_t)slot * num_qo_heads + hq) * D + col * 8, out);
    if (col == 0)
      part_lse[(int64_t)slot * num_qo_heads + hq] =
          st.l[g] > 0.f ? st.m[g] + __log2f(st.l[g]) : -INFINITY;
  }
}

// ----------------------------------------------------------------- merge ---
// One workgroup of MT threads per (row, q head) of a split row.  LPT lanes
// cover one partial row of D floats; the workgroup takes RPI partial rows per
// pass and issues up to kMergeBatch passes of loads (each partial's lse and
// output together) before folding any of them, so a row of up to
// RPI * kMergeBatch items costs one memory round trip.  Each thread folds its
// partials online (running max, weight sum, weighted output); the threads'
// states are combined with xor shuffles inside a wave and through LDS across
// waves.  MT is one wave when the plan averages a few items per row (the
// ragged batch-64 case: ~5), four waves when rows hold tens of items, eight
// beyond 96.
constexpr int kMergeBatch = 8;
constexpr int kMergeFewItems = 8;  // average items per row up to which one wave merges
// Average slots per row above which eight waves merge (a row of ~128 items:
// 1 x 32K tokens, plan + decode + merge 36.7 -> 35.7 us; at ~33 items per
// row (4 x 2112) four waves stay 0.25 us faster, and at ~69 (the same rows
// with their 2048-token prefix shared: 64 prefix chunks each) 5.2 -> 4.9 us).
constexpr int kMergeManyItems = 96;
constexpr int kMergeCUs = 256;  // MI355X

// Workgroups per (row, head) of the merge: the head's dims split as far as
// 4 while the launch stays within one workgroup per CU (a full-chip launch
// gains nothing from it).
__host__ __device__ constexpr int merge_dim_split(int head_dim, int pairs) {
  return (head_dim % 32 == 0 && pairs * 4 <= kMergeCUs) ? 4 : (head_dim % 16 == 0 && pairs * 2 <= kMergeCUs) ? 2 : 1;
}

struct MergeState {
  float m, w, a[8];  // log2 max, sum of weights, weighted output (8 dims)
  __device__ __forceinline__ void add(float m_o, float w_o, const float (&a_o)[8]) {
    const float m_new = fmaxf(m, m_o);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float s = fast_exp2(m - m_use), so = fast_exp2(m_o - m_use);
    w = w * s + w_o * so;
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = a[i] * s + a_o[i] * so;
    m = m_new;
  }
};

// The o_proj module's LoRA shrink, folded into the merge (decoder layers):
// the merged output of the attention is o_proj's input, so each workgroup
// multiplies its slice of the (row, head) output, rounded to T as stored, by
// the same columns of the row's adapter's A rows and writes the rank-space
// partial sums, one per (head, dim slice): part[b * ld + (hq * DS + ds) * R
// + r].  The A rows are read from the shuffled [W_o; A_o] weight: adapter a's
// rank r is row a_row0 + a * R + r.  An adapter outside [0, n_adapters)
// gives adapter 0's products (its consumer does not apply them).
struct OShrink {
  const void* A;
  int ksteps;       // o_proj's in_features / 32 (num_qo_heads * D / 32)
  int a_row0;
  int adapter;      // >= 0: every row's adapter; -1: ids[b]
  const int32_t* ids;
  int n_adapters;
  float* part;
  int64_t ld;
};

// DS: the head's dims split over DS workgroups (each folds every partial of
// its D / DS dims), for launches with few (row, head) pairs: one row of 32
// heads is otherwise 32 workgroups, each reading 64 KB of partials alone.
// OR > 0: the OShrink products of rank OR are formed too, and single-item
// rows (published as one partial) are merged as well.
template <typename T, int D, int MT, int DS = 1, int OR = 0>
__global__ __launch_bounds__(MT) void merge_kernel(
    const int2* __restrict__ row_info, const float* __restrict__ part_lse,
    const float* __restrict__ part_o, T* __restrict__ o, int64_t o_sb, int64_t o_sh,
    float* __restrict__ lse, const int* __restrict__ header, int batch, int num_qo_heads,
    int max_items, Direct dir, OShrink os) {
  static_assert((D / 8) % DS == 0, "whole 8-dim slices per workgroup");
  static_assert(OR == 0 || OR == 8 || OR == 16, "o shrink ranks 8 or 16");
  constexpr int LPT = D / 8 / DS, RPI = MT / LPT, NWV = MT / kWave;
  constexpr int NP = OR * LPT, PPT = OR > 0 ? (NP + MT - 1) / MT : 1;  // shrink products, per thread
  constexpr int kMinItems = OR > 0 ? 1 : 2;
  __shared__ float s_m[NWV][LPT], s_w[NWV][LPT], s_a[NWV][LPT][8];
  __shared__ float s_ov[OR > 0 ? LPT : 1][8];
  // the partials' addresses are read with the first arguments (held in
  // scalar registers): left to their first use, they come from another
  // cache line of the arguments, a round trip after the row's range
  uint64_t plse_u = (uint64_t)(uintptr_t)part_lse, po_u = (uint64_t)(uintptr_t)part_o;
  asm volatile("" : "+s"(plse_u), "+s"(po_u));
  part_lse = gptr<const float*>(plse_u);
  part_o = gptr<const float*>(po_u);
  const int pair = blockIdx.x / DS, ds = blockIdx.x % DS;
  if (pair >= batch * num_qo_heads) return;
  const int b = pair / num_qo_heads;
  const int hq = pair - b * num_qo_heads;
  // the A pieces' addresses (they need only the row's adapter); the loads
  // go out after the first batch of partials, so the fold does not wait
  // for them (loads complete in order)
  [[maybe_unused]] uint4 ap[PPT];
  [[maybe_unused]] const T* ap_src[PPT];
  if constexpr (OR > 0) {
    const int a_raw = os.adapter >= 0 ? os.adapter : os.ids[b];
    const int aa = (a_raw >= 0 && a_raw < os.n_adapters) ? a_raw : 0;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int i = min((int)threadIdx.x + j * MT, NP - 1);
      const int r = i / LPT, c = i - r * LPT;
      const int64_t n = (int64_t)os.a_row0 + (int64_t)aa * OR + r;
      const int k = hq * D + (ds * LPT + c) * 8;
      ap_src[j] = (const T*)os.A + (((n / 16) * os.ksteps + k / 32) * 64 + ((k % 32) / 8) * 16 + n % 16) * 8;
    }
  }
  int first, n;
  if (dir.indptr != nullptr) {  // direct items (uniform): the row's slots from indptr
    direct_row(dir, batch, b, first, n);
    if (!((n >= kMinItems) & (first >= 0) & (first + n <= max_items))) return;
  } else {
    // One combined check that needs all three loads, so they are issued
    // together (separate early exits would sink each load below the last).
    const int stamp_batch = uniform(header[2]), stamp = uniform(header[3]);
    const int2 info = row_info[b];
    first = uniform(info.x), n = uniform(info.y);
    const bool planned = (stamp_batch == batch) & (stamp == plan_stamp(batch, max_items));
    if (!(planned & (n >= kMinItems) & (first >= 0) & (first + n <= max_items))) return;
  }

  const int r = threadIdx.x / LPT, col = threadIdx.x % LPT;
  const int dcol = ds * LPT + col;  // the thread's 8-dim slice of the head
  MergeState st{-INFINITY, 0.f, {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}};
  for (int c0 = 0; c0 < n; c0 += RPI * kMergeBatch) {
    float lv[kMergeBatch];
    float4 oa[kMergeBatch], ob[kMergeBatch];
    // passes of this batch that hold any item (uniform): a row of a few items
    // issues one pass of loads, not kMergeBatch passes of re-reads
    const int passes = min(kMergeBatch, (n - c0 + RPI - 1) / RPI);
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      if (k < passes) {
        // past the last item: re-read the last one (in bounds); its weight is dropped below
        const int c = min(c0 + r + k * RPI, n - 1);
        const int64_t slot = (int64_t)(first + c) * num_qo_heads + hq;
        lv[k] = part_lse[slot];
        oa[k] = *reinterpret_cast<const float4*>(part_o + slot * D + dcol * 8);
        ob[k] = *reinterpret_cast<const float4*>(part_o + slot * D + dcol * 8 + 4);
      }
    }
    if constexpr (OR > 0) {
      if (c0 == 0) {
#pragma unroll
        for (int j = 0; j < PPT; ++j) ap[j] = *reinterpret_cast<const uint4*>(ap_src[j]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // the whole batch in flight before the first fold
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      if (k < passes) {
        const bool on = c0 + r + k * RPI < n;
        const float v[8] = {oa[k].x, oa[k].y, oa[k].z, oa[k].w, ob[k].x, ob[k].y, ob[k].z, ob[k].w};
        st.add(on ? lv[k] : -INFINITY, on ? 1.f : 0.f, v);
      }
    }
  }
  // fold the RPI rows: within a wave (xor over the row bits of the lane id) ...
#pragma unroll
  for (int off = LPT; off < kWave; off <<= 1) {
    float a_o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) a_o[i] = __shfl_xor(st.a[i], off);
    const float m_o = __shfl_xor(st.m, off), w_o = __shfl_xor(st.w, off);
    st.add(m_o, w_o, a_o);
  }
  // ... then across the waves through LDS
  if constexpr (NWV > 1) {
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (lane < LPT) {
      s_m[wave][col] = st.m;
      s_w[wave][col] = st.w;
#pragma unroll
      for (int i = 0; i < 8; ++i) s_a[wave][col][i] = st.a[i];
    }
    __syncthreads();
  }
  if (threadIdx.x < LPT) {
#pragma unroll
    for (int w = 1; w < NWV; ++w) {
      float a_o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) a_o[i] = s_a[w][col][i];
      st.add(s_m[w][col], s_w[w][col], a_o);
    }
    const float inv = st.w > 0.f ? 1.f / st.w : 0.f;
    T* op = o + (int64_t)b * o_sb + (int64_t)hq * o_sh + dcol * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const T v = from_float<T>(st.a[i] * inv);
      op[i] = v;
      if constexpr (OR > 0) s_ov[col][i] = to_float<T>(v);
    }
    if (lse != nullptr && dcol == 0) {
      constexpr float kLn2 = 0.69314718055994530942f;
      const float m_use = st.m == -INFINITY ? 0.f : st.m;
      lse[(int64_t)b * num_qo_heads + hq] = st.w > 0.f ? (m_use + __log2f(st.w)) * kLn2 : -INFINITY;
    }
  }
  if constexpr (OR > 0) {
    __syncthreads();
    // products of the A pieces with the stored output, summed over the LPT
    // consecutive lanes of each rank (DPP, fixed order)
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int i = (int)threadIdx.x + j * MT;
      const int r = i / LPT, c = i - r * LPT;
      float f[8];
      unpack2<T>(ap[j].x, f[0], f[1]);
      unpack2<T>(ap[j].y, f[2], f[3]);
      unpack2<T>(ap[j].z, f[4], f[5]);
      unpack2<T>(ap[j].w, f[6], f[7]);
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(s_ov[c][e], f[e], acc);
      acc = group_sum(acc, LPT == 16 ? 4 : LPT == 8 ? 3 : LPT == 4 ? 2 : LPT == 2 ? 1 : 0);
      if (c == 0 && i < NP) os.part[(int64_t)b * os.ld + (int64_t)(hq * DS + ds) * OR + r] = acc;
    }
  }
}

// ------------------------------------------------------------- dispatch ---
struct RunArgs {
  const void* q; int64_t q_sb, q_sh;
  const void* kc; const void* vc; int64_t page_stride, token_stride, head_stride;
  const int32_t* indices; const int32_t* last;
  void* o; int64_t o_sb, o_sh; float* lse;
  int batch, hq, hkv, page_size; int64_t num_pages; float scale_log2;
  int kv_split;  // virtual kv heads per real one (hkv counts the virtual heads)
  const int* header; const Item* items; int max_items; const int2* row_info;
  float* part_lse; float* part_o; int flags;
  Direct dir;  // dir.indptr != nullptr: items derived from indptr (no plan kernel)
  int grid_items;  // work items the decode grid covers (max_items, the slot count, unless a prefix is shared)
  OShrink os;      // os.part != nullptr: the merge forms o_proj's LoRA shrink partials (rank os_rank)
  int os_rank;
  hipStream_t stream;
};

template <typename T, int D, int G, bool FUSED = false, int R = 0, bool SMALL = false>
int launch(const RunArgs& a, const QkvIn& qin = QkvIn{}) {
  if (!(a.flags & PL_DECODE_MERGE_ONLY)) {
    const int64_t waves = (int64_t)a.grid_items * a.hkv;
    constexpr int wpg = waves_per_wg<FUSED>();
    const int grid = (int)((waves + wpg - 1) / wpg);
    auto go = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, dim3(grid), dim3(kWave * wpg), 0, a.stream, (const T*)a.q, a.q_sb, a.q_sh,
                         (const T*)a.kc, (const T*)a.vc, a.page_stride, a.token_stride, a.head_stride, a.indices,
                         a.last, (T*)a.o, a.o_sb, a.o_sh, a.lse, a.hq, a.hkv, a.page_size, a.num_pages,
                         a.scale_log2, a.header, a.items, a.batch, a.max_items, a.part_lse, a.part_o, qin,
                         a.kv_split, a.dir);
    };
    if constexpr (FUSED) {
      if (a.dir.shared > 0)
        go(decode_kernel<T, D, G, FUSED, R, SMALL, true>);
      else
        go(decode_kernel<T, D, G, FUSED, R, SMALL, false>);
    } else {
      go(decode_kernel<T, D, G, FUSED, R, SMALL, false>);
    }
    PL_LAUNCH_CHECK("decode_kernel");
  }
  if (!(a.flags & PL_DECODE_SKIP_MERGE)) {
    const int pairs = a.batch * a.hq;
    const int ds = merge_dim_split(D, pairs);
    auto go = [&](auto mt, auto dsc) {
      constexpr int MT = decltype(mt)::value, DS = decltype(dsc)::value;
      auto with = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(pairs * DS), dim3(MT), 0, a.stream, a.row_info, a.part_lse, a.part_o,
                           (T*)a.o, a.o_sb, a.o_sh, a.lse, a.header, a.batch, a.hq, a.max_items, a.dir, a.os);
      };
      if constexpr (FUSED && D == 128) {
        if (a.os.part != nullptr && a.os_rank == 16) return with(merge_kernel<T, D, MT, DS, 16>);
        if (a.os.part != nullptr && a.os_rank == 8) return with(merge_kernel<T, D, MT, DS, 8>);
      }
      with(merge_kernel<T, D, MT, DS, 0>);
    };
    auto by_ds = [&](auto mt) {
      if constexpr (D % 32 == 0)
        if (ds == 4) return go(mt, std::integral_constant<int, 4>{});
      if constexpr (D % 16 == 0)
        if (ds == 2) return go(mt, std::integral_constant<int, 2>{});
      go(mt, std::integral_constant<int, 1>{});
    };
    if (a.max_items <= kMergeFewItems * a.batch)
      by_ds(std::integral_constant<int, kWave>{});
    else if (a.max_items <= kMergeManyItems * a.batch)
      by_ds(std::integral_constant<int, 4 * kWave>{});
    else
      by_ds(std::integral_constant<int, 8 * kWave>{});
    PL_LAUNCH_CHECK("merge_kernel");
  }
  return ok();
}

constexpr int kMaxGroup = 8;          // query heads per wave (larger GQA groups are split)
constexpr int kMaxPageSize = 1 << 16; // tokens per page

template <typename T, int D, bool SMALL>
int by_group(const RunArgs& a, int g) {
  switch (g) {
    case 1: return launch<T, D, 1, false, 0, SMALL>(a);
    case 2: return launch<T, D, 2, false, 0, SMALL>(a);
    case 3: return launch<T, D, 3, false, 0, SMALL>(a);
    case 4: return launch<T, D, 4, false, 0, SMALL>(a);
    case 5: return launch<T, D, 5, false, 0, SMALL>(a);
    case 6: return launch<T, D, 6, false, 0, SMALL>(a);
    case 7: return launch<T, D, 7, false, 0, SMALL>(a);
    case 8: return launch<T, D, 8, false, 0, SMALL>(a);
  }
  return fail(PL_ERR_UNSUPPORTED, "GQA group size %d per wave not built (1..%d)", g, kMaxGroup);
}

template <typename T, bool SMALL>
int by_dim(const RunArgs& a, int d, int g) {
  switch (d) {
    case 64: return by_group<T, 64, SMALL>(a, g);
    case 128: return by_group<T, 128, SMALL>(a, g);
    case 256: return by_group<T, 256, SMALL>(a, g);
  }
  return fail(PL_ERR_UNSUPPORTED, "head_dim %d not built (64, 128, 256)", d);
}

// Launch decode (+ merge) for pages of a multiple of 16 tokens
// (paged_decode.hip) or of any other size (paged_decode_small.hip); g is the
// query heads per wave (1..8).
int run_multiple16_pages(const RunArgs& a, int dtype, int d, int g);
int run_small_pages(const RunArgs& a, int dtype, int d, int g);

}  // namespace decode
}  // namespace pl
