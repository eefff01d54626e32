// Paged prefill (multi-query) attention for gfx950.
//
// For request r with query rows qo_indptr[r] .. qo_indptr[r+1] (qo_len of
// them, the LAST qo_len positions of its kv_len-token sequence) and kv
// pages kv_indices[kv_indptr[r] ..] (all full but the last, which holds
// kv_last_page_len[r] tokens):
//   o[t, h] = softmax(q[t, h] . K^T * sm_scale  [+ causal mask]) . V
// With `causal`, query j of the request sees kv positions
// p <= kv_len - qo_len + j (bottom-right aligned, as FlashInfer's
// BatchPrefillWithPagedKVCacheWrapper); kv head = h / g, g = Hq / Hkv.
//
// Work decomposition.  A request's rows are (query position, head of the
// GQA group) pairs, row = pos * g + hg, so one kv head's K/V tile serves
// all g heads.  A work item is 64 consecutive rows of one request; the
// host plan lists items longest first (causal items near the end of a
// long prompt see the most tiles).  Grid = (items, kv heads), 4 waves of
// 16 rows each.
//
// Per kv tile (64 tokens; 32 at head_dim 256): K and V (both row-major)
// are staged in LDS straight from the pages while the next tile's loads are
// already in flight in registers.  Each wave computes S^T = K Q^T (MFMA
// 16x16x32, Q held in registers as the B operand), so a lane holds one
// query and 16 of the tile's tokens: masking and the fp32 online softmax
// (log2 domain) reduce within the lane and across the column's four lanes.
// The probabilities are then already in the B-operand layout of
// O^T += V^T P^T (no LDS round trip).  For bf16, P (in [0, 1]) is split into
// bf16 hi + lo parts and P V runs as two MFMAs, so P carries ~16 mantissa
// bits instead of 8 (fp16's 11 bits are used as is).  The V operand pairs
// two adjacent head-dim rows per lane: tile 2a holds d = 32a + 2c and tile
// 2a+1 holds d = 32a + 2c + 1, so a lane builds both A operands from eight
// 32-bit LDS reads and byte permutes, and writes both outputs as one
// 32-bit store.
//
// Reference: FlashInferAttentionBackend.plan_prefill / run_prefill
// (model/flashinfer/attention_backend.py:133-190); q / query_rescale with
// sm_scale * query_rescale there is the same softmax as here.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "pl_common.h"

namespace pl {
namespace prefill {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kRows = 16 * kWaves;  // rows per work item
constexpr int kPlanTile = 64;       // kv tokens per unit of the plan's work estimate

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <typename T> __device__ __forceinline__ f32x4 mfma32(u32x4 a, u32x4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma32<bf16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma32<f16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

// Tile geometry per head dim.  KT kv tokens per tile (64, or 32 at
// D = 256 to bound registers and LDS), NB 16-token blocks of S^T, NKC
// 32-token k-chunks of P V.
// Two probabilities (finite, in [0, 1]) packed as the PV operand type with
// the hardware round-to-nearest-even conversion: v_cvt_pk_bf16_f32 for bf16,
// one instruction per pair instead of the bit-level rounding the outputs use
// (which also handles NaN).
typedef float f32x2_pp __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ uint32_t pack_p(float a, float b);
template <> __device__ __forceinline__ uint32_t pack_p<bf16_t>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_pp{a, b}, bf16x2_t));
}
template <> __device__ __forceinline__ uint32_t pack_p<f16_t>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_pp{a, b}, half2_t));
}

template <int D>
struct Cfg {
  static constexpr int KT = D <= 128 ? 64 : 32;
  static constexpr int NB = KT / 16;
  static constexpr int NKC = KT / 32;
  static constexpr int CH = D / 8;                // 16-byte chunks per token row
  static constexpr int PER = KT * CH / kThreads;  // chunks per thread per tile (K and V each)
  static constexpr int KSTEPS = D / 32;           // MFMA k-steps of S over the head dim
  static constexpr int NPAIR = D / 32;            // pairs of 16-dim O tiles
  static constexpr int KP = D + 8;                // K row pitch (elements): conflict-free 16-byte reads
  static constexpr int VPW = D / 2 + 4;           // V row pitch (words): rows 4 apart land 16 banks apart
  static_assert(KT * CH % kThreads == 0, "tile must split evenly");
};

// Loads this thread's K and V chunks of kv tile `tile` into registers.
// Chunk j of a thread holds token RPP*j + threadIdx.x / CH of the tile
// (RPP = kThreads / CH token rows per pass).  ALIGNED (page_size a multiple
// of RPP): the RPP tokens of a pass lie in one page, so the page id and the
// pass's base offset are the same for the whole workgroup and come from
// scalar loads and scalar arithmetic; each lane only adds its fixed offset.
template <typename T, int D, bool ALIGNED>
__device__ __forceinline__ void load_tile(const T* __restrict__ kc, const T* __restrict__ vc,
                                          const int32_t* __restrict__ ind, int tile, int kv_len, int page_size,
                                          int64_t num_pages, int64_t page_stride, int64_t token_stride,
                                          int64_t head_off, u32x4 (&kr)[Cfg<D>::PER], u32x4 (&vr)[Cfg<D>::PER]) {
  constexpr int CH = Cfg<D>::CH;
  constexpr int RPP = kThreads / CH;
  if constexpr (ALIGNED) {
    const int tok0 = threadIdx.x / CH;
    const int64_t lane_off = (int64_t)tok0 * token_stride + head_off + (threadIdx.x % CH) * 8;
    auto pass_base = [&](int g0) -> int64_t {  // g0: first token of the pass (< kv_len)
      int64_t page = uniform(ind[g0 / page_size]);
      page = page < 0 ? 0 : (page >= num_pages ? num_pages - 1 : page);
      return page * page_stride + (int64_t)(g0 % page_size) * token_stride;
    };
    if (uniform((tile + 1) * Cfg<D>::KT <= kv_len ? 1 : 0)) {
      // a whole tile: every token exists, no zero fill
#pragma unroll
      for (int j = 0; j < Cfg<D>::PER; ++j) {
        const int64_t base = pass_base(uniform(tile * Cfg<D>::KT + RPP * j));
        kr[j] = *reinterpret_cast<const u32x4*>(kc + base + lane_off);
        vr[j] = *reinterpret_cast<const u32x4*>(vc + base + lane_off);
      }
    } else {
      // the row's last tile: tokens past kv_len read as zeros (their scores
      // are masked, and a zero V keeps an unused slot's contents out of P V)
#pragma unroll
      for (int j = 0; j < Cfg<D>::PER; ++j) {
        const int g0 = uniform(tile * Cfg<D>::KT + RPP * j);
        kr[j] = u32x4{0u, 0u, 0u, 0u};
        vr[j] = u32x4{0u, 0u, 0u, 0u};
        if (g0 < kv_len) {
          const int64_t base = pass_base(g0);
          if (g0 + tok0 < kv_len) {
            kr[j] = *reinterpret_cast<const u32x4*>(kc + base + lane_off);
            vr[j] = *reinterpret_cast<const u32x4*>(vc + base + lane_off);
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < Cfg<D>::PER; ++j) {
      const int c = threadIdx.x + j * kThreads;
      const int tok = c / CH, ch = c % CH;
      const int pos = tile * Cfg<D>::KT + tok;
      kr[j] = u32x4{0u, 0u, 0u, 0u};
      vr[j] = u32x4{0u, 0u, 0u, 0u};
      if (pos < kv_len) {
        int64_t page = ind[pos / page_size];
        page = page < 0 ? 0 : (page >= num_pages ? num_pages - 1 : page);
        const int64_t off = page * page_stride + (int64_t)(pos % page_size) * token_stride + head_off + ch * 8;
        kr[j] = *reinterpret_cast<const u32x4*>(kc + off);
        vr[j] = *reinterpret_cast<const u32x4*>(vc + off);
      }
    }
  }
}

// S^T = K Q^T: kv tokens are the MFMA rows and the wave's 16 query rows the
// columns, so a lane holds one query (column lr) and tokens 4*grp + i of
// each 16-token block.  The softmax then reduces within the lane and across
// the four lanes of the column, and the scores are already in the B-operand
// layout of O^T += V^T P^T: MFMA only needs A and B to agree on which token
// each k index is, so k index 8*grp + e of a 32-token chunk stands for token
// 4*grp + e (e < 4) or 16 + 4*grp + (e - 4) (e >= 4) in both operands.  No
// LDS round trip for P.
template <typename T, int D, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void prefill_kernel(
    const T* __restrict__ q, int64_t q_st, int64_t q_sh, const T* __restrict__ kc, const T* __restrict__ vc,
    int64_t page_stride, int64_t token_stride, int64_t head_stride, int64_t num_pages,
    const int32_t* __restrict__ qo_indptr, const int32_t* __restrict__ kv_indptr,
    const int32_t* __restrict__ kv_indices, const int32_t* __restrict__ kv_last, const int2* __restrict__ items,
    int n_items, T* __restrict__ o, int64_t o_st, int64_t o_sh, int batch, int hq, int hkv, int page_size,
    int causal, float scale_log2) {
  using C = Cfg<D>;
  constexpr int KT = C::KT, NB = C::NB, NKC = C::NKC, CH = C::CH, PER = C::PER;
  constexpr int KSTEPS = C::KSTEPS, NPAIR = C::NPAIR, KP = C::KP, VPW = C::VPW;
  constexpr int NPP = std::is_same<T, bf16_t>::value ? 2 : 1;  // P planes: hi (+ lo)
  __shared__ __align__(16) uint16_t s_k[KT * KP];
  __shared__ __align__(16) uint32_t s_v[KT * VPW];

  const int item = blockIdx.x;
  const int h = blockIdx.y;  // kv head
  if (item >= n_items || h >= hkv) return;
  const int2 it = items[item];
  const int r = uniform(it.x), row0 = uniform(it.y);
  if (r < 0 || r >= batch) return;
  const int g = hq / hkv;
  const int qo_begin = uniform(qo_indptr[r]);
  const int qo_len = uniform(qo_indptr[r + 1]) - qo_begin;
  const int pb = uniform(kv_indptr[r]), pe = uniform(kv_indptr[r + 1]);
  int last = uniform(kv_last[r]);
  last = last < 1 ? 1 : (last > page_size ? page_size : last);
  const int kv_len = pe > pb ? (pe - pb - 1) * page_size + last : 0;
  const int n_rows = qo_len * g;
  const int32_t* ind = kv_indices + pb;
  const int64_t head_off = (int64_t)h * head_stride;

  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int lr = lane % 16, grp = lane / 16;

  // this lane's query row (column lr of the wave's tile) and its last visible kv position
  const int qrow = row0 + wave * 16 + lr;
  const int q_pos = qrow / g, q_hg = qrow - q_pos * g;
  const bool q_ok = qrow < n_rows;
  const int lim = min(!q_ok ? -1 : (causal ? kv_len - qo_len + q_pos : kv_len - 1), kv_len - 1);

  // Q as the B operand: column lr, head-dim 32*ks + 8*grp .. +8
  u32x4 qb[KSTEPS];
  {
    const T* qp = q + (int64_t)(qo_begin + q_pos) * q_st + (int64_t)(h * g + q_hg) * q_sh + grp * 8;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      qb[ks] = q_ok ? *reinterpret_cast<const u32x4*>(qp + ks * 32) : u32x4{0u, 0u, 0u, 0u};
  }

  // O^T tiles: tile 2a holds dims 32a + 2*(4*grp + i), tile 2a+1 the next dim; column lr
  f32x4 acc[2 * NPAIR];
#pragma unroll
  for (int nt = 0; nt < 2 * NPAIR; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;  // this query's online-softmax state (log2 domain)

  // kv tiles this item needs: up to the largest causal limit among its rows
  const int last_row = min(row0 + kRows, n_rows) - 1;
  const int max_pos = min(causal ? kv_len - qo_len + last_row / g : kv_len - 1, kv_len - 1);
  const int n_tiles = uniform(max_pos < 0 ? 0 : max_pos / KT + 1);

  u32x4 kr[PER], vr[PER];
  if (n_tiles > 0)
    load_tile<T, D, ALIGNED>(kc, vc, ind, 0, kv_len, page_size, num_pages, page_stride, token_stride, head_off, kr, vr);

  for (int tile = 0; tile < n_tiles; ++tile) {
    // ---- registers -> LDS, then start the next tile's loads
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = threadIdx.x + j * kThreads;
      const int tok = c / CH, ch = c % CH;
      *reinterpret_cast<u32x4*>(&s_k[tok * KP + ch * 8]) = kr[j];
      *reinterpret_cast<u32x4*>(&s_v[tok * VPW + ch * 4]) = vr[j];
    }
    __syncthreads();
    if (tile + 1 < n_tiles)
      load_tile<T, D, ALIGNED>(kc, vc, ind, tile + 1, kv_len, page_size, num_pages, page_stride, token_stride, head_off, kr,
                      vr);

    // ---- S^T for NB 16-token blocks: lane holds tokens blk*16 + 4*grp + i of query lr
    f32x4 s[NB];
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      s[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(&s_k[(blk * 16 + lr) * KP + ks * 32 + grp * 8]);
        s[blk] = mfma32<T>(ka, qb[ks], s[blk]);
      }
    }
    // ---- mask, online softmax: reduce over the lane's tokens, then the column's 4 lanes
    float mx = -INFINITY;
    const int t0 = tile * KT + 4 * grp;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = t0 + blk * 16 + i <= lim ? s[blk][i] * scale_log2 : -INFINITY;
        s[blk][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    float ps = 0.f;
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = fast_exp2(s[blk][i] - m_use);
        s[blk][i] = e;
        ps += e;
      }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    l = l * alpha + ps;
    // Rescale the accumulators only when some query's running max rose in
    // this tile (alpha is exactly 1 everywhere else); after the first tiles
    // that is the exception, and the rescale is 32 multiplies plus the moves
    // of the accumulators between register files.
    const bool rose = m_new > m;
    m = m_new;
    if (__builtin_amdgcn_ballot_w64(rose) != 0) {
#pragma unroll
      for (int nt = 0; nt < 2 * NPAIR; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[nt][i] *= alpha;
    }

    // ---- O^T += V^T P^T per 32-token chunk
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
      // P^T as the B operand: k = 8*grp + e <-> tokens of blocks 2kc (e < 4) and 2kc+1 (e >= 4)
      u32x4 pbv[NPP];
      {
        const f32x4 a0 = s[2 * kc], a1 = s[2 * kc + 1];
        const float pv[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hw[e] = pack_p<T>(pv[2 * e], pv[2 * e + 1]);
          if constexpr (NPP == 2) {
            float h0, h1;
            unpack2<T>(hw[e], h0, h1);
            lw[e] = pack_p<T>(pv[2 * e] - h0, pv[2 * e + 1] - h1);
          }
        }
        pbv[0] = u32x4{hw[0], hw[1], hw[2], hw[3]};
        if constexpr (NPP == 2) pbv[NPP - 1] = u32x4{lw[0], lw[1], lw[2], lw[3]};
      }
      // V^T as the A operand: row lr = dims 32a + 2lr (lo) / +1 (hi), the same 8 tokens
      int trow[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) trow[e] = (kc * 32 + (e < 4 ? 4 * grp + e : 16 + 4 * grp + e - 4)) * VPW;
#pragma unroll
      for (int a = 0; a < NPAIR; ++a) {
        uint32_t w[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = s_v[trow[e] + 16 * a + lr];
        u32x4 a_lo, a_hi;
        a_lo.x = __builtin_amdgcn_perm(w[1], w[0], 0x05040100u);
        a_hi.x = __builtin_amdgcn_perm(w[1], w[0], 0x07060302u);
        a_lo.y = __builtin_amdgcn_perm(w[3], w[2], 0x05040100u);
        a_hi.y = __builtin_amdgcn_perm(w[3], w[2], 0x07060302u);
        a_lo.z = __builtin_amdgcn_perm(w[5], w[4], 0x05040100u);
        a_hi.z = __builtin_amdgcn_perm(w[5], w[4], 0x07060302u);
        a_lo.w = __builtin_amdgcn_perm(w[7], w[6], 0x05040100u);
        a_hi.w = __builtin_amdgcn_perm(w[7], w[6], 0x07060302u);
#pragma unroll
        for (int pl = 0; pl < NPP; ++pl) {
          acc[2 * a] = mfma32<T>(a_lo, pbv[pl], acc[2 * a]);
          acc[2 * a + 1] = mfma32<T>(a_hi, pbv[pl], acc[2 * a + 1]);
        }
      }
    }
    __syncthreads();  // the next tile overwrites s_k / s_v
  }

  // ---- write: query lr, dims 32a + 8*grp + 2i and +1 as one 32-bit store
  if (q_ok) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    T* op = o + (int64_t)(qo_begin + q_pos) * o_st + (int64_t)(h * g + q_hg) * o_sh + 8 * grp;
#pragma unroll
    for (int a = 0; a < NPAIR; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<uint32_t*>(op + 32 * a + 2 * i) = pack2<T>(acc[2 * a][i] * inv, acc[2 * a + 1][i] * inv);
  }
}

template <typename T, int D>
int launch(dim3 grid, hipStream_t s, const void* q, int64_t q_st, int64_t q_sh, const void* kc, const void* vc,
           int64_t ps_, int64_t ts, int64_t hs, int64_t np, const int32_t* qo, const int32_t* kvi,
           const int32_t* ind, const int32_t* last, const int2* items, int n_items, void* o, int64_t o_st,
           int64_t o_sh, int batch, int hq, int hkv, int page_size, int causal, float sl2) {
  // pages a whole number of token rows per load pass: scalar page addressing
  const bool aligned = page_size % (kThreads / Cfg<D>::CH) == 0;
  auto kern = aligned ? prefill_kernel<T, D, true> : prefill_kernel<T, D, false>;
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, s, (const T*)q, q_st, q_sh, (const T*)kc,
                     (const T*)vc, ps_, ts, hs, np, qo, kvi, ind, last, items, n_items, (T*)o, o_st, o_sh, batch,
                     hq, hkv, page_size, causal, sl2);
  PL_LAUNCH_CHECK("prefill_kernel");
  return ok();
}

}  // namespace prefill
}  // namespace pl

using namespace pl;
using namespace pl::prefill;

extern "C" int pl_prefill_plan(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                               const int32_t* kv_last_page_len_h, int batch, int num_qo_heads, int num_kv_heads,
                               int page_size, int causal, int32_t* items_h, int max_items, int* num_items_h) {
  if (!num_items_h) return fail(PL_ERR_INVALID, "num_items_h must not be null");
  *num_items_h = 0;
  if (batch < 0) return fail(PL_ERR_INVALID, "batch must be >= 0");
  if (batch > 0 && (!qo_indptr_h || !kv_indptr_h || !kv_last_page_len_h))
    return fail(PL_ERR_INVALID, "null table pointer");
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads)
    return fail(PL_ERR_INVALID, "num_qo_heads (%d) must be a multiple of num_kv_heads (%d)", num_qo_heads,
                num_kv_heads);
  if (page_size <= 0) return fail(PL_ERR_INVALID, "page_size must be > 0");
  const int g = num_qo_heads / num_kv_heads;
  if (batch > 0 && (qo_indptr_h[0] != 0 || kv_indptr_h[0] != 0))
    return fail(PL_ERR_INVALID, "qo_indptr_h[0] and kv_indptr_h[0] must be 0");
  struct Entry {
    int64_t work;
    int32_t r, row0;
  };
  std::vector<Entry> list;
  for (int r = 0; r < batch; ++r) {
    const int qo_len = qo_indptr_h[r + 1] - qo_indptr_h[r];
    const int pages = kv_indptr_h[r + 1] - kv_indptr_h[r];
    if (qo_len < 0) return fail(PL_ERR_INVALID, "qo_indptr_h must be non-decreasing (row %d)", r);
    if (pages < 0) return fail(PL_ERR_INVALID, "kv_indptr_h must be non-decreasing (row %d)", r);
    const int last = kv_last_page_len_h[r];
    if (pages > 0 && (last < 1 || last > page_size))
      return fail(PL_ERR_INVALID, "last_page_len[%d] = %d outside [1, %d]", r, last, page_size);
    const int64_t kv_len = pages > 0 ? (int64_t)(pages - 1) * page_size + last : 0;
    if (kv_len > INT32_MAX / 2) return fail(PL_ERR_INVALID, "row %d: kv_len %lld too large", r, (long long)kv_len);
    if (causal && qo_len > kv_len)
      return fail(PL_ERR_INVALID, "row %d: qo_len %d exceeds kv_len %lld under the causal mask", r, qo_len,
                  (long long)kv_len);
    if (qo_len > 0 && kv_len == 0) return fail(PL_ERR_INVALID, "row %d has queries but no kv", r);
    const int64_t rows = (int64_t)qo_len * g;
    if (rows > INT32_MAX / 2) return fail(PL_ERR_INVALID, "row %d: %lld query rows too many", r, (long long)rows);
    for (int64_t r0 = 0; r0 < rows; r0 += kRows) {
      const int64_t last_row = std::min<int64_t>(r0 + kRows, rows) - 1;
      const int64_t max_pos = causal ? kv_len - qo_len + last_row / g : kv_len - 1;
      list.push_back(Entry{max_pos / kPlanTile + 1, r, (int32_t)r0});
    }
  }
  if (list.size() > (size_t)INT32_MAX / 2) return fail(PL_ERR_INVALID, "too many prefill work items");
  // longest first, so the causal tail of a long prompt does not finish last
  std::stable_sort(list.begin(), list.end(), [](const Entry& a, const Entry& b) { return a.work > b.work; });
  *num_items_h = (int)list.size();
  if (items_h == nullptr) return ok();
  if ((int)list.size() > max_items)
    return fail(PL_ERR_WORKSPACE, "%zu prefill work items exceed the %d provided", list.size(), max_items);
  for (size_t i = 0; i < list.size(); ++i) {
    items_h[2 * i] = list[i].r;
    items_h[2 * i + 1] = list[i].row0;
  }
  return ok();
}

extern "C" int pl_prefill_run(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                              const void* v_cache, int64_t page_stride, int64_t token_stride, int64_t head_stride,
                              int64_t num_pages, const int32_t* qo_indptr, const int32_t* kv_indptr,
                              const int32_t* kv_indices, const int32_t* kv_last_page_len, const int32_t* items,
                              int num_items, void* o, int64_t o_stride_t, int64_t o_stride_h, int batch,
                              int num_qo_heads, int num_kv_heads, int head_dim, int page_size, int causal,
                              float sm_scale, int dtype, void* stream) {
  if (num_items < 0 || batch < 0) return fail(PL_ERR_INVALID, "num_items and batch must be >= 0");
  if (num_items == 0 || batch == 0) return ok();
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads)
    return fail(PL_ERR_INVALID, "num_qo_heads (%d) must be a multiple of num_kv_heads (%d)", num_qo_heads,
                num_kv_heads);
  if (page_size <= 0 || num_pages <= 0) return fail(PL_ERR_INVALID, "page_size and num_pages must be > 0");
  if (!q || !k_cache || !v_cache || !qo_indptr || !kv_indptr || !kv_indices || !kv_last_page_len || !items || !o)
    return fail(PL_ERR_INVALID, "null pointer argument");
  const int64_t strides[] = {q_stride_t, q_stride_h, o_stride_t, o_stride_h, page_stride, token_stride, head_stride};
  for (int64_t st : strides)
    if (st % 8) return fail(PL_ERR_INVALID, "strides must be multiples of 8 elements");
  const void* ptrs[] = {q, k_cache, v_cache, o};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return fail(PL_ERR_INVALID, "q, o and the caches must be 16-byte aligned");
  if (num_kv_heads > 65535) return fail(PL_ERR_INVALID, "num_kv_heads %d exceeds the grid limit", num_kv_heads);
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "prefill dtype must be F16 or BF16 (got %d)", dtype);
  const dim3 grid(num_items, num_kv_heads);
  hipStream_t s = (hipStream_t)stream;
  const float sl2 = sm_scale * 1.44269504088896340736f;
  const int2* it = reinterpret_cast<const int2*>(items);
  const bool bf = dtype == PL_DTYPE_BF16;
#define PL_PREFILL_ARGS                                                                                            \
  grid, s, q, q_stride_t, q_stride_h, k_cache, v_cache, page_stride, token_stride, head_stride, num_pages,         \
      qo_indptr, kv_indptr, kv_indices, kv_last_page_len, it, num_items, o, o_stride_t, o_stride_h, batch,        \
      num_qo_heads, num_kv_heads, page_size, causal, sl2
  switch (head_dim) {
    case 64: return bf ? launch<bf16_t, 64>(PL_PREFILL_ARGS) : launch<f16_t, 64>(PL_PREFILL_ARGS);
    case 128: return bf ? launch<bf16_t, 128>(PL_PREFILL_ARGS) : launch<f16_t, 128>(PL_PREFILL_ARGS);
    case 256: return bf ? launch<bf16_t, 256>(PL_PREFILL_ARGS) : launch<f16_t, 256>(PL_PREFILL_ARGS);
  }
#undef PL_PREFILL_ARGS
  return fail(PL_ERR_UNSUPPORTED, "prefill head_dim %d not built (64, 128, 256)", head_dim);
}
