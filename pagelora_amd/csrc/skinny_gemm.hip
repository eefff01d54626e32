// Decode-sized GEMM on pre-shuffled weights (gfx950):  out = x . W^T (+ bias)
// for few tokens (T <= 64) with W [N, K] streamed once from HBM.
//
// Weight layout.  MFMA 16x16x32's B operand gives lane l the 8 k-values
// (l / 16) * 8 .. +8 of column l % 16, so a wave reading a row-major W
// touches 16 rows x 64 bytes per instruction.  pl_weight_shuffle stores W
// once, at load time, as 1 KiB blocks in exactly that lane order:
//   block (nb, ks) = rows nb*16 .. +16, k = ks*32 .. +32;
//   element e of lane l at  ((nb * K/32 + ks) * 64 + l) * 8 + e
//                        =  W[nb*16 + l%16][ks*32 + (l/16)*8 + e]
// (rows past N are zero).  Every wave load is then one contiguous,
// fully coalesced 1 KiB read that lands directly in MFMA registers; a
// wave's k-range of a row block is contiguous in memory.
//
// shuffled_gemm_kernel  one workgroup of 16 waves per 16 output columns
//                       (x one 16-token tile); the waves split K, each
//                       streams its contiguous run of blocks four at a time
//                       (non-temporal loads) against x rows read from L2,
//                       and the 16 partial tiles are summed through LDS.
//                       Eight at a time measured slower at every decode
//                       shape (74 VGPRs: one workgroup per CU instead of two).
//
// Reference: the base F.linear of project_qkv_packed / project_gate_up_packed
// / project_linear (model/flashinfer/packed_ops.py:143, 179, 251-265) and
// LoRALinear.forward (multilora/linear.py:226-231) at decode batch sizes.
#include <algorithm>
#include <type_traits>

#include "lora_up.h"
#include "pl_common.h"

namespace pl {
namespace sgemm {

constexpr int kWave = 64;
constexpr int kWaves = 16;
constexpr int kThreads = kWave * kWaves;
constexpr int kUnroll = 4;
constexpr int kBlockElems = 512;  // 16 rows x 32 k

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T> __device__ __forceinline__ f32x4 mfma32(u32x4 a, u32x4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma32<bf16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma32<f16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

// The cross-wave sum of one cell of a workgroup's 16-token x 16-column tile
// (s_red[wave][token * 16 + column]): lane l of wave w takes token
// 4 * w + l / 16 and column l % 16, so at most four waves work and at four
// tokens one wave finishes the tile in one pass (one wave looping over the
// cells measured 0.4-0.5 us slower per launch at 4 tokens).  Lanes past the
// tile's nt tokens sum token 0's cell and return false.
__device__ __forceinline__ bool tile_cell_sum(const float (*s_red)[256], int wave, int lane, int nt, int& tl,
                                              float& sum) {
  tl = wave * 4 + lane / 16;
  const bool live = tl < nt;
  const int cell = (live ? tl : 0) * 16 + lane % 16;
  sum = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) sum += s_red[w][cell];
  return live;
}

// One thread per 16-byte piece of the shuffled buffer (N_pad x K elements).
__global__ void shuffle_kernel(const uint16_t* __restrict__ W, int64_t ldw, int N, int K, uint16_t* __restrict__ Ws,
                               int64_t pieces) {
  const int ksteps = K / 32;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t blk = i / 64;
    const int l = (int)(i % 64);
    const int ks = (int)(blk % ksteps);
    const int64_t n = (blk / ksteps) * 16 + l % 16;
    const int k = ks * 32 + (l / 16) * 8;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (n < N) v = *reinterpret_cast<const uint4*>(W + n * ldw + k);
    *reinterpret_cast<uint4*>(Ws + i * 8) = v;
  }
}

// The inverse of shuffle_kernel: one thread per 16-byte piece, rows < N
// written back to the row-major W (row stride ldw).
__global__ void unshuffle_kernel(const uint16_t* __restrict__ Ws, int N, int K, uint16_t* __restrict__ W,
                                 int64_t ldw, int64_t pieces) {
  const int ksteps = K / 32;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t blk = i / 64;
    const int l = (int)(i % 64);
    const int ks = (int)(blk % ksteps);
    const int64_t n = (blk / ksteps) * 16 + l % 16;
    const int k = ks * 32 + (l / 16) * 8;
    if (n < N) *reinterpret_cast<uint4*>(W + n * ldw + k) = *reinterpret_cast<const uint4*>(Ws + i * 8);
  }
}

// PARTIAL: split-K over gridDim.z workgroups per row block; workgroup z sums
// k-steps [z*K/32/splits, ..) and writes its fp32 tile to plane z of
// `partial` (row t at t * ldp, planes plane_stride apart) instead of `out`.
// SIDE: row blocks below main_tiles are computed whole into `out`; the
// blocks from main_tiles on (the LoRA A rows stacked under W) are split-K
// over side_splits small workgroups each, appended to the grid, into fp32
// planes of `partial` (column n - 16 * main_tiles).  A row-block count that
// is a multiple of the CU count then stays one: one more whole block costs a
// CU two blocks' time (o_proj, 4 tokens: 4096 rows 7.6 us, 4112 rows 10.1).
template <typename T, bool PARTIAL, bool SIDE = false>
__global__ __launch_bounds__(kThreads) void shuffled_gemm_kernel(const T* __restrict__ x, int64_t ldx, int tokens,
                                                                 int K, const T* __restrict__ Ws, int N,
                                                                 const T* __restrict__ bias, T* __restrict__ out,
                                                                 int64_t ldo, float* __restrict__ partial,
                                                                 int64_t ldp, int64_t plane_stride,
                                                                 int main_tiles = 0, int side_splits = 1) {
  __shared__ float s_red[kWaves][256];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int lr = lane % 16, kq = (lane / 16) * 8;
  const bool side = SIDE && (int)blockIdx.x >= main_tiles;
  const int se_idx = (int)blockIdx.x - main_tiles;
  const int nb = side ? main_tiles + se_idx / side_splits : (int)blockIdx.x, t0 = blockIdx.y * 16;
  const int zs = SIDE ? (side ? se_idx % side_splits : 0) : (int)blockIdx.z;
  const int nz = SIDE ? (side ? side_splits : 1) : (int)gridDim.z;
  const int t = t0 + lr;
  const bool t_ok = t < tokens;
  const int ksteps = K / 32;
  const int chunk = (ksteps + nz - 1) / nz;
  const int kb0 = min(ksteps, zs * chunk), ke0 = min(ksteps, kb0 + chunk);
  const int per = (ke0 - kb0 + kWaves - 1) / kWaves;
  const int sb = min(ke0, kb0 + wave * per), se = min(ke0, sb + per);
  const u32x4* wb = reinterpret_cast<const u32x4*>(Ws + (int64_t)nb * ksteps * kBlockElems) + lane;
  const T* xr = x + (int64_t)(t_ok ? t : 0) * ldx + kq;

  // A rows of tokens >= `tokens` read token 0's row (xr is clamped): row i of
  // the MFMA result depends only on row i of A, and those rows are never
  // written, so the loads need no condition (a condition here becomes a
  // branch around each load, and a wait before the next batch).
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int s = sb;
  for (; s + kUnroll <= se; s += kUnroll) {
    u32x4 b[kUnroll], a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) b[u] = __builtin_nontemporal_load(wb + (s + u) * kWave);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = *reinterpret_cast<const u32x4*>(xr + (s + u) * 32);
    // all of a batch's loads before its first MFMA (measured: lm_head at 4
    // tokens 180.9 -> 175.6 us, down_proj split 3 20.0 -> 19.7 us)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc = mfma32<T>(a[u], b[u], acc);
  }
  for (; s < se; ++s) {
    const u32x4 b = __builtin_nontemporal_load(wb + s * kWave);
    const u32x4 a = *reinterpret_cast<const u32x4*>(xr + s * 32);
    acc = mfma32<T>(a, b, acc);
  }
  // D: rows = tokens 4*(lane/16)+i of the tile, column = lr
#pragma unroll
  for (int i = 0; i < 4; ++i) s_red[wave][((lane / 16) * 4 + i) * 16 + lr] = acc[i];
  __syncthreads();
  const int nt = min(16, tokens - t0);
  if (wave * 4 >= nt) return;
  const int n = nb * 16 + lr;
  const float bv = (!PARTIAL && !side && bias != nullptr && n < N) ? to_float<T>(bias[n]) : 0.f;
  int tl;
  float sum;
  if (tile_cell_sum(s_red, wave, lane, nt, tl, sum) && n < N) {
    const int tr = t0 + tl;
    if (PARTIAL)
      partial[(int64_t)blockIdx.z * plane_stride + (int64_t)tr * ldp + n] = sum;
    else if (side)
      partial[(int64_t)zs * plane_stride + (int64_t)tr * ldp + (n - main_tiles * 16)] = sum;
    else
      out[(int64_t)tr * ldo + n] = from_float<T>(sum + bv);
  }
}

// ------------------------------------------------------- norm prologue ---
// out = RMSNorm(x) . W^T: the workgroup normalizes the rows of its token
// tile into LDS (x * rsqrt(mean(x^2) + eps) * w rounded to T, as
// rmsnorm_kernel forms it), with its waves' first batch of weight blocks
// already in flight, and the waves then take their MFMA A operands from LDS.
// PPT: 16-byte pieces of the tile's rows per thread (the tile's rows are
// K / 8 * nt pieces, a multiple of 64 per row: K % 512 == 0).  The LDS rows
// are kNormRowPad elements longer than K, so the rows of a lane group's
// tokens start 64 bytes apart in the banks; after the main loop the same
// LDS holds the cross-wave partial tiles.
constexpr int kNormMaxPieces = 4;    // per thread
constexpr int kNormRowPad = 32;      // elements
constexpr int kNormMaxTokens = 8;
constexpr int kRedBytes = kWaves * 256 * 4;

// the tile's rows (padded), then the norm weight; the partial tiles of the
// cross-wave sum reuse the space after the main loop
__host__ __device__ constexpr int norm_lds_bytes(int nt, int K) {
  return nt * (K + kNormRowPad) * 2 + K * 2 > kRedBytes ? nt * (K + kNormRowPad) * 2 + K * 2 : kRedBytes;
}

// HOLD: the rows stay in registers across the first barrier (no LDS copy of
// the raw rows) and only the first batch of weights is preloaded: faster
// for a grid that fits the chip at once (q/k/v at 4 tokens: 12.7 vs 13.5
// us), where a second preloaded batch costs registers that the raw-row LDS
// copy makes room for; a grid of several rounds (gate/up) overlaps the
// prologue with other workgroups' streams and keeps the two-batch preload
// (34.1 vs 35.6 us).
// j / d for 0 <= j < 2^14 through the reciprocal r of d (1 ulp): (j + 1/2) / d
// lies 1 / (2d) or more from an integer, and the product's error, a few ulp
// of a value below 2^14 / d, is far below that, so truncation gives the
// quotient exactly.  Saves the integer division's ~30 instructions per use.
__device__ __forceinline__ int piece_row(int j, float r) { return (int)(((float)j + 0.5f) * r); }

template <typename T, int PPT, bool HOLD>
__global__ __launch_bounds__(kThreads) void shuffled_gemm_norm_kernel(
    const T* __restrict__ x, int64_t ldx, int tokens, int K, const T* __restrict__ nw, float eps,
    const T* __restrict__ Ws, int N, T* __restrict__ out, int64_t ldo, T* __restrict__ xn_out, int64_t ldxn) {
  extern __shared__ __align__(16) unsigned char s_dyn[];
  __shared__ float s_ss[kThreads * PPT / kWave];  // one sum per 64-piece slice of a row
  T* xs = reinterpret_cast<T*>(s_dyn);
  float (*s_red)[256] = reinterpret_cast<float (*)[256]>(s_dyn);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int lr = lane % 16, kq = (lane / 16) * 8;
  const int nb = blockIdx.x, t0 = blockIdx.y * 16;
  const int nt = min(16, tokens - t0);
  const int ksteps = K / 32;
  const int per = (ksteps + kWaves - 1) / kWaves;
  const int sb = min(ksteps, wave * per), se = min(ksteps, sb + per);
  const u32x4* wb = reinterpret_cast<const u32x4*>(Ws + (int64_t)nb * ksteps * kBlockElems) + lane;
  const int Kp = K + kNormRowPad;

  // the tile's rows, PPT pieces per thread (pieces past the tile re-read
  // piece 0), and the norm weight go to LDS as they are; the sums of squares
  // come from the same registers (a wave's 64 pieces of pass c are one slice
  // of one row), so no row value stays in a register across the barrier
  const int rp = K / 8, pieces = nt * rp;
  const float rrp = __builtin_amdgcn_rcpf((float)rp);
  uint4* sw8 = reinterpret_cast<uint4*>(xs + nt * Kp);  // the norm weight, K / 8 pieces
  uint4 hv[PPT];
#pragma unroll
  for (int c = 0; c < PPT; ++c) {
    const int j = threadIdx.x + c * kThreads;
    const int jj = j < pieces ? j : 0;
    const int tt = piece_row(jj, rrp), cc = jj - tt * rp;
    hv[c] = *reinterpret_cast<const uint4*>(x + (int64_t)(t0 + tt) * ldx + cc * 8);
  }
  const int wc = threadIdx.x < rp ? threadIdx.x : 0;
  const uint4 wv = *reinterpret_cast<const uint4*>(nw + wc * 8);
  // Then the wave's first two batches of weight blocks (its whole k-range at
  // K = 4096), in flight while the rows are normalized.  After the rows:
  // loads complete in order, so the rows' wait does not wait for these.
  __builtin_amdgcn_sched_barrier(0);
  u32x4 b[kUnroll], b1[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) b[u] = __builtin_nontemporal_load(wb + min(sb + u, ksteps - 1) * kWave);
  if constexpr (!HOLD) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      b1[u] = __builtin_nontemporal_load(wb + min(sb + kUnroll + u, ksteps - 1) * kWave);
  }
  __builtin_amdgcn_sched_barrier(0);
  // unconditional (threads past the K / 8 pieces rewrite piece 0 with its
  // own value): a store under a test drags its load below the weights'
  sw8[wc] = wv;  // rp <= kThreads: K <= 8192
#pragma unroll
  for (int c = 0; c < PPT; ++c) {
    const int j = threadIdx.x + c * kThreads;
    if (!HOLD && j < pieces) {
      const int tt = piece_row(j, rrp), cc = j - tt * rp;
      *reinterpret_cast<uint4*>(xs + tt * Kp + cc * 8) = hv[c];
    }
    float f[8];
    unpack2<T>(hv[c].x, f[0], f[1]);
    unpack2<T>(hv[c].y, f[2], f[3]);
    unpack2<T>(hv[c].z, f[4], f[5]);
    unpack2<T>(hv[c].w, f[6], f[7]);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(f[i], f[i], ss);
    ss = wave_sum(ss);
    if (lane == 0) s_ss[wave + c * kWaves] = ss;
  }
  __syncthreads();
  const int slices = rp / kWave;  // per row
  auto normalize_piece = [&](int c, const uint4& held) {
    const int j = threadIdx.x + c * kThreads;
    if (j < pieces) {
      const int tt = piece_row(j, rrp), cc = j - tt * rp;
      float tot = 0.f;
      for (int s = 0; s < slices; ++s) tot += s_ss[tt * slices + s];
      const float rstd = rsqrtf(tot / (float)K + eps);
      const uint4 hw = HOLD ? held : *reinterpret_cast<const uint4*>(xs + tt * Kp + cc * 8), ww = sw8[cc];
      auto norm2 = [&](uint32_t h2, uint32_t w2) {
        float f0, f1, w0, w1;
        unpack2<T>(h2, f0, f1);
        unpack2<T>(w2, w0, w1);
        return pack2_hw<T>(f0 * rstd * w0, f1 * rstd * w1);
      };
      const uint4 o = make_uint4(norm2(hw.x, ww.x), norm2(hw.y, ww.y), norm2(hw.z, ww.z), norm2(hw.w, ww.w));
      *reinterpret_cast<uint4*>(xs + tt * Kp + cc * 8) = o;
      if (xn_out != nullptr && blockIdx.x == 0)
        *reinterpret_cast<uint4*>(xn_out + (int64_t)(t0 + tt) * ldxn + cc * 8) = o;
    }
  };
  if constexpr (HOLD) {
    // the held rows: unrolled, so they stay in registers (a loop index into
    // them would place them in scratch memory)
#pragma unroll
    for (int c = 0; c < PPT; ++c) normalize_piece(c, hv[c]);
  } else {
    // one piece at a time: the weight batches are live here, and two
    // pieces' temporaries at once would raise the kernel's register count
#pragma unroll 1
    for (int c = 0; c < PPT; ++c) normalize_piece(c, hv[0]);
  }
  __syncthreads();

  // Lanes of tokens past the tile read token 0's row (their MFMA rows are
  // never written).
  const T* xr = xs + (lr < nt ? lr : 0) * Kp + kq;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int s = sb;
  if (s + kUnroll <= se) {
    u32x4 a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = *reinterpret_cast<const u32x4*>(xr + (s + u) * 32);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc = mfma32<T>(a[u], b[u], acc);
    s += kUnroll;
    if (!HOLD && s + kUnroll <= se) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) a[u] = *reinterpret_cast<const u32x4*>(xr + (s + u) * 32);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc = mfma32<T>(a[u], b1[u], acc);
      s += kUnroll;
    }
  }
  for (; s + kUnroll <= se; s += kUnroll) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) b[u] = __builtin_nontemporal_load(wb + (s + u) * kWave);
    u32x4 a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = *reinterpret_cast<const u32x4*>(xr + (s + u) * 32);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc = mfma32<T>(a[u], b[u], acc);
  }
  for (; s < se; ++s) {
    const u32x4 bb = __builtin_nontemporal_load(wb + s * kWave);
    const u32x4 a = *reinterpret_cast<const u32x4*>(xr + s * 32);
    acc = mfma32<T>(a, bb, acc);
  }
  __syncthreads();  // every wave is done with the rows before the tiles reuse the LDS
#pragma unroll
  for (int i = 0; i < 4; ++i) s_red[wave][((lane / 16) * 4 + i) * 16 + lr] = acc[i];
  __syncthreads();
  if (wave * 4 >= nt) return;
  const int n = nb * 16 + lr;
  int tl;
  float sum;
  if (tile_cell_sum(s_red, wave, lane, nt, tl, sum) && n < N) out[(int64_t)(t0 + tl) * ldo + n] = from_float<T>(sum);
}

// ------------------------------------ norm from the producer's squares ---
// out = RMSNorm(x) . W^T where the kernel that wrote x also wrote its sums
// of squares in pieces, sq[t * ldsq + j] for j < parts
// (pl_linear_shuffled_add's sq_out): wave t of the workgroup adds token t's
// pieces in a fixed order (QPL float4 per lane, then the wave's DPP tree),
// so no row goes through LDS and one barrier separates the loads from the
// main loop.  The MFMA A operands are the rows read from global memory as
// in shuffled_gemm_kernel, normalized in registers as rmsnorm_kernel forms
// them, (x * rstd) * w rounded to T, with w from an LDS copy.
template <typename T, int QPL, bool XN>
__global__ __launch_bounds__(kThreads) void shuffled_gemm_normsq_kernel(
    const T* __restrict__ x, int64_t ldx, int tokens, int K, const T* __restrict__ nw, float eps,
    const float* __restrict__ sq, int64_t ldsq, int parts, const T* __restrict__ Ws, int N, T* __restrict__ out,
    int64_t ldo, T* __restrict__ xn_out, int64_t ldxn) {
  __shared__ float s_red[kWaves][256];
  __shared__ uint4 s_w[8192 / 8];  // the norm weight, K / 8 pieces (K <= 8192)
  __shared__ float s_rstd[16];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int lr = lane % 16, kq = (lane / 16) * 8;
  const int nb = blockIdx.x, t0 = blockIdx.y * 16;
  const int nt = min(16, tokens - t0);
  const int ksteps = K / 32;
  const int per = (ksteps + kWaves - 1) / kWaves;
  const int sb = min(ksteps, wave * per), se = min(ksteps, sb + per);
  const u32x4* wb = reinterpret_cast<const u32x4*>(Ws + (int64_t)nb * ksteps * kBlockElems) + lane;
  const int tok = lr < nt ? lr : 0;
  const T* xr = x + (int64_t)(t0 + tok) * ldx + kq;

  // the loads the barrier waits for first (they complete in order): wave w <
  // nt takes token w's pieces (pieces past `parts` re-read piece 0 and are
  // masked), every thread one piece of the norm weight (threads past K / 8
  // re-read piece 0 and rewrite it with its own value)
  const int tw = wave < nt ? wave : 0;
  float4 qv[QPL];
#pragma unroll
  for (int c = 0; c < QPL; ++c) {
    const int j = (lane + c * kWave) * 4;
    qv[c] = *reinterpret_cast<const float4*>(sq + (int64_t)(t0 + tw) * ldsq + (j < parts ? j : 0));
  }
  const int wc = (int)threadIdx.x < K / 8 ? (int)threadIdx.x : 0;
  const uint4 wv = *reinterpret_cast<const uint4*>(nw + wc * 8);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 b[kUnroll], a[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int s = min(sb + u, ksteps - 1);
    b[u] = __builtin_nontemporal_load(wb + s * kWave);
    a[u] = *reinterpret_cast<const u32x4*>(xr + s * 32);
  }
  __builtin_amdgcn_sched_barrier(0);
  s_w[wc] = wv;
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < QPL; ++c) {
    const int j = (lane + c * kWave) * 4;
    ss += (j + 0 < parts ? qv[c].x : 0.f) + (j + 1 < parts ? qv[c].y : 0.f) +
          (j + 2 < parts ? qv[c].z : 0.f) + (j + 3 < parts ? qv[c].w : 0.f);
  }
  ss = wave_sum(ss);
  if (lane == 0 && wave < nt) s_rstd[wave] = rsqrtf(ss / (float)K + eps);
  __syncthreads();
  const float rstd = s_rstd[tok];
  [[maybe_unused]] const bool xn_store = XN && blockIdx.x == 0 && lr < nt;
  // x -> (x * rstd) * w rounded to T, in place
  auto normalize = [&](u32x4& v, int s) {
    const uint4 w8 = s_w[(s * 32 + kq) / 8];
    auto n2 = [&](uint32_t h2, uint32_t w2) {
      float f0, f1, w0, w1;
      unpack2<T>(h2, f0, f1);
      unpack2<T>(w2, w0, w1);
      return pack2_hw<T>(f0 * rstd * w0, f1 * rstd * w1);
    };
    v = u32x4{n2(v.x, w8.x), n2(v.y, w8.y), n2(v.z, w8.z), n2(v.w, w8.w)};
    if constexpr (XN)
      if (xn_store) *reinterpret_cast<u32x4*>(xn_out + (int64_t)(t0 + lr) * ldxn + s * 32 + kq) = v;
  };

  // (one operand at a time: the scheduler would otherwise normalize the
  // batch's four operands together and raise the kernel's register count)
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int s = sb;
  if (s + kUnroll <= se) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      normalize(a[u], s + u);
      acc = mfma32<T>(a[u], b[u], acc);
      __builtin_amdgcn_sched_barrier(0);
    }
    s += kUnroll;
  }
  for (; s + kUnroll <= se; s += kUnroll) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) b[u] = __builtin_nontemporal_load(wb + (s + u) * kWave);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = *reinterpret_cast<const u32x4*>(xr + (s + u) * 32);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      normalize(a[u], s + u);
      acc = mfma32<T>(a[u], b[u], acc);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  for (; s < se; ++s) {
    const u32x4 bb = __builtin_nontemporal_load(wb + s * kWave);
    u32x4 aa = *reinterpret_cast<const u32x4*>(xr + s * 32);
    normalize(aa, s);
    acc = mfma32<T>(aa, bb, acc);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) s_red[wave][((lane / 16) * 4 + i) * 16 + lr] = acc[i];
  __syncthreads();
  if (wave * 4 >= nt) return;
  const int n = nb * 16 + lr;
  int tl;
  float sum;
  if (tile_cell_sum(s_red, wave, lane, nt, tl, sum) && n < N) out[(int64_t)(t0 + tl) * ldo + n] = from_float<T>(sum);
}

// --------------------------------------------- residual + LoRA epilogue ---
// residual += round(round(x . W^T) + scale * y . B_a^T) for the first N
// rows of the shuffled weight.  y comes as fp32 partial sums written by the
// producer of x: flat index f = (t * (R/4) + q) * G + p (G = parts rounded up
// to a power of two, p >= parts reading as 0) over the tile's tokens, one
// float4 of ranks 4q .. 4q+3 per f, YPT of them per thread.  They are loaded
// before the weights and summed while the first batch of weight blocks is in
// flight: over min(G, 64) lanes with DPP (group_sum), then the per-wave
// slices of groups wider than a wave in order through LDS.  The epilogue
// gives every (token, column) cell its own lane (tile_cell_sum): one wave
// looping over the tokens cost 1.1 us more per launch at o_proj's and
// down_proj's shapes.
//
// NB > 0: every wave has exactly NB batches of weight blocks (K = 16 * 4 *
// NB * 32) and the grid is at most one workgroup per CU, so a wave may hold
// 128 registers: two batches are kept in flight (the next but one is issued
// after each batch's MFMAs) instead of one.  NB == 0: any K, one batch at a
// time, at most 64 registers.
constexpr int kAddMaxYPT = 4;

template <typename T, int R, int YPT, int NB>
__global__ __launch_bounds__(kThreads) void shuffled_gemm_add_kernel(
    const T* __restrict__ x, int64_t ldx, int tokens, int K, const T* __restrict__ Ws, int N,
    T* __restrict__ res, int64_t ldr, LoraUp lora, const float* __restrict__ yp, int64_t ldyp, int parts, int lg,
    const int32_t* __restrict__ ids, int n_adapters, T* __restrict__ out, int64_t ldo, float* __restrict__ sq_out,
    int64_t ldsq) {
  constexpr int Q = R > 0 ? R / 4 : 1;
  __shared__ float s_red[kWaves][256];
  // (t, q) group x slice: at most YPT * kThreads / kWave entries (G <= 64:
  // one slice per group, nt * Q <= 64 groups; G > 64: nt * Q * G / 64)
  __shared__ float4 s_y[R > 0 ? kAddMaxYPT * kThreads / kWave : 1];
  // the epilogue's inputs: the residual tile (loaded with the partials) and
  // the B pieces of the workgroup's 16 columns (token tl, column c, ranks
  // 8k ..; loaded after the weights' first batches)
  __shared__ float s_res[16 * 16];
  __shared__ uint4 s_b[R > 0 ? 16 * 16 * (R / 8) : 1];
  __shared__ int s_ok[16];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int lr = lane % 16, kq = (lane / 16) * 8;
  const int nb = blockIdx.x, t0 = blockIdx.y * 16;
  const int nt = min(16, tokens - t0);
  const int t = t0 + lr;
  const bool t_ok = t < tokens;
  // NB > 0: K is NB * kWaves * kUnroll k-steps, a constant, and no batch
  // runs past the end (no clamped index: the loads take immediate offsets)
  const int ksteps = NB > 0 ? NB * kWaves * kUnroll : K / 32;
  const int per = NB > 0 ? NB * kUnroll : (ksteps + kWaves - 1) / kWaves;
  const int sb = min(ksteps, wave * per), se = min(ksteps, sb + per);
  const u32x4* wb = reinterpret_cast<const u32x4*>(Ws + (int64_t)nb * ksteps * kBlockElems) + lane;
  const T* xr = x + (int64_t)(t_ok ? t : 0) * ldx + kq;
  const int G = 1 << lg;                  // parts rounded up to a power of two
  const int lgw = lg < 6 ? lg : 6;        // butterfly width 2^lgw lanes
  const int slices = 1 << (lg - lgw);

  // (a partial past `parts` or the tile re-reads partial 0 of token t0 and
  // is masked to zero after the weight loads are issued: a select on the
  // loaded value here would wait for the load first)
  [[maybe_unused]] float4 yv[YPT];
  [[maybe_unused]] bool yon[YPT];
  if constexpr (R > 0) {
#pragma unroll
    for (int c = 0; c < YPT; ++c) {
      const int f = threadIdx.x + c * kThreads;
      const int p = f & (G - 1), tq = f >> lg;
      const int tt = tq / Q, q = tq - tt * Q;
      yon[c] = (p < parts) & (tt < nt);
      const float* src = yp + (int64_t)(t0 + (yon[c] ? tt : 0)) * ldyp + (yon[c] ? p : 0) * R + q * 4;
      yv[c] = *reinterpret_cast<const float4*>(src);
    }
  }
  // residual tile: thread i < nt * 16 reads token i / 16, column i % 16
  // (threads past it re-read the last entry; the stores below are
  // unconditional, so no load waits under a test)
  const int ri = min((int)threadIdx.x, nt * 16 - 1);
  const T rv_ld = res[(int64_t)(t0 + ri / 16) * ldr + min(nb * 16 + ri % 16, N - 1)];
  // The token's adapter id: an unconditional load (a bound adapter reads a
  // dummy word of the weight), so no load sits under a test: a test would
  // make the compiler wait for every load in flight where the paths join,
  // the weights' first batch included.  The B piece it addresses goes out
  // after the weights' first batches, and reaches LDS after the main loop.
  [[maybe_unused]] int id_ld = 0;
  if constexpr (R > 0) {
    constexpr int KB = R / 8;
    const int bi = min((int)threadIdx.x, nt * 16 * KB - 1);
    const int tl = bi / (16 * KB);
    id_ld = *(lora.adapter >= 0 ? reinterpret_cast<const int32_t*>(Ws) : ids + t0 + tl);
  }
  constexpr int NQ = NB > 0 ? NB : 1;
  u32x4 b[NQ][kUnroll], a[NQ][kUnroll];
  // NB > 0: s0 counts from the wave's first k-step, so every load is the
  // wave's base plus a constant offset
  const u32x4* wq = wb + (NB > 0 ? sb : 0) * kWave;
  const T* xq = xr + (NB > 0 ? sb : 0) * 32;
  auto issue = [&](int q, int s0) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = NB > 0 ? s0 + u : min(s0 + u, ksteps - 1);
      b[q][u] = __builtin_nontemporal_load(wq + s * kWave);
      a[q][u] = *reinterpret_cast<const u32x4*>(xq + s * 32);
    }
  };
  issue(0, NB > 0 ? 0 : sb);
  if constexpr (NB > 1) issue(1, kUnroll);
  __builtin_amdgcn_sched_barrier(0);  // every weight and x load of the first batches out first
  s_res[ri] = to_float<T>(rv_ld);
  [[maybe_unused]] uint4 bpc;
  if constexpr (R > 0) {
    constexpr int KB = R / 8;
    const int bi = min((int)threadIdx.x, nt * 16 * KB - 1);
    const int col = (bi / KB) % 16, kb = bi % KB;
    const int a_raw = lora.adapter >= 0 ? lora.adapter : id_ld;
    const int a_ok_ld = (a_raw >= 0) & (a_raw < n_adapters);
    const int nc = min(nb * 16 + col, N - 1);
    bpc = *lora_b_piece<T, R>(lora, a_ok_ld ? a_raw : 0, nc & ~7, nc & 7, kb);
    if (bi % (16 * KB) == 0) s_ok[bi / (16 * KB)] = a_ok_ld;
  }
  if constexpr (R > 0) {
#pragma unroll
    for (int c = 0; c < YPT; ++c) {
      const float m = yon[c] ? 1.f : 0.f;
      float4 v = make_float4(yv[c].x * m, yv[c].y * m, yv[c].z * m, yv[c].w * m);
      v = make_float4(group_sum(v.x, lgw), group_sum(v.y, lgw), group_sum(v.z, lgw), group_sum(v.w, lgw));
      const int f = threadIdx.x + c * kThreads;
      const int p = f & (G - 1), tq = f >> lg;
      if ((p & ((1 << lgw) - 1)) == 0 && tq < nt * Q) s_y[tq * slices + (p >> lgw)] = v;
    }
  }

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (NB > 0) {
    // batch i + 2 reuses batch i's registers once its MFMAs have read them
#pragma unroll
    for (int i = 0; i < NB; ++i) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc = mfma32<T>(a[i][u], b[i][u], acc);
      if (i + 2 < NB) issue(i + 2, (i + 2) * kUnroll);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    int s = sb;
    if (s + kUnroll <= se) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc = mfma32<T>(a[0][u], b[0][u], acc);
      s += kUnroll;
    }
    for (; s + kUnroll <= se; s += kUnroll) {
      issue(0, s);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc = mfma32<T>(a[0][u], b[0][u], acc);
    }
    for (; s < se; ++s) {
      const u32x4 bb = __builtin_nontemporal_load(wb + s * kWave);
      const u32x4 aa = *reinterpret_cast<const u32x4*>(xr + s * 32);
      acc = mfma32<T>(aa, bb, acc);
    }
  }
  if constexpr (R > 0) s_b[min((int)threadIdx.x, nt * 16 * (R / 8) - 1)] = bpc;
#pragma unroll
  for (int i = 0; i < 4; ++i) s_red[wave][((lane / 16) * 4 + i) * 16 + lr] = acc[i];
  __syncthreads();
  if (wave * 4 >= nt) return;
  int tl;
  float sum;
  const bool live = tile_cell_sum(s_red, wave, lane, nt, tl, sum);
  const int tr = t0 + tl, tc = live ? tl : 0;
  const int cell = tc * 16 + lr;
  float xa = through<T>(sum);
  if constexpr (R > 0) {
    // y of the token, 8 ranks per piece: the wave slices in order, rounded to T
    constexpr int KB = R / 8;
    float d = 0.f;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      const int g0 = (tc * KB + k) * 2;  // the two quads of ranks 8k ..
      float4 lo = s_y[g0 * slices], hi = s_y[(g0 + 1) * slices];
#pragma unroll 1
      for (int sl = 1; sl < slices; ++sl) {
        const float4 l2 = s_y[g0 * slices + sl], h2 = s_y[(g0 + 1) * slices + sl];
        lo.x += l2.x; lo.y += l2.y; lo.z += l2.z; lo.w += l2.w;
        hi.x += h2.x; hi.y += h2.y; hi.z += h2.z; hi.w += h2.w;
      }
      const uint4 yr = make_uint4(pack2<T>(lo.x, lo.y), pack2<T>(lo.z, lo.w), pack2<T>(hi.x, hi.y), pack2<T>(hi.z, hi.w));
      d = dot8<T>(yr, s_b[cell * KB + k], d);
    }
    d *= lora.scale;
    xa = through<T>(xa + (s_ok[tc] ? d : -0.f));
  }
  const T v = from_float<T>(s_res[cell] + xa);
  const int n = nb * 16 + lr;
  if (live && n < N) {
    res[(int64_t)tr * ldr + n] = v;
    if (out != nullptr) out[(int64_t)tr * ldo + n] = from_float<T>(sum);
  }
  if (sq_out != nullptr) {
    // the squares of the stored residual over the block's columns (the 16
    // lanes of this token's group), for the next RMSNorm
    const float vf = n < N ? to_float<T>(v) : 0.f;
    const float q = row16_sum(vf * vf);
    if (live && lr == 0) sq_out[(int64_t)tr * ldsq + nb] = q;
  }
}

}  // namespace sgemm
}  // namespace pl

using namespace pl;
using namespace pl::sgemm;

extern "C" size_t pl_weight_shuffled_bytes(int out_features, int in_features) {
  if (out_features <= 0 || in_features <= 0 || in_features % 32) return 0;
  return (size_t)((out_features + 15) / 16) * 16 * in_features * 2;
}

extern "C" int pl_weight_shuffle(const void* weight, int64_t ldw, int out_features, int in_features, void* shuffled,
                                 size_t shuffled_bytes, int dtype, void* stream) {
  if (out_features <= 0 || in_features <= 0 || in_features % 32)
    return fail(PL_ERR_INVALID, "out_features > 0 and in_features a positive multiple of 32 required");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "shuffled weights are F16 or BF16 (got %d)", dtype);
  if (!weight || !shuffled) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldw < in_features || ldw % 8 || (uintptr_t)weight % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "weight rows and the shuffled buffer must be 16-byte aligned");
  const size_t need = pl_weight_shuffled_bytes(out_features, in_features);
  if (shuffled_bytes < need)
    return fail(PL_ERR_WORKSPACE, "shuffled buffer of %zu bytes < %zu needed", shuffled_bytes, need);
  const int64_t pieces = (int64_t)need / 16;
  const int64_t blocks = std::min<int64_t>((pieces + 255) / 256, 65536);
  hipLaunchKernelGGL(shuffle_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)weight, ldw, out_features, in_features, (uint16_t*)shuffled, pieces);
  PL_LAUNCH_CHECK("shuffle_kernel");
  return ok();
}

extern "C" int pl_weight_unshuffle(const void* shuffled, size_t shuffled_bytes, int out_features, int in_features,
                                   void* weight, int64_t ldw, int dtype, void* stream) {
  if (out_features <= 0 || in_features <= 0 || in_features % 32)
    return fail(PL_ERR_INVALID, "out_features > 0 and in_features a positive multiple of 32 required");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "shuffled weights are F16 or BF16 (got %d)", dtype);
  if (!weight || !shuffled) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldw < in_features || ldw % 8 || (uintptr_t)weight % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "weight rows and the shuffled buffer must be 16-byte aligned");
  const size_t need = pl_weight_shuffled_bytes(out_features, in_features);
  if (shuffled_bytes < need)
    return fail(PL_ERR_WORKSPACE, "shuffled buffer of %zu bytes < %zu needed", shuffled_bytes, need);
  const int64_t pieces = (int64_t)need / 16;
  const int64_t blocks = std::min<int64_t>((pieces + 255) / 256, 65536);
  hipLaunchKernelGGL(unshuffle_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)shuffled, out_features, in_features, (uint16_t*)weight, ldw, pieces);
  PL_LAUNCH_CHECK("unshuffle_kernel");
  return ok();
}

extern "C" int pl_linear_shuffled(const void* x, int64_t ldx, int num_tokens, int in_features, const void* shuffled,
                                  int out_features, const void* bias, void* out, int64_t ldo, int dtype,
                                  void* stream) {
  if (num_tokens < 0 || num_tokens > PL_LINEAR_MAX_TOKENS)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", PL_LINEAR_MAX_TOKENS, num_tokens);
  if (num_tokens == 0) return ok();
  if (in_features <= 0 || in_features % 32 || out_features <= 0)
    return fail(PL_ERR_INVALID, "in_features must be a positive multiple of 32 and out_features > 0");
  if (!x || !shuffled || !out) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx < in_features || ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "x rows and the shuffled weight must be 16-byte aligned");
  if (ldo < out_features) return fail(PL_ERR_INVALID, "ldo < out_features");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_linear_shuffled dtype must be F16 or BF16 (got %d)", dtype);
  const dim3 grid((out_features + 15) / 16, (num_tokens + 15) / 16);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PL_DTYPE_BF16)
    hipLaunchKernelGGL((shuffled_gemm_kernel<bf16_t, false>), grid, dim3(kThreads), 0, s, (const bf16_t*)x, ldx,
                       num_tokens, in_features, (const bf16_t*)shuffled, out_features, (const bf16_t*)bias,
                       (bf16_t*)out, ldo, nullptr, 0, 0);
  else
    hipLaunchKernelGGL((shuffled_gemm_kernel<f16_t, false>), grid, dim3(kThreads), 0, s, (const f16_t*)x, ldx,
                       num_tokens, in_features, (const f16_t*)shuffled, out_features, (const f16_t*)bias,
                       (f16_t*)out, ldo, nullptr, 0, 0);
  PL_LAUNCH_CHECK("shuffled_gemm_kernel");
  return ok();
}

extern "C" int pl_linear_shuffled_split(const void* x, int64_t ldx, int num_tokens, int in_features,
                                        const void* shuffled, int out_features, int splits, float* partials,
                                        int64_t ld, int64_t plane_stride, int dtype, void* stream) {
  if (num_tokens < 0 || num_tokens > PL_LINEAR_MAX_TOKENS)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", PL_LINEAR_MAX_TOKENS, num_tokens);
  if (num_tokens == 0) return ok();
  if (in_features <= 0 || in_features % 32 || out_features <= 0)
    return fail(PL_ERR_INVALID, "in_features must be a positive multiple of 32 and out_features > 0");
  if (splits < 1 || splits > 16 || splits > in_features / 32)
    return fail(PL_ERR_INVALID, "splits must be 1..min(16, in_features/32) (got %d)", splits);
  if (!x || !shuffled || !partials) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx < in_features || ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "x rows and the shuffled weight must be 16-byte aligned");
  if (ld < out_features || plane_stride < ld * num_tokens)
    return fail(PL_ERR_INVALID, "partial planes overlap (ld %lld, plane_stride %lld)", (long long)ld,
                (long long)plane_stride);
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_linear_shuffled_split dtype must be F16 or BF16 (got %d)", dtype);
  const dim3 grid((out_features + 15) / 16, (num_tokens + 15) / 16, splits);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PL_DTYPE_BF16)
    hipLaunchKernelGGL((shuffled_gemm_kernel<bf16_t, true>), grid, dim3(kThreads), 0, s, (const bf16_t*)x, ldx,
                       num_tokens, in_features, (const bf16_t*)shuffled, out_features, nullptr, nullptr, 0,
                       partials, ld, plane_stride);
  else
    hipLaunchKernelGGL((shuffled_gemm_kernel<f16_t, true>), grid, dim3(kThreads), 0, s, (const f16_t*)x, ldx,
                       num_tokens, in_features, (const f16_t*)shuffled, out_features, nullptr, nullptr, 0,
                       partials, ld, plane_stride);
  PL_LAUNCH_CHECK("shuffled_gemm_kernel");
  return ok();
}

extern "C" int pl_linear_shuffled_side(const void* x, int64_t ldx, int num_tokens, int in_features,
                                       const void* shuffled, int out_features, int main_features, void* out,
                                       int64_t ldo, int side_splits, float* side_partials, int64_t ld_side,
                                       int64_t side_plane_stride, int dtype, void* stream) {
  if (num_tokens < 0 || num_tokens > PL_LINEAR_MAX_TOKENS)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", PL_LINEAR_MAX_TOKENS, num_tokens);
  if (num_tokens == 0) return ok();
  if (in_features <= 0 || in_features % 32 || out_features <= 0)
    return fail(PL_ERR_INVALID, "in_features must be a positive multiple of 32 and out_features > 0");
  if (main_features <= 0 || main_features % 16 || main_features >= out_features)
    return fail(PL_ERR_INVALID, "main_features must be a positive multiple of 16 below out_features (got %d of %d)",
                main_features, out_features);
  if (side_splits < 1 || side_splits > 64 || side_splits > in_features / 32)
    return fail(PL_ERR_INVALID, "side_splits must be 1..min(64, in_features/32) (got %d)", side_splits);
  if (!x || !shuffled || !out || !side_partials) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx < in_features || ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "x rows and the shuffled weight must be 16-byte aligned");
  if (ldo < main_features) return fail(PL_ERR_INVALID, "ldo < main_features");
  const int side_features = out_features - main_features;
  if (ld_side < side_features || side_plane_stride < ld_side * num_tokens)
    return fail(PL_ERR_INVALID, "side planes overlap (ld %lld, plane_stride %lld)", (long long)ld_side,
                (long long)side_plane_stride);
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_linear_shuffled_side dtype must be F16 or BF16 (got %d)", dtype);
  const int main_tiles = main_features / 16;
  const int side_tiles = (out_features + 15) / 16 - main_tiles;
  const dim3 grid(main_tiles + side_tiles * side_splits, (num_tokens + 15) / 16, 1);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PL_DTYPE_BF16)
    hipLaunchKernelGGL((shuffled_gemm_kernel<bf16_t, false, true>), grid, dim3(kThreads), 0, s, (const bf16_t*)x,
                       ldx, num_tokens, in_features, (const bf16_t*)shuffled, out_features, nullptr, (bf16_t*)out,
                       ldo, side_partials, ld_side, side_plane_stride, main_tiles, side_splits);
  else
    hipLaunchKernelGGL((shuffled_gemm_kernel<f16_t, false, true>), grid, dim3(kThreads), 0, s, (const f16_t*)x,
                       ldx, num_tokens, in_features, (const f16_t*)shuffled, out_features, nullptr, (f16_t*)out,
                       ldo, side_partials, ld_side, side_plane_stride, main_tiles, side_splits);
  PL_LAUNCH_CHECK("shuffled_gemm_kernel");
  return ok();
}

constexpr int kGemmCUs = 256;  // MI355X

template <typename T, int PPT>
static void launch_norm_gemm(const void* x, int64_t ldx, int num_tokens, int K, const void* nw, float eps,
                             const void* Ws, int N, void* out, int64_t ldo, void* xn, int64_t ldxn, hipStream_t s) {
  const int nt = std::min(num_tokens, 16);
  const dim3 grid((N + 15) / 16, (num_tokens + 15) / 16);
  // two workgroups per CU: a grid of at most that many runs in one round
  if ((int64_t)grid.x * grid.y <= 2 * kGemmCUs)
    hipLaunchKernelGGL((shuffled_gemm_norm_kernel<T, PPT, true>), grid, dim3(kThreads), norm_lds_bytes(nt, K), s,
                       (const T*)x, ldx, num_tokens, K, (const T*)nw, eps, (const T*)Ws, N, (T*)out, ldo, (T*)xn, ldxn);
  else
    hipLaunchKernelGGL((shuffled_gemm_norm_kernel<T, PPT, false>), grid, dim3(kThreads), norm_lds_bytes(nt, K), s,
                       (const T*)x, ldx, num_tokens, K, (const T*)nw, eps, (const T*)Ws, N, (T*)out, ldo, (T*)xn, ldxn);
}

template <typename T>
static int norm_gemm_t(const void* x, int64_t ldx, int num_tokens, int K, const void* nw, float eps, const void* Ws,
                       int N, void* out, int64_t ldo, void* xn, int64_t ldxn, hipStream_t s) {
  const int pieces = std::min(num_tokens, 16) * (K / 8);
  if (pieces <= kThreads)
    launch_norm_gemm<T, 1>(x, ldx, num_tokens, K, nw, eps, Ws, N, out, ldo, xn, ldxn, s);
  else if (pieces <= 2 * kThreads)
    launch_norm_gemm<T, 2>(x, ldx, num_tokens, K, nw, eps, Ws, N, out, ldo, xn, ldxn, s);
  else
    launch_norm_gemm<T, 4>(x, ldx, num_tokens, K, nw, eps, Ws, N, out, ldo, xn, ldxn, s);
  PL_LAUNCH_CHECK("shuffled_gemm_norm_kernel");
  return ok();
}

template <typename T>
static int normsq_gemm_t(const void* x, int64_t ldx, int num_tokens, int K, const void* nw, float eps,
                         const float* sq, int64_t ldsq, int parts, const void* Ws, int N, void* out, int64_t ldo,
                         void* xn, int64_t ldxn, hipStream_t s) {
  const dim3 grid((N + 15) / 16, (num_tokens + 15) / 16);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, (const T*)x, ldx, num_tokens, K, (const T*)nw, eps, sq,
                       ldsq, parts, (const T*)Ws, N, (T*)out, ldo, (T*)xn, ldxn);
  };
  auto by_qpl = [&](auto xn) {
    constexpr bool XN = decltype(xn)::value;
    if (parts <= kWave * 4)
      go(shuffled_gemm_normsq_kernel<T, 1, XN>);
    else if (parts <= kWave * 8)
      go(shuffled_gemm_normsq_kernel<T, 2, XN>);
    else
      go(shuffled_gemm_normsq_kernel<T, 4, XN>);
  };
  if (xn != nullptr)
    by_qpl(std::true_type{});
  else
    by_qpl(std::false_type{});
  PL_LAUNCH_CHECK("shuffled_gemm_normsq_kernel");
  return ok();
}

extern "C" int pl_linear_shuffled_norm(const void* x, int64_t ldx, int num_tokens, int in_features,
                                       const void* norm_weight, float eps, const float* sq_partials, int64_t ld_sq,
                                       int sq_parts, const void* shuffled, int out_features, void* out, int64_t ldo,
                                       void* x_norm_out, int64_t ld_norm_out, int dtype, void* stream) {
  const int max_tokens = sq_partials ? 16 : kNormMaxTokens;
  if (num_tokens < 0 || num_tokens > max_tokens)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..%d (got %d)", max_tokens, num_tokens);
  if (num_tokens == 0) return ok();
  if (sq_partials ? (in_features <= 0 || in_features % 32 || in_features > 8192)
                  : (in_features <= 0 || in_features % 512 || in_features > 8192 || num_tokens * in_features > 32768))
    return fail(PL_ERR_UNSUPPORTED,
                "in_features must be a multiple of 32 (with sq_partials) or of 512 with num_tokens * in_features <= "
                "32768 (without), up to 8192 (got %d x %d)", num_tokens, in_features);
  if (out_features <= 0) return fail(PL_ERR_INVALID, "out_features must be > 0");
  if (!x || !norm_weight || !shuffled || !out) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx < in_features || ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)shuffled % 16 || (uintptr_t)norm_weight % 16)
    return fail(PL_ERR_INVALID, "x rows, the norm weight and the shuffled weight must be 16-byte aligned");
  if (ldo < out_features) return fail(PL_ERR_INVALID, "ldo < out_features");
  if (x_norm_out && (ld_norm_out < in_features || ld_norm_out % 8 || (uintptr_t)x_norm_out % 16))
    return fail(PL_ERR_INVALID, "x_norm_out rows must be 16-byte aligned with ld_norm_out >= in_features");
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_linear_shuffled_norm dtype must be F16 or BF16 (got %d)", dtype);
  hipStream_t s = (hipStream_t)stream;
  if (sq_partials != nullptr) {
    if (sq_parts < 1 || sq_parts > kWave * 16 || ld_sq < sq_parts || ld_sq % 4 || (uintptr_t)sq_partials % 16)
      return fail(PL_ERR_INVALID, "sq_partials: 1..%d parts per row, ld_sq >= parts and a multiple of 4, 16-byte "
                  "aligned (got %d parts, ld %lld)", kWave * 16, sq_parts, (long long)ld_sq);
    if (dtype == PL_DTYPE_BF16)
      return normsq_gemm_t<bf16_t>(x, ldx, num_tokens, in_features, norm_weight, eps, sq_partials, ld_sq, sq_parts,
                                   shuffled, out_features, out, ldo, x_norm_out, ld_norm_out, s);
    return normsq_gemm_t<f16_t>(x, ldx, num_tokens, in_features, norm_weight, eps, sq_partials, ld_sq, sq_parts,
                                shuffled, out_features, out, ldo, x_norm_out, ld_norm_out, s);
  }
  if (dtype == PL_DTYPE_BF16)
    return norm_gemm_t<bf16_t>(x, ldx, num_tokens, in_features, norm_weight, eps, shuffled, out_features, out, ldo,
                               x_norm_out, ld_norm_out, s);
  return norm_gemm_t<f16_t>(x, ldx, num_tokens, in_features, norm_weight, eps, shuffled, out_features, out, ldo,
                            x_norm_out, ld_norm_out, s);
}

template <typename T, int R, int YPT>
static void launch_add_gemm(const void* x, int64_t ldx, int num_tokens, int K, const void* Ws, int N, void* res,
                            int64_t ldr, const LoraUp& lu, const pl_lora_partials* yp, int lg, const int32_t* ids,
                            int na, void* out, int64_t ldo, float* sq, int64_t ldsq, hipStream_t s) {
  const dim3 grid((N + 15) / 16, (num_tokens + 15) / 16);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, (const T*)x, ldx, num_tokens, K, (const T*)Ws, N,
                       (T*)res, ldr, lu, yp ? yp->partials : nullptr, yp ? yp->ld : 0, yp ? yp->parts : 0, lg, ids,
                       na, (T*)out, ldo, sq, ldsq);
  };
  // two batches in flight per wave where the grid is one workgroup per CU
  // and K splits into whole batches per wave (o_proj 4096, down_proj 12288)
  const int ksteps = K / 32;
  const int nb = ksteps % (kWaves * kUnroll) == 0 ? ksteps / (kWaves * kUnroll) : 0;
  const bool one_round = (int64_t)grid.x * grid.y <= kGemmCUs;
  if (one_round && nb == 2) go(shuffled_gemm_add_kernel<T, R, YPT, 2>);
  else if (one_round && nb == 6) go(shuffled_gemm_add_kernel<T, R, YPT, 6>);
  else go(shuffled_gemm_add_kernel<T, R, YPT, 0>);
}

template <typename T>
static int add_gemm_t(const void* x, int64_t ldx, int num_tokens, int K, const void* Ws, int N, void* res,
                      int64_t ldr, const LoraUp& lu, int rank, const pl_lora_partials* yp, int lg, int ypt,
                      const int32_t* ids, int na, void* out, int64_t ldo, float* sq, int64_t ldsq, hipStream_t s) {
  switch (rank) {
    case 0: launch_add_gemm<T, 0, 1>(x, ldx, num_tokens, K, Ws, N, res, ldr, lu, yp, lg, ids, na, out, ldo, sq, ldsq, s); break;
    case 8:
      if (ypt <= 1) launch_add_gemm<T, 8, 1>(x, ldx, num_tokens, K, Ws, N, res, ldr, lu, yp, lg, ids, na, out, ldo, sq, ldsq, s);
      else if (ypt <= 2) launch_add_gemm<T, 8, 2>(x, ldx, num_tokens, K, Ws, N, res, ldr, lu, yp, lg, ids, na, out, ldo, sq, ldsq, s);
      else launch_add_gemm<T, 8, 4>(x, ldx, num_tokens, K, Ws, N, res, ldr, lu, yp, lg, ids, na, out, ldo, sq, ldsq, s);
      break;
    default:
      if (ypt <= 1) launch_add_gemm<T, 16, 1>(x, ldx, num_tokens, K, Ws, N, res, ldr, lu, yp, lg, ids, na, out, ldo, sq, ldsq, s);
      else if (ypt <= 2) launch_add_gemm<T, 16, 2>(x, ldx, num_tokens, K, Ws, N, res, ldr, lu, yp, lg, ids, na, out, ldo, sq, ldsq, s);
      else launch_add_gemm<T, 16, 4>(x, ldx, num_tokens, K, Ws, N, res, ldr, lu, yp, lg, ids, na, out, ldo, sq, ldsq, s);
      break;
  }
  PL_LAUNCH_CHECK("shuffled_gemm_add_kernel");
  return ok();
}

extern "C" int pl_linear_shuffled_add(const void* x, int64_t ldx, int num_tokens, int in_features,
                                      const void* shuffled, int out_features, void* residual, int64_t ldr,
                                      const pl_lora_up* lora, const pl_lora_partials* lora_y,
                                      const int32_t* adapter_ids, int num_adapters, void* out, int64_t ldo,
                                      float* sq_out, int64_t ld_sq, int dtype, void* stream) {
  if (num_tokens < 0 || num_tokens > 16)
    return fail(PL_ERR_INVALID, "num_tokens must be 0..16 (got %d)", num_tokens);
  if (num_tokens == 0) return ok();
  if (in_features <= 0 || in_features % 32 || out_features <= 0)
    return fail(PL_ERR_INVALID, "in_features must be a positive multiple of 32 and out_features > 0");
  if (!x || !shuffled || !residual) return fail(PL_ERR_INVALID, "null pointer argument");
  if (ldx < in_features || ldx % 8 || (uintptr_t)x % 16 || (uintptr_t)shuffled % 16)
    return fail(PL_ERR_INVALID, "x rows and the shuffled weight must be 16-byte aligned");
  if (ldr < out_features || (out && ldo < out_features))
    return fail(PL_ERR_INVALID, "residual / out rows shorter than out_features");
  if (sq_out && ld_sq < (out_features + 15) / 16)
    return fail(PL_ERR_INVALID, "sq_out rows need ld_sq >= %d (one sum per 16 columns)", (out_features + 15) / 16);
  if (dtype != PL_DTYPE_BF16 && dtype != PL_DTYPE_F16)
    return fail(PL_ERR_UNSUPPORTED, "pl_linear_shuffled_add dtype must be F16 or BF16 (got %d)", dtype);
  if ((lora == nullptr) != (lora_y == nullptr))
    return fail(PL_ERR_INVALID, "lora and lora_y are given together or not at all");
  LoraUp lu{};
  int rank = 0, G = 1, lg = 0, ypt = 1;
  if (lora) {
    if (const int st = lora_adapters_checked(lora, 1, adapter_ids, num_adapters, "linear_shuffled_add LoRA"))
      return st;
    if (!lora->B || (uintptr_t)lora->B % 16) return fail(PL_ERR_INVALID, "LoRA B must be non-null and 16-byte aligned");
    if (lora->rank != 8 && lora->rank != 16)
      return fail(PL_ERR_UNSUPPORTED, "pl_linear_shuffled_add: LoRA rank %d not built (8, 16)", lora->rank);
    if (lora->out_features < out_features)
      return fail(PL_ERR_INVALID, "LoRA B has %d output features, %d needed", lora->out_features, out_features);
    if (lora->b_layout != PL_LORA_B_ROWS && (lora->b_layout != PL_LORA_B_CHUNK8 || lora->out_features % 8))
      return fail(PL_ERR_INVALID, "unknown or unusable LoRA b_layout %d", lora->b_layout);
    if (lora_y->rank != lora->rank) return fail(PL_ERR_INVALID, "lora_y rank %d != LoRA rank %d", lora_y->rank, lora->rank);
    if (!lora_y->partials || (uintptr_t)lora_y->partials % 16 || lora_y->parts < 1 ||
        lora_y->ld < (int64_t)lora_y->parts * lora_y->rank || lora_y->ld % 4)
      return fail(PL_ERR_INVALID, "lora_y: 16-byte aligned partials, parts >= 1, ld >= parts * rank (a multiple of 4)");
    rank = lora->rank;
    while (G < lora_y->parts) G <<= 1, ++lg;
    const int groups = std::min(num_tokens, 16) * (rank / 4);
    const int64_t f = (int64_t)groups * G;
    if (f > (int64_t)kAddMaxYPT * kThreads)
      return fail(PL_ERR_UNSUPPORTED, "lora_y: %d parts for %d tokens exceed the %d partial sums a workgroup adds",
                  lora_y->parts, num_tokens, kAddMaxYPT * kThreads * 4);
    ypt = (int)((f + kThreads - 1) / kThreads);
    lu = LoraUp{nullptr, 0, 0, lora->B, lora->out_features, lora->rank, lora->scale, lora->b_layout, lora->adapter};
  }
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PL_DTYPE_BF16)
    return add_gemm_t<bf16_t>(x, ldx, num_tokens, in_features, shuffled, out_features, residual, ldr, lu, rank, lora_y,
                              lg, ypt, adapter_ids, num_adapters, out, ldo, sq_out, ld_sq, s);
  return add_gemm_t<f16_t>(x, ldx, num_tokens, in_features, shuffled, out_features, residual, ldr, lu, rank, lora_y,
                           lg, ypt, adapter_ids, num_adapters, out, ldo, sq_out, ld_sq, s);
}
