// Batched single-token paged attention for gfx950 (MI355X).
//
// Three kernels, all launched with a grid that depends only on the batch
// size and the workspace plan, never on sequence lengths, so a captured
// hipGraph replays across decode steps while rows grow:
//
//   plan_kernel    one workgroup; reads indptr[B+1] and cuts every row into
//                  chunks of `chunk_pages` pages (chunk_pages chosen on the
//                  device from the total page count) -> a work list of
//                  (row, page range) items, full-size chunks first and the
//                  rows' shorter last chunks after them, longest first.
//   decode_kernel  one wavefront per (item, kv head).  Streams the item's
//                  pages 16 tokens at a time straight from HBM into VGPRs
//                  (16 lanes x 16 B cover one 128-dim token row, so one
//                  dwordx4 load instruction reads 4 token rows), scores them
//                  against the g query heads of the kv head with v_dot2 and
//                  DPP row reductions (GQA 4 at head_dim 128 in 16-bit
//                  types: on MFMA, DecodeWaveMfma), and keeps an online
//                  softmax per lane row in fp32.  Rows with one item write
//                  the output directly; split rows write (o, lse) partials.
//   merge_kernel   one wavefront per (row, q head) of a split row: the
//                  LSE-weighted sum of its partials.  A separate launch, so
//                  the kernel boundary orders the partials across the eight
//                  XCD L2 caches without per-wave L2 write-back fences.
//
// Mathematics: o = softmax(q . K^T * sm_scale) . V, as the reference's
// FlashInferAttentionBackend.run_decode (model/flashinfer/attention_backend.py
// :120-131) obtains from FlashInfer with q/16 and sm_scale 16/sqrt(D).
#include <cstdlib>
#include <mutex>
#include <unordered_map>

#include "decode_kernels.h"

namespace pl {
namespace decode {

// ------------------------------------------------------------------ plan ---
constexpr int kPlanThreads = 1024;
constexpr int kPlanBuckets = 1024;  // size classes of the rows' last (short) chunks
constexpr int kPlanOwnChunks = 8;   // rows of up to this many chunks are written by their own thread
static_assert(kPlanBuckets == kPlanThreads, "the class scan takes one class per thread");


// Exclusive prefix sum of one int per thread over the 1024-thread block
// (shuffles inside each wave, then the 16 wave totals); returns the prefix,
// writes the block total to *total.  Every thread of the block must call it.
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_wave, int* total) {
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    x += lane >= off ? y : 0;
  }
  if (lane == 63) s_wave[wave] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) {
    const int t = s_wave[w];
    before += w < wave ? t : 0;
    all += t;
  }
  __syncthreads();  // s_wave may be reused by the next scan
  *total = all;
  return before + x - v;
}

// Cuts every row into chunks of `chunk` pages and writes the work list.
//
// Two orders are involved.  A row's items get consecutive *slots* (its
// partial outputs and row_info use them, so the merge reads a row's partials
// as one range).  The *list* order, which is the order the hardware
// dispatches the items' waves in, is: every full-size chunk first (row by
// row), then the rows' last, shorter chunks from the longest to the shortest,
// so the waves that start last are the ones that finish soonest.  Measured on
// the ragged batch-64 workload: 743.5 us in row order, 721.2 us in this order.
// An item's slot travels in its flags (bits 2 and up).
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(
    const int32_t* __restrict__ indptr, int batch, int indices_capacity, int target_items,
    int min_chunk_pages, int max_items, Item* __restrict__ items,
    int2* __restrict__ row_info, int* __restrict__ header) {
  __shared__ int s_wave[kPlanThreads / 64];
  __shared__ int s_hist[kPlanBuckets];
  __shared__ int s_chunk;
  const int tid = threadIdx.x;
  // Page ranges are clamped to [0, indices_capacity] so a malformed indptr
  // can never send a reader outside the indices buffer.
  auto clampi = [&](int v) { return v < 0 ? 0 : (v > indices_capacity ? indices_capacity : v); };
  if (tid == 0) {
    const int total = clampi(indptr[batch]) - clampi(indptr[0]);
    int c = (total + target_items - 1) / target_items;
    c = c > min_chunk_pages ? c : min_chunk_pages;
    s_chunk = c > 1 ? c : 1;
  }
  for (int i = tid; i < kPlanBuckets; i += kPlanThreads) s_hist[i] = 0;
  __syncthreads();
  const int chunk = s_chunk;
  // size class of a short chunk of `pages` pages (< chunk): longest first
  auto bucket = [&](int pages) {
    const int64_t k = chunk - 1 - pages;  // 0 for the longest possible
    return chunk <= kPlanBuckets ? (int)k : (int)(k * kPlanBuckets / chunk);
  };
  auto row_pages = [&](int r, int& pb, int& pe) {
    pb = clampi(indptr[r]);
    pe = clampi(indptr[r + 1]);
    pe = pe > pb ? pe : pb;
  };
  const int per = (batch + kPlanThreads - 1) / kPlanThreads;
  const int r0 = tid * per;
  const int r1 = min(batch, r0 + per);
  // pass 1: per-thread counts of slots and full chunks; size classes of the
  // short chunks (their rank inside the class parked in row_info until pass 2)
  int n_slots = 0, n_full = 0;
  for (int r = r0; r < r1; ++r) {
    int pb, pe;
    row_pages(r, pb, pe);
    const int n = pe - pb;
    const int nch = n > 0 ? (n + chunk - 1) / chunk : 1;
    const int full = n / chunk;
    n_slots += nch;
    n_full += full;
    if (nch > full) {
      const int k = bucket(n - full * chunk);
      row_info[r] = make_int2(k, atomicAdd(&s_hist[k], 1));
    }
  }
  int total_items, total_full;
  int slot = block_exclusive_scan(n_slots, s_wave, &total_items);
  int fpos = block_exclusive_scan(n_full, s_wave, &total_full);
  // exclusive scan of the size classes (one per thread), offset past the full chunks
  int hist_total;
  const int hcount = s_hist[tid];
  const int hstart = block_exclusive_scan(hcount, s_wave, &hist_total);
  s_hist[tid] = total_full + hstart;
  __syncthreads();
  // pass 2: row_info, then the items.  A row of a few chunks is written by
  // its own thread; a longer row is broadcast to its wave, whose 64 lanes
  // write its chunks together (a single 32K-token row cut into 128 items took
  // 16 us in one thread; walking every lane's row through the whole wave cost
  // the batch-64 plan ~12 us instead).
  const int lane = tid % 64;
  for (int k = 0; k < per; ++k) {  // the same trip count in every thread
    const int r = r0 + k;
    int pb = 0, pe = 0, nch = 0, full = 0, short_pos = -1;
    const int my_slot = slot, my_fpos = fpos;
    if (r < r1) {
      row_pages(r, pb, pe);
      const int n = pe - pb;
      nch = n > 0 ? (n + chunk - 1) / chunk : 1;
      full = n / chunk;
      if (nch > full) {
        const int2 kr = row_info[r];  // this thread's own pass-1 write
        short_pos = s_hist[kr.x] + kr.y;
      }
      const int room = max_items - slot;
      row_info[r] = make_int2(slot < max_items ? slot : max_items, nch < room ? nch : (room > 0 ? room : 0));
      slot += nch;
      fpos += full;
    }
    // item j of a row: list position, slot, page range, flags
    auto put = [&](int rr, int pb_, int pe_, int n_, int full_, int slot_, int fpos_, int short_, int j) {
      const int pos = j < full_ ? fpos_ + j : short_;
      const int sl = slot_ + j;
      if (pos < 0 || pos >= max_items || sl >= max_items) return;  // unreachable by construction; keeps writes in bounds
      const int a = pb_ + j * chunk;
      const int e = min(pe_, a + chunk);
      Item item;
      item.row = rr;
      item.page_begin = a;
      item.page_end = e;
      item.flags = (sl << 2) | (n_ == 1 ? 1 : 0) | (e == pe_ ? 2 : 0);
      items[pos] = item;
    };
    if (nch <= kPlanOwnChunks)
      for (int j = 0; j < nch; ++j) put(r, pb, pe, nch, full, my_slot, my_fpos, short_pos, j);
    uint64_t long_rows = __builtin_amdgcn_ballot_w64(nch > kPlanOwnChunks);
    while (long_rows) {  // the same mask in every lane: a uniform loop
      const int src = __builtin_ctzll(long_rows);
      long_rows &= long_rows - 1;
      const int nL = __builtin_amdgcn_readlane(nch, src);
      const int rL = __builtin_amdgcn_readlane(r, src), pbL = __builtin_amdgcn_readlane(pb, src);
      const int peL = __builtin_amdgcn_readlane(pe, src), fullL = __builtin_amdgcn_readlane(full, src);
      const int slotL = __builtin_amdgcn_readlane(my_slot, src), fposL = __builtin_amdgcn_readlane(my_fpos, src);
      const int shortL = __builtin_amdgcn_readlane(short_pos, src);
      for (int j = lane; j < nL; j += 64) put(rL, pbL, peL, nL, fullL, slotL, fposL, shortL, j);
    }
  }
  for (int i = total_items + tid; i < max_items; i += kPlanThreads) {
    Item item;
    item.row = -1;
    item.page_begin = item.page_end = item.flags = 0;
    items[i] = item;
  }
  if (tid == 0) {
    header[0] = chunk;
    header[1] = total_items;
    header[2] = batch;
    header[3] = plan_stamp(batch, max_items);
  }
}

// The folded q/k/v epilogue: 16-bit types, head_dim 128, GQA 4, LoRA rank 0/8/16.
template <typename T>
int by_rank_qkv(const RunArgs& a, const QkvIn& qin, int rank) {
  switch (rank) {
    case 0: return launch<T, 128, 4, true, 0>(a, qin);
    case 8: return launch<T, 128, 4, true, 8>(a, qin);
    case 16: return launch<T, 128, 4, true, 16>(a, qin);
  }
  return fail(PL_ERR_UNSUPPORTED, "LoRA rank %d not built for the folded q/k/v epilogue (0, 8, 16)", rank);
}

int run_multiple16_pages(const RunArgs& a, int dtype, int d, int g) {
  switch (dtype) {
    case PL_DTYPE_F32: return by_dim<float, false>(a, d, g);
    case PL_DTYPE_F16: return by_dim<f16_t, false>(a, d, g);
    case PL_DTYPE_BF16: return by_dim<bf16_t, false>(a, d, g);
  }
  return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
}

}  // namespace decode
}  // namespace pl

using namespace pl;
using namespace pl::decode;

// Direct-item plans (batches of up to kDirectMaxBatch rows): pl_decode_plan
// launches nothing and records, per workspace, where the page table's indptr
// lives and how to split it; the runs on that workspace pass it to their
// kernels, which derive the items themselves.  The record is host state of
// the library, read when a run is enqueued (or captured into a graph).
// PAGELORA_DECODE_PLAN_KERNEL=1 keeps the plan kernel for every batch.
namespace {
struct DirectRec {
  const int32_t* indptr;
  int batch, capacity, target_items, min_chunk, shared, pchunk;
};
std::mutex g_direct_mutex;
std::unordered_map<const void*, DirectRec> g_direct;

bool direct_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("PAGELORA_DECODE_PLAN_KERNEL");
    return !(e != nullptr && e[0] == '1');
  }();
  return on;
}

// The direct plan recorded for `workspace`, if it matches this run.
Direct direct_for(const void* workspace, int batch, int target_items) {
  Direct d{nullptr, 0, 1, 1, 0, 1};
  std::lock_guard<std::mutex> lock(g_direct_mutex);
  const auto it = g_direct.find(workspace);
  if (it != g_direct.end() && it->second.batch == batch && it->second.target_items == target_items)
    d = Direct{it->second.indptr, it->second.capacity, it->second.target_items, it->second.min_chunk,
               it->second.shared, it->second.pchunk};
  return d;
}

// Slot capacity (max_items) and decode grid items of a run: the plan's
// target_items + batch, plus with a shared prefix of n_pref items one slot
// per row for each and grid items for the prefix workgroups (four prefix
// items of one kv head per workgroup).
void run_sizes(int batch, int target_items, const Direct& d, int& max_items, int& grid_items) {
  const int n_pref = d.shared > 0 ? (d.shared + d.pchunk - 1) / d.pchunk : 0;
  max_items = target_items + batch + batch * n_pref;
  grid_items = target_items + batch + (n_pref + 3) / 4 * 4;
}
}  // namespace

extern "C" size_t pl_decode_workspace_size(int batch, int target_items, int num_qo_heads,
                                           int head_dim) {
  if (batch < 0 || target_items <= 0 || num_qo_heads <= 0 || head_dim <= 0) return 0;
  return layout(batch, target_items + batch, num_qo_heads, head_dim).total;
}

extern "C" int pl_decode_plan(const int32_t* indptr, int batch, int indices_capacity,
                              int num_qo_heads, int head_dim, int target_items,
                              int min_chunk_pages, void* workspace, size_t workspace_bytes,
                              void* stream) {
  return pl_decode_plan_shared(indptr, batch, indices_capacity, num_qo_heads, head_dim, target_items,
                               min_chunk_pages, 0, 1, workspace, workspace_bytes, stream);
}

extern "C" int pl_decode_forget(const void* workspace) {
  std::lock_guard<std::mutex> lock(g_direct_mutex);
  g_direct.erase(workspace);
  return ok();
}

extern "C" size_t pl_decode_workspace_size_shared(int batch, int target_items, int num_qo_heads, int head_dim,
                                                  int shared_pages, int prefix_chunk_pages) {
  if (batch < 0 || target_items <= 0 || num_qo_heads <= 0 || head_dim <= 0 || shared_pages < 0 ||
      prefix_chunk_pages <= 0)
    return 0;
  int max_items, grid_items;
  run_sizes(batch, target_items, Direct{nullptr, 0, 1, 1, shared_pages, prefix_chunk_pages}, max_items, grid_items);
  return layout(batch, max_items, num_qo_heads, head_dim).total;
}

extern "C" int pl_decode_plan_shared(const int32_t* indptr, int batch, int indices_capacity,
                                     int num_qo_heads, int head_dim, int target_items,
                                     int min_chunk_pages, int shared_pages, int prefix_chunk_pages,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  if (shared_pages < 0 || prefix_chunk_pages <= 0 || (shared_pages > 0 && shared_pages % prefix_chunk_pages))
    return fail(PL_ERR_INVALID, "shared_pages must be a multiple of prefix_chunk_pages (got %d, %d)", shared_pages,
                prefix_chunk_pages);
  // A shared prefix is attended once only on direct plans (up to
  // kDirectMaxBatch rows, plan kernel not forced); otherwise the batch is
  // planned unshared, every row reading its own copy of the prefix pages.
  if (shared_pages > 0 && (batch > kDirectMaxBatch || !direct_enabled())) {
    shared_pages = 0;
    prefix_chunk_pages = 1;
  }
  if (batch < 0) return fail(PL_ERR_INVALID, "batch must be >= 0 (got %d)", batch);
  if (target_items <= 0) return fail(PL_ERR_INVALID, "target_items must be > 0");
  if (num_qo_heads <= 0 || head_dim <= 0) return fail(PL_ERR_INVALID, "bad head shape");
  if (indices_capacity < 0) return fail(PL_ERR_INVALID, "indices_capacity must be >= 0");
  if (batch == 0) return ok();
  if (indptr == nullptr || workspace == nullptr) return fail(PL_ERR_INVALID, "null pointer");
  if ((uintptr_t)workspace % 256) return fail(PL_ERR_INVALID, "workspace must be 256-byte aligned");
  const int max_items = target_items + batch;
  int shared_max_items, grid_items;
  run_sizes(batch, target_items, Direct{nullptr, 0, 1, 1, shared_pages, prefix_chunk_pages}, shared_max_items,
            grid_items);
  const Layout L = layout(batch, shared_max_items, num_qo_heads, head_dim);
  if (L.total > workspace_bytes)
    return fail(PL_ERR_WORKSPACE, "workspace of %zu bytes < %zu needed", workspace_bytes, L.total);
  const int min_chunk = min_chunk_pages < 1 ? 1 : min_chunk_pages;
  {
    std::lock_guard<std::mutex> lock(g_direct_mutex);
    if (direct_enabled() && batch <= kDirectMaxBatch) {
      g_direct[workspace] =
          DirectRec{indptr, batch, indices_capacity, target_items, min_chunk, shared_pages, prefix_chunk_pages};
      return ok();
    }
    g_direct.erase(workspace);
  }
  char* ws = (char*)workspace;
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, indptr,
                     batch, indices_capacity, target_items, min_chunk_pages < 1 ? 1 : min_chunk_pages, max_items,
                     (Item*)(ws + L.items), (int2*)(ws + L.row_info), (int*)(ws + L.header));
  PL_LAUNCH_CHECK("plan_kernel");
  return ok();
}

static int decode_run_common(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const void* k_cache, const void* v_cache, int64_t page_stride,
                             int64_t token_stride, int64_t head_stride, int64_t num_pages,
                             const int32_t* indices, const int32_t* last_page_len, void* o, int64_t o_stride_b,
                             int64_t o_stride_h, float* lse, int batch, int num_qo_heads,
                             int num_kv_heads, int head_dim, int page_size, float sm_scale,
                             int dtype, int target_items, int flags, void* workspace,
                             size_t workspace_bytes, void* stream, const QkvIn* qin = nullptr,
                             int qin_rank = 0, const OShrink* os = nullptr, int os_rank = 0) {
  if (batch < 0) return fail(PL_ERR_INVALID, "batch must be >= 0");
  if (batch == 0) return ok();
  if (num_kv_heads <= 0 || num_qo_heads <= 0 || num_qo_heads % num_kv_heads)
    return fail(PL_ERR_INVALID, "num_qo_heads (%d) must be a positive multiple of num_kv_heads (%d)",
                num_qo_heads, num_kv_heads);
  if (page_size <= 0 || page_size > kMaxPageSize)
    return fail(PL_ERR_UNSUPPORTED, "page_size %d: must be 1..%d", page_size, kMaxPageSize);
  if (qin && page_size % kBlockTokens)
    return fail(PL_ERR_UNSUPPORTED, "the folded q/k/v epilogue needs pages of a multiple of %d tokens (got %d)",
                kBlockTokens, page_size);
  if (target_items <= 0) return fail(PL_ERR_INVALID, "target_items must be > 0");
  if (num_pages <= 0) return fail(PL_ERR_INVALID, "num_pages must be > 0");
  if ((!q && !qin) || !k_cache || !v_cache || !indices || !last_page_len || !o || !workspace)
    return fail(PL_ERR_INVALID, "null pointer argument");
  if (dtype != PL_DTYPE_F32 && dtype != PL_DTYPE_F16 && dtype != PL_DTYPE_BF16)
    return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
  // Every lane issues 16-byte loads of 8 consecutive elements.
  const int64_t strides[] = {q_stride_b, q_stride_h, page_stride, token_stride, head_stride,
                             o_stride_b, o_stride_h};
  for (int64_t s : strides)
    if (s % 8) return fail(PL_ERR_INVALID, "every stride must be a multiple of 8 elements");
  const void* ptrs[] = {qin ? k_cache : q, k_cache, v_cache, o};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return fail(PL_ERR_INVALID, "q, caches and o must be 16-byte aligned");
  Direct dir = direct_for(workspace, batch, target_items);
  // a shared prefix is attended by prefix items in the folded q/k/v kernel
  // only, for up to 4 rows with one bound adapter, whole 16-token blocks and
  // one 32-token MFMA step per item; anything else reads every page per row
  if (dir.shared > 0) {
    const bool ok_shared = qin != nullptr && batch <= kPrefixMaxRows && page_size % kBlockTokens == 0 &&
                           dir.pchunk * page_size == kPrefixTokens && head_dim == 128 &&
                           num_qo_heads == 4 * num_kv_heads && (qin_rank == 0 || qin->m[0].adapter >= 0);
    if (!ok_shared) dir.shared = 0;
  }
  int max_items, grid_items;
  run_sizes(batch, target_items, dir, max_items, grid_items);
  const Layout L = layout(batch, max_items, num_qo_heads, head_dim);
  if (L.total > workspace_bytes)
    return fail(PL_ERR_WORKSPACE, "workspace of %zu bytes < %zu needed", workspace_bytes, L.total);
  char* ws = (char*)workspace;
  RunArgs a;
  a.q = q; a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.kc = k_cache; a.vc = v_cache;
  a.page_stride = page_stride; a.token_stride = token_stride; a.head_stride = head_stride;
  a.indices = indices; a.last = last_page_len;
  a.o = o; a.o_sb = o_stride_b; a.o_sh = o_stride_h; a.lse = lse;
  a.batch = batch; a.hq = num_qo_heads; a.hkv = num_kv_heads; a.page_size = page_size;
  a.kv_split = 1;
  a.num_pages = num_pages; a.header = (const int*)(ws + L.header);
  a.scale_log2 = sm_scale * 1.44269504088896340736f;
  a.items = (const Item*)(ws + L.items); a.max_items = max_items;
  a.row_info = (const int2*)(ws + L.row_info);
  a.flags = flags;
  a.part_lse = (float*)(ws + L.lse); a.part_o = (float*)(ws + L.partial_o);
  a.dir = dir;
  a.grid_items = grid_items;
  a.os = os ? *os : OShrink{};
  a.os_rank = os ? os_rank : 0;
  a.stream = (hipStream_t)stream;
  const int g = num_qo_heads / num_kv_heads;
  if (qin) {
    if (head_dim != 128 || g != 4 || (dtype != PL_DTYPE_F16 && dtype != PL_DTYPE_BF16))
      return fail(PL_ERR_UNSUPPORTED, "the folded q/k/v epilogue is built for 16-bit types, head_dim 128, GQA 4");
    return dtype == PL_DTYPE_F16 ? by_rank_qkv<f16_t>(a, *qin, qin_rank) : by_rank_qkv<bf16_t>(a, *qin, qin_rank);
  }
  switch (dtype) {
    case PL_DTYPE_F32:
    case PL_DTYPE_F16:
    case PL_DTYPE_BF16: {
      // GQA groups above 8 heads: virtual kv heads of at most 8 query heads
      // each (the largest divisor of g up to 8), kv_split of them per kv head
      int gw = g;
      if (g > kMaxGroup) {
        gw = 1;
        for (int d = kMaxGroup; d >= 1; --d)
          if (g % d == 0) { gw = d; break; }
      }
      a.kv_split = g / gw;
      a.hkv = num_kv_heads * a.kv_split;
      if (page_size % kBlockTokens) return run_small_pages(a, dtype, head_dim, gw);
      return run_multiple16_pages(a, dtype, head_dim, gw);
    }
  }
  return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
}

extern "C" int pl_decode_run(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const void* k_cache, const void* v_cache, int64_t page_stride,
                             int64_t token_stride, int64_t head_stride, int64_t num_pages,
                             const int32_t* indices, const int32_t* last_page_len, void* o, int64_t o_stride_b,
                             int64_t o_stride_h, float* lse, int batch, int num_qo_heads,
                             int num_kv_heads, int head_dim, int page_size, float sm_scale,
                             int dtype, int target_items, int flags, void* workspace,
                             size_t workspace_bytes, void* stream) {
  return decode_run_common(q, q_stride_b, q_stride_h, k_cache, v_cache, page_stride, token_stride, head_stride,
                           num_pages, indices, last_page_len, o, o_stride_b, o_stride_h, lse, batch, num_qo_heads,
                           num_kv_heads, head_dim, page_size, sm_scale, dtype, target_items, flags, workspace,
                           workspace_bytes, stream);
}

static int decode_run_qkv_common(const void* qkv, int64_t ld_qkv, const pl_lora_up* lora_qkv_h,
                                 const int32_t* adapter_ids, int num_adapters, const void* q_norm_weight,
                                 const void* k_norm_weight, const float* rope_cos_sin, const int64_t* page_id,
                                 const int64_t* offset, float eps, void* k_cache, void* v_cache,
                                 int64_t page_stride, int64_t token_stride, int64_t head_stride, int64_t num_pages,
                                 const int32_t* indices, const int32_t* last_page_len, void* o, int64_t o_stride_b,
                                 int64_t o_stride_h, float* lse, int batch, int num_qo_heads, int num_kv_heads,
                                 int head_dim, int page_size, float sm_scale, int dtype, int target_items, int flags,
                                 void* workspace, size_t workspace_bytes, void* stream,
                                 const pl_lora_a_rows* o_a = nullptr, const pl_lora_partials* o_y = nullptr) {
  if (batch < 0) return fail(PL_ERR_INVALID, "batch must be >= 0");
  if (batch == 0) return ok();
  if (!qkv || !rope_cos_sin || !page_id || !offset) return fail(PL_ERR_INVALID, "null pointer argument");
  if (num_qo_heads <= 0 || num_kv_heads <= 0) return fail(PL_ERR_INVALID, "bad head counts");
  const int64_t row_cols = (int64_t)(num_qo_heads + 2 * num_kv_heads) * head_dim;
  if (ld_qkv < row_cols || ld_qkv % 8 || (uintptr_t)qkv % 16)
    return fail(PL_ERR_INVALID, "qkv rows need ld >= %lld (a multiple of 8) and 16-byte alignment",
                (long long)row_cols);
  if ((uintptr_t)rope_cos_sin % 16) return fail(PL_ERR_INVALID, "rope_cos_sin must be 16-byte aligned");
  if ((uintptr_t)q_norm_weight % 16 || (uintptr_t)k_norm_weight % 16)
    return fail(PL_ERR_INVALID, "norm weights must be 16-byte aligned");
  QkvIn qin{};
  qin.qkv = qkv; qin.ld = ld_qkv; qin.q_norm_w = q_norm_weight; qin.k_norm_w = k_norm_weight;
  qin.rope = rope_cos_sin; qin.page_id = page_id; qin.page_off = offset; qin.eps = eps;
  // ids is read unconditionally: with a uniform adapter (no ids) it points at
  // offset, an int64[batch] array, read as int32 and ignored
  qin.ids = adapter_ids ? adapter_ids : reinterpret_cast<const int32_t*>(offset);
  qin.n_adapters = num_adapters;
  qin.m[0].adapter = -1;  // no LoRA: the kernel's adapter test is off (rank 0)
  int rank = 0;
  if (lora_qkv_h) {
    if (const int st = lora_adapters_checked(lora_qkv_h, 3, adapter_ids, num_adapters, "decode q/k/v LoRA")) return st;
    const int need[3] = {num_qo_heads * head_dim, num_kv_heads * head_dim, num_kv_heads * head_dim};
    const char* names[3] = {"q LoRA", "k LoRA", "v LoRA"};
    for (int m = 0; m < 3; ++m)
      if (const int st = lora_up_checked(&lora_qkv_h[m], need[m], &qin.m[m], names[m])) return st;
    rank = lora_qkv_h[0].rank;
    if (lora_qkv_h[1].rank != rank || lora_qkv_h[2].rank != rank)
      return fail(PL_ERR_INVALID, "q, k and v LoRA must share one rank");
  }
  OShrink os{};
  int os_rank = 0;
  if (o_a != nullptr || o_y != nullptr) {
    if (!o_a || !o_y) return fail(PL_ERR_INVALID, "o_proj's A rows and partials are given together");
    if (flags & (PL_DECODE_SKIP_MERGE | PL_DECODE_MERGE_ONLY))
      return fail(PL_ERR_INVALID, "the o_proj shrink runs in the merge: no PL_DECODE_SKIP_MERGE / MERGE_ONLY");
    const int K = num_qo_heads * head_dim;
    if (o_a->rank != 8 && o_a->rank != 16)
      return fail(PL_ERR_UNSUPPORTED, "o_proj shrink rank %d not built (8, 16)", o_a->rank);
    if (!o_a->shuffled || (uintptr_t)o_a->shuffled % 16 || o_a->in_features != K || o_a->a_row0 < 0 ||
        (int64_t)o_a->a_row0 + (int64_t)num_adapters * o_a->rank > o_a->out_features)
      return fail(PL_ERR_INVALID,
                  "o_proj A rows: a 16-byte aligned shuffled weight %d wide (got %d) whose %d rows hold rows "
                  "a_row0 (%d) .. + %d adapters x rank %d",
                  K, o_a->in_features, o_a->out_features, o_a->a_row0, num_adapters, o_a->rank);
    if (o_a->adapter < -1 || o_a->adapter >= num_adapters || num_adapters < 1 ||
        (o_a->adapter < 0 && !adapter_ids))
      return fail(PL_ERR_INVALID, "o_proj A rows: adapter %d with %d adapters (per-row ids need adapter_ids)",
                  o_a->adapter, num_adapters);
    // partials per row: one per (head, dim slice), the slice count the merge picks
    const int ds = merge_dim_split(head_dim, batch * num_qo_heads);
    if (!o_y->partials || o_y->rank != o_a->rank || o_y->parts != num_qo_heads * ds ||
        o_y->ld < (int64_t)o_y->parts * o_y->rank)
      return fail(PL_ERR_INVALID, "o_proj partials: rank %d, %d parts per row (num_qo_heads x %d), ld >= %d",
                  o_a->rank, num_qo_heads * ds, ds, num_qo_heads * ds * o_a->rank);
    os = OShrink{o_a->shuffled, K / 32, o_a->a_row0, o_a->adapter,
                 adapter_ids ? adapter_ids : reinterpret_cast<const int32_t*>(offset), num_adapters,
                 o_y->partials, o_y->ld};
    os_rank = o_a->rank;
    qin.no_direct = 1;
  }
  return decode_run_common(nullptr, 0, 0, k_cache, v_cache, page_stride, token_stride, head_stride, num_pages,
                           indices, last_page_len, o, o_stride_b, o_stride_h, lse, batch, num_qo_heads, num_kv_heads,
                           head_dim, page_size, sm_scale, dtype, target_items, flags, workspace, workspace_bytes,
                           stream, &qin, rank, os_rank ? &os : nullptr, os_rank);
}

extern "C" int pl_decode_run_qkv(const void* qkv, int64_t ld_qkv, const pl_lora_up* lora_qkv_h,
                                 const int32_t* adapter_ids, int num_adapters, const void* q_norm_weight,
                                 const void* k_norm_weight, const float* rope_cos_sin, const int64_t* page_id,
                                 const int64_t* offset, float eps, void* k_cache, void* v_cache,
                                 int64_t page_stride, int64_t token_stride, int64_t head_stride, int64_t num_pages,
                                 const int32_t* indices, const int32_t* last_page_len, void* o, int64_t o_stride_b,
                                 int64_t o_stride_h, float* lse, int batch, int num_qo_heads, int num_kv_heads,
                                 int head_dim, int page_size, float sm_scale, int dtype, int target_items, int flags,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  return decode_run_qkv_common(qkv, ld_qkv, lora_qkv_h, adapter_ids, num_adapters, q_norm_weight, k_norm_weight,
                               rope_cos_sin, page_id, offset, eps, k_cache, v_cache, page_stride, token_stride,
                               head_stride, num_pages, indices, last_page_len, o, o_stride_b, o_stride_h, lse, batch,
                               num_qo_heads, num_kv_heads, head_dim, page_size, sm_scale, dtype, target_items, flags,
                               workspace, workspace_bytes, stream);
}

extern "C" int pl_decode_run_qkv_oshrink(
    const void* qkv, int64_t ld_qkv, const pl_lora_up* lora_qkv_h, const int32_t* adapter_ids, int num_adapters,
    const void* q_norm_weight, const void* k_norm_weight, const float* rope_cos_sin, const int64_t* page_id,
    const int64_t* offset, float eps, void* k_cache, void* v_cache, int64_t page_stride, int64_t token_stride,
    int64_t head_stride, int64_t num_pages, const int32_t* indices, const int32_t* last_page_len, void* o,
    int64_t o_stride_b, int64_t o_stride_h, float* lse, int batch, int num_qo_heads, int num_kv_heads, int head_dim,
    int page_size, float sm_scale, int dtype, int target_items, int flags, void* workspace, size_t workspace_bytes,
    const pl_lora_a_rows* o_lora_a, const pl_lora_partials* o_lora_y, void* stream) {
  if (!o_lora_a || !o_lora_y) return fail(PL_ERR_INVALID, "null o_proj A rows or partials");
  return decode_run_qkv_common(qkv, ld_qkv, lora_qkv_h, adapter_ids, num_adapters, q_norm_weight, k_norm_weight,
                               rope_cos_sin, page_id, offset, eps, k_cache, v_cache, page_stride, token_stride,
                               head_stride, num_pages, indices, last_page_len, o, o_stride_b, o_stride_h, lse, batch,
                               num_qo_heads, num_kv_heads, head_dim, page_size, sm_scale, dtype, target_items, flags,
                               workspace, workspace_bytes, stream, o_lora_a, o_lora_y);
}

// ------------------------------------------------- allocation-free entry ---
// pl_decode_noalloc keeps its work list and partials in this file-scope
// device array instead of a caller workspace.  Each GPU the library runs on
// holds its own copy for the life of the process.  In host code `scratch`
// names a host-side stand-in, never the device memory: its device address
// comes from hipGetSymbolAddress, once per device with that device current,
// and only that address is handed to kernels.
constexpr size_t kNoAllocScratchBytes = PL_DECODE_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

#include <mutex>

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch`, per device id
}  // namespace

// The device address of `scratch` on the current device (looked up on the
// first call on that device).  `stream` must belong to the current device.
static int scratch_of_current_device(void* stream, void** out) {
  int dev = -1;
  PL_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(PL_ERR_UNSUPPORTED, "device %d: the allocation-free entry serves devices 0..%d", dev,
                kMaxScratchDevices - 1);
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    PL_HIP_CHECK(hipStreamGetDevice((hipStream_t)stream, &sdev));
    if ((int)sdev != dev)
      return fail(PL_ERR_INVALID, "the stream belongs to device %d but device %d is current", (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(PL_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PL_OK;
}

extern "C" int pl_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                                 const void* v_cache, int64_t page_stride, int64_t token_stride,
                                 int64_t head_stride, int64_t num_pages, const int32_t* indptr,
                                 int indices_capacity, const int32_t* indices, const int32_t* last_page_len,
                                 void* o, int64_t o_stride_b, int64_t o_stride_h, float* lse, int batch,
                                 int num_qo_heads, int num_kv_heads, int head_dim, int page_size, float sm_scale,
                                 int dtype, int target_items, int min_chunk_pages, void* stream) {
  if (batch < 0) return fail(PL_ERR_INVALID, "batch must be >= 0 (got %d)", batch);
  if (target_items <= 0) return fail(PL_ERR_INVALID, "target_items must be > 0");
  if (num_qo_heads <= 0 || head_dim <= 0) return fail(PL_ERR_INVALID, "bad head shape");
  if (batch == 0) return ok();
  // Host-side size check first: a plan that does not fit is rejected
  // before any HIP call.
  const size_t need = layout(batch, target_items + batch, num_qo_heads, head_dim).total;
  if (need > kNoAllocScratchBytes)
    return fail(PL_ERR_WORKSPACE,
                "decode plan of %d rows x %d items x %d heads x dim %d needs %zu bytes of scratch, more than the "
                "%zu-byte maximum of pl_decode_noalloc (use pl_decode_plan + pl_decode_run with a workspace)",
                batch, target_items, num_qo_heads, head_dim, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (const int st = scratch_of_current_device(stream, &ws)) return st;
  // The plan rewrites the header, the whole work list and the row table on
  // every call, and the run reads only what this call's plan and decode
  // kernels wrote, so nothing needs clearing between calls.
  if (const int st = pl_decode_plan(indptr, batch, indices_capacity, num_qo_heads, head_dim, target_items,
                                    min_chunk_pages, ws, kNoAllocScratchBytes, stream))
    return st;
  return pl_decode_run(q, q_stride_b, q_stride_h, k_cache, v_cache, page_stride, token_stride, head_stride,
                       num_pages, indices, last_page_len, o, o_stride_b, o_stride_h, lse, batch, num_qo_heads,
                       num_kv_heads, head_dim, page_size, sm_scale, dtype, target_items, 0, ws,
                       kNoAllocScratchBytes, stream);
}
