// Device-side advance of a batched paged-KV page table by one decode token
// (gfx950).
//
// Every row of the CSR table (indptr[B+1], indices, last_page_len[B]) gains
// one token.  A row whose last page still has room keeps its pages and its
// fill grows by one; a row whose last page is full (or that has no page)
// takes the next page of its reserve ring and that page starts with fill 1.
// The kernel also writes each row's decode inputs: the token's position and
// the (page, offset) slot its K/V row is appended to.
//
// Replaces the per-step host bookkeeping of the reference's batched decode
// loop (model/flashinfer/generation.py:1011-1035): reserve_chunk(request, 1)
// per row (paged_kvcache_manager.py:195-213 -> paged_kv_store.py:113-190:
// extend the partial last span, else allocate a page and append the span
// (page, 0, 1)), then the repack of every row's spans into the reusable
// table (flashinfer_page_table.py:89-121).  Done on the device it needs no
// host table and no upload, so a captured decode step replays step after
// step while rows grow.
//
// Reserve ring: row b owns reserve[b * slots + s] for s < slots; reserve_head
// [b] counts the pages row b has taken, and the next page is slot
// head % slots.  A taken slot is set to -1; the host refills slots ahead of
// use.  A row that needs a page and finds -1 is an error (bit 1 of status),
// as is a table that would outgrow the indices buffer (bit 2) or a malformed
// table (bit 4): then the table is left unchanged and every row's slot is
// set to page -1, which the append kernels skip.
//
// One workgroup does it all.  Room for the new pages is made by moving
// indices toward the end in place: every row's entries move right by the
// number of rows before it that take a page, a map that is strictly
// increasing, so tiles processed from the end of the table, all reads of a
// tile before any of its writes, never overwrite an entry not yet read.
#include "pl_common.h"

namespace pl {
namespace pt {

constexpr int kThreads = 1024;
constexpr int kPerThread = 8;                 // entries each thread carries per move tile
constexpr int kTile = kThreads * kPerThread;  // entries per move tile
constexpr int kMaxRows = 4096;                // rows per table (LDS-resident row data)

enum : int { kMissingPage = 1, kNoRoom = 2, kBadTable = 4 };

__global__ __launch_bounds__(kThreads) void advance_kernel(
    int32_t* __restrict__ indptr, int32_t* __restrict__ indices, int64_t capacity,
    int32_t* __restrict__ last_page_len, int batch, int page_size, int32_t* __restrict__ reserve,
    int slots, int32_t* __restrict__ head, int64_t* __restrict__ positions,
    int64_t* __restrict__ page_id, int64_t* __restrict__ page_offset, int32_t* __restrict__ status) {
  __shared__ int s_ptr[kMaxRows + 1];    // indptr before the advance
  __shared__ int s_shift[kMaxRows + 1];  // rows before b that take a page
  __shared__ int s_last[kMaxRows];       // last_page_len before the advance (0: no page)
  __shared__ int s_scan[kThreads];
  __shared__ int s_err, s_first;
  const int tid = threadIdx.x;
  if (tid == 0) {
    s_err = 0;
    s_first = batch;
  }
  for (int b = tid; b <= batch; b += kThreads) s_ptr[b] = indptr[b];
  __syncthreads();

  // Each thread owns a contiguous run of rows, so a scan over threads is a
  // scan over rows.
  const int per = (batch + kThreads - 1) / kThreads;
  const int r0 = min(batch, tid * per), r1 = min(batch, r0 + per);
  int err = 0, grows = 0, first = batch;
  for (int r = r0; r < r1; ++r) {
    const int a = s_ptr[r], e = s_ptr[r + 1];
    int last = 0;
    if (a < 0 || e < a || (int64_t)e > capacity) {
      err |= kBadTable;
    } else if (e > a) {
      last = last_page_len[r];
      if (last < 1 || last > page_size) err |= kBadTable;
    }
    s_last[r] = last;
    if (last == 0 || last == page_size) {  // no page yet, or the last one is full
      const int h = head[r];
      if (h < 0 || reserve[(int64_t)r * slots + h % slots] < 0) err |= kMissingPage;
      ++grows;
      first = min(first, r);
    }
  }
  s_scan[tid] = grows;
  if (err) atomicOr(&s_err, err);
  if (first < batch) atomicMin(&s_first, first);
  __syncthreads();
  for (int off = 1; off < kThreads; off <<= 1) {  // inclusive scan of page takers
    const int v = tid >= off ? s_scan[tid - off] : 0;
    __syncthreads();
    s_scan[tid] += v;
    __syncthreads();
  }
  const int total_grow = s_scan[kThreads - 1];
  const int old_total = s_ptr[batch];
  {
    int base = s_scan[tid] - grows;
    for (int r = r0; r < r1; ++r) {
      s_shift[r] = base;
      base += (s_last[r] == 0 || s_last[r] == page_size) ? 1 : 0;
    }
  }
  if (tid == 0) {
    s_shift[batch] = total_grow;
    if ((int64_t)old_total + total_grow > capacity) s_err |= kNoRoom;
  }
  __syncthreads();

  if (s_err) {  // leave the table alone; point every slot nowhere
    for (int r = tid; r < batch; r += kThreads) {
      const int n = s_ptr[r + 1] - s_ptr[r];
      positions[r] = n > 0 && s_last[r] > 0 ? (int64_t)(n - 1) * page_size + s_last[r] : 0;
      page_id[r] = -1;
      page_offset[r] = -1;
    }
    if (tid == 0) status[0] = status[0] | s_err;
    return;
  }

  // Move every entry of the rows after the first page taker right by its
  // row's shift, tile by tile from the end of the table.
  const int begin = s_first < batch ? s_ptr[s_first + 1] : old_total;
  for (int hi = old_total; hi > begin; hi -= kTile) {
    const int lo = max(begin, hi - kTile);
    int val[kPerThread], dst[kPerThread];
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
      const int p = lo + tid + k * kThreads;
      dst[k] = -1;
      if (p < hi) {
        // the row holding entry p: the last b with s_ptr[b] <= p (p < s_ptr[batch])
        int lo_b = 0, hi_b = batch;  // s_ptr[lo_b] <= p < s_ptr[hi_b]
        while (hi_b - lo_b > 1) {
          const int mid = (lo_b + hi_b) >> 1;
          if (s_ptr[mid] <= p) lo_b = mid; else hi_b = mid;
        }
        val[k] = indices[p];
        dst[k] = p + s_shift[lo_b];
      }
    }
    __syncthreads();  // every read of this tile precedes any write of it
#pragma unroll
    for (int k = 0; k < kPerThread; ++k)
      if (dst[k] >= 0) indices[dst[k]] = val[k];
  }
  __syncthreads();  // the moved entries are visible to the whole workgroup

  for (int r = r0; r < r1; ++r) {
    const int n = s_ptr[r + 1] - s_ptr[r], last = s_last[r];
    const int na = s_ptr[r] + s_shift[r];
    int pg, fill, pages;
    if (last == 0 || last == page_size) {
      const int h = head[r];
      int32_t* slot = reserve + (int64_t)r * slots + h % slots;
      pg = *slot;
      *slot = -1;
      head[r] = h + 1;
      indices[na + n] = pg;
      fill = 1;
      pages = n + 1;
    } else {
      pg = indices[na + n - 1];
      fill = last + 1;
      pages = n;
    }
    indptr[r] = na;
    last_page_len[r] = fill;
    positions[r] = (int64_t)(pages - 1) * page_size + fill - 1;
    page_id[r] = pg;
    page_offset[r] = fill - 1;
  }
  if (tid == 0) indptr[batch] = old_total + total_grow;
}

}  // namespace pt
}  // namespace pl

using namespace pl;

extern "C" int pl_page_table_advance(int32_t* indptr, int32_t* indices, int64_t indices_capacity,
                                     int32_t* last_page_len, int batch, int page_size, int32_t* reserve,
                                     int reserve_slots, int32_t* reserve_head, int64_t* positions,
                                     int64_t* page_id, int64_t* page_offset, int32_t* status, void* stream) {
  if (batch < 0) return fail(PL_ERR_INVALID, "batch must be >= 0");
  if (batch == 0) return ok();
  if (batch > pt::kMaxRows) return fail(PL_ERR_UNSUPPORTED, "batch %d exceeds %d rows", batch, pt::kMaxRows);
  if (page_size <= 0) return fail(PL_ERR_INVALID, "page_size must be > 0");
  if (reserve_slots <= 0) return fail(PL_ERR_INVALID, "reserve_slots must be > 0");
  if (indices_capacity <= 0 || indices_capacity > INT32_MAX)
    return fail(PL_ERR_INVALID, "indices_capacity must be in [1, 2^31)");
  if (!indptr || !indices || !last_page_len || !reserve || !reserve_head || !positions || !page_id ||
      !page_offset || !status)
    return fail(PL_ERR_INVALID, "null pointer argument");
  hipLaunchKernelGGL(pt::advance_kernel, dim3(1), dim3(pt::kThreads), 0, (hipStream_t)stream, indptr, indices,
                     indices_capacity, last_page_len, batch, page_size, reserve, reserve_slots, reserve_head,
                     positions, page_id, page_offset, status);
  PL_LAUNCH_CHECK("page_table_advance");
  return ok();
}
