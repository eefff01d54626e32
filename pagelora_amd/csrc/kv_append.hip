// Write the decode token's K and V rows into their pages (gfx950).
//   K[page_id[b], offset[b], h, :] = k[b, h, :],  V likewise.
// One thread moves 16 bytes; consecutive threads cover one head row, so every
// row is read and written with full 16-byte vector accesses.
//
// Replaces _append_decode_kv_static (model/flashinfer/layer_runner.py:399-412):
// layer_cache.index_put_((page_id, 0|1, offset), k|v).
#include "pl_common.h"

namespace pl {
namespace append {

constexpr int kThreads = 256;

template <int EB>  // element bytes
__global__ __launch_bounds__(kThreads) void append_kernel(
    const char* __restrict__ k, const char* __restrict__ v, int64_t k_sb, int64_t k_sh,
    int64_t v_sb, int64_t v_sh, char* __restrict__ kc, char* __restrict__ vc,
    int64_t page_stride, int64_t token_stride, int64_t head_stride,
    const int64_t* __restrict__ page_id, const int64_t* __restrict__ offset, int batch,
    int num_kv_heads, int head_dim, int64_t num_pages, int page_size) {
  constexpr int kElems = 16 / EB;  // elements per thread
  const int per_row = head_dim / kElems;
  const int64_t total = (int64_t)batch * num_kv_heads * per_row * 2;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kThreads) {
    int64_t r = i;
    const int c = (int)(r % per_row); r /= per_row;
    const int h = (int)(r % num_kv_heads); r /= num_kv_heads;
    const int b = (int)(r % batch);
    const int which = (int)(r / batch);  // 0 = K, 1 = V
    const int64_t p = page_id[b], off = offset[b];
    if (p < 0 || p >= num_pages || off < 0 || off >= page_size) continue;  // outside the pool
    const char* src = which == 0 ? k + (((int64_t)b * k_sb + (int64_t)h * k_sh) + c * kElems) * EB
                                 : v + (((int64_t)b * v_sb + (int64_t)h * v_sh) + c * kElems) * EB;
    char* dst = (which == 0 ? kc : vc) +
                (p * page_stride + off * token_stride + (int64_t)h * head_stride + c * kElems) * EB;
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  }
}

}  // namespace append
}  // namespace pl

using namespace pl;

extern "C" int pl_kv_append(const void* k, const void* v, int64_t k_stride_b, int64_t k_stride_h,
                            int64_t v_stride_b, int64_t v_stride_h, void* k_cache, void* v_cache,
                            int64_t page_stride, int64_t token_stride, int64_t head_stride,
                            int64_t num_pages, int page_size, const int64_t* page_id,
                            const int64_t* offset, int batch, int num_kv_heads, int head_dim,
                            int dtype, void* stream) {
  if (batch < 0 || num_kv_heads <= 0 || head_dim <= 0) return fail(PL_ERR_INVALID, "bad shape");
  if (batch == 0) return ok();
  if (!k || !v || !k_cache || !v_cache || !page_id || !offset)
    return fail(PL_ERR_INVALID, "null pointer argument");
  if (num_pages <= 0 || page_size <= 0) return fail(PL_ERR_INVALID, "num_pages and page_size must be > 0");
  if (dtype != PL_DTYPE_F32 && dtype != PL_DTYPE_F16 && dtype != PL_DTYPE_BF16)
    return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
  const int eb = dtype_bytes(dtype);
  const int per = 16 / eb;
  if (head_dim % per) return fail(PL_ERR_INVALID, "head_dim must be a multiple of %d", per);
  const int64_t strides[] = {k_stride_b, k_stride_h, v_stride_b, v_stride_h, page_stride,
                             token_stride, head_stride};
  for (int64_t s : strides)
    if (s % per) return fail(PL_ERR_INVALID, "strides must be multiples of %d elements", per);
  const void* ptrs[] = {k, v, k_cache, v_cache};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return fail(PL_ERR_INVALID, "k, v and caches must be 16-byte aligned");
  const int64_t work = (int64_t)batch * num_kv_heads * (head_dim / per) * 2;
  int64_t grid = (work + append::kThreads - 1) / append::kThreads;
  if (grid > 4096) grid = 4096;
  hipStream_t s = (hipStream_t)stream;
  if (eb == 4)
    hipLaunchKernelGGL(append::append_kernel<4>, dim3((unsigned)grid), dim3(append::kThreads), 0, s,
                       (const char*)k, (const char*)v, k_stride_b, k_stride_h, v_stride_b, v_stride_h,
                       (char*)k_cache, (char*)v_cache, page_stride, token_stride, head_stride,
                       page_id, offset, batch, num_kv_heads, head_dim, num_pages, page_size);
  else
    hipLaunchKernelGGL(append::append_kernel<2>, dim3((unsigned)grid), dim3(append::kThreads), 0, s,
                       (const char*)k, (const char*)v, k_stride_b, k_stride_h, v_stride_b, v_stride_h,
                       (char*)k_cache, (char*)v_cache, page_stride, token_stride, head_stride,
                       page_id, offset, batch, num_kv_heads, head_dim, num_pages, page_size);
  PL_LAUNCH_CHECK("kv append_kernel");
  return ok();
}
