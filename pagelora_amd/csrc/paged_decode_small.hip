// Batched paged decode attention for pages whose size is not a multiple of
// 16 tokens (FlashInfer's decode takes any page size; the reference's own
// tests run 2- and 4-token pages: test_paged_kvcache_manager.py:429-543,
// test_flashinfer_backend.py:157-177).  The kernels are those of
// decode_kernels.h with SMALL = true; compiled on its own so the two page
// families build in parallel.
#include "decode_kernels.h"

namespace pl {
namespace decode {

int run_small_pages(const RunArgs& a, int dtype, int d, int g) {
  switch (dtype) {
    case PL_DTYPE_F32: return by_dim<float, true>(a, d, g);
    case PL_DTYPE_F16: return by_dim<f16_t, true>(a, d, g);
    case PL_DTYPE_BF16: return by_dim<bf16_t, true>(a, d, g);
  }
  return fail(PL_ERR_UNSUPPORTED, "dtype %d", dtype);
}

}  // namespace decode
}  // namespace pl
