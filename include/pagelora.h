/*
 * pagelora.h — C ABI of the MI355X (gfx950) paged-decode + no-merge LoRA library.
 *
 * Every entry point is stream ordered: it enqueues work on `stream` (a
 * hipStream_t passed as void*, NULL = the legacy default stream) and returns
 * without synchronising.  None of them allocates device memory: scratch space
 * is the caller's `workspace` (pl_decode_noalloc: a fixed array the library
 * holds per device).  Return value: PL_OK (0) or a pl_status code;
 * pl_last_error() then holds a message for the calling thread.
 *
 * Pointers are device pointers unless a parameter name ends in `_h` (host).
 * Strides are in elements, not bytes.
 */
#ifndef PAGELORA_H_
#define PAGELORA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  PL_DTYPE_F32 = 0,
  PL_DTYPE_F16 = 1,
  PL_DTYPE_BF16 = 2,
} pl_dtype;

typedef enum {
  PL_OK = 0,
  PL_ERR_INVALID = 1,      /* bad argument (shape, stride, null pointer)     */
  PL_ERR_UNSUPPORTED = 2,  /* valid but not built (head_dim, group, dtype)  */
  PL_ERR_WORKSPACE = 3,    /* workspace too small for the requested plan    */
  PL_ERR_HIP = 4,          /* a HIP runtime call failed                     */
} pl_status;

/* Message describing the last failure on this thread ("" if none). */
const char* pl_last_error(void);

/* Library ABI version: (major << 16) | minor. */
int pl_version(void);

/* ------------------------------------------------------------------------ */
/* Paged decode attention                                                    */
/* ------------------------------------------------------------------------ */

/*
 * Bytes of workspace that pl_decode_plan / pl_decode_run need for `batch`
 * rows, `target_items` split-KV work items, `num_qo_heads` query heads and
 * `head_dim`.  The plan may create up to target_items + batch items.
 *
 * Replaces the workspace sizing of FlashInferAttentionBackend.__init__
 * (model/flashinfer/attention_backend.py:42-43): the reference hands a fixed
 * 128 MiB buffer to FlashInfer; here the caller can size it exactly.
 */
size_t pl_decode_workspace_size(int batch, int target_items, int num_qo_heads,
                                int head_dim);

/*
 * Device-side split-KV planning for one decode step.  Reads the page-table
 * row pointer `indptr` [batch+1] (int32, device) and writes into `workspace`
 * a work list of (row, page range) items of near-equal size:
 *   chunk_pages = max(min_chunk_pages, ceil(total_pages / target_items)).
 * Page ranges are clamped to [0, indices_capacity], the length of the
 * indices buffer the run will read.
 * No host read-back: the plan runs on the stream, so it can sit inside a
 * captured hipGraph and one graph replays across steps whatever the lengths.
 * For batches of up to 16 rows nothing is launched: the library records
 * the indptr pointer and the split parameters against `workspace` (host
 * state of the library), and the runs on that workspace derive the same
 * chunking from indptr inside their kernels (items in row order).  indptr is
 * then not snapshotted: the runs read it when they execute, so it must stay
 * valid (and hold the step's row pointer) until then, and a workspace that
 * is freed should be released with pl_decode_forget.
 * PAGELORA_DECODE_PLAN_KERNEL=1 in the environment keeps the plan kernel for
 * every batch.
 *
 * Replaces FlashInferAttentionBackend.plan_decode / _call_plan
 * (model/flashinfer/attention_backend.py:63-118, 229-285), which call
 * flashinfer.BatchDecodeWithPagedKVCacheWrapper.plan with a host read-back
 * of indptr.
 */
int pl_decode_plan(const int32_t* indptr, int batch, int indices_capacity,
                   int num_qo_heads, int head_dim, int target_items,
                   int min_chunk_pages, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * Drops the direct plan the library holds for `workspace` (see
 * pl_decode_plan), so a later allocation at the same address cannot inherit
 * it; runs on that workspace then need a fresh plan.  Call it before freeing
 * a decode workspace.  Returns PL_OK whether or not a plan was held.  No
 * counterpart in the reference: FlashInfer's wrapper keeps its plan in the
 * wrapper object (attention_backend.py:63-118), whose lifetime is the
 * workspace's.
 */
int pl_decode_forget(const void* workspace);

/*
 * pl_decode_plan for a batch whose rows all begin with the same
 * shared_pages page ids (a shared prompt prefix held in shared pages; a
 * multiple of prefix_chunk_pages, and fewer than every row's page count).
 * pl_decode_run_qkv then attends the prefix once for all rows: items of
 * prefix_chunk_pages pages, each scoring every row's query heads of one kv
 * head as the columns of one MFMA tile, and each row's own items cover its
 * pages after the prefix; the merge combines both.  Taken when the batch
 * has at most 4 rows, GQA 4, head_dim 128, prefix_chunk_pages * page_size
 * == 32 and the LoRA (if any) binds one adapter; otherwise, and in
 * pl_decode_run, every row reads every page as after pl_decode_plan.  The
 * results equal the unshared run's up to the order of the softmax merge.
 * Needs the direct plan (batch <= 16, see above) and a workspace of
 * pl_decode_workspace_size_shared bytes; a larger batch, or the plan kernel
 * forced by PAGELORA_DECODE_PLAN_KERNEL=1, is planned as by pl_decode_plan
 * (shared_pages ignored).  No counterpart in the reference:
 * its decode wrapper reads a shared page once per row (FlashInfer's
 * BatchDecodeWithPagedKVCacheWrapper, attention_backend.py:63-131).
 */
size_t pl_decode_workspace_size_shared(int batch, int target_items,
                                       int num_qo_heads, int head_dim,
                                       int shared_pages,
                                       int prefix_chunk_pages);
int pl_decode_plan_shared(const int32_t* indptr, int batch,
                          int indices_capacity, int num_qo_heads,
                          int head_dim, int target_items, int min_chunk_pages,
                          int shared_pages, int prefix_chunk_pages,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/*
 * Batched single-token paged attention:
 *   o[b, hq] = softmax(q[b, hq] . K_b[:, hq / g]^T * sm_scale) . V_b
 * with g = num_qo_heads / num_kv_heads, K_b / V_b gathered from the pages
 * indices[indptr[b] .. indptr[b+1]) (all full except the last, which holds
 * last_page_len[b] tokens).  Token t of page p, kv head h, dim d lives at
 *   k_cache[p * page_stride + t * token_stride + h * head_stride + d]
 * (same for v_cache; page ids outside [0, num_pages) are clamped into the
 * pool rather than read out of bounds), which covers the reference's NHD pool
 * [P, 2, page, Hkv, D] (k_cache = pool, v_cache = pool + page*Hkv*D,
 * page_stride = 2*page*Hkv*D) as well as split K/V tensors and HND pages.
 * q is [batch, num_qo_heads, head_dim] with strides (q_stride_b,
 * q_stride_h, 1); o likewise.  lse (nullable) receives the natural-log
 * log-sum-exp of the scaled scores, [batch, num_qo_heads] fp32.
 * q, caches and o share `dtype`; accumulation is fp32.
 * Requires a pl_decode_plan on the same workspace earlier on the stream.
 * head_dim: 64, 128 or 256.  num_qo_heads / num_kv_heads: any positive
 * integer (groups above 8 run as several waves of at most 8 query heads per
 * kv head).  page_size: 1..65536; pages of a multiple of 16 tokens take the
 * scalar-addressed path, other sizes a per-lane page lookup.
 *
 * Replaces FlashInferAttentionBackend.run_decode / _call_run
 * (model/flashinfer/attention_backend.py:120-131, 287-292), i.e.
 * flashinfer.BatchDecodeWithPagedKVCacheWrapper.run(q / 16, cache) with
 * sm_scale 16/sqrt(D) (attention_backend.py:97) — the same softmax.
 */
int pl_decode_run(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                  const void* k_cache, const void* v_cache,
                  int64_t page_stride, int64_t token_stride,
                  int64_t head_stride, int64_t num_pages,
                  const int32_t* indices,
                  const int32_t* last_page_len, void* o, int64_t o_stride_b,
                  int64_t o_stride_h, float* lse, int batch, int num_qo_heads,
                  int num_kv_heads, int head_dim, int page_size,
                  float sm_scale, int dtype, int target_items, int flags,
                  void* workspace, size_t workspace_bytes, void* stream);

/* pl_decode_run flags.  0 launches both of the run's kernels: the split-KV
 * decode kernel and the merge of split rows.  A caller may launch them as
 * two calls (SKIP_MERGE, then MERGE_ONLY with the same arguments) to place
 * other work or timing events between them. */
#define PL_DECODE_SKIP_MERGE 1
#define PL_DECODE_MERGE_ONLY 2

/*
 * Plan + run of one decode step with no caller workspace and no allocation:
 * pl_decode_plan(indptr, ...) followed by pl_decode_run(..., flags 0), with
 * the work list and split partials in a fixed scratch array the library
 * holds on each device (PL_DECODE_NOALLOC_MAX_BYTES; every GPU the library
 * runs on keeps its copy until the process ends).  Arguments are those of
 * the two calls.  A plan that needs more scratch than the maximum
 * (pl_decode_workspace_size(batch, target_items, num_qo_heads, head_dim))
 * is rejected with PL_ERR_WORKSPACE before any HIP call.  `stream` must
 * belong to the current device.  Every call on a GPU shares that GPU's
 * scratch and re-plans into it, so calls that overlap on one GPU (other
 * streams, other threads) race; calls ordered on one stream do not.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate:
 * code under hipGraph capture, tight serving loops, and harnesses that
 * forbid hipMalloc.
 */
#define PL_DECODE_NOALLOC_MAX_BYTES ((size_t)16 << 20)
int pl_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                      const void* k_cache, const void* v_cache,
                      int64_t page_stride, int64_t token_stride,
                      int64_t head_stride, int64_t num_pages,
                      const int32_t* indptr, int indices_capacity,
                      const int32_t* indices, const int32_t* last_page_len,
                      void* o, int64_t o_stride_b, int64_t o_stride_h,
                      float* lse, int batch, int num_qo_heads,
                      int num_kv_heads, int head_dim, int page_size,
                      float sm_scale, int dtype, int target_items,
                      int min_chunk_pages, void* stream);

/*
 * Write one decode token per row into its page:
 *   K[page_id[b], offset[b], h, :] = k[b, h, :]   (and V from v)
 * with the cache addressed as in pl_decode_run.  k and v are
 * [batch, num_kv_heads, head_dim] with strides (k_stride_b, k_stride_h, 1).
 * page_id / offset are int64 (the graph-owned buffers of the reference);
 * a row whose page_id is outside [0, num_pages) or whose offset is outside
 * [0, page_size) is skipped rather than written out of bounds.
 *
 * Replaces _append_decode_kv_static (model/flashinfer/layer_runner.py:399-412),
 * two torch index_put_ calls into the paged pool.
 */
int pl_kv_append(const void* k, const void* v, int64_t k_stride_b,
                 int64_t k_stride_h, int64_t v_stride_b, int64_t v_stride_h,
                 void* k_cache, void* v_cache, int64_t page_stride,
                 int64_t token_stride, int64_t head_stride, int64_t num_pages,
                 int page_size, const int64_t* page_id, const int64_t* offset,
                 int batch, int num_kv_heads, int head_dim, int dtype,
                 void* stream);

/* ------------------------------------------------------------------------ */
/* Paged prefill attention                                                   */
/* ------------------------------------------------------------------------ */

/*
 * Host-side plan of a paged prefill: validates the host tables qo_indptr_h
 * [batch+1], kv_indptr_h [batch+1] and kv_last_page_len_h [batch] (int32)
 * and writes the work list items_h (int32 pairs (request, first row),
 * longest first) for pl_prefill_run, which reads it from device memory.
 * *num_items_h receives the item count; with items_h == NULL only the count
 * is computed.  A request's rows are its
 * qo_len * (num_qo_heads / num_kv_heads) (position, group head) pairs, 64
 * per item.  Under `causal` every request needs qo_len <= kv_len.
 * PL_ERR_WORKSPACE if more than max_items items are needed.
 *
 * Replaces FlashInferAttentionBackend.plan_prefill
 * (model/flashinfer/attention_backend.py:133-170), i.e.
 * flashinfer.BatchPrefillWithPagedKVCacheWrapper.plan.
 */
int pl_prefill_plan(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                    const int32_t* kv_last_page_len_h, int batch,
                    int num_qo_heads, int num_kv_heads, int page_size,
                    int causal, int32_t* items_h, int max_items,
                    int* num_items_h);

/*
 * Multi-token paged attention over packed queries:
 *   o[t, hq] = softmax(q[t, hq] . K_r[:, hq / g]^T * sm_scale [+ mask]) . V_r
 * for the tokens t of request r, qo_indptr[r] <= t < qo_indptr[r+1], which
 * are the LAST qo_len positions of the request's kv_len tokens (pages
 * kv_indices[kv_indptr[r] ..], addressed as in pl_decode_run).  With
 * `causal`, query j of a request sees kv positions <= kv_len - qo_len + j.
 * q and o are [tokens, num_qo_heads, head_dim] with strides (stride_t,
 * stride_h, 1); all tables and `items` (from pl_prefill_plan) are device
 * arrays.  q, caches and o share `dtype` (F16 or BF16); accumulation is
 * fp32.  head_dim: 64, 128 or 256.  Strides must be multiples of 8
 * elements and q, o and the caches 16-byte aligned.
 *
 * Replaces FlashInferAttentionBackend.run_prefill
 * (model/flashinfer/attention_backend.py:172-190), i.e.
 * BatchPrefillWithPagedKVCacheWrapper.run(q / 16, cache) with sm_scale
 * 16/sqrt(D) — the same softmax.
 */
int pl_prefill_run(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                   const void* k_cache, const void* v_cache,
                   int64_t page_stride, int64_t token_stride,
                   int64_t head_stride, int64_t num_pages,
                   const int32_t* qo_indptr, const int32_t* kv_indptr,
                   const int32_t* kv_indices,
                   const int32_t* kv_last_page_len, const int32_t* items,
                   int num_items, void* o, int64_t o_stride_t,
                   int64_t o_stride_h, int batch, int num_qo_heads,
                   int num_kv_heads, int head_dim, int page_size, int causal,
                   float sm_scale, int dtype, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused element-wise ops of the decode layer                                */
/* ------------------------------------------------------------------------ */

/*
 * out[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * weight, fp32 statistics, one
 * rounding.  rows x hidden with row strides ldx / ldo; hidden % 8 == 0.
 * Replaces apply_rmsnorm (model/flashinfer/norm.py:15-24, 60-65).
 */
int pl_rmsnorm(const void* x, int64_t ldx, const void* weight, void* out,
               int64_t ldo, int rows, int hidden, float eps, int dtype,
               void* stream);

/*
 * residual[r] += x[r] (stored in the storage type), then
 * out[r] = rmsnorm(residual[r]) as pl_rmsnorm.
 * Replaces add_residual_rmsnorm (model/flashinfer/norm.py:27-57).
 */
int pl_add_rmsnorm(void* residual, int64_t ldr, const void* x, int64_t ldx,
                   const void* weight, void* out, int64_t ldo, int rows,
                   int hidden, float eps, int dtype, void* stream);

/*
 * out[r, i] = silu(gate_up[r, i]) * gate_up[r, inter + i], fp32, one rounding.
 * Replaces apply_gate_up_activation / flashinfer.silu_and_mul
 * (model/flashinfer/packed_ops.py:230-239).
 */
int pl_silu_mul(const void* gate_up, int64_t ldg, void* out, int64_t ldo,
                int rows, int inter, int dtype, void* stream);

/*
 * Per decode token b, from the packed projection row qkv[b] = [q | k | v]
 * (num_qo_heads, num_kv_heads, num_kv_heads heads of head_dim):
 *   q_out[b, h] = rope(rmsnorm(q[b, h]) * q_norm_weight)     (norm skipped if the weight is NULL)
 *   K[page_id[b], offset[b], h] = rope(rmsnorm(k[b, h]) * k_norm_weight)
 *   V[page_id[b], offset[b], h] = v[b, h]
 * rope: non-interleaved rotate-half, angle(i) = positions[b] * inv_freq[i]
 * in fp32, inv_freq[head_dim/2] (fp32, device) being the caller's table
 * (1 / theta^(2i/head_dim), divided by a linear rope scale).  K/V addressed
 * as in pl_decode_run; a slot outside the pool is skipped.  q_out is
 * [batch, num_qo_heads, head_dim].
 * Replaces project_qkv_with_optional_norm's head norm + apply_rope_pos_ids
 * + _append_decode_kv_static (model/flashinfer/projection.py:155-190,
 * 248-260; layer_runner.py:399-412).
 */
int pl_qk_norm_rope_append(const void* qkv, int64_t ld_qkv,
                           const void* q_norm_weight, const void* k_norm_weight,
                           const int64_t* positions, const int64_t* page_id,
                           const int64_t* offset, void* q_out, void* k_cache,
                           void* v_cache, int64_t page_stride,
                           int64_t token_stride, int64_t head_stride,
                           int64_t num_pages, int page_size, int batch,
                           int num_qo_heads, int num_kv_heads, int head_dim,
                           const float* inv_freq, float eps, int dtype,
                           void* stream);

/* ------------------------------------------------------------------------ */
/* The same ops with the LoRA up-projection of their input applied first     */
/* ------------------------------------------------------------------------ */

/*
 * The up-projection (expand) half of a no-merge LoRA module, applied by the
 * kernel that consumes the module's output.  The producer GEMM ran on the
 * base weight with the adapters' A rows stacked under it ([W; A_0; A_1 ..]),
 * so its output row t holds, besides the base columns, the rank-space
 * intermediate y[t, a] = x[t] . A_a^T of every adapter a (in the storage
 * type, as the reference's F.linear(x, A) returns it) at columns
 * y_offset + a * rank .. + rank of y (row stride ldy).  For the token's
 * adapter a = adapter_ids[t] (0 <= a < num_adapters; other ids add nothing):
 *   value[t, c] = round(base[t, c] + scale * sum_j y[t, a, j] * B[a][c][j])
 * with B [num_adapters, out_features, rank] (rank % 8 == 0, <= 128).  That
 * is LoRALinear.forward / _packed_lora_delta's module output
 * (multilora/linear.py:226-231, model/flashinfer/packed_ops.py:314-325)
 * without a separate expand kernel.
 *
 * b_layout says how B is stored.  PL_LORA_B_ROWS: row-major
 * [num_adapters, out_features, rank], the nn.Linear weight of lora_B.
 * PL_LORA_B_CHUNK8 (out_features % 8 == 0): the same values as
 * [num_adapters, nblk, 8, rank / 8, 64, 8] with nblk = ceil(out_features /
 * 512), element (a, j, i, k, l, e) = B[a][8 (64 j + l) + i][8k + e] (zero
 * past out_features).  A wave whose 64 threads own 8 consecutive output
 * columns each reads its block j as one contiguous region, every load
 * instruction 1 KiB contiguous, where the row-major layout makes each
 * thread's 16-byte piece a separate cache line.
 */
#define PL_LORA_B_ROWS 0
#define PL_LORA_B_CHUNK8 1
/*
 * adapter: -1 selects each token's adapter from adapter_ids (as above).
 * 0 <= adapter < num_adapters binds that one adapter to every token, the
 * reference's model (one active adapter per batch, multilora/runtime.py:
 * 138-174); adapter_ids may then be null.  Kernels then skip the
 * adapter-id load, and its dependent round trip, in front of the y and B
 * reads.  All modules of one call must agree on it.
 */
typedef struct {
  const void* y;
  int64_t ldy;
  int y_offset;
  const void* B;
  int out_features;
  int rank;
  float scale;
  int b_layout;
  int adapter;
} pl_lora_up;

/*
 * A GEMM output given as split-K partial sums (pl_linear_shuffled_split):
 * element (t, c) is the fp32 sum over planes s = 0, 1, .. splits-1, in that
 * order, of partials[s * plane_stride + t * ld + c], rounded to the storage
 * type -- the value the unsplit GEMM's output would hold.  ld and
 * plane_stride are multiples of 8; partials is 16-byte aligned.
 */
typedef struct {
  const float* partials;
  int splits;
  int64_t ld;
  int64_t plane_stride;
} pl_split_out;

/*
 * pl_add_rmsnorm with x = the o_proj / down_proj output whose module is
 * lora_h: residual[r] += round(x[r] + delta[r]), then the norm.  With
 * x_split_h (nullable) x and the module's y are read from the split-K
 * partial planes instead (x and lora_h->y are then ignored).
 * Replaces LoRALinear.forward's delta on project_linear's output followed
 * by add_residual_rmsnorm (packed_ops.py:251-265, norm.py:27-57).
 */
int pl_add_rmsnorm_lora(void* residual, int64_t ldr, const void* x,
                        int64_t ldx, const pl_split_out* x_split_h,
                        const pl_lora_up* lora_h,
                        const int32_t* adapter_ids, int num_adapters,
                        const void* weight, void* out, int64_t ldo, int rows,
                        int hidden, float eps, int dtype, void* stream);

/*
 * pl_add_rmsnorm_lora with the module's y read from the side planes of
 * pl_linear_shuffled_side (y_side_h: 1..64 planes, adapter a's rank-space
 * row at columns lora_h->y_offset + a * rank; lora_h->y is ignored), x
 * whole.  The planes are summed in order per rank, then rounded to the
 * dtype as the reference's F.linear(x, A) output is.  16-bit dtypes,
 * hidden <= 8192, rank 8 or 16.  Replaces the same reference code as
 * pl_add_rmsnorm_lora.
 */
int pl_add_rmsnorm_lora_side(void* residual, int64_t ldr, const void* x,
                             int64_t ldx, const pl_split_out* y_side_h,
                             const pl_lora_up* lora_h,
                             const int32_t* adapter_ids, int num_adapters,
                             const void* weight, void* out, int64_t ldo,
                             int rows, int hidden, float eps, int dtype,
                             void* stream);

/*
 * pl_silu_mul with the gate and up modules' deltas (lora_gate_up_h[0] for
 * the gate columns, [1] for the up columns) added to gate_up first.
 * Replaces project_gate_up_packed's delta + silu_and_mul
 * (packed_ops.py:168-203, 230-239).
 */
int pl_silu_mul_lora(const void* gate_up, int64_t ldg,
                     const pl_lora_up* lora_gate_up_h,
                     const int32_t* adapter_ids, int num_adapters, void* out,
                     int64_t ldo, int rows, int inter, int dtype,
                     void* stream);

/*
 * pl_qk_norm_rope_append with the q, k and v modules' deltas
 * (lora_qkv_h[0..2], columns head-major within each module) added to the
 * packed row first.  With qkv_split_h (nullable) the packed rows and the
 * modules' y come from split-K partial planes (qkv and the y pointers are
 * then ignored).  Replaces project_qkv_packed's delta followed by the head
 * norm, RoPE and append (packed_ops.py:105-165, projection.py:155-190).
 */
int pl_qk_norm_rope_append_lora(const void* qkv, int64_t ld_qkv,
                                const pl_split_out* qkv_split_h,
                                const pl_lora_up* lora_qkv_h,
                                const int32_t* adapter_ids, int num_adapters,
                                const void* q_norm_weight,
                                const void* k_norm_weight,
                                const int64_t* positions,
                                const int64_t* page_id, const int64_t* offset,
                                void* q_out, void* k_cache, void* v_cache,
                                int64_t page_stride, int64_t token_stride,
                                int64_t head_stride, int64_t num_pages,
                                int page_size, int batch, int num_qo_heads,
                                int num_kv_heads, int head_dim,
                                const float* inv_freq, float eps, int dtype,
                                void* stream);

/*
 * cos and sin of positions[b] * inv_freq[i] for every row b < batch and
 * rotation pair i < half_dim, as out[b][i] = {cos, sin} (fp32).  The angles
 * of one decode step, which every layer's RoPE shares: the same fp32 product
 * and sincosf as pl_qk_norm_rope_append, computed once per step for
 * pl_decode_run_qkv.  No counterpart in the reference (FlashInfer computes
 * the angles inside apply_rope_pos_ids, projection.py:181).
 */
int pl_rope_cos_sin(const int64_t* positions, int batch, const float* inv_freq,
                    int half_dim, float* out, void* stream);

/*
 * pl_decode_run with the q/k/v epilogue folded in: the kernel reads the
 * packed projection rows qkv [batch, ld_qkv] (q heads, then k heads, then v
 * heads, head-major, head_dim each) instead of a finished q, and
 *   - forms each q head as pl_qk_norm_rope_append(_lora) does: the q
 *     module's LoRA delta (lora_qkv_h[0], nullable as a whole for no LoRA),
 *     RMSNorm with q_norm_weight (nullable), RoPE with the step's angles
 *     rope_cos_sin (from pl_rope_cos_sin);
 *   - appends each row's new token: k (k LoRA, k-norm, RoPE) and v (v LoRA)
 *     of every kv head into (page_id[b], offset[b]) -- slots outside the pool
 *     are skipped -- and attends over the row, that token included.  The
 *     slot is expected where a decode step puts it: the row's last token
 *     (offset last_page_len[b] - 1 of the row's last page), whose K/V the
 *     kernel takes from registers; a slot elsewhere is written, but this
 *     call may read the old contents there;
 *   - attends as pl_decode_run.
 * The plan (pl_decode_plan on the same workspace) must already count the new
 * token.  Built for 16-bit dtypes, head_dim 128, num_qo_heads / num_kv_heads
 * == 4 and LoRA rank 0, 8 or 16 (the three modules share it); other shapes
 * return PL_ERR_UNSUPPORTED (use pl_qk_norm_rope_append + pl_decode_run).
 * q differs from the two-call path by at most the rounding of the head
 * norm's sum (another summation order).  No single counterpart in the
 * reference: it replaces project_qkv_packed's delta, the head norm, RoPE and
 * append (packed_ops.py:105-165, projection.py:155-190,
 * layer_runner.py:399-412) followed by run_decode (attention_backend.py:
 * 120-131) within one decode layer.
 */
int pl_decode_run_qkv(const void* qkv, int64_t ld_qkv,
                      const pl_lora_up* lora_qkv_h, const int32_t* adapter_ids,
                      int num_adapters, const void* q_norm_weight,
                      const void* k_norm_weight, const float* rope_cos_sin,
                      const int64_t* page_id, const int64_t* offset, float eps,
                      void* k_cache, void* v_cache, int64_t page_stride,
                      int64_t token_stride, int64_t head_stride,
                      int64_t num_pages, const int32_t* indices,
                      const int32_t* last_page_len, void* o,
                      int64_t o_stride_b, int64_t o_stride_h, float* lse,
                      int batch, int num_qo_heads, int num_kv_heads,
                      int head_dim, int page_size, float sm_scale, int dtype,
                      int target_items, int flags, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* No-merge multi-adapter LoRA delta                                         */
/* ------------------------------------------------------------------------ */

/*
 * One LoRA-wrapped linear module of a group that shares its input x
 * (q/k/v, or gate/up, or a lone o_proj / down_proj).
 *   A    : [num_adapters, rank, in_features]   (dtype of x)
 *   B    : [num_adapters, out_features, rank]  (dtype of x)
 *   out  : rows t of out[t * ldo + j], j < out_features, receive
 *          out += scale * B[a_t] . (A[a_t] . x_t)
 */
typedef struct {
  const void* A;
  const void* B;
  void* out;
  int64_t ldo;
  int out_features;
  int rank;
  float scale;
} pl_lora_module;

/* Most modules in one group (q, k, v). */
#define PL_LORA_MAX_MODULES 4

/* Workspace bytes for pl_lora_shrink / pl_lora_expand (and pl_linear's
 * LoRA epilogue): the shrink's fp32 partial sums, [k-slices][num_tokens]
 * [sum(rank) rounded up to 32], the slice count depending on num_tokens and
 * in_features.  Calls that share a workspace must be stream ordered; shrink
 * writes it, expand reads it. */
size_t pl_lora_workspace_size(int num_tokens, int in_features,
                              const pl_lora_module* modules_h, int num_modules);

/* One group of modules sharing the input x [num_tokens, in_features] (row
 * stride ldx), for pl_lora_delta_groups. */
typedef struct {
  const void* x;
  int64_t ldx;
  int in_features;
  int num_modules;
  const pl_lora_module* modules;  /* host array of num_modules */
} pl_lora_group;

/* Most groups in one pl_lora_delta_groups call (a decoder layer's four:
 * q/k/v, o, gate/up, down). */
#define PL_LORA_MAX_GROUPS 4

/* Workspace bytes for pl_lora_delta / pl_lora_delta_groups.  The workspace
 * of these two entry points must be zero-filled once before its first use
 * (e.g. at allocation): the decode path keeps double-buffered intermediate
 * accumulators and their parity there from call to call.  Keep it for these
 * two entry points (not pl_lora_shrink, pl_lora_expand or pl_linear), one
 * call at a time (stream-ordered).  Returns 0 for an invalid group list. */
size_t pl_lora_delta_workspace_size(const pl_lora_group* groups_h, int num_groups,
                                    int num_tokens, int num_adapters);

/*
 * out_m[t] += scale_m * B_m[a_t] . (A_m[a_t] . x[t]) for every module m of the
 * group and every token t with adapter_ids[t] in [0, num_adapters); tokens
 * with a negative id are left untouched.  x is [num_tokens, in_features]
 * with row stride ldx.  `dtype` is that of x, A and B (F16 or BF16);
 * `out_dtype` that of the outputs (F16, BF16 or F32).  The rank-r
 * intermediate is rounded to `dtype` before the expand, as the reference's
 * two chained F.linear calls do.
 *
 * Replaces the packed / per-module LoRA delta of the no-merge path:
 * _packed_lora_delta + _cached_packed_lora_delta
 * (model/flashinfer/packed_ops.py:314-384; A concatenated, B block-diagonal
 * with the scale folded in), _lora_delta (packed_ops.py:534-553) and the
 * delta term of LoRALinear.forward (multilora/linear.py:226-231).  Per-token
 * adapter ids generalise the reference's single bound adapter
 * (multilora/runtime.py:138-174).
 *
 * Workspace: pl_lora_delta_workspace_size of the one group, zero-filled
 * before its first use (see there).  Up to 64 tokens and 64 adapters, with
 * ranks, out_features and ldo multiples of 8 and B and the outputs 16-byte
 * aligned, the call is two launches built for decode latency; otherwise the
 * general shrink + expand pair (same results to the stated tolerance).
 *
 * Non-finite values propagate as the reference's packed product
 * F.linear(F.linear(x, A_cat), B_bd) propagates them: a NaN or infinity in
 * x or A makes the intermediate of that (token, rank) NaN or infinite, and
 * the expand carries it into every output column of the group for that
 * token (0 * inf = NaN through the block-diagonal B, as in the reference's
 * dense B_bd).  Tokens of other adapters are not affected by x or A; a
 * non-finite value in the B of an adapter reaches every token of the call.
 * The decode path sums the k-split in fixed point: a finite partial of
 * magnitude above 2^31 saturates there.
 */
int pl_lora_delta(const void* x, int64_t ldx, int num_tokens, int in_features,
                  const pl_lora_module* modules_h, int num_modules,
                  const int32_t* adapter_ids, int num_adapters, int dtype,
                  int out_dtype, void* workspace, size_t workspace_bytes,
                  void* stream);

/*
 * pl_lora_delta for up to PL_LORA_MAX_GROUPS groups with their own inputs
 * (e.g. a decoder layer's q/k/v, o, gate/up and down deltas when their
 * inputs are at hand together), one adapter id per token shared by all
 * groups.  At decode sizes (<= 64 tokens, <= 64 adapters) all groups share
 * the same two launches; otherwise they run one after another.  Groups must
 * not write the same outputs.  No counterpart in the reference, which runs
 * each module's delta inside its projection (packed_ops.py:105-265).
 */
int pl_lora_delta_groups(const pl_lora_group* groups_h, int num_groups, int num_tokens,
                         const int32_t* adapter_ids, int num_adapters, int dtype,
                         int out_dtype, void* workspace, size_t workspace_bytes,
                         void* stream);

/* The two stages of pl_lora_delta, for callers that overlap them with the
 * base GEMM: shrink writes the fp32 partial sums into the workspace, expand
 * reduces them and accumulates into the outputs. */
int pl_lora_shrink(const void* x, int64_t ldx, int num_tokens,
                   int in_features, const pl_lora_module* modules_h,
                   int num_modules, const int32_t* adapter_ids,
                   int num_adapters, int dtype, void* workspace,
                   size_t workspace_bytes, void* stream);
int pl_lora_expand(int num_tokens, int in_features,
                   const pl_lora_module* modules_h, int num_modules,
                   const int32_t* adapter_ids, int num_adapters, int dtype,
                   int out_dtype, const void* workspace,
                   size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Decode-sized linear layer with the fused LoRA expand                      */
/* ------------------------------------------------------------------------ */

/* Most tokens pl_linear takes (it re-reads W once per 16 tokens). */
#define PL_LINEAR_MAX_TOKENS 64

/* A LoRA module whose delta pl_linear adds to its output columns
 * [col_offset, col_offset + out_features); B as in pl_lora_module. */
typedef struct {
  const void* B;
  int col_offset;
  int out_features;
  int rank;
  float scale;
} pl_linear_lora;

/*
 * out[t, :] = x[t] . W^T (+ bias) (+ sum_m scale_m * B_m[a_t] . y_m[t])
 * for num_tokens <= PL_LINEAR_MAX_TOKENS, W [out_features, in_features]
 * (row stride ldw) streamed once, fp32 accumulation, one rounding.
 * With num_lora > 0, y is the rank-r intermediate of the same group
 * produced by pl_lora_shrink on lora_workspace just before (same x, same
 * modules in the same order, same adapter_ids): the expand runs in this
 * kernel's epilogue instead of a separate pl_lora_expand launch.
 * dtype: F16 or BF16 for x, W, bias, B and out.
 *
 * Replaces the base F.linear of the packed / per-module projections
 * (model/flashinfer/packed_ops.py:143, 179, 251-265) together with the
 * LoRA up-projection of _packed_lora_delta / LoRALinear.forward
 * (packed_ops.py:325; multilora/linear.py:230-231).
 */
int pl_linear(const void* x, int64_t ldx, int num_tokens, int in_features,
              const void* weight, int64_t ldw, int out_features,
              const void* bias, void* out, int64_t ldo,
              const pl_linear_lora* lora_h, int num_lora,
              const int32_t* adapter_ids, int num_adapters,
              const void* lora_workspace, size_t lora_workspace_bytes,
              int dtype, void* stream);

/* ------------------------------------------------------------------------ */
/* Decode-sized linear layer on pre-shuffled weights                          */
/* ------------------------------------------------------------------------ */

/*
 * Bytes of the shuffled copy of a [out_features, in_features] weight
 * (rows padded to a multiple of 16); 0 when in_features is not a positive
 * multiple of 32.
 */
size_t pl_weight_shuffled_bytes(int out_features, int in_features);

/*
 * Re-lays a row-major weight W [out_features, in_features] (row stride ldw,
 * F16 or BF16) once, at load time, into 1 KiB blocks in the lane order of
 * the MFMA B operand:
 *   shuffled[((nb * in/32 + ks) * 64 + l) * 8 + e]
 *     = W[nb*16 + l%16][ks*32 + (l/16)*8 + e]      (0 for rows >= out_features)
 * so that pl_linear_shuffled reads every weight byte with fully coalesced
 * 1 KiB wave loads.  shuffled_bytes >= pl_weight_shuffled_bytes(...).
 * No counterpart in the reference: the weight layout of the decode GEMM.
 */
int pl_weight_shuffle(const void* weight, int64_t ldw, int out_features,
                      int in_features, void* shuffled, size_t shuffled_bytes,
                      int dtype, void* stream);

/*
 * The inverse of pl_weight_shuffle: rows 0 .. out_features of the row-major
 * weight (row stride ldw, 16-byte aligned rows) from its shuffled copy.  The
 * decoder keeps only the shuffled copy of its projection weights and runs
 * this per layer into one reusable buffer when a library GEMM (prefill)
 * needs the row-major form.  No counterpart in the reference, which keeps
 * nn.Linear weights row-major.
 */
int pl_weight_unshuffle(const void* shuffled, size_t shuffled_bytes, int out_features,
                        int in_features, void* weight, int64_t ldw, int dtype,
                        void* stream);

/*
 * out[t, n] = x[t] . W[n]^T (+ bias[n]) for t < num_tokens (<= 64) from the
 * shuffled weight of pl_weight_shuffle (same out_features / in_features).
 * x [num_tokens, in_features] with row stride ldx, out with ldo; fp32
 * accumulation, one rounding.  Replaces the base F.linear of
 * project_qkv_packed / project_gate_up_packed / project_linear
 * (model/flashinfer/packed_ops.py:143, 179, 251-265) at decode batch sizes.
 */
int pl_linear_shuffled(const void* x, int64_t ldx, int num_tokens,
                       int in_features, const void* shuffled,
                       int out_features, const void* bias, void* out,
                       int64_t ldo, int dtype, void* stream);

/*
 * pl_linear_shuffled with K split over `splits` workgroups per 16-column
 * block: workgroup s sums k in [s*K/splits, (s+1)*K/splits) (whole 32-wide
 * steps) and writes fp32 plane s of partials (row t at t * ld, planes
 * plane_stride >= num_tokens * ld apart), no bias.  The consumer sums the
 * planes in order (pl_split_out).  More workgroups for narrow projections
 * (o_proj, down_proj: 257 row blocks for 4096 outputs) without a
 * cross-workgroup reduction inside the kernel.
 */
int pl_linear_shuffled_split(const void* x, int64_t ldx, int num_tokens,
                             int in_features, const void* shuffled,
                             int out_features, int splits, float* partials,
                             int64_t ld, int64_t plane_stride, int dtype,
                             void* stream);

/*
 * pl_linear_shuffled whose last out_features - main_features outputs (the
 * LoRA A rows stacked under W) are split-K: columns c < main_features are
 * written whole to out (no bias); the others, as in pl_linear_shuffled_split,
 * to side_splits fp32 planes of side_partials (column c - main_features, row
 * t at t * ld_side, planes side_plane_stride apart), computed by side_splits
 * small workgroups per 16-column block appended to the grid.  main_features
 * must be a multiple of 16.  With main_features a multiple of 16 x the CU
 * count (4096 on 256 CUs) every CU streams one whole block, where one more
 * whole block would cost some CU two.  The consumer reads y from the planes
 * (pl_add_rmsnorm_lora_side).  No counterpart in the reference: it computes
 * the same x . [W; A]^T as project_linear with its LoRA shrink
 * (packed_ops.py:251-265, linear.py:226-231).
 */
int pl_linear_shuffled_side(const void* x, int64_t ldx, int num_tokens,
                            int in_features, const void* shuffled,
                            int out_features, int main_features, void* out,
                            int64_t ldo, int side_splits, float* side_partials,
                            int64_t ld_side, int64_t side_plane_stride,
                            int dtype, void* stream);

/*
 * The rank-space row y = x . A_a^T of a LoRA module for each token's own
 * adapter a, as fp32 partial sums written by the kernel that produces x:
 * y[t][r] is the sum over p = 0 .. parts-1 of partials[t * ld + p * rank + r].
 * The consumer adds them in a fixed order, so repeated calls give the same
 * bits.  ld >= parts * rank.
 */
typedef struct {
  float* partials;
  int64_t ld;
  int parts;
  int rank;
} pl_lora_partials;

/*
 * A LoRA module's A rows inside its shuffled weight (pl_weight_shuffle of
 * the out_features rows [W; A_0; A_1; ..], in_features wide): adapter a's
 * rank r is row a_row0 + a * rank + r, and a_row0 + num_adapters * rank <=
 * out_features.  adapter >= 0 binds that adapter to every token; -1 takes
 * each token's adapter from the call's adapter_ids.  A token whose adapter
 * lies outside [0, num_adapters) gets partials of adapter 0, which the
 * consumer then does not apply.
 */
typedef struct {
  const void* shuffled;
  int in_features;
  int out_features;
  int a_row0;
  int rank;
  int adapter;
} pl_lora_a_rows;

/*
 * out = RMSNorm(x) . W^T on a shuffled weight for decode batches: the norm
 * (x * rsqrt(mean(x^2) + eps)) * norm_weight, rounded to dtype (the
 * arithmetic of pl_rmsnorm), is formed inside the GEMM, so no normalized row
 * goes through memory.  The sum of squares of row t comes from sq_partials
 * when given -- sq_parts pieces sq_partials[t * ld_sq + j] added in order j =
 * 0, 1, .., as pl_linear_shuffled_add writes them for its output -- and is
 * otherwise formed by every workgroup from the rows (staged in LDS).
 * x_norm_out (nullable, row stride ld_norm_out) also receives the normalized
 * rows.  With sq_partials: num_tokens <= 16, in_features a multiple of 32 up
 * to 8192, sq_parts <= 1024 (ld_sq a multiple of 4); without: num_tokens <=
 * 8, in_features a multiple of 512 up to 8192 with num_tokens * in_features
 * <= 32768.  No counterpart in the reference: it computes the RMSNorm
 * (model/flashinfer/norm.py:15-57) and the projection that reads it
 * (packed_ops.py:143, 179) in one launch.
 */
int pl_linear_shuffled_norm(const void* x, int64_t ldx, int num_tokens,
                            int in_features, const void* norm_weight,
                            float eps, const float* sq_partials, int64_t ld_sq,
                            int sq_parts, const void* shuffled,
                            int out_features, void* out, int64_t ldo,
                            void* x_norm_out, int64_t ld_norm_out, int dtype,
                            void* stream);

/*
 * residual[t][c] += round(round(x . W^T)[t][c] + delta[t][c]) for c <
 * out_features (rows of the shuffled weight past out_features, e.g. LoRA A
 * rows stacked under W, are not read): the projection, its LoRA
 * up-projection delta = scale * y . B_a^T with y from lora_y's partial sums
 * rounded to dtype, and the residual add, rounded as the reference's module
 * output followed by `hidden + out`.  lora / lora_y are both NULL (no
 * delta) or both given (lora->y is ignored; rank 8 or 16); adapter ids
 * as in pl_add_rmsnorm_lora.  out (nullable) receives round(x . W^T).
 * sq_out (nullable) receives, for the next RMSNorm (pl_linear_shuffled_norm's
 * sq_partials), the fp32 sum of squares of the new residual over each block
 * of 16 columns: sq_out[t * ld_sq + j] for columns 16j .. 16j+15 below
 * out_features, ld_sq >= ceil(out_features / 16).  num_tokens <= 16.  No
 * counterpart in the reference: it computes project_linear with
 * LoRALinear.forward's delta (packed_ops.py:251-265,
 * multilora/linear.py:226-231) and the residual add that precedes the next
 * RMSNorm (norm.py:27-57) in one launch.
 */
int pl_linear_shuffled_add(const void* x, int64_t ldx, int num_tokens,
                           int in_features, const void* shuffled,
                           int out_features, void* residual, int64_t ldr,
                           const pl_lora_up* lora,
                           const pl_lora_partials* lora_y,
                           const int32_t* adapter_ids, int num_adapters,
                           void* out, int64_t ldo, float* sq_out,
                           int64_t ld_sq, int dtype, void* stream);

/*
 * pl_decode_run_qkv whose merge also forms o_proj's LoRA shrink: the
 * attention output of each (row, head) -- the input of o_proj -- rounded to
 * dtype as stored, times the same columns of the row's adapter's A rows
 * (o_lora_a, in_features = num_qo_heads * head_dim), as fp32 partial sums
 * o_lora_y: one per (head, dim slice) of each row, parts = num_qo_heads x
 * the merge's dim split (4 while batch * num_qo_heads * 4 <= 256, else 2
 * while batch * num_qo_heads * 2 <= 256, else 1), for pl_linear_shuffled_add.
 * Every row then goes through the merge, single-item rows included.  Rank 8
 * or 16; the adapter binding follows o_lora_a->adapter with adapter_ids and
 * num_adapters as for the q/k/v LoRA.  flags may not skip the merge.  No
 * counterpart in the reference: it computes the first F.linear of o_proj's
 * LoRALinear.forward delta (multilora/linear.py:226-231) inside the decode
 * call.
 */
int pl_decode_run_qkv_oshrink(
    const void* qkv, int64_t ld_qkv, const pl_lora_up* lora_qkv_h,
    const int32_t* adapter_ids, int num_adapters, const void* q_norm_weight,
    const void* k_norm_weight, const float* rope_cos_sin,
    const int64_t* page_id, const int64_t* offset, float eps, void* k_cache,
    void* v_cache, int64_t page_stride, int64_t token_stride,
    int64_t head_stride, int64_t num_pages, const int32_t* indices,
    const int32_t* last_page_len, void* o, int64_t o_stride_b,
    int64_t o_stride_h, float* lse, int batch, int num_qo_heads,
    int num_kv_heads, int head_dim, int page_size, float sm_scale, int dtype,
    int target_items, int flags, void* workspace, size_t workspace_bytes,
    const pl_lora_a_rows* o_lora_a, const pl_lora_partials* o_lora_y,
    void* stream);

/*
 * pl_silu_mul_lora that also forms down_proj's LoRA shrink: the stored
 * output act (down_proj's input), times the same columns of the row's
 * adapter's A rows (down_lora_a, in_features = inter, binding the gate / up
 * modules' adapter), as fp32 partial sums down_lora_y with one part per 256
 * columns (parts = ceil(inter / 256); ld a multiple of 4), for
 * pl_linear_shuffled_add.  16-bit dtypes, gate / up rank up to 16, down rank
 * 8 or 16, inter a multiple of 32.  No counterpart in the reference: it
 * computes the first F.linear of down_proj's LoRALinear.forward delta
 * (multilora/linear.py:226-231) with silu_and_mul (packed_ops.py:230-239).
 */
int pl_silu_mul_lora_shrink(const void* gate_up, int64_t ldg,
                            const pl_lora_up* lora_gate_up_h,
                            const int32_t* adapter_ids, int num_adapters,
                            void* out, int64_t ldo, int rows, int inter,
                            const pl_lora_a_rows* down_lora_a,
                            const pl_lora_partials* down_lora_y, int dtype,
                            void* stream);

/*
 * Advance every row of a batched page table by one decode token, in place
 * on the device (one kernel, no host table, safe to capture in a graph).
 * indptr [batch+1], indices (capacity indices_capacity entries) and
 * last_page_len [batch] are int32 device buffers in the layout pl_decode_plan
 * reads.  A row whose last page has room grows its fill by one; a row whose
 * last page is full, or that has no page, takes page
 * reserve[b * reserve_slots + reserve_head[b] % reserve_slots] (int32), sets
 * that slot to -1 and increments reserve_head[b]; its new page starts with
 * fill 1.  Entries of later rows move right to make room.  The kernel
 * writes each row's decode inputs (int64): positions[b] = the token's
 * position, page_id[b] / page_offset[b] = the slot its K/V row goes to.
 *
 * Errors found on the device leave the table unchanged, set page_id[b] =
 * page_offset[b] = -1 for every row (the append entry points skip such
 * rows) and OR a bit into status[0]: 1 = a row needed a page and its
 * reserve slot held -1, 2 = the table would outgrow indices_capacity,
 * 4 = a malformed table (indptr decreasing or outside [0, capacity],
 * last_page_len outside [1, page_size] on a row with pages).  batch is at
 * most 4096.
 *
 * Replaces the per-step host bookkeeping of the batched decode loop
 * (model/flashinfer/generation.py:1011-1035): reserve_chunk(request, 1) per
 * row (model/kvcache/paged_kvcache_manager.py:195-213 ->
 * model/kvcache/paged_kv_store.py:113-190) and the repack of all rows into
 * the reusable table (model/kvcache/flashinfer_page_table.py:89-121).
 */
int pl_page_table_advance(int32_t* indptr, int32_t* indices,
                          int64_t indices_capacity, int32_t* last_page_len,
                          int batch, int page_size, int32_t* reserve,
                          int reserve_slots, int32_t* reserve_head,
                          int64_t* positions, int64_t* page_id,
                          int64_t* page_offset, int32_t* status, void* stream);

/*
 * Greedy next token: next_tokens[r] = the index of the largest of
 * logits[r, 0 .. vocab) (row stride ld elements, rows 16-byte aligned),
 * int64.  Ties go to the first index and a NaN counts as the largest value
 * (the first NaN wins), as torch.argmax does.  tokens_out (nullable)
 * receives the same indices: the decode step's input-token buffer, so the
 * next step needs no copy.  Each row is split over many workgroups whose
 * partial maxima go to the caller's workspace
 * (pl_greedy_argmax_workspace_size bytes, 8-byte aligned); a second kernel
 * folds them.
 *
 * Replaces greedy_argmax_token (model/flashinfer/sampling.py:8-15).
 */
size_t pl_greedy_argmax_workspace_size(int rows, int vocab, int dtype);
int pl_greedy_argmax(const void* logits, int64_t ld, int rows, int vocab,
                     int dtype, int64_t* next_tokens, int64_t* tokens_out,
                     void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGELORA_H_ */
