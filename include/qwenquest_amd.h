/*
 * qwenquest_amd - C ABI of the MI355X (gfx950) Quest sparse-decode library.
 *
 * Every entry point enqueues HIP kernels on `stream` (a hipStream_t passed as
 * void*; NULL = the default stream) and returns a status:
 *   QQ_OK (0), QQ_EINVAL (bad argument; the Python side raises ValueError),
 *   QQ_ERUNTIME (ordering / capacity; RuntimeError), QQ_EHIP (a HIP error).
 * qq_last_error() returns the message of the last failure on this thread.
 *
 * The library never allocates: the caller owns every buffer (device memory
 * for tensors and workspaces, pinned host memory for the HiSparse host tier)
 * and passes raw pointers plus explicit geometry.  All tensors are dense,
 * row-major, in the layouts of the reference (wengyinqi/QwenQuest):
 *   page_k_bounds  [L, R, MP, KV, D, 2] bf16  (min, max) interleaved
 *   running_k_min/max [L, R, KV, D] bf16, running counters [R] int32
 *   req_to_token   [R, max_ctx] int32,  K/V pool of a layer [rows, KV, D]
 * bf16 tensors are passed as uint16_t bit patterns.
 *
 * Reference file:line citations are relative to the reference repository root.
 */
#ifndef QWENQUEST_AMD_H
#define QWENQUEST_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QQ_OK 0
#define QQ_EINVAL (-1)
#define QQ_ERUNTIME (-2)
#define QQ_EHIP (-3)

#define QQ_DTYPE_BF16 0
#define QQ_DTYPE_F32 1

/* Library version (major*10000 + minor*100 + patch). */
int qq_version(void);
/* Message of the last failing call on this thread ("" if none). */
const char* qq_last_error(void);

/* ------------------------------------------------------------ Quest storage
 * Replaces QuestAlgorithm.init_storage's sentinel fill (src/qwenquest/quest.py:194-208)
 * and QuestAlgorithm.invalidate_request (src/qwenquest/quest.py:468-479):
 * resets requests [req_begin, req_begin + req_count) in every layer - page
 * bounds to (min=+bf16max, max=-bf16max), running bounds to the same
 * sentinels, both counters to 0. */
int qq_quest_reset(uint16_t* page_k_bounds, uint16_t* running_k_min, uint16_t* running_k_max,
                   int32_t* running_token_count, int32_t* running_page_idx, int num_layers,
                   int max_reqs, int max_pages, int kv_heads, int head_dim, int req_begin,
                   int req_count, void* stream);

/* Replaces QuestAlgorithm.update_prefill_representations
 * (src/qwenquest/quest.py:231-280), fused over `n_layers` consecutive layers
 * starting at layer offset `layer_begin` (upstream's
 * update_prefill_representations_fused).  Keys of layer (layer_begin + i) are
 * read from `k_base + i * k_layer_stride` (elements, `k_rows` rows of KV*D
 * elements; rows outside [0, k_rows) are skipped), gathered through
 * `prefill_indices` (int32 or int64, `n_tokens` entries in position order).
 * Complete pages go to page_k_bounds, the partial tail to the running bounds;
 * when `set_counters` the request's counters become (n % P, n / P)
 * (the reference does this on the last layer, quest.py:278-280). */
int qq_quest_prefill_bounds(const void* k_base, int64_t k_layer_stride, int k_dtype,
                            int64_t k_rows, const void* prefill_indices, int indices_are_int64, int64_t n_tokens,
                            int req, int layer_begin, int n_layers, int set_counters,
                            uint16_t* page_k_bounds, uint16_t* running_k_min,
                            uint16_t* running_k_max, int32_t* running_token_count,
                            int32_t* running_page_idx, int num_layers, int max_reqs, int max_pages,
                            int kv_heads, int head_dim, int page_size, void* stream);

/* Replaces QuestAlgorithm.update_decode_representations
 * (src/qwenquest/quest.py:284-302) for layers [layer_begin, layer_begin + n_layers):
 * folds the key at row `device_locs[i]` into request `req_indices[i]`'s
 * running min/max.  An entry with device_locs[i] < 0 is skipped entirely (the
 * reference drops such requests from the call: quest_only.py:88-92).  With `finalize` != 0 (requires the full layer range) it
 * also performs maybe_finalize_decode_representations (quest.py:304-321) in
 * the same pass - upstream's update_decode_representations_fused. */
int qq_quest_decode_update(const void* k_base, int64_t k_layer_stride, int k_dtype,
                           int64_t k_rows, const int64_t* req_indices, const int64_t* device_locs, int n,
                           int layer_begin, int n_layers, int finalize, uint16_t* page_k_bounds,
                           uint16_t* running_k_min, uint16_t* running_k_max,
                           int32_t* running_token_count, int32_t* running_page_idx,
                           int num_layers, int max_reqs, int max_pages, int kv_heads,
                           int head_dim, int page_size, void* stream);

/* Replaces the row lookup of QuestOnlyBackend._do_quest_decode_step_update
 * (src/qwenquest/attention/quest_only.py:84-97): for batch entry i, request
 * r = req_pool_indices[i], the previous step's token sits at position
 * p = max(seq_lens[i] - 2, 0); device_locs_out[i] = req_to_token[r * r2t_stride + p],
 * or -1 when the request is on its first decode step after prefill (skip_first[r] !=
 * 0) or r lies outside the table's r2t_rows rows or p outside its r2t_cols columns
 * (r2t_stride >= r2t_cols: a strided view of a wider table is read only within its
 * own columns).  skip_first[r] is then cleared for every listed
 * request (after all lookups, so a request listed twice reads the flag once as
 * set).  The result feeds qq_quest_decode_update. */
int qq_quest_decode_step_locs(const int64_t* req_pool_indices, const int64_t* seq_lens, int bs,
                              uint8_t* skip_first, const int32_t* req_to_token, int64_t r2t_rows,
                              int64_t r2t_cols, int64_t r2t_stride, int64_t* device_locs_out, void* stream);

/* Replaces QuestAlgorithm.maybe_finalize_decode_representations
 * (src/qwenquest/quest.py:304-321): for requests whose running_token_count is
 * P-1, copy the running bounds into page running_page_idx (all layers), reset
 * them, advance the page index; every listed request's count becomes (c+1)%P. */
int qq_quest_decode_finalize(const int64_t* req_indices, int n, uint16_t* page_k_bounds,
                             uint16_t* running_k_min, uint16_t* running_k_max,
                             int32_t* running_token_count, int32_t* running_page_idx,
                             int num_layers, int max_reqs, int max_pages, int kv_heads,
                             int head_dim, int page_size, void* stream);

/* Replaces QuestAlgorithm.prepare_step (src/qwenquest/quest.py:325-362):
 * actual_lens = min(seq, top_k); candidate_limit = seq / P, or max(seq/P - 1, 0)
 * with avoid_recent_overlap.  The recent window and the dense layout are
 * produced directly by qq_quest_retrieve_topk. */
int qq_quest_prepare_step(const int64_t* seq_lens, int bs, int page_size, int top_k,
                          int avoid_recent_overlap, int32_t* actual_lens,
                          int32_t* candidate_limit, void* stream);

/* Bytes of the sync buffer qq_quest_decode_step takes for `bs` batch entries (one
 * counter per entry, each on its own 128-byte line). */
int64_t qq_quest_decode_step_sync_bytes(int bs);

/* Replaces one decode step's Quest bookkeeping as QuestOnlyBackend.init_forward_metadata
 * runs it, in one launch: the previous token's row per request
 * (src/qwenquest/attention/quest_only.py:84-97), QuestAlgorithm.update_decode_representations
 * and maybe_finalize_decode_representations over every layer (src/qwenquest/quest.py:284-321)
 * and QuestAlgorithm.prepare_step (quest.py:325-362).  The results are those of
 * qq_quest_decode_step_locs, qq_quest_decode_update (finalize, layers [0, num_layers)) and
 * qq_quest_prepare_step called in that order, for a batch that lists each request once (as
 * the reference's batches do; a request listed twice would be folded and advanced once per
 * entry).  device_locs_out (optional, [bs]) receives the rows looked up.  sync:
 * qq_quest_decode_step_sync_bytes(bs) bytes, zero before the first call; each call leaves
 * it zero. */
int qq_quest_decode_step(const int64_t* req_pool_indices, const int64_t* seq_lens, int bs,
                         uint8_t* skip_first, const int32_t* req_to_token, int64_t r2t_rows,
                         int64_t r2t_cols, int64_t r2t_stride, int64_t* device_locs_out,
                         const void* k_base, int64_t k_layer_stride, int k_dtype, int64_t k_rows,
                         uint16_t* page_k_bounds, uint16_t* running_k_min, uint16_t* running_k_max,
                         int32_t* running_token_count, int32_t* running_page_idx, int num_layers,
                         int max_reqs, int max_pages, int kv_heads, int head_dim, int page_size,
                         int top_k, int avoid_recent_overlap, int32_t* actual_lens,
                         int32_t* candidate_limit, void* sync, int64_t sync_bytes, void* stream);

/* Replaces QuestAlgorithm.retrieve_topk (src/qwenquest/quest.py:409-464)
 * including group_queries (:366-391) and page_scores (:393-405), for layer
 * offset `layer`.  q: [bs, num_q_heads, D] (bf16 or fp32) with batch stride
 * `q_batch_stride` elements.  Writes positions [bs, top_k] int32 (long
 * requests: the top_k/P - 1 best complete pages by descending score, ties to
 * the lowest page index, expanded x P, then the recent window; short
 * requests: 0..seq-1 padded with seq-1).  Page scores of candidate pages are
 * left in scores_ws [bs, max_pages] fp32. */
int qq_quest_retrieve_topk(const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                           const uint16_t* page_k_bounds, int layer, const int64_t* req_pool_indices,
                           const int64_t* seq_lens, const int32_t* candidate_limit, int bs,
                           int max_reqs, int max_pages, int kv_heads, int head_dim, int page_size,
                           int top_k, float* scores_ws, int32_t* positions, void* stream);

/* Replaces QuestAlgorithm.group_queries (src/qwenquest/quest.py:366-391):
 * out[b, h, d] = mean over the G = num_q_heads / kv_heads query heads of KV
 * head h (fp32 sum in head order, / G, one rounding to q's dtype). */
int qq_quest_group_queries(const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                           int kv_heads, int head_dim, int bs, void* out, void* stream);

/* Replaces QuestAlgorithm.page_scores (src/qwenquest/quest.py:393-405):
 * scores[b, p] = sum_{h,d} (qbar >= 0 ? qbar*kmax : qbar*kmin) over every page
 * slot p < max_pages of request req_pool_indices[b] at layer offset `layer`,
 * fp32 products summed in the canonical order (64 lanes of ceil(KV*D/64)
 * channels, then a halving tree). */
int qq_quest_page_scores(const void* grouped_q, int q_dtype, int64_t q_batch_stride,
                         const uint16_t* page_k_bounds, int layer, const int64_t* req_pool_indices,
                         int bs, int max_reqs, int max_pages, int kv_heads, int head_dim,
                         float* scores, void* stream);

/* Workspace bytes qq_*_decode_attention needs for `bs` requests of up to
 * `max_rows` rows each with `num_q_heads` x `head_dim` outputs. */
int64_t qq_decode_attention_workspace_bytes(int bs, int max_rows, int num_q_heads, int head_dim);

/* Replaces the Mode-2 gather + attention of QuestOnlyBackend.forward_decode
 * (src/qwenquest/attention/quest_only.py:149-159) and decode_attention
 * (src/qwenquest/attention/ops.py:48-66): for request i, attends q[i] over rows
 * req_to_token[req_pool_indices[i], positions[i, j]] for j < actual_lens[i]
 * (duplicates counted), softmax(q.k * scale) in fp32, output [bs, H*D] in
 * q's dtype.  k_layer/v_layer: this layer's [kv_rows, KV, D] pool;
 * req_to_token: [req_to_token_rows, req_to_token_stride] int32.  Out-of-range
 * requests, positions or rows read the padding row 0 instead of faulting. */
int qq_quest_decode_attention(const void* q, int q_dtype, int64_t q_batch_stride,
                              int num_q_heads, const void* k_layer, const void* v_layer,
                              int kv_dtype, int64_t kv_rows, int kv_heads, int head_dim,
                              const int32_t* req_to_token, int64_t req_to_token_stride,
                              int64_t req_to_token_rows, const int64_t* req_pool_indices,
                              const int32_t* positions,
                              int64_t positions_stride, const int32_t* actual_lens, int bs,
                              float scale, void* out, void* workspace, int64_t workspace_bytes,
                              void* stream);

/* Replaces the Mode-3 attention of QuestHiSparseBackend.forward_decode
 * (src/qwenquest/attention/quest_hisparse.py:294-300): like
 * qq_quest_decode_attention but rows come directly from `rows` [bs, rows_stride]
 * int64 (the hot-buffer rows returned by the swap-in).  With `sync` (>=
 * qq_quest_layer_step_sync_bytes(bs, kv_heads), zeroed before the first call),
 * bf16, KV*D = 4*128, G <= 16 and rows_stride <= 4096 slots, it runs the
 * attention kernel of qq_quest_forward_decode's fused path over the given rows
 * (same arithmetic in the same slot order: pass `sync` exactly when
 * qq_quest_fused_step holds for the quest configuration, and quest_hisparse
 * matches quest bit for bit); otherwise chunked MFMA attention + merge, as
 * qq_quest_decode_attention. */
int qq_decode_attention_rows(const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                             const void* k_layer, const void* v_layer, int kv_dtype,
                             int64_t kv_rows, int kv_heads, int head_dim, const int64_t* rows,
                             int64_t rows_stride, const int32_t* actual_lens, int bs, float scale,
                             void* out, void* workspace, int64_t workspace_bytes, void* sync,
                             int64_t sync_bytes, void* stream);

/* 1 when qq_quest_forward_decode with a sync buffer runs the fused layer step
 * for these shapes (bf16, KV*D = 4*128, G <= 16, page 64, at most 64 selected
 * pages, top_k <= 4096, max_pages <= 8192; new_dtype -1 = no new token), else
 * 0.  No counterpart in the reference: it lets a caller of
 * qq_decode_attention_rows choose the same attention arithmetic. */
int qq_quest_fused_step(int q_dtype, int kv_dtype, int new_dtype, int num_q_heads, int kv_heads,
                        int head_dim, int page_size, int top_k, int max_pages);

/* Bytes of the sync buffer qq_quest_forward_decode's two-launch path uses for
 * `bs` requests (one counter per (request, KV head), each on its own 128-byte
 * line).  The caller zeroes it once; every call leaves it zeroed again. */
int64_t qq_quest_layer_step_sync_bytes(int bs, int kv_heads);

/* Replaces QuestOnlyBackend.forward_decode (src/qwenquest/attention/quest_only.py:132-159)
 * for one layer: the new tokens' K/V (k_new/v_new [bs, KV, D]) go to rows
 * out_cache_loc of k_layer/v_layer (memory.py:114-120; skipped when k_new is
 * NULL), retrieve_topk (quest.py:409-464) writes positions [bs, top_k], and
 * attention over req_to_token[req, positions[:n]] writes out [bs, H*D]
 * (ops.py:48-66; rows equal to out_cache_loc[i] attend the new K/V, as after
 * set_kv_buffer).  seq_lens / candidate_limit / actual_lens are the step's
 * prepare_step outputs; workspace sized by
 * qq_decode_attention_workspace_bytes(bs, top_k, H, D).
 * With `sync` (>= qq_quest_layer_step_sync_bytes, zeroed before the first
 * call) and the shapes of qq_quest_fused_step (bf16 tensors, KV*D = 4*128,
 * page 64, top_k/P - 1 <= 64, max_pages <= 8192), the layer runs as two launches (page
 * scores + new token, then per (request, KV head, part) the request's selection,
 * layout, attention and the merge of the parts, handed off inside the launch);
 * otherwise, or with sync == NULL, as four launches.  Calls sharing one sync
 * buffer must not overlap (one stream). */
int qq_quest_forward_decode(const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                            const void* k_new, const void* v_new, int new_dtype,
                            const int64_t* out_cache_loc, void* k_layer, void* v_layer,
                            int kv_dtype, int64_t kv_rows, const uint16_t* page_k_bounds,
                            int layer, const int64_t* req_pool_indices, const int64_t* seq_lens,
                            const int32_t* candidate_limit, const int32_t* actual_lens, int bs,
                            int max_reqs, int max_pages, int kv_heads, int head_dim,
                            int page_size, int top_k, const int32_t* req_to_token,
                            int64_t req_to_token_stride, int64_t req_to_token_rows, float scale,
                            float* scores_ws, int32_t* positions, void* out, void* workspace,
                            int64_t workspace_bytes, void* sync, int64_t sync_bytes, void* stream);

/* qq_quest_forward_decode without caller workspaces: the page scores, the
 * attention partials and the hand-off counters live in one fixed device array
 * of qq_quest_forward_decode_noalloc_max_bytes() bytes (16 MiB: 64 KiB of
 * counters, 4 MiB - 64 KiB of scores, 12 MiB of partials) that each GPU holds
 * until the process ends.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The call allocates nothing; the
 * first call on a device looks the array up and clears its counters on
 * `stream`.  Sizes beyond the array (bs * max_pages * 4 B of scores, the
 * qq_decode_attention_workspace_bytes(bs, top_k, H, D) of partials) return
 * QQ_EINVAL.  Every call on a device shares its array: calls that overlap on
 * one GPU (two streams, two threads) race.  Arguments and results otherwise
 * as qq_quest_forward_decode (same kernels, bit-identical outputs). */
int qq_quest_forward_decode_noalloc(const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                                    const void* k_new, const void* v_new, int new_dtype,
                                    const int64_t* out_cache_loc, void* k_layer, void* v_layer,
                                    int kv_dtype, int64_t kv_rows, const uint16_t* page_k_bounds,
                                    int layer, const int64_t* req_pool_indices, const int64_t* seq_lens,
                                    const int32_t* candidate_limit, const int32_t* actual_lens, int bs,
                                    int max_reqs, int max_pages, int kv_heads, int head_dim,
                                    int page_size, int top_k, const int32_t* req_to_token,
                                    int64_t req_to_token_stride, int64_t req_to_token_rows, float scale,
                                    int32_t* positions, void* out, void* stream);
/* Bytes of qq_quest_forward_decode_noalloc's per-device scratch array. */
int64_t qq_quest_forward_decode_noalloc_max_bytes(void);

/* qq_quest_forward_decode split into its two stages, for callers that run
 * other work between them or time them separately: phase 1 = page scoring and
 * the new token's K/V store, phase 2 = selection + layout + attention
 * (consumes the scores phase 1 left in `scores_ws`), phase 3 = both.
 * `positions` and `out` are complete after phase 2.  Arguments as for
 * qq_quest_forward_decode; no counterpart in the reference. */
int qq_quest_forward_decode_phase(const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                                  const void* k_new, const void* v_new, int new_dtype,
                                  const int64_t* out_cache_loc, void* k_layer, void* v_layer,
                                  int kv_dtype, int64_t kv_rows, const uint16_t* page_k_bounds,
                                  int layer, const int64_t* req_pool_indices, const int64_t* seq_lens,
                                  const int32_t* candidate_limit, const int32_t* actual_lens, int bs,
                                  int max_reqs, int max_pages, int kv_heads, int head_dim,
                                  int page_size, int top_k, const int32_t* req_to_token,
                                  int64_t req_to_token_stride, int64_t req_to_token_rows, float scale,
                                  float* scores_ws, int32_t* positions, void* out, void* workspace,
                                  int64_t workspace_bytes, void* sync, int64_t sync_bytes, int phase,
                                  void* stream);

/* Replaces DenseBackend.forward_decode (src/qwenquest/attention/dense.py:26-42) for
 * one layer: the new tokens' K/V (k_new/v_new [bs, KV, D]; NULL: none) go to rows
 * out_cache_loc (memory.py:114-120), then request i attends
 * req_to_token[req_pool_indices[i], 0 .. seq_lens[i]) (ops.py:48-66) -> out
 * [bs, H*D].  bf16 queries and K/V, KV*D = 4*128, H/KV <= 16 (QQ_EINVAL
 * otherwise); seq_lens[i] <= req_to_token_stride.  sync as for
 * qq_quest_forward_decode (>= qq_quest_layer_step_sync_bytes(bs, 4), zeroed
 * once, left zeroed); workspace >= qq_dense_decode_workspace_bytes(bs,
 * req_to_token_stride, H, KV).  Two launches: the K/V store, then the
 * attention (per (request, KV head, part of at most 4096 rows), parts merged
 * inside the launch). */
int qq_dense_forward_decode(const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                            const void* k_new, const void* v_new, int new_dtype,
                            const int64_t* out_cache_loc, void* k_layer, void* v_layer, int kv_dtype,
                            int64_t kv_rows, int kv_heads, int head_dim,
                            const int64_t* req_pool_indices, const int64_t* seq_lens, int bs,
                            const int32_t* req_to_token, int64_t req_to_token_stride,
                            int64_t req_to_token_rows, float scale, void* out, void* workspace,
                            int64_t workspace_bytes, void* sync, int64_t sync_bytes, void* stream);

/* Workspace bytes of qq_dense_forward_decode for contexts of up to max_rows
 * tokens (no counterpart in the reference). */
int64_t qq_dense_decode_workspace_bytes(int bs, int64_t max_rows, int num_q_heads, int kv_heads);

/* Replaces MHATokenToKVPool.set_kv_buffer (src/qwenquest/memory.py:114-120):
 * k_layer[locs[i]] = k[i], v_layer[locs[i]] = v[i] (row = KV*D elements),
 * converting src_dtype -> buf_dtype. */
int qq_kv_scatter(void* k_layer, void* v_layer, int buf_dtype, int64_t kv_rows, const void* k,
                  const void* v, int src_dtype, const int64_t* locs, int n, int64_t row_elems,
                  void* stream);

/* ------------------------------------------------------------- HiSparse tier
 * Layouts of the reference HiSparseCoordinator (src/qwenquest/hisparse/coordinator.py:103-131):
 * device_k/v[layer] [R*(buf+1), KV, D] (request r owns rows r*(buf+1) + slot,
 * slot buf = newest token), buffer_tokens/lru_slots [L, R, buf] int64,
 * req_to_host_pool [R, max_ctx] int64 (-1 = none), host_k/v[layer]
 * [host_rows, KV, D] in pinned host memory that the kernels read and write
 * directly (device-accessible pointer from qq_host_device_pointer). */

/* Replaces HiSparseCoordinator.swap_in_selected_pages / _swap_in_long
 * (coordinator.py:232-304) for one layer: rows_out [bs, top_k] int64 (-1 past
 * actual_lens) index device_k/v of the layer; misses are loaded from the host
 * tier into the least recently used slots (deduplicated by first occurrence),
 * buffer_tokens / lru_slots of the layer are updated exactly as the reference
 * does, stats[0..2] += (hits, misses, fast-path calls).  copy_dst/copy_src
 * [bs, top_k] int64 and copy_count [bs] int32 are workspaces.  Too few victims
 * (coordinator.py:278-279) sets bit 1 of *error_flags, a missing host row
 * (:285-286) bit 2; that request's state is then left unchanged and its rows
 * are all -1 (the rows attention then outputs NaN for it).  error_mirror (a
 * device-accessible pointer to 3 int32 in pinned host memory, or NULL) gets
 * word 0 / word 1 set to 1 with the same conditions, so the host can poll for
 * errors without a device synchronisation.  new_k / new_v (both or neither): the
 * step's new K and V rows ([bs] rows of row_bytes, the hot buffer's dtype), which
 * the plan also writes into each request's newest slot, row
 * req * (buf + 1) + min(seq - 1, buf) - HiSparseCoordinator.write_new_token
 * (coordinator.py:217-228) in the same launch. */
int qq_hisparse_swap_in(const int32_t* positions, int64_t positions_stride,
                        const int32_t* actual_lens, const int64_t* seq_lens,
                        const int64_t* req_pool_indices, int bs, int max_reqs,
                        int device_buffer_size, int top_k, int64_t* buffer_tokens_layer,
                        int64_t* lru_slots_layer, const int64_t* req_to_host_pool,
                        int64_t max_context_len, void* device_k_layer, void* device_v_layer,
                        const void* host_k_layer, const void* host_v_layer, int64_t row_bytes,
                        int64_t host_rows, int64_t* rows_out, int64_t* copy_dst,
                        int64_t* copy_src, int32_t* copy_count, uint64_t* stats,
                        int32_t* error_flags, int32_t* error_mirror, const void* new_k,
                        const void* new_v, void* stream);

/* qq_hisparse_swap_in without its copy: the plan only (rows_out, buffer_tokens,
 * lru_slots, stats and errors as there); the layer's misses are left in
 * copy_dst / copy_src [bs, top_k] (hot-buffer row <- host row, copy_count[b] of
 * them per request) for the caller to copy.  Serves the swap-in route the
 * reference's upstream takes (coordinator.py:282-291: pinned-host
 * hipMemcpyAsync on a side stream), which the coordinator offers as
 * swap_route="memcpy" to measure it against the in-kernel copy. */
int qq_hisparse_swap_plan(const int32_t* positions, int64_t positions_stride,
                          const int32_t* actual_lens, const int64_t* seq_lens,
                          const int64_t* req_pool_indices, int bs, int max_reqs,
                          int device_buffer_size, int top_k, int64_t* buffer_tokens_layer,
                          int64_t* lru_slots_layer, const int64_t* req_to_host_pool,
                          int64_t max_context_len, int64_t* rows_out, int64_t* copy_dst,
                          int64_t* copy_src, int32_t* copy_count, uint64_t* stats,
                          int32_t* error_flags, int32_t* error_mirror, void* stream);

/* Row copies over n_layers layers: dst[layer][dst_idx[i]] = src[layer][src_idx[i]]
 * (row_bytes each; indices outside [0, rows) are skipped).  Carries the
 * admission copies (coordinator.py:158-164: token pool -> host tier and hot
 * buffer) and the eager backup (coordinator.py:211-215: hot buffer -> host). */
int qq_copy_rows(const void* src, int64_t src_layer_stride_bytes, int64_t src_rows,
                 const int64_t* src_idx, void* dst, int64_t dst_layer_stride_bytes,
                 int64_t dst_rows, const int64_t* dst_idx, int n, int n_layers,
                 int64_t row_bytes, void* stream);

/* Per-request LRU state.  release == 0 (admit, coordinator.py:155, 166-167):
 * buffer_tokens[:, req, s] = s, lru_slots[:, req, s] = s, req_to_host_pool[req, :n]
 * = host_idx, the rest -1.  release != 0 (coordinator.py:312-314):
 * buffer_tokens = -1, lru_slots = identity, req_to_host_pool[req] = -1. */
int qq_hisparse_request_state(int64_t* buffer_tokens, int64_t* lru_slots, int num_layers,
                              int max_reqs, int device_buffer_size, int64_t* req_to_host_pool,
                              int64_t max_context_len, int req, const int64_t* host_idx, int64_t n,
                              int release, void* stream);

/* Replaces the eager backup's bookkeeping of HiSparseCoordinator.prepare_decode_step
 * (coordinator.py:183-212) without host synchronisation: batch entry b (request
 * req_pool_indices[b], previous position seq_lens[b]-2) is skipped, and its
 * request's skip flag cleared, when skip_flags[req] is set (the first decode step
 * after admission, coordinator.py:193-195); otherwise it takes the next free host
 * row in batch order from the device free list (free_ring / free_state, see
 * qq_hisparse_ring_alloc), req_to_host_pool[req, seq-2] = that row,
 * host_idx[b] = that row and device_rows[b] = req*(buf+1) + min(seq-2, buf) (the
 * previous token's hot-buffer row); skipped entries get -1 in both.  Fewer free
 * rows than entries (TokenToKVPoolAllocator.alloc's error, memory.py:62-66):
 * bit 4 of *error_flags (and error_mirror word 2), nothing taken: host_idx[b] = -1
 * and req_to_host_pool unchanged, but device_rows[b] is still written for every
 * entry that wanted a backup, since the reference folds the previous token into the
 * bounds (coordinator.py:204-208) before its alloc fails (:210). */
int qq_hisparse_backup_step(const int64_t* req_pool_indices, const int64_t* seq_lens, int bs,
                            uint8_t* skip_flags, int device_buffer_size, int max_reqs,
                            int64_t* req_to_host_pool, int64_t max_context_len, const int64_t* free_ring,
                            int64_t* free_state, int64_t free_cap, int64_t* host_idx, int64_t* device_rows,
                            int32_t* error_flags, int32_t* error_mirror, void* stream);

/* The host tier's TokenToKVPoolAllocator (memory.py:47-70) kept on the device so that
 * a decode step needs no host synchronisation: free_ring [free_cap] int64 with
 * free_state = {head, count} int64 holds the free rows in order,
 * free_ring[(head + i) % free_cap] for i < count.  alloc(n): out[i] = the i-th free
 * row (fewer than n free: bit 4 of *error_flags, error_mirror word 2, out = -1,
 * nothing taken). */
int qq_hisparse_ring_alloc(const int64_t* free_ring, int64_t* free_state, int64_t free_cap, int64_t n,
                           int64_t* out, int32_t* error_flags, int32_t* error_mirror, void* stream);

/* free(rows): the entries rows[i] > 0 are appended at the tail in order
 * (TokenToKVPoolAllocator.free, memory.py:68-72). */
int qq_hisparse_ring_free(int64_t* free_ring, int64_t* free_state, int64_t free_cap, const int64_t* rows,
                          int64_t n, void* stream);

/* Replaces HiSparseCoordinator.write_new_token (coordinator.py:217-228): the new
 * K/V of request i goes to hot-buffer slot min(seq_lens[i]-1, buf). */
int qq_hisparse_write_new_token(void* device_k_layer, void* device_v_layer, int buf_dtype,
                                const void* k, const void* v, int src_dtype,
                                const int64_t* req_pool_indices, const int64_t* seq_lens, int bs,
                                int device_buffer_size, int max_reqs, int64_t row_elems,
                                void* stream);

/* Device-side address of pinned host memory (hipHostGetDevicePointer). */
int qq_host_device_pointer(void* host_ptr, void** device_ptr);

/* Replaces the allocation of the reference's host tier (host_k / host_v,
 * src/qwenquest/hisparse/coordinator.py:104-110, torch.zeros on the host device):
 * `bytes` of pinned host memory at exactly that size (hipHostMalloc, default flags:
 * mapped into the device's address space), contents undefined; QQ_EHIP when the
 * system cannot pin that much.  qq_host_free releases it. */
int qq_host_alloc(int64_t bytes, void** host_ptr);
int qq_host_free(void* host_ptr);

#ifdef __cplusplus
}
#endif

#endif /* QWENQUEST_AMD_H */
