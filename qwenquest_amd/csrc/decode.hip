// One Quest decode layer for a batch, as QuestOnlyBackend.forward_decode does it
// (reference src/qwenquest/attention/quest_only.py:132-159): store the new
// token's K/V, select the positions, gather through req_to_token and attend.
//
// Four launches on one stream, each consuming the previous one's output:
//   score (all CUs) -> select + new-token store (one block per request)
//   -> chunk attention (MFMA) -> merge.
// The new token's K/V is written by the select launch, which runs before the
// attention launch reads the pool; the scoring launch never reads the pool.
#include "qq_kernels.h"

using namespace qq;

extern "C" int qq_quest_forward_decode(
    const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads, const void* k_new,
    const void* v_new, int new_dtype, const int64_t* out_cache_loc, void* k_layer, void* v_layer,
    int kv_dtype, int64_t kv_rows, const uint16_t* page_k_bounds, int layer,
    const int64_t* req_pool_indices, const int64_t* seq_lens, const int32_t* candidate_limit,
    const int32_t* actual_lens, int bs, int max_reqs, int max_pages, int kv_heads, int head_dim,
    int page_size, int top_k, const int32_t* req_to_token, int64_t req_to_token_stride,
    int64_t req_to_token_rows, float scale, float* scores_ws, int32_t* positions, void* out,
    void* workspace, int64_t workspace_bytes, void* stream) {
  const char* what = "qq_quest_forward_decode";
  QQ_REQUIRE(dtype_ok(q_dtype) && dtype_ok(kv_dtype) && dtype_ok(new_dtype), "%s: unsupported dtype",
             what);
  QQ_REQUIRE(kv_heads > 0 && head_dim > 0 && num_q_heads > 0 && num_q_heads % kv_heads == 0,
             "%s: q_heads %d not divisible by kv_heads %d", what, num_q_heads, kv_heads);
  QQ_REQUIRE(page_size > 0 && top_k > 0 && top_k % page_size == 0,
             "%s: top_k %d must be a positive multiple of page_size %d", what, top_k, page_size);
  const int C = kv_heads * head_dim;
  const int k_sel = top_k / page_size - 1;
  QQ_REQUIRE(C <= 1024, "%s: kv_heads*head_dim %d exceeds 1024", what, C);
  QQ_REQUIRE(k_sel <= 1024, "%s: %d selected pages exceed 1024", what, k_sel);
  QQ_REQUIRE(bs >= 0 && bs <= max_reqs && layer >= 0, "%s: bad batch/layer", what);
  QQ_REQUIRE(q && k_layer && v_layer && page_k_bounds && req_pool_indices && seq_lens &&
                 candidate_limit && actual_lens && req_to_token && scores_ws && positions && out,
             "%s: null pointer", what);
  QQ_REQUIRE(!k_new || (v_new && out_cache_loc), "%s: new K without V or locations", what);
  if (bs == 0) return QQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);

  SelectArgs sa;
  sa.q = q;
  sa.q_dtype = q_dtype;
  sa.q_bstride = q_batch_stride;
  sa.H = num_q_heads;
  sa.bounds_layer =
      reinterpret_cast<const uint32_t*>(page_k_bounds) + (int64_t)layer * max_reqs * max_pages * C;
  sa.rpi = req_pool_indices;
  sa.seq = seq_lens;
  sa.limit = candidate_limit;
  sa.R = max_reqs;
  sa.MP = max_pages;
  sa.KV = kv_heads;
  sa.D = head_dim;
  sa.C = C;
  sa.m = (C + 63) / 64;
  sa.P = page_size;
  sa.top_k = top_k;
  sa.k_sel = k_sel;
  sa.ppb = 32;
  sa.scores = scores_ws;
  sa.positions = positions;
  sa.new_k = k_new;
  sa.new_v = v_new;
  sa.new_dtype = new_dtype;
  sa.new_locs = out_cache_loc;
  sa.k_pool = k_layer;
  sa.v_pool = v_layer;
  sa.pool_dtype = kv_dtype;
  sa.pool_rows = kv_rows;
  int st = launch_retrieve(sa, bs, s);
  if (st != QQ_OK) return st;

  AttnArgs aa;
  aa.q = q;
  aa.q_dtype = q_dtype;
  aa.q_bstride = q_batch_stride;
  aa.H = num_q_heads;
  aa.k = k_layer;
  aa.v = v_layer;
  aa.kv_rows = kv_rows;
  aa.KV = kv_heads;
  aa.D = head_dim;
  aa.r2t = req_to_token;
  aa.r2t_stride = req_to_token_stride;
  aa.r2t_rows = req_to_token_rows;
  aa.rpi = req_pool_indices;
  aa.positions = positions;
  aa.rows = nullptr;
  aa.pos_stride = top_k;
  aa.actual = actual_lens;
  aa.scale = scale;
  aa.out = out;
  return launch_attention(aa, kv_dtype, bs, workspace_bytes, workspace, s, what);
}
