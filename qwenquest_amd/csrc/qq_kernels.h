// Kernel argument blocks and launchers shared by the entry points.
#pragma once

#include "qq_common.h"

namespace qq {

struct SelectArgs {
  const void* q;
  int q_dtype;
  int64_t q_bstride;
  int H;
  const uint32_t* bounds_layer;  // [R, MP, C] (min, max) words of this layer
  // rpi .. limit adjacent: the attention launch reads them in its first batch of
  // argument loads
  const int64_t* rpi;
  const int64_t* seq;
  float* scores;
  int R, MP;
  const int32_t* limit;
  int KV, D, C, m, P, top_k, k_sel, ppb;
  int32_t* positions;
  // optional: store the decoded token's K/V (memory.py:114-120) before attention reads it
  const void* new_k;
  const void* new_v;
  int new_dtype;
  const int64_t* new_locs;
  void* k_pool;
  void* v_pool;
  int pool_dtype;
  int64_t pool_rows;
};

struct AttnArgs {
  const void* q;
  int q_dtype;
  int64_t q_bstride;
  int H;
  const void* k;
  const void* v;
  int64_t kv_rows;
  int KV, D;
  const int32_t* r2t;
  int64_t r2t_stride;
  int64_t r2t_rows;
  const int64_t* rpi;
  const int32_t* positions;
  const int64_t* rows;
  int64_t pos_stride;
  const int32_t* actual;
  float scale;
  void* out;
  float* ws_o;   // [bs, max_chunks, H, D]
  float* ws_ml;  // [bs, max_chunks, H, 2]
  int max_chunks;
};

// Page scoring + selection + layout of one layer (qq_quest_retrieve_topk).
int launch_retrieve(const SelectArgs& a, int bs, hipStream_t stream);

// Selection + layout only (one block per request), from scores already in a.scores.
void launch_select(const SelectArgs& a, int bs, int max_pages, int k_sel, hipStream_t stream);

// Page scoring only (scores of long requests' candidate pages); with
// `store_new` the new token's K/V is stored as well (blocks x == 0).
int launch_score(const SelectArgs& a, int bs, bool store_new, hipStream_t stream);

// Chunk attention + merge; `workspace` holds the (m, l, o) partials.
int launch_attention(AttnArgs& a, int kv_dtype, int bs, int64_t workspace_bytes, void* workspace,
                     hipStream_t stream, const char* what);

// The fused layer step's attention kernel over given rows (`slots` per request,
// rows[b * slots + i]); QQ_OK when launched, 1 when the shape or the buffers do
// not allow it.  Callers check bf16 and KV * D = 4 * 128.
int attend_rows_fused(const void* q, int64_t q_bstride, int num_q_heads, const void* k_layer, const void* v_layer,
                      int64_t kv_rows, const int64_t* rows, int64_t slots, const int32_t* actual, int bs, float scale,
                      void* out, void* workspace, int64_t workspace_bytes, void* sync, int64_t sync_bytes,
                      hipStream_t s);

}  // namespace qq
