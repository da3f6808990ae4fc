// One Quest decode layer for a batch, as QuestOnlyBackend.forward_decode does it
// (reference src/qwenquest/attention/quest_only.py:132-159): store the new
// token's K/V, select the positions, gather through req_to_token and attend.
//
// Fused path (bf16, KV*D = 4*128, page 64, at most 64 selected pages, at most
// 4096 pages per request, and a zeroed sync buffer from the caller): two
// launches, each small enough per block that the whole grid is resident at
// once, so every block's chain of dependent memory round trips overlaps the
// others' streaming:
//   1. score + select, one block per (request, 32 candidate pages): 4 waves x
//      8 pages scored, scores out with agent-scope stores, then the block
//      counts itself on its request's counter.  The block that completes the
//      count selects the request's pages (filter top-k over the scores) and
//      writes the layout: positions [bs, top_k], the pool rows they map to
//      through req_to_token (workspace), and the new token's K/V
//      (set_kv_buffer, memory.py:114-120).
//   2. attention + merge, one block per (request, 4 chunks of 64 layout rows,
//      KV head): each wave attends one chunk with MFMA, the 4 waves combine in
//      LDS into an (m, l, o) partial (agent-scope stores); the block that
//      completes a (request, KV head) count merges the partials into the
//      output.
// The counters return to zero before each launch ends, so the next call (or a
// graph replay) starts clean.
//
// Other shapes: four launches on one stream, each consuming the previous one's
// output: score (all CUs) -> select + new-token store (one block per request)
// -> chunk attention (MFMA) -> merge.
#include "qq_quest_dev.h"

namespace qq {
namespace {

constexpr int kStepKV = 4;            // KV heads of the fused path (KV*D = 512)
constexpr int kStepM = 8;             // bounds words per lane (512 / 64)
constexpr int kStepPagesPerTile = 32; // score tile: 4 waves x 8 pages
constexpr int kStepMaxG = 16;
constexpr int kMaxSelFused = 64;
constexpr int kStepMaxNT = (kMaxSelFused + 1 + 3) / 4;  // 64-row chunks / 4 per tile

struct StepArgs {
  SelectArgs s;            // scoring, selection, positions, new token
  const uint16_t* k;       // this layer's pool [kv_rows, KV, 128]
  const uint16_t* v;
  int64_t kv_rows;
  const int32_t* r2t;
  int64_t r2t_stride, r2t_rows;
  float sl2;               // scale * log2(e)
  uint16_t* out;           // [bs, H * 128] bf16
  float* part_o;           // [bs, KV, NT, G, 128]
  float* part_ml;          // [bs, KV, NT, G, 2] (m in log2 units, l)
  int32_t* rows;           // [bs, top_k] pool rows of the layout
  uint32_t* sync;
  int bs, tiles_s, nt, G;
};

// sync layout (uint32 words, each counter on its own 128-byte line):
//   score count [bs], attention count [KV][bs].
__device__ inline uint32_t* score_count(const StepArgs& a, int b) { return a.sync + b * 32; }
__device__ inline uint32_t* attn_count(const StepArgs& a, int b, int h) { return a.sync + ((1 + h) * a.bs + b) * 32; }

__device__ inline bool needs_selection(const SelectArgs& sa, int64_t s) { return s > sa.top_k && sa.k_sel > 0; }

template <int KPT>
union ScoreSmem {
  float q[kMaxC];
  SelectSmem<KPT> sel;
};

// The request's selection and layout (quest.py:409-464), run by the block
// that completed its score count: positions, pool rows (quest_only.py:149-151)
// and the new token's K/V (C = 512 bf16 = 256 words per row).
template <int KPT>
__device__ void select_request(const StepArgs& a, int b, ScoreSmem<KPT>& sm) {
  const SelectArgs& sa = a.s;
  const int tid = threadIdx.x;
  const int64_t s = sa.seq[b];
  const int64_t req = sa.rpi[b];
  const bool req_ok = req >= 0 && req < sa.R;
  const int lim = req_ok ? min(sa.limit[b], sa.MP) : 0;
  const int k = sa.k_sel, P = sa.P, top_k = sa.top_k;
  const bool long_b = needs_selection(sa, s);
  const int64_t loc = sa.new_k ? sa.new_locs[b] : -1;
  uint32_t kw = 0u, vw = 0u;
  if (sa.new_k) {
    kw = static_cast<const uint32_t*>(sa.new_k)[(int64_t)b * 256 + tid];
    vw = static_cast<const uint32_t*>(sa.new_v)[(int64_t)b * 256 + tid];
  }
  if (long_b) {
    const float* sc = sa.scores + (int64_t)b * sa.MP;
    float sv[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int p = tid + kBlock * i;
      sv[i] = p < lim ? ld_agent(sc + p) : 0.0f;
    }
    select_topk_block<KPT>(sv, lim, max(lim, k), k, sm.sel);
  }
  // layout slot -> position (pages by rank, then the recent window; or dense)
  int32_t* pos = sa.positions + (int64_t)b * top_k;
  int32_t* rows = a.rows + (int64_t)b * top_k;
  const bool r2t_ok = req >= 0 && req < a.r2t_rows;
  for (int slot0 = 0; slot0 < top_k; slot0 += kBlock * 8) {
    int64_t pv[8];
    int32_t rv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int slot = slot0 + tid + kBlock * i;
      int64_t p;
      if (!long_b)
        p = s <= top_k ? min((int64_t)slot, max(s - 1, (int64_t)0)) : min(max(s - P, (int64_t)0) + slot, s - 1);
      else if (slot < k * P)
        p = (int64_t)sm.sel.order[slot / P] * P + slot % P;
      else
        p = min(max(s - P, (int64_t)0) + (slot - k * P), s - 1);
      pv[i] = p;
      rv[i] = (slot < top_k && r2t_ok && p >= 0 && p < a.r2t_stride) ? a.r2t[req * a.r2t_stride + p] : 0;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int slot = slot0 + tid + kBlock * i;
      if (slot < top_k) {
        pos[slot] = (int32_t)pv[i];
        const int64_t row = rv[i];
        rows[slot] = (row >= 0 && row < a.kv_rows) ? (int32_t)row : 0;
      }
    }
  }
  if (loc >= 0 && loc < sa.pool_rows) {
    static_cast<uint32_t*>(sa.k_pool)[loc * 256 + tid] = kw;
    static_cast<uint32_t*>(sa.v_pool)[loc * 256 + tid] = vw;
  }
}

template <int KPT>
__global__ __launch_bounds__(kBlock) void quest_score_select_kernel(StepArgs a) {
  __shared__ ScoreSmem<KPT> sm;
  __shared__ uint32_t s_last;
  const SelectArgs& sa = a.s;
  const int tid = threadIdx.x;
  const int b = blockIdx.x / a.tiles_s, t = blockIdx.x - b * a.tiles_s;
  const int64_t s = sa.seq[b];
  const int64_t req = sa.rpi[b];
  const int lim = (req >= 0 && req < sa.R) ? min(sa.limit[b], sa.MP) : 0;
  const int p0 = t * kStepPagesPerTile;
  if (needs_selection(sa, s) && p0 < lim) {  // block-uniform
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int pw = p0 + wave * 8;
    uint32_t w[8][kStepM];
    load_8pages<kStepM>(w, sa.bounds_layer + req * sa.MP * (64 * kStepM), pw, lim, lane);
    block_qbar(sm.q, sa, b);
    __syncthreads();
    if (pw < lim) {
      const float v = score_8pages<kStepM>(w, sm.q, lane);
      const int p = pw + (lane >> 3);
      if ((lane & 7) == 0 && p < lim) st_agent(sa.scores + (int64_t)b * sa.MP + p, v);
    }
  }
  wait_memory();
  __syncthreads();
  if (tid == 0) s_last = add_agent(score_count(a, b), 1u) == (uint32_t)(a.tiles_s - 1);
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) st_agent(score_count(a, b), 0u);
  select_request<KPT>(a, b, sm);
}

struct AttnSmem {
  const uint16_t* kp[kBlockWaves][64];
  const uint16_t* vp[kBlockWaves][64];
  float m[kBlockWaves][kStepMaxG];
  float l[kBlockWaves][kStepMaxG];
  float o[kBlockWaves][kStepMaxG][kMfmaDim];
};

__global__ __launch_bounds__(kBlock) void quest_attend_merge_kernel(StepArgs a) {
  __shared__ AttnSmem sm_attn;
  __shared__ uint32_t s_last;
  const SelectArgs& sa = a.s;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int per_req = kStepKV * a.nt;
  const int b = blockIdx.x / per_req, rem = blockIdx.x - b * per_req;
  const int j = rem / kStepKV, h = rem - j * kStepKV;  // the 4 heads of a row block are adjacent
  const int64_t s = sa.seq[b];
  const int n = (int)min(max(s, (int64_t)0), (int64_t)sa.top_k);  // actual_lens (quest.py:345)
  const int c = j * kBlockWaves + wave;  // this wave's chunk of 64 layout slots
  const int cnt = max(0, min(64, n - c * 64));
  {
    constexpr int kRow = kStepKV * kMfmaDim;
    const int64_t row = lane < cnt ? a.rows[(int64_t)b * sa.top_k + c * 64 + lane] : 0;
    sm_attn.kp[wave][lane] = a.k + row * kRow + h * kMfmaDim;
    sm_attn.vp[wave][lane] = a.v + row * kRow + h * kMfmaDim;
  }
  __syncthreads();
  const int G = a.G;
  const int lo = lane & 15, hi = lane >> 4;
  float mx, sum;
  float4_t o[8];
  const uint16_t* qh =
      static_cast<const uint16_t*>(sa.q) + (int64_t)b * sa.q_bstride + (int64_t)h * G * kMfmaDim;
  AttnSmem& sm = sm_attn;
  attn_wave64(sm.kp[wave], sm.vp[wave], qh, G, cnt, a.sl2, mx, sum, o);
  // combine the 4 waves' chunks in LDS
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int head = hi * 4 + i;
    if (head < G) {
      float* dst = &sm.o[wave][head][lo * 8];
      *reinterpret_cast<float4*>(dst) = make_float4(o[0][i], o[1][i], o[2][i], o[3][i]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4][i], o[5][i], o[6][i], o[7][i]);
    }
  }
  if (hi == 0 && lo < G) {
    sm.m[wave][lo] = mx;
    sm.l[wave][lo] = sum;
  }
  __syncthreads();
  const int64_t part = ((int64_t)b * kStepKV + h) * a.nt + j;
#pragma unroll
  for (int r = 0; r < kStepMaxG * kMfmaDim / kBlock; ++r) {
    const int idx = tid + kBlock * r;
    const int head = idx >> 7, d = idx & 127;
    if (head < G) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kBlockWaves; ++w) M = fmaxf(M, sm.m[w][head]);
      float L = 0.0f, O = 0.0f;
#pragma unroll
      for (int w = 0; w < kBlockWaves; ++w) {
        const float mw = sm.m[w][head];
        const float wgt = mw == -INFINITY ? 0.0f : exp2f(mw - M);
        L += wgt * sm.l[w][head];
        O += wgt * sm.o[w][head][d];
      }
      st_agent(a.part_o + (part * G + head) * kMfmaDim + d, O);
      if (d == 0) {
        st_agent(a.part_ml + (part * G + head) * 2, M);
        st_agent(a.part_ml + (part * G + head) * 2 + 1, L);
      }
    }
  }
  wait_memory();
  __syncthreads();
  if (tid == 0) s_last = add_agent(attn_count(a, b, h), 1u) == (uint32_t)(a.nt - 1);
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) st_agent(attn_count(a, b, h), 0u);
  // merge the NT partials of (request b, KV head h) into the output: each
  // thread one head x 4 channels, all of its partial loads in flight at once
  const int64_t part0 = ((int64_t)b * kStepKV + h) * a.nt;
  const __amdgpu_buffer_rsrc_t ro =
      agent_rsrc(a.part_o + part0 * G * kMfmaDim, (uint32_t)(a.nt * G * kMfmaDim * sizeof(float)));
  const uint64_t* ml64 = reinterpret_cast<const uint64_t*>(a.part_ml) + part0 * G;
  for (int grp = tid; grp < G * (kMfmaDim / 4); grp += kBlock) {
    const int head = grp >> 5, d4 = (grp & 31) * 4;
    float4 ov[kStepMaxNT];
    uint64_t mlv[kStepMaxNT];
#pragma unroll
    for (int jj = 0; jj < kStepMaxNT; ++jj) {
      if (jj < a.nt) {
        ov[jj] = ld_agent_x4(ro, (uint32_t)(((jj * G + head) * kMfmaDim + d4) * sizeof(float)));
        mlv[jj] = ld_agent(ml64 + jj * G + head);
      }
    }
    float M = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < kStepMaxNT; ++jj)
      if (jj < a.nt) M = fmaxf(M, __uint_as_float((uint32_t)mlv[jj]));
    float L = 0.0f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int jj = 0; jj < kStepMaxNT; ++jj) {
      if (jj < a.nt) {
        const float mj = __uint_as_float((uint32_t)mlv[jj]);
        const float wgt = mj == -INFINITY ? 0.0f : exp2f(mj - M);
        L += wgt * __uint_as_float((uint32_t)(mlv[jj] >> 32));
        O.x += wgt * ov[jj].x;
        O.y += wgt * ov[jj].y;
        O.z += wgt * ov[jj].z;
        O.w += wgt * ov[jj].w;
      }
    }
    uint16_t* dst = a.out + (int64_t)b * sa.H * kMfmaDim + (int64_t)(h * G + head) * kMfmaDim + d4;
    const bool any = L > 0.0f;
    const uint32_t lo2 = (uint32_t)f2bf(any ? O.x / L : 0.0f) | ((uint32_t)f2bf(any ? O.y / L : 0.0f) << 16);
    const uint32_t hi2 = (uint32_t)f2bf(any ? O.z / L : 0.0f) | ((uint32_t)f2bf(any ? O.w / L : 0.0f) << 16);
    *reinterpret_cast<uint2*>(dst) = make_uint2(lo2, hi2);
  }
}

}  // namespace
}  // namespace qq

using namespace qq;

extern "C" int64_t qq_quest_layer_step_sync_bytes(int bs, int kv_heads) {
  if (bs <= 0 || kv_heads <= 0) return 0;
  return (int64_t)(1 + kStepKV) * bs * 32 * (int64_t)sizeof(uint32_t);
}

extern "C" int qq_quest_forward_decode(
    const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads, const void* k_new,
    const void* v_new, int new_dtype, const int64_t* out_cache_loc, void* k_layer, void* v_layer,
    int kv_dtype, int64_t kv_rows, const uint16_t* page_k_bounds, int layer,
    const int64_t* req_pool_indices, const int64_t* seq_lens, const int32_t* candidate_limit,
    const int32_t* actual_lens, int bs, int max_reqs, int max_pages, int kv_heads, int head_dim,
    int page_size, int top_k, const int32_t* req_to_token, int64_t req_to_token_stride,
    int64_t req_to_token_rows, float scale, float* scores_ws, int32_t* positions, void* out,
    void* workspace, int64_t workspace_bytes, void* sync, int64_t sync_bytes, void* stream) {
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

  const int G = num_q_heads / kv_heads;
  const int chunks = top_k / page_size;
  const int nt = ceil_div(chunks, kBlockWaves);
  const int64_t part_bytes = (int64_t)bs * kStepKV * nt * G * (kMfmaDim + 2) * (int64_t)sizeof(float);
  const int64_t rows_bytes = (int64_t)bs * top_k * (int64_t)sizeof(int32_t);
  const bool fused = sync && sync_bytes >= qq_quest_layer_step_sync_bytes(bs, kv_heads) &&
                     q_dtype == QQ_DTYPE_BF16 && kv_dtype == QQ_DTYPE_BF16 &&
                     (!k_new || new_dtype == QQ_DTYPE_BF16) && kv_heads == kStepKV &&
                     head_dim == kMfmaDim && G <= kStepMaxG && page_size == 64 && k_sel <= kMaxSelFused &&
                     max_pages <= 16 * kBlock && workspace && workspace_bytes >= part_bytes + rows_bytes;
  if (fused) {
    StepArgs a;
    a.s = sa;
    a.k = static_cast<const uint16_t*>(k_layer);
    a.v = static_cast<const uint16_t*>(v_layer);
    a.kv_rows = kv_rows;
    a.r2t = req_to_token;
    a.r2t_stride = req_to_token_stride;
    a.r2t_rows = req_to_token_rows;
    a.sl2 = scale * kLog2e;
    a.out = static_cast<uint16_t*>(out);
    a.part_o = static_cast<float*>(workspace);
    a.part_ml = a.part_o + (int64_t)bs * kStepKV * nt * G * kMfmaDim;
    a.rows = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + part_bytes);
    a.sync = static_cast<uint32_t*>(sync);
    a.bs = bs;
    a.tiles_s = ceil_div(max(max_pages, 1), kStepPagesPerTile);
    a.nt = nt;
    a.G = G;
    const int score_blocks = bs * a.tiles_s;
    const int n_max = max(max_pages, k_sel);
    if (n_max <= 4 * kBlock)
      quest_score_select_kernel<4><<<score_blocks, kBlock, 0, s>>>(a);
    else if (n_max <= 8 * kBlock)
      quest_score_select_kernel<8><<<score_blocks, kBlock, 0, s>>>(a);
    else if (n_max <= 12 * kBlock)
      quest_score_select_kernel<12><<<score_blocks, kBlock, 0, s>>>(a);
    else
      quest_score_select_kernel<16><<<score_blocks, kBlock, 0, s>>>(a);
    quest_attend_merge_kernel<<<bs * kStepKV * nt, kBlock, 0, s>>>(a);
    return check_launch(what);
  }

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
