// Gather + split-K decode attention over an explicit row list.
//
// Reference: decode_attention (src/qwenquest/attention/ops.py:48-66) applied per
// request to rows req_to_token[req, positions[:n]] (quest_only.py:149-159) or to
// hot-buffer rows (quest_hisparse.py:294-300).  Rows are attended exactly as
// listed (a duplicate counts twice); scores, softmax and PV accumulate in fp32.
//
// Grid (chunks, bs): block (c, b) takes rows [c*64, c*64 + 64) of request b,
// gathers them through the row map, computes per q head the chunk max m,
// sum l = sum exp(s - m) and o = sum exp(s - m) v, and writes (m, l, o) to the
// workspace.  The last chunk block of a request to finish (agent-scope ticket)
// merges the partials: out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.
#include "qq_common.h"

namespace qq {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 64;

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
  int32_t* tickets;
};

__device__ inline float ldkv(const uint16_t* p, int64_t i) { return bf2f(p[i]); }
__device__ inline float ldkv(const float* p, int64_t i) { return p[i]; }

template <typename KVT>
__global__ __launch_bounds__(kThreads) void attn_chunk_kernel(AttnArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int c = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int n = (int)min((int64_t)a.actual[b], a.pos_stride);
  const int nc = (n + kChunk - 1) / kChunk;
  if (c >= nc) return;
  const int H = a.H, D = a.D;
  const int r0 = c * kChunk, cnt = min(kChunk, n - r0);
  int64_t* s_rows = reinterpret_cast<int64_t*>(smem_raw);
  float* s_q = reinterpret_cast<float*>(s_rows + kChunk);
  float* s_p = s_q + H * D;
  float* s_m = s_p + H * kChunk;
  float* s_l = s_m + H;
  __shared__ int s_last;

  if (tid < cnt) {
    int64_t row;
    if (a.rows) {
      row = a.rows[(int64_t)b * a.pos_stride + r0 + tid];
    } else {
      const int64_t p = a.positions[(int64_t)b * a.pos_stride + r0 + tid];
      const int64_t req = a.rpi[b];
      const bool ok = p >= 0 && p < a.r2t_stride && req >= 0 && req < a.r2t_rows;
      row = ok ? (int64_t)a.r2t[req * a.r2t_stride + p] : 0;
    }
    s_rows[tid] = (row >= 0 && row < a.kv_rows) ? row : 0;
  }
  for (int i = tid; i < H * D; i += kThreads)
    s_q[i] = load_as_float(a.q, (int64_t)b * a.q_bstride + i, a.q_dtype);
  __syncthreads();

  const int G = H / a.KV;
  const int64_t rowe = (int64_t)a.KV * D;
  const KVT* K = static_cast<const KVT*>(a.k);
  const KVT* V = static_cast<const KVT*>(a.v);
  for (int idx = tid; idx < H * cnt; idx += kThreads) {
    const int h = idx / cnt, j = idx - h * cnt;
    const KVT* kp = K + s_rows[j] * rowe + (int64_t)(h / G) * D;
    const float* qp = s_q + h * D;
    float dot = 0.0f;
    for (int d = 0; d < D; ++d) dot += qp[d] * ldkv(kp, d);
    s_p[h * kChunk + j] = dot * a.scale;
  }
  __syncthreads();
  for (int h = tid; h < H; h += kThreads) {
    float m = -INFINITY;
    for (int j = 0; j < cnt; ++j) m = fmaxf(m, s_p[h * kChunk + j]);
    float l = 0.0f;
    for (int j = 0; j < cnt; ++j) {
      const float e = expf(s_p[h * kChunk + j] - m);
      s_p[h * kChunk + j] = e;
      l += e;
    }
    s_m[h] = m;
    s_l[h] = l;
  }
  __syncthreads();
  const int64_t part = (int64_t)b * a.max_chunks + c;
  float* wo = a.ws_o + part * H * D;
  for (int idx = tid; idx < H * D; idx += kThreads) {
    const int h = idx / D, d = idx - h * D;
    const int64_t hoff = (int64_t)(h / G) * D + d;
    float acc = 0.0f;
    for (int j = 0; j < cnt; ++j) acc += s_p[h * kChunk + j] * ldkv(V + s_rows[j] * rowe, hoff);
    wo[idx] = acc;
  }
  for (int h = tid; h < H; h += kThreads) {
    a.ws_ml[(part * H + h) * 2 + 0] = s_m[h];
    a.ws_ml[(part * H + h) * 2 + 1] = s_l[h];
  }

  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (tid == 0) s_last = (ticket_arrive(&a.tickets[b]) == nc - 1);
  __syncthreads();
  if (!s_last) return;
  acquire_fence();
  const int64_t base = (int64_t)b * a.max_chunks;
  for (int idx = tid; idx < H * D; idx += kThreads) {
    const int h = idx / D;
    float M = -INFINITY;
    for (int cc = 0; cc < nc; ++cc) M = fmaxf(M, a.ws_ml[((base + cc) * H + h) * 2]);
    float L = 0.0f, O = 0.0f;
    for (int cc = 0; cc < nc; ++cc) {
      const float w = expf(a.ws_ml[((base + cc) * H + h) * 2] - M);
      L += w * a.ws_ml[((base + cc) * H + h) * 2 + 1];
      O += w * a.ws_o[(base + cc) * H * D + idx];
    }
    const float r = O / L;
    if (a.q_dtype == QQ_DTYPE_BF16)
      static_cast<uint16_t*>(a.out)[(int64_t)b * H * D + idx] = f2bf(r);
    else
      static_cast<float*>(a.out)[(int64_t)b * H * D + idx] = r;
  }
  if (tid == 0) a.tickets[b] = 0;
}

int launch_attention(AttnArgs& a, int kv_dtype, int bs, int64_t workspace_bytes, void* workspace,
                     void* stream, const char* what) {
  const int64_t need = qq_decode_attention_workspace_bytes(bs, (int)a.pos_stride, a.H, a.D);
  QQ_REQUIRE(workspace && workspace_bytes >= need, "%s: workspace %lld bytes < %lld needed", what,
             (long long)workspace_bytes, (long long)need);
  a.max_chunks = ceil_div(a.pos_stride, kChunk);
  a.ws_o = static_cast<float*>(workspace);
  a.ws_ml = a.ws_o + (int64_t)bs * a.max_chunks * a.H * a.D;
  const size_t smem = kChunk * sizeof(int64_t) + (size_t)(a.H * a.D + a.H * kChunk + 2 * a.H) * 4;
  QQ_REQUIRE(smem <= 64 * 1024, "%s: %d heads x %d dims need too much LDS", what, a.H, a.D);
  dim3 grid(max(1, a.max_chunks), bs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (kv_dtype == QQ_DTYPE_BF16)
    attn_chunk_kernel<uint16_t><<<grid, kThreads, smem, s>>>(a);
  else
    attn_chunk_kernel<float><<<grid, kThreads, smem, s>>>(a);
  return check_launch(what);
}

int fill_common(AttnArgs& a, const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                const void* k_layer, const void* v_layer, int kv_dtype, int64_t kv_rows,
                int kv_heads, int head_dim, const int32_t* actual_lens, float scale, void* out,
                int32_t* tickets, const char* what) {
  QQ_REQUIRE(dtype_ok(q_dtype) && dtype_ok(kv_dtype), "%s: unsupported dtype", what);
  QQ_REQUIRE(kv_heads > 0 && head_dim > 0 && num_q_heads > 0 && num_q_heads % kv_heads == 0,
             "%s: q_heads %d not divisible by kv_heads %d", what, num_q_heads, kv_heads);
  QQ_REQUIRE(q && k_layer && v_layer && actual_lens && out && tickets, "%s: null pointer", what);
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_bstride = q_batch_stride;
  a.H = num_q_heads;
  a.k = k_layer;
  a.v = v_layer;
  a.kv_rows = kv_rows;
  a.KV = kv_heads;
  a.D = head_dim;
  a.actual = actual_lens;
  a.scale = scale;
  a.out = out;
  a.tickets = tickets;
  a.r2t = nullptr;
  a.r2t_stride = 0;
  a.r2t_rows = 0;
  a.rpi = nullptr;
  a.positions = nullptr;
  a.rows = nullptr;
  return QQ_OK;
}

}  // namespace
}  // namespace qq

using namespace qq;

extern "C" int64_t qq_decode_attention_workspace_bytes(int bs, int max_rows, int num_q_heads,
                                                       int head_dim) {
  const int64_t chunks = (max_rows + kChunk - 1) / kChunk;
  return (int64_t)bs * chunks * num_q_heads * (head_dim + 2) * (int64_t)sizeof(float);
}

extern "C" int qq_quest_decode_attention(const void* q, int q_dtype, int64_t q_batch_stride,
                                         int num_q_heads, const void* k_layer, const void* v_layer,
                                         int kv_dtype, int64_t kv_rows, int kv_heads, int head_dim,
                                         const int32_t* req_to_token, int64_t req_to_token_stride,
                                         int64_t req_to_token_rows, const int64_t* req_pool_indices, const int32_t* positions,
                                         int64_t positions_stride, const int32_t* actual_lens,
                                         int bs, float scale, void* out, void* workspace,
                                         int64_t workspace_bytes, int32_t* tickets, void* stream) {
  const char* what = "qq_quest_decode_attention";
  if (bs == 0) return QQ_OK;
  AttnArgs a;
  int st = fill_common(a, q, q_dtype, q_batch_stride, num_q_heads, k_layer, v_layer, kv_dtype,
                       kv_rows, kv_heads, head_dim, actual_lens, scale, out, tickets, what);
  if (st != QQ_OK) return st;
  QQ_REQUIRE(req_to_token && req_pool_indices && positions && positions_stride > 0,
             "%s: null row map", what);
  a.r2t = req_to_token;
  a.r2t_stride = req_to_token_stride;
  a.r2t_rows = req_to_token_rows;
  a.rpi = req_pool_indices;
  a.positions = positions;
  a.pos_stride = positions_stride;
  return launch_attention(a, kv_dtype, bs, workspace_bytes, workspace, stream, what);
}

extern "C" int qq_decode_attention_rows(const void* q, int q_dtype, int64_t q_batch_stride,
                                        int num_q_heads, const void* k_layer, const void* v_layer,
                                        int kv_dtype, int64_t kv_rows, int kv_heads, int head_dim,
                                        const int64_t* rows, int64_t rows_stride,
                                        const int32_t* actual_lens, int bs, float scale, void* out,
                                        void* workspace, int64_t workspace_bytes, int32_t* tickets,
                                        void* stream) {
  const char* what = "qq_decode_attention_rows";
  if (bs == 0) return QQ_OK;
  AttnArgs a;
  int st = fill_common(a, q, q_dtype, q_batch_stride, num_q_heads, k_layer, v_layer, kv_dtype,
                       kv_rows, kv_heads, head_dim, actual_lens, scale, out, tickets, what);
  if (st != QQ_OK) return st;
  QQ_REQUIRE(rows && rows_stride > 0, "%s: null row list", what);
  a.rows = rows;
  a.pos_stride = rows_stride;
  return launch_attention(a, kv_dtype, bs, workspace_bytes, workspace, stream, what);
}
