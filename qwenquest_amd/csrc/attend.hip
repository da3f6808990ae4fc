// Gather + split-K decode attention over an explicit row list.
//
// Reference: decode_attention (src/qwenquest/attention/ops.py:48-66) applied per
// request to rows req_to_token[req, positions[:n]] (quest_only.py:149-159) or to
// hot-buffer rows (quest_hisparse.py:294-300).  Rows are attended exactly as
// listed (a duplicate counts twice); scores, softmax and PV accumulate in fp32.
//
// Two launches per call:
//   1. chunk kernel, grid (chunks, bs): block (c, b) takes rows [64c, 64c + 64)
//      of request b, gathers them through the row map and writes per q head the
//      chunk max m, l = sum exp(s - m) and o = sum exp(s - m) v to the workspace.
//      bf16 / head_dim 128 / group <= 16 uses MFMA (one wave per KV head):
//        S^T = K Q^T with v_mfma_f32_16x16x32_bf16 - K rows are the A operand,
//        16 bytes per lane straight from HBM, Q^T the B operand (query heads on
//        N, padded to 16); the S^T accumulator gives each lane one head and 4
//        consecutive tokens, which is exactly the A-operand layout of
//        v_mfma_f32_16x16x16bf16_1k, so P = exp(S - m) (bf16) feeds O = P V
//        without an LDS round trip; V comes in 16-byte row slices (8 channels)
//        transposed 4x8 in registers, channel d = 8*(lane % 16) + e.
//      Other shapes / fp32 use a scalar kernel with the same partial format.
//   2. merge kernel, grid (H, bs): out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.
#include "qq_quest_dev.h"

namespace qq {
namespace {

constexpr int kThreads = kBlock;
constexpr int kChunk = 64;



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

  int bad = 0;  // given rows: a real slot without a row (a failed swap-in) poisons the output
  if (tid < cnt) {
    int64_t row;
    if (a.rows) {
      row = a.rows[(int64_t)b * a.pos_stride + r0 + tid];
      bad = row < 0;
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
  const bool poison = __syncthreads_or(bad) != 0;

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
    s_l[h] = poison ? __builtin_nanf("") : l;  // NaN survives every weight of the merge
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

}

__device__ inline int64_t chunk_row(const AttnArgs& a, int b, int i) {
  int64_t row;
  if (a.rows) {
    row = a.rows[(int64_t)b * a.pos_stride + i];
  } else {
    const int64_t p = a.positions[(int64_t)b * a.pos_stride + i];
    const int64_t req = a.rpi[b];
    const bool ok = p >= 0 && p < a.r2t_stride && req >= 0 && req < a.r2t_rows;
    row = ok ? (int64_t)a.r2t[req * a.r2t_stride + p] : 0;
  }
  return (row >= 0 && row < a.kv_rows) ? row : 0;
}

// bf16, head_dim 128, G = H/KV <= 16: one wave per KV head, 64 rows per block.
template <int KV>
__global__ __launch_bounds__(64 * KV) void attn_mfma_kernel(AttnArgs a) {
  const int c = blockIdx.x, b = blockIdx.y;
  const int n = (int)min((int64_t)a.actual[b], a.pos_stride);
  const int nc = (n + kChunk - 1) / kChunk;
  if (c >= nc) return;
  const int r0 = c * kChunk, cnt = min(kChunk, n - r0);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int lo = l & 15, hi = l >> 4;
  const int G = a.H / KV;
  constexpr int kRow = KV * kMfmaDim;  // elements per pool row
  // row pointers per KV head (row base + head * 128 channels)
  __shared__ const uint16_t* s_kp[KV][kChunk];
  __shared__ const uint16_t* s_vp[KV][kChunk];
  int bad = 0;  // given rows: a real slot without a row (a failed swap-in) poisons the output
  if (threadIdx.x < kChunk) {
    if (a.rows && threadIdx.x < cnt) bad = a.rows[(int64_t)b * a.pos_stride + r0 + threadIdx.x] < 0;
    const int64_t row = threadIdx.x < cnt ? chunk_row(a, b, r0 + threadIdx.x) : 0;
#pragma unroll
    for (int h = 0; h < KV; ++h) {
      s_kp[h][threadIdx.x] = static_cast<const uint16_t*>(a.k) + row * kRow + h * kMfmaDim;
      s_vp[h][threadIdx.x] = static_cast<const uint16_t*>(a.v) + row * kRow + h * kMfmaDim;
    }
  }
  const bool poison = __syncthreads_or(bad) != 0;
  float mx, sum;
  float4_t o[8];
  const uint16_t* qh = static_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_bstride + (int64_t)w * G * kMfmaDim;
  attn_wave64(s_kp[w], s_vp[w], qh, G, cnt, a.scale * kLog2e, mx, sum, o);

  const int64_t part = (int64_t)b * a.max_chunks + c;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int head = hi * 4 + i;
    if (head < G) {
      float* dst = a.ws_o + (part * a.H + w * G + head) * kMfmaDim + lo * 8;
      *reinterpret_cast<float4*>(dst) = make_float4(o[0][i], o[1][i], o[2][i], o[3][i]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4][i], o[5][i], o[6][i], o[7][i]);
    }
  }
  if (hi == 0 && lo < G) {
    float* ml = a.ws_ml + (part * a.H + w * G + lo) * 2;
    ml[0] = mx * kLn2;
    ml[1] = poison ? __builtin_nanf("") : sum;
  }
}

// Combines the chunk partials of one (head, request): grid (H, bs), one thread
// per channel.  Each thread issues the loads of up to 32 chunks' (m, l, o) at
// once, then folds them with the online-softmax update
// (M' = max(M, m_c), L = L e^(M - M') + l_c e^(m_c - M'), same for O).
constexpr int kMaxChunks = 1024;
constexpr int kMergeGroup = 32;

__global__ __launch_bounds__(kThreads) void attn_merge_kernel(AttnArgs a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int n = (int)min((int64_t)a.actual[b], a.pos_stride);
  const int nc = (n + kChunk - 1) / kChunk;
  const int H = a.H, D = a.D;
  const int64_t base = (int64_t)b * a.max_chunks;
  const float* ml = a.ws_ml + (base * H + h) * 2;
  const int64_t mls = (int64_t)H * 2;
  const float* op = a.ws_o + (base * H + h) * D;
  const int64_t os = (int64_t)H * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += kMergeGroup) {
      float mv[kMergeGroup], lv[kMergeGroup], ov[kMergeGroup];
#pragma unroll
      for (int u = 0; u < kMergeGroup; ++u) {
        const bool ok = c0 + u < nc;
        mv[u] = ok ? ml[(c0 + u) * mls] : -INFINITY;
        lv[u] = ok ? ml[(c0 + u) * mls + 1] : 0.0f;
        ov[u] = ok ? op[(c0 + u) * os + d] : 0.0f;
      }
      float gm = M;
#pragma unroll
      for (int u = 0; u < kMergeGroup; ++u) gm = fmaxf(gm, mv[u]);
      const float sc = (M == -INFINITY) ? 0.0f : expf(M - gm);
      L *= sc;
      O *= sc;
#pragma unroll
      for (int u = 0; u < kMergeGroup; ++u) {
        const float wgt = (mv[u] == -INFINITY) ? 0.0f : expf(mv[u] - gm);
        L += wgt * lv[u];
        O += wgt * ov[u];
      }
      M = gm;
    }
    const float r = nc > 0 ? O / L : 0.0f;
    const int64_t oi = ((int64_t)b * H + h) * D + d;
    if (a.q_dtype == QQ_DTYPE_BF16)
      static_cast<uint16_t*>(a.out)[oi] = f2bf(r);
    else
      static_cast<float*>(a.out)[oi] = r;
  }
}

// Fast merge (nc <= 64 chunks, D a multiple of 64): lane c < nc loads (m_c,
// l_c) of its chunk; wave reductions give M and L, the chunk weights e^(m_c - M)
// go through LDS; every thread issued its channel's o_c loads before all that.
__global__ __launch_bounds__(1024) void attn_merge64_kernel(AttnArgs a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int n = (int)min((int64_t)a.actual[b], a.pos_stride);
  const int nc = (n + kChunk - 1) / kChunk;
  const int H = a.H, D = a.D;
  const int64_t base = (int64_t)b * a.max_chunks;
  const int d = threadIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float* op = a.ws_o + (base * H + h) * D + d;
  const int64_t os = (int64_t)H * D;
  float ov[64];
#pragma unroll
  for (int u = 0; u < 64; ++u) ov[u] = u < nc ? op[u * os] : 0.0f;
  float2 ml = make_float2(-INFINITY, 0.0f);
  if (lane < nc) ml = *reinterpret_cast<const float2*>(a.ws_ml + ((base + lane) * H + h) * 2);
  float M = ml.x;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  const float wgt = lane < nc ? expf(ml.x - M) : 0.0f;
  float L = wgt * ml.y;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) L += __shfl_xor(L, off, 64);
  __shared__ float s_w[16][64];
  s_w[wave][lane] = wgt;
  __syncthreads();
  const float* w = s_w[wave];
  float O = 0.0f;
#pragma unroll
  for (int u = 0; u < 64; ++u) O += w[u] * ov[u];
  const float r = nc > 0 ? O / L : 0.0f;
  const int64_t oi = ((int64_t)b * H + h) * D + d;
  if (a.q_dtype == QQ_DTYPE_BF16)
    static_cast<uint16_t*>(a.out)[oi] = f2bf(r);
  else
    static_cast<float*>(a.out)[oi] = r;
}

}  // namespace

int launch_attention(AttnArgs& a, int kv_dtype, int bs, int64_t workspace_bytes, void* workspace,
                     hipStream_t s, const char* what) {
  const int64_t need = qq_decode_attention_workspace_bytes(bs, (int)a.pos_stride, a.H, a.D);
  QQ_REQUIRE(workspace && workspace_bytes >= need, "%s: workspace %lld bytes < %lld needed", what,
             (long long)workspace_bytes, (long long)need);
  a.max_chunks = ceil_div(a.pos_stride, kChunk);
  QQ_REQUIRE(a.max_chunks <= kMaxChunks, "%s: %lld rows per request exceed %d", what,
             (long long)a.pos_stride, kMaxChunks * kChunk);
  a.ws_o = static_cast<float*>(workspace);
  a.ws_ml = a.ws_o + (int64_t)bs * a.max_chunks * a.H * a.D;
  const size_t smem = kChunk * sizeof(int64_t) + (size_t)(a.H * a.D + a.H * kChunk + 2 * a.H) * 4;
  QQ_REQUIRE(smem <= 64 * 1024, "%s: %d heads x %d dims need too much LDS", what, a.H, a.D);
  dim3 grid(max(1, a.max_chunks), bs);
  const int G = a.H / a.KV;
  const bool mfma = a.q_dtype == QQ_DTYPE_BF16 && kv_dtype == QQ_DTYPE_BF16 && a.D == kMfmaDim &&
                    G <= 16 && (a.KV == 1 || a.KV == 2 || a.KV == 4 || a.KV == 8);
  if (mfma) {
    switch (a.KV) {
      case 1: attn_mfma_kernel<1><<<grid, 64, 0, s>>>(a); break;
      case 2: attn_mfma_kernel<2><<<grid, 128, 0, s>>>(a); break;
      case 4: attn_mfma_kernel<4><<<grid, 256, 0, s>>>(a); break;
      default: attn_mfma_kernel<8><<<grid, 512, 0, s>>>(a); break;
    }
  } else if (kv_dtype == QQ_DTYPE_BF16) {
    attn_chunk_kernel<uint16_t><<<grid, kThreads, smem, s>>>(a);
  } else {
    attn_chunk_kernel<float><<<grid, kThreads, smem, s>>>(a);
  }
  if (a.max_chunks <= 64 && a.D % 64 == 0 && a.D <= 1024)
    attn_merge64_kernel<<<dim3(a.H, bs), a.D, 0, s>>>(a);
  else
    attn_merge_kernel<<<dim3(a.H, bs), a.D <= 128 ? 128 : kThreads, 0, s>>>(a);
  return check_launch(what);
}

int fill_common(AttnArgs& a, const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                const void* k_layer, const void* v_layer, int kv_dtype, int64_t kv_rows,
                int kv_heads, int head_dim, const int32_t* actual_lens, float scale, void* out,
                const char* what) {
  QQ_REQUIRE(dtype_ok(q_dtype) && dtype_ok(kv_dtype), "%s: unsupported dtype", what);
  QQ_REQUIRE(kv_heads > 0 && head_dim > 0 && num_q_heads > 0 && num_q_heads % kv_heads == 0,
             "%s: q_heads %d not divisible by kv_heads %d", what, num_q_heads, kv_heads);
  QQ_REQUIRE(q && k_layer && v_layer && actual_lens && out, "%s: null pointer", what);
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
  a.r2t = nullptr;
  a.r2t_stride = 0;
  a.r2t_rows = 0;
  a.rpi = nullptr;
  a.positions = nullptr;
  a.rows = nullptr;
  return QQ_OK;
}

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
                                         int64_t workspace_bytes, void* stream) {
  const char* what = "qq_quest_decode_attention";
  if (bs == 0) return QQ_OK;
  AttnArgs a;
  int st = fill_common(a, q, q_dtype, q_batch_stride, num_q_heads, k_layer, v_layer, kv_dtype,
                       kv_rows, kv_heads, head_dim, actual_lens, scale, out, what);
  if (st != QQ_OK) return st;
  QQ_REQUIRE(req_to_token && req_pool_indices && positions && positions_stride > 0,
             "%s: null row map", what);
  a.r2t = req_to_token;
  a.r2t_stride = req_to_token_stride;
  a.r2t_rows = req_to_token_rows;
  a.rpi = req_pool_indices;
  a.positions = positions;
  a.pos_stride = positions_stride;
  return launch_attention(a, kv_dtype, bs, workspace_bytes, workspace, static_cast<hipStream_t>(stream), what);
}

extern "C" int qq_decode_attention_rows(const void* q, int q_dtype, int64_t q_batch_stride,
                                        int num_q_heads, const void* k_layer, const void* v_layer,
                                        int kv_dtype, int64_t kv_rows, int kv_heads, int head_dim,
                                        const int64_t* rows, int64_t rows_stride,
                                        const int32_t* actual_lens, int bs, float scale, void* out,
                                        void* workspace, int64_t workspace_bytes, void* sync,
                                        int64_t sync_bytes, void* stream) {
  const char* what = "qq_decode_attention_rows";
  if (bs == 0) return QQ_OK;
  AttnArgs a;
  int st = fill_common(a, q, q_dtype, q_batch_stride, num_q_heads, k_layer, v_layer, kv_dtype,
                       kv_rows, kv_heads, head_dim, actual_lens, scale, out, what);
  if (st != QQ_OK) return st;
  QQ_REQUIRE(rows && rows_stride > 0, "%s: null row list", what);
  if (sync && q_dtype == QQ_DTYPE_BF16 && kv_dtype == QQ_DTYPE_BF16 && kv_heads == 4 && head_dim == kMfmaDim &&
      attend_rows_fused(q, q_batch_stride, num_q_heads, k_layer, v_layer, kv_rows, rows, rows_stride, actual_lens, bs,
                        scale, out, workspace, workspace_bytes, sync, sync_bytes,
                        static_cast<hipStream_t>(stream)) == QQ_OK)
    return check_launch(what);
  a.rows = rows;
  a.pos_stride = rows_stride;
  return launch_attention(a, kv_dtype, bs, workspace_bytes, workspace, static_cast<hipStream_t>(stream), what);
}
