// Quest page bounds: sentinel reset, prefill build, decode fold + finalize,
// per-step layout scalars, and the KV-pool scatter write.
//
// Layouts (reference src/qwenquest/quest.py:194-208):
//   page_k_bounds [L, R, MP, C, 2] bf16 with C = KV*D; one (min, max) pair is one
//   32-bit word, so a page of one layer is C contiguous words (2 KiB at C=512).
//   running_k_min/max [L, R, C] bf16.
#include "qq_common.h"

namespace qq {
namespace {

constexpr int kThreads = 256;

__device__ inline uint32_t pack_pair(uint16_t mn, uint16_t mx) {
  return (uint32_t)mn | ((uint32_t)mx << 16);
}

// One block per (request-run chunk, request, layer) writes sentinel pairs.
__global__ __launch_bounds__(kThreads) void reset_bounds_kernel(uint32_t* bounds, int R, int64_t page_words,
                                                              int req_begin, int64_t chunk) {
  const int req = req_begin + blockIdx.y;
  const int layer = blockIdx.z;
  uint32_t* base = bounds + ((int64_t)layer * R + req) * page_words;
  const int64_t begin = (int64_t)blockIdx.x * chunk;
  const int64_t end = min(begin + chunk, page_words);
  for (int64_t i = begin + threadIdx.x; i < end; i += kThreads) base[i] = kSentinelPair;
}

__global__ __launch_bounds__(kThreads) void reset_running_kernel(uint16_t* rmin, uint16_t* rmax, int32_t* count,
                                                               int32_t* page_idx, int R, int C,
                                                               int req_begin, int req_count) {
  const int layer = blockIdx.y;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < (int64_t)req_count * C;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t off = ((int64_t)layer * R + req_begin) * C + i;
    rmin[off] = kBf16Max;
    rmax[off] = kBf16Min;
  }
  if (layer == 0 && blockIdx.x == 0) {
    for (int r = threadIdx.x; r < req_count; r += kThreads) {
      count[req_begin + r] = 0;
      page_idx[req_begin + r] = 0;
    }
  }
}

struct PrefillArgs {
  const char* k_base;
  int64_t k_layer_stride_bytes;
  int k_dtype;
  int64_t k_rows;
  const void* idx;
  int idx64;
  int64_t n;
  int req, layer_begin, n_layers, set_counters;
  uint32_t* bounds;
  uint16_t *rmin, *rmax;
  int32_t *count, *page_idx;
  int R, MP, C, P;
  int64_t full_pages;
};

__device__ inline int64_t load_index(const void* p, int is64, int64_t i) {
  return is64 ? static_cast<const int64_t*>(p)[i] : (int64_t) static_cast<const int32_t*>(p)[i];
}

// quest.py:256-276 - blockIdx.x = page (the last one may be the partial tail),
// blockIdx.y = layer within the fused range.  The page's row indices are staged
// in LDS (chunks of kRowChunk), then every thread folds its channels over the
// rows with independent loads (one row = KV*D contiguous elements, so each
// row step of the block is one coalesced KV*D-element read).
constexpr int kRowChunk = 256;

__global__ __launch_bounds__(kThreads) void prefill_bounds_kernel(PrefillArgs a) {
  const int64_t page = blockIdx.x;
  const int li = blockIdx.y;
  const int layer = a.layer_begin + li;
  const int64_t begin = page * a.P;
  const int64_t end = min(begin + (int64_t)a.P, a.n);
  if (a.set_counters && page == 0 && li == a.n_layers - 1 && threadIdx.x == 0) {
    a.count[a.req] = (int32_t)(a.n - a.full_pages * a.P);
    a.page_idx[a.req] = (int32_t)a.full_pages;
  }
  if (begin >= end) return;
  const void* kl = a.k_base + (int64_t)li * a.k_layer_stride_bytes;
  __shared__ int64_t s_rows[kRowChunk];
  constexpr int kMaxCPerThread = 8;  // C <= 2048
  // start from +inf / -inf so the first valid row wins every comparison
  uint16_t mn[kMaxCPerThread], mx[kMaxCPerThread];
#pragma unroll
  for (int i = 0; i < kMaxCPerThread; ++i) {
    mn[i] = 0x7F80;
    mx[i] = 0xFF80;
  }
  for (int64_t t0 = begin; t0 < end; t0 += kRowChunk) {
    const int cnt = (int)min((int64_t)kRowChunk, end - t0);
    __syncthreads();
    for (int t = threadIdx.x; t < cnt; t += kThreads) {
      const int64_t row = load_index(a.idx, a.idx64, t0 + t);
      s_rows[t] = (row >= 0 && row < a.k_rows) ? row : -1;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kMaxCPerThread; ++i) {
      const int c = threadIdx.x + i * kThreads;
      if (c >= a.C) break;
#pragma unroll 8
      for (int t = 0; t < cnt; ++t) {
        const int64_t row = s_rows[t];
        if (row < 0) continue;
        const uint16_t v = load_as_bf16(kl, row * a.C + c, a.k_dtype);
        mn[i] = bmin(mn[i], v);
        mx[i] = bmax(mx[i], v);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kMaxCPerThread; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c >= a.C) break;
    const int64_t rc = ((int64_t)layer * a.R + a.req) * a.C + c;
    if (page < a.full_pages) {
      if (page < a.MP)
        a.bounds[(((int64_t)layer * a.R + a.req) * a.MP + page) * a.C + c] = pack_pair(mn[i], mx[i]);
    } else {
      a.rmin[rc] = mn[i];
      a.rmax[rc] = mx[i];
    }
  }
}

struct DecodeArgs {
  const char* k_base;
  int64_t k_layer_stride_bytes;
  int k_dtype;
  int64_t k_rows;
  const int64_t *reqs, *locs;
  int layer_begin, finalize;
  uint32_t* bounds;
  uint16_t *rmin, *rmax;
  const int32_t *count, *page_idx;
  int R, MP, C, P;
};

// quest.py:297-302 (+ 312-319 when finalize): blockIdx.x = listed request, blockIdx.y = layer.
__global__ __launch_bounds__(kThreads) void decode_update_kernel(DecodeArgs a) {
  const int i = blockIdx.x;
  const int li = blockIdx.y;
  const int layer = a.layer_begin + li;
  const int64_t req = a.reqs[i];
  const int64_t row = a.locs[i];
  if (req < 0 || req >= a.R || row < 0) return;  // row < 0: request skipped this step
  const bool row_ok = row < a.k_rows;
  const bool complete = a.finalize && a.count[req] == a.P - 1;
  const int64_t page = a.page_idx[req];
  const void* kl = a.k_base + (int64_t)li * a.k_layer_stride_bytes;
  for (int c = threadIdx.x; c < a.C; c += kThreads) {
    const int64_t rc = ((int64_t)layer * a.R + req) * a.C + c;
    uint16_t mn = a.rmin[rc], mx = a.rmax[rc];
    if (row_ok) {
      const uint16_t v = load_as_bf16(kl, row * a.C + c, a.k_dtype);
      mn = bmin(mn, v);
      mx = bmax(mx, v);
    }
    if (complete) {
      if (page >= 0 && page < a.MP)
        a.bounds[(((int64_t)layer * a.R + req) * a.MP + page) * a.C + c] = pack_pair(mn, mx);
      a.rmin[rc] = kBf16Max;
      a.rmax[rc] = kBf16Min;
    } else {
      a.rmin[rc] = mn;
      a.rmax[rc] = mx;
    }
  }
}

// quest.py:312-319 without the fold: blockIdx.x = listed request, blockIdx.y = layer.
__global__ __launch_bounds__(kThreads) void finalize_pages_kernel(const int64_t* reqs, uint32_t* bounds,
                                                                uint16_t* rmin, uint16_t* rmax,
                                                                const int32_t* count,
                                                                const int32_t* page_idx, int R,
                                                                int MP, int C, int P) {
  const int64_t req = reqs[blockIdx.x];
  const int layer = blockIdx.y;
  if (req < 0 || req >= R || count[req] != P - 1) return;
  const int64_t page = page_idx[req];
  for (int c = threadIdx.x; c < C; c += kThreads) {
    const int64_t rc = ((int64_t)layer * R + req) * C + c;
    if (page >= 0 && page < MP)
      bounds[(((int64_t)layer * R + req) * MP + page) * C + c] = pack_pair(rmin[rc], rmax[rc]);
    rmin[rc] = kBf16Max;
    rmax[rc] = kBf16Min;
  }
}

// quest.py:312-321 counters: runs after every layer's finalize.
// `locs` (optional): entries with locs[i] < 0 are skipped, as in decode_update_kernel.
__global__ __launch_bounds__(kThreads) void advance_counters_kernel(const int64_t* reqs, const int64_t* locs,
                                                                  int n, int32_t* count,
                                                                  int32_t* page_idx, int R, int P) {
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const int64_t req = reqs[i];
    if (req < 0 || req >= R || (locs && locs[i] < 0)) continue;
    const int32_t c = count[req];
    if (c == P - 1) page_idx[req] += 1;
    count[req] = (c + 1) % P;
  }
}

// quest.py:343-352.
__global__ __launch_bounds__(kThreads) void prepare_step_kernel(const int64_t* seq, int bs, int P, int top_k,
                                                              int avoid, int32_t* actual,
                                                              int32_t* limit) {
  for (int i = blockIdx.x * kThreads + threadIdx.x; i < bs; i += gridDim.x * kThreads) {
    const int64_t s = seq[i];
    actual[i] = (int32_t)min(s, (int64_t)top_k);
    const int64_t full = s / P;
    limit[i] = (int32_t)(avoid ? max(full - 1, (int64_t)0) : full);
  }
}

template <typename Dst, typename Src>
__device__ inline Dst convert(Src v);
template <> __device__ inline uint16_t convert<uint16_t, uint16_t>(uint16_t v) { return v; }
template <> __device__ inline float convert<float, float>(float v) { return v; }
template <> __device__ inline uint16_t convert<uint16_t, float>(float v) { return f2bf(v); }
template <> __device__ inline float convert<float, uint16_t>(uint16_t v) { return bf2f(v); }

// memory.py:117-120: dst[locs[i]] = src[i] for K and V.
template <typename Dst, typename Src>
__global__ __launch_bounds__(kThreads) void kv_scatter_kernel(Dst* k_dst, Dst* v_dst, int64_t rows,
                                                            const Src* k_src, const Src* v_src,
                                                            const int64_t* locs, int64_t row_elems) {
  const int64_t loc = locs[blockIdx.x];
  if (loc < 0 || loc >= rows) return;
  const Src* ks = k_src + (int64_t)blockIdx.x * row_elems;
  const Src* vs = v_src + (int64_t)blockIdx.x * row_elems;
  Dst* kd = k_dst + loc * row_elems;
  Dst* vd = v_dst + loc * row_elems;
  for (int64_t e = threadIdx.x; e < row_elems; e += kThreads) {
    kd[e] = convert<Dst, Src>(ks[e]);
    vd[e] = convert<Dst, Src>(vs[e]);
  }
}

}  // namespace
}  // namespace qq

using namespace qq;

extern "C" int qq_quest_reset(uint16_t* page_k_bounds, uint16_t* running_k_min,
                              uint16_t* running_k_max, int32_t* running_token_count,
                              int32_t* running_page_idx, int num_layers, int max_reqs,
                              int max_pages, int kv_heads, int head_dim, int req_begin,
                              int req_count, void* stream) {
  QQ_REQUIRE(page_k_bounds && running_k_min && running_k_max && running_token_count &&
                 running_page_idx,
             "qq_quest_reset: null pointer");
  QQ_REQUIRE(num_layers > 0 && max_reqs > 0 && max_pages >= 0 && kv_heads > 0 && head_dim > 0,
             "qq_quest_reset: bad geometry");
  QQ_REQUIRE(req_begin >= 0 && req_count >= 0 && req_begin + req_count <= max_reqs,
             "qq_quest_reset: request range [%d, %d) outside [0, %d)", req_begin,
             req_begin + req_count, max_reqs);
  if (req_count == 0) return QQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int C = kv_heads * head_dim;
  const int64_t page_words = (int64_t)max_pages * C;
  if (page_words > 0) {
    const int64_t chunk = 16384;
    dim3 grid(ceil_div(page_words, chunk), req_count, num_layers);
    reset_bounds_kernel<<<grid, kThreads, 0, s>>>(reinterpret_cast<uint32_t*>(page_k_bounds),
                                                  max_reqs, page_words, req_begin, chunk);
  }
  dim3 g2(min(ceil_div((int64_t)req_count * C, kThreads), 1024), num_layers);
  reset_running_kernel<<<g2, kThreads, 0, s>>>(running_k_min, running_k_max, running_token_count,
                                               running_page_idx, max_reqs, C, req_begin, req_count);
  return check_launch("qq_quest_reset");
}

extern "C" int qq_quest_prefill_bounds(const void* k_base, int64_t k_layer_stride, int k_dtype,
                                       int64_t k_rows, const void* prefill_indices,
                                       int indices_are_int64, int64_t n_tokens, int req,
                                       int layer_begin, int n_layers, int set_counters,
                                       uint16_t* page_k_bounds, uint16_t* running_k_min,
                                       uint16_t* running_k_max, int32_t* running_token_count,
                                       int32_t* running_page_idx, int num_layers, int max_reqs,
                                       int max_pages, int kv_heads, int head_dim, int page_size,
                                       void* stream) {
  QQ_REQUIRE(dtype_ok(k_dtype), "qq_quest_prefill_bounds: unsupported key dtype %d", k_dtype);
  QQ_REQUIRE(page_size > 0 && kv_heads > 0 && head_dim > 0, "qq_quest_prefill_bounds: bad geometry");
  QQ_REQUIRE(req >= 0 && req < max_reqs, "qq_quest_prefill_bounds: request %d out of range", req);
  QQ_REQUIRE(layer_begin >= 0 && n_layers > 0 && layer_begin + n_layers <= num_layers,
             "qq_quest_prefill_bounds: layer range out of range");
  QQ_REQUIRE(n_tokens >= 0 && (n_tokens == 0 || prefill_indices), "qq_quest_prefill_bounds: bad indices");
  QQ_REQUIRE(kv_heads * head_dim <= 8 * kThreads,
             "qq_quest_prefill_bounds: kv_heads*head_dim %d exceeds %d", kv_heads * head_dim,
             8 * kThreads);
  const int64_t full = n_tokens / page_size;
  QQ_REQUIRE(full <= max_pages, "qq_quest_prefill_bounds: %lld tokens exceed %d pages",
             (long long)n_tokens, max_pages);
  PrefillArgs a;
  a.k_base = static_cast<const char*>(k_base);
  a.k_layer_stride_bytes = k_layer_stride * dtype_size(k_dtype);
  a.k_dtype = k_dtype;
  a.k_rows = k_rows;
  a.idx = prefill_indices;
  a.idx64 = indices_are_int64;
  a.n = n_tokens;
  a.req = req;
  a.layer_begin = layer_begin;
  a.n_layers = n_layers;
  a.set_counters = set_counters;
  a.bounds = reinterpret_cast<uint32_t*>(page_k_bounds);
  a.rmin = running_k_min;
  a.rmax = running_k_max;
  a.count = running_token_count;
  a.page_idx = running_page_idx;
  a.R = max_reqs;
  a.MP = max_pages;
  a.C = kv_heads * head_dim;
  a.P = page_size;
  a.full_pages = full;
  const int pages = max(1, ceil_div(n_tokens, page_size));
  dim3 grid(pages, n_layers);
  prefill_bounds_kernel<<<grid, kThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
  return check_launch("qq_quest_prefill_bounds");
}

extern "C" int qq_quest_decode_update(const void* k_base, int64_t k_layer_stride, int k_dtype,
                                      int64_t k_rows, const int64_t* req_indices,
                                      const int64_t* device_locs, int n, int layer_begin,
                                      int n_layers, int finalize, uint16_t* page_k_bounds,
                                      uint16_t* running_k_min, uint16_t* running_k_max,
                                      int32_t* running_token_count, int32_t* running_page_idx,
                                      int num_layers, int max_reqs, int max_pages, int kv_heads,
                                      int head_dim, int page_size, void* stream) {
  QQ_REQUIRE(dtype_ok(k_dtype), "qq_quest_decode_update: unsupported key dtype %d", k_dtype);
  QQ_REQUIRE(n >= 0, "qq_quest_decode_update: negative count");
  QQ_REQUIRE(layer_begin >= 0 && n_layers > 0 && layer_begin + n_layers <= num_layers,
             "qq_quest_decode_update: layer range out of range");
  QQ_REQUIRE(!finalize || (layer_begin == 0 && n_layers == num_layers),
             "qq_quest_decode_update: finalize needs the full layer range");
  if (n == 0) return QQ_OK;
  DecodeArgs a;
  a.k_base = static_cast<const char*>(k_base);
  a.k_layer_stride_bytes = k_layer_stride * dtype_size(k_dtype);
  a.k_dtype = k_dtype;
  a.k_rows = k_rows;
  a.reqs = req_indices;
  a.locs = device_locs;
  a.layer_begin = layer_begin;
  a.finalize = finalize;
  a.bounds = reinterpret_cast<uint32_t*>(page_k_bounds);
  a.rmin = running_k_min;
  a.rmax = running_k_max;
  a.count = running_token_count;
  a.page_idx = running_page_idx;
  a.R = max_reqs;
  a.MP = max_pages;
  a.C = kv_heads * head_dim;
  a.P = page_size;
  hipStream_t s = static_cast<hipStream_t>(stream);
  decode_update_kernel<<<dim3(n, n_layers), kThreads, 0, s>>>(a);
  if (finalize)
    advance_counters_kernel<<<1, kThreads, 0, s>>>(req_indices, device_locs, n,
                                                   running_token_count, running_page_idx,
                                                   max_reqs, page_size);
  return check_launch("qq_quest_decode_update");
}

extern "C" int qq_quest_decode_finalize(const int64_t* req_indices, int n, uint16_t* page_k_bounds,
                                        uint16_t* running_k_min, uint16_t* running_k_max,
                                        int32_t* running_token_count, int32_t* running_page_idx,
                                        int num_layers, int max_reqs, int max_pages, int kv_heads,
                                        int head_dim, int page_size, void* stream) {
  QQ_REQUIRE(n >= 0 && num_layers > 0, "qq_quest_decode_finalize: bad arguments");
  if (n == 0) return QQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  finalize_pages_kernel<<<dim3(n, num_layers), kThreads, 0, s>>>(
      req_indices, reinterpret_cast<uint32_t*>(page_k_bounds), running_k_min, running_k_max,
      running_token_count, running_page_idx, max_reqs, max_pages, kv_heads * head_dim, page_size);
  advance_counters_kernel<<<1, kThreads, 0, s>>>(req_indices, nullptr, n, running_token_count,
                                                 running_page_idx, max_reqs, page_size);
  return check_launch("qq_quest_decode_finalize");
}

extern "C" int qq_quest_prepare_step(const int64_t* seq_lens, int bs, int page_size, int top_k,
                                     int avoid_recent_overlap, int32_t* actual_lens,
                                     int32_t* candidate_limit, void* stream) {
  QQ_REQUIRE(page_size > 0 && top_k > 0 && bs >= 0, "qq_quest_prepare_step: bad arguments");
  if (bs == 0) return QQ_OK;
  prepare_step_kernel<<<ceil_div(bs, kThreads), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      seq_lens, bs, page_size, top_k, avoid_recent_overlap, actual_lens, candidate_limit);
  return check_launch("qq_quest_prepare_step");
}

extern "C" int qq_kv_scatter(void* k_layer, void* v_layer, int buf_dtype, int64_t kv_rows,
                             const void* k, const void* v, int src_dtype, const int64_t* locs,
                             int n, int64_t row_elems, void* stream) {
  QQ_REQUIRE(dtype_ok(buf_dtype) && dtype_ok(src_dtype), "qq_kv_scatter: unsupported dtype");
  QQ_REQUIRE(n >= 0 && row_elems > 0, "qq_kv_scatter: bad sizes");
  if (n == 0) return QQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (buf_dtype == QQ_DTYPE_BF16 && src_dtype == QQ_DTYPE_BF16)
    kv_scatter_kernel<uint16_t, uint16_t><<<n, kThreads, 0, s>>>(
        (uint16_t*)k_layer, (uint16_t*)v_layer, kv_rows, (const uint16_t*)k, (const uint16_t*)v,
        locs, row_elems);
  else if (buf_dtype == QQ_DTYPE_BF16)
    kv_scatter_kernel<uint16_t, float><<<n, kThreads, 0, s>>>(
        (uint16_t*)k_layer, (uint16_t*)v_layer, kv_rows, (const float*)k, (const float*)v, locs,
        row_elems);
  else if (src_dtype == QQ_DTYPE_BF16)
    kv_scatter_kernel<float, uint16_t><<<n, kThreads, 0, s>>>(
        (float*)k_layer, (float*)v_layer, kv_rows, (const uint16_t*)k, (const uint16_t*)v, locs,
        row_elems);
  else
    kv_scatter_kernel<float, float><<<n, kThreads, 0, s>>>((float*)k_layer, (float*)v_layer,
                                                           kv_rows, (const float*)k,
                                                           (const float*)v, locs, row_elems);
  return check_launch("qq_kv_scatter");
}
