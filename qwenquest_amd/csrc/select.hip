// Quest page scoring + top-k page selection + token layout.
//
// Reference: src/qwenquest/quest.py:366-464 (group_queries, page_scores,
// retrieve_topk) and the layout of prepare_step (quest.py:333-342).
//
// Launch 1, grid (page blocks, bs): each block averages q over the GQA group
// (once, into LDS) while its 4 waves' page loads are in flight; each wave then
// scores 8 candidate pages of [0, candidate_limit): lane l holds
// channels [l*m, l*m + m) of the page (m = ceil(KV*D / 64)), so a wave reads a
// page's KV*D (min, max) words as one coalesced 2 KiB stream at KV*D = 512.
// Per page the lane adds its m fp32 products in channel order and the 64 lane
// sums are combined by a halving tree (acc[l] += acc[l + w], w = 32 .. 1) - the
// canonical order the oracle reproduces.
// Launch 2, one block per request: the top k = top_k/P - 1 pages by (score desc,
// page asc), then positions (pages x P, then the recent window); short requests
// get the dense layout.  k <= 64 over <= 4096 pages: a threshold from the
// per-thread maxima filters the keys, survivors are rank-counted; otherwise a 4-pass radix
// select on order-preserving 32-bit keys with ties at the threshold to the
// lowest page index.
#include "qq_quest_dev.h"

namespace qq {
namespace {

constexpr int kThreads = kBlock;
constexpr int kMaxSel = 1024;  // top_k / P - 1
constexpr int kPagesPerBlock = 32;



// Block-wide inclusive suffix sum over 256 entries of `v` (in place).
__device__ inline void suffix_sum_256(uint32_t* v) {
  const int t = threadIdx.x;
  for (int off = 1; off < 256; off <<= 1) {
    __syncthreads();
    const uint32_t add = (t + off < 256) ? v[t + off] : 0u;
    __syncthreads();
    v[t] += add;
  }
  __syncthreads();
}

// Block-wide exclusive prefix sum over 256 entries (in place).
__device__ inline void prefix_sum_256_exclusive(int* v) {
  const int t = threadIdx.x;
  const int mine = v[t];
  for (int off = 1; off < 256; off <<= 1) {
    __syncthreads();
    const int add = (t >= off) ? v[t - off] : 0;
    __syncthreads();
    v[t] += add;
  }
  __syncthreads();
  v[t] -= mine;
  __syncthreads();
}

// This lane's m channels of one page, products summed in channel order.
template <int M>
__device__ inline float lane_partial(const uint32_t (&w)[M], const float (&qreg)[M], int lane, int m,
                                     int C) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const int c = lane * m + j;
    const float qv = qreg[j];
    const float kv = qv >= 0.0f ? bf2f((uint16_t)(w[j] >> 16)) : bf2f((uint16_t)(w[j] & 0xFFFFu));
    const float prod = (j < m && c < C) ? __fmul_rn(qv, kv) : 0.0f;
    if (j == 0)
      acc = prod;
    else if (j < m)
      acc = __fadd_rn(acc, prod);
  }
  return acc;
}

template <int M>
__device__ inline void load_lane_words(uint32_t (&w)[M], const uint32_t* pb, int lane, int m, int C,
                                       bool valid) {
  if (!valid) {
#pragma unroll
    for (int j = 0; j < M; ++j) w[j] = 0u;
  } else if (M % 4 == 0 && m == M && C == 64 * M) {
    const uint4* p4 = reinterpret_cast<const uint4*>(pb + lane * M);
#pragma unroll
    for (int i = 0; i < M / 4; ++i) {
      const uint4 v = p4[i];
      w[4 * i + 0] = v.x;
      w[4 * i + 1] = v.y;
      w[4 * i + 2] = v.z;
      w[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < M; ++j) {
      const int c = lane * m + j;
      w[j] = (j < m && c < C) ? pb[c] : 0u;
    }
  }
}

// Scores the candidate pages [0, candidate_limit) of long requests: each wave
// 8 pages.  The bounds loads are issued first; q-bar is then computed once per
// block into LDS while they are in flight (the barrier does not wait for them).
template <int M>
__global__ __launch_bounds__(kThreads) void score_candidates_kernel(SelectArgs a, int store_new) {
  const int b = blockIdx.y;
  // the three per-request words are loaded together, before any branch on them
  const int64_t s = a.seq[b];
  const int lim = min(a.limit[b], a.MP);
  const int64_t req = a.rpi[b];
  if (store_new && blockIdx.x == 0) store_new_token(a, b);
  const int p0 = blockIdx.x * a.ppb;
  // dense layout / recent window only / no candidates here / no request slot
  if (s <= a.top_k || a.k_sel == 0 || p0 >= lim || req < 0 || req >= a.R) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pw = p0 + wave * 8;  // this wave's 8 pages
  const uint32_t* pbase = a.bounds_layer + req * a.MP * a.C;
  uint32_t w[8][M];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    load_lane_words<M>(w[i], pbase + (int64_t)(pw + i) * a.C, lane, a.m, a.C, pw + i < lim);
  __shared__ float s_q[kMaxC];
  block_qbar(s_q, a, b);
  __syncthreads();
  if (pw >= lim) return;
  float qreg[M];
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const int c = lane * a.m + j;
    qreg[j] = (j < a.m && c < a.C) ? s_q[c] : 0.0f;
  }
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = lane_partial<M>(w[i], qreg, lane, a.m, a.C);
  const float v = reduce8_pages(acc, lane);
  const int p = pw + (lane >> 3);
  if ((lane & 7) == 0 && p < lim) a.scores[(int64_t)b * a.MP + p] = v;
}

// score_candidates_kernel for KV*D == 64*M (M a multiple of 4): lane l holds
// channels [l*M, l*M + M) as M/4 16-byte loads.  The page addresses are wave
// uniform (scalar base + the lane's offset), min-or-max is one byte permute per
// channel picked by q-bar's sign, and the products and sums are the same fp32
// operations in the same order as lane_partial.  Pages past the candidate limit
// re-read the limit's last page and are not stored, so every load is issued
// unconditionally.
//
// Tile 0 of a request also stores the new token's K/V (set_kv_buffer); its
// loads go out with the page loads and its stores after the scores, so that
// the block's pages are not held back by the copy's round trips.
template <int M>
__global__ __launch_bounds__(kThreads) void score_pages_fast_kernel(SelectArgs a, int store_new) {
  constexpr int C = 64 * M;
  const int b = blockIdx.y;
  const int64_t s = a.seq[b];
  const int lim = min(a.limit[b], a.MP);
  const int64_t req = a.rpi[b];
  const int p0 = blockIdx.x * a.ppb;
  const bool copy_new = store_new && blockIdx.x == 0;
  if (s <= a.top_k || a.k_sel == 0 || p0 >= lim || req < 0 || req >= a.R) {
    if (copy_new) store_new_token(a, b);
    return;
  }
  // the new token as 16-byte pieces of bf16 rows of C elements, one per thread
  static_assert(C / 8 <= kThreads, "one 16-byte piece of K and of V per thread");
  const bool copy_fast = copy_new && a.new_k && a.new_dtype == QQ_DTYPE_BF16 && a.pool_dtype == QQ_DTYPE_BF16;
  uint4 nk = make_uint4(0u, 0u, 0u, 0u), nv = nk;
  int64_t loc = -1;
  if (copy_fast && threadIdx.x < C / 8) {
    loc = a.new_locs[b];
    nk = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.new_k) + (int64_t)b * C)[threadIdx.x];
    nv = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.new_v) + (int64_t)b * C)[threadIdx.x];
  }
  // bf16 queries with G <= 8: the request's query words are loaded before the
  // pages and q-bar is computed while the pages are in flight (the same fp32
  // operations in the same order as block_qbar); other queries after them
  const int G = a.H / a.KV;
  const bool q_early = a.q_dtype == QQ_DTYPE_BF16 && a.D % 2 == 0 && G > 1 && G <= 8;
  constexpr int kPairs = (C / 2 + kThreads - 1) / kThreads;  // channel pairs per thread
  uint32_t qw[kPairs][8];
  if (q_early) {
#pragma unroll
    for (int j = 0; j < kPairs; ++j) {
      const int c = (threadIdx.x + kThreads * j) * 2;
      if (c < C) {
        const int h = c / a.D, d = c - h * a.D;
        const uint32_t* qp = reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.q) +
                                                               (int64_t)b * a.q_bstride + (int64_t)h * G * a.D + d);
#pragma unroll
        for (int g = 0; g < 8; ++g) qw[j][g] = g < G ? qp[(int64_t)g * (a.D / 2)] : 0u;
      }
    }
    __asm__ volatile("" ::: "memory");  // the query loads go out before the page loads
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int pw = p0 + wave * 8;  // this wave's 8 pages
  uint32_t w[8][M];
  load_8pages<M>(w, a.bounds_layer + req * a.MP * C, pw, lim, lane);
  __shared__ float s_q[kMaxC];
  if (q_early) {
#pragma unroll
    for (int j = 0; j < kPairs; ++j) {
      const int c = (threadIdx.x + kThreads * j) * 2;
      if (c < C) {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          if (g < G) {
            a0 = __fadd_rn(a0, bf2f((uint16_t)(qw[j][g] & 0xFFFFu)));
            a1 = __fadd_rn(a1, bf2f((uint16_t)(qw[j][g] >> 16)));
          }
        }
        s_q[c] = bf2f(f2bf(a0 / (float)G));
        s_q[c + 1] = bf2f(f2bf(a1 / (float)G));
      }
    }
  } else {
    block_qbar(s_q, a, b);
  }
  lds_barrier();  // s_q is written; the page loads stay in flight
  if (pw < lim) {
    const float v = score_8pages<M>(w, s_q, lane);
    const int p = pw + (lane >> 3);
    if ((lane & 7) == 0 && p < lim) a.scores[(int64_t)b * a.MP + p] = v;
  }
  if (copy_fast) {
    if (threadIdx.x < C / 8 && loc >= 0 && loc < a.pool_rows) {
      reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.k_pool) + loc * C)[threadIdx.x] = nk;
      reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.v_pool) + loc * C)[threadIdx.x] = nv;
    }
  } else if (copy_new) {
    store_new_token(a, b);
  }
}

// score_pages_fast_kernel at KV*D = 4*128 with bf16 queries and 2 <= G <= 8 (the
// shape of the fused layer step), in a shape that reads the bounds faster: each
// wave scores 4 pages, a 256-thread block 16, and the kernel fits 64 VGPRs, so
// eight waves per SIMD hold every block of a batch of 16 at 128K at once (2048
// blocks; 8 x 16-byte loads per lane in flight instead of 16).  Each load
// instruction reads 1 KiB of a page: lane l holds words [4l, 4l + 4) of the page's
// first half and of its second.  The canonical lane partials (lane L: channels
// 8L .. 8L+7 summed in order) are rebuilt exactly: an even lane's four products
// are the first half of an odd lane's sum, which continues it after one DPP move,
// so odd lane 2m+1 holds the partials of canonical lanes m (first half) and m + 32
// (second half).  Their sum is the tree's first level; the levels 16 .. 1 pair
// odd lanes 32, 16, 8, 4 and 2 apart, the 4 pages' trees interleaved as in
// reduce8_pages.  Lane 16p + 1 ends with page p's score, bit-identical to
// score_8pages.  The query words of the GQA mean are loaded unconditionally (heads
// past G re-read the last one and are not summed).  One extra block per request
// (blockIdx.x == 0; page tiles follow it) stores the new token's K/V, so that its
// registers are not held across the page loads.
constexpr int kPagesPerBlock4 = 16;

// v of lane l - 1 for odd lanes (quad_perm [0, 0, 2, 2])
__device__ inline float lane_from_even(float v) { return dpp_f32<0xA0>(v); }

// Canonical partial of one 16-byte piece of each half page (words [4l, 4l + 4) and
// [256 + 4l, 256 + 4l + 4)), summed over both halves: valid in odd lanes.
__device__ inline float half_pages_partial(const uint4 (&w)[2], const float4 (&q)[2]) {
  float u = 0.0f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t ws[4] = {w[h].x, w[h].y, w[h].z, w[h].w};
    const float qs[4] = {q[h].x, q[h].y, q[h].z, q[h].w};
    float pr[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      pr[k] = __fmul_rn(qs[k], __uint_as_float(__builtin_amdgcn_perm(ws[k], ws[k], qs[k] >= 0.0f ? 0x03020C0Cu
                                                                                                  : 0x01000C0Cu)));
    const float first = __fadd_rn(__fadd_rn(__fadd_rn(pr[0], pr[1]), pr[2]), pr[3]);  // an even lane's 4
    float t = lane_from_even(first);                                                 // odd lanes: continue it
#pragma unroll
    for (int k = 0; k < 4; ++k) t = __fadd_rn(t, pr[k]);
    u = h == 0 ? t : __fadd_rn(u, t);  // tree level 32: canonical lanes m and m + 32
  }
  return u;
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void score_pages_fast4_kernel(SelectArgs a, int store_new) {
  constexpr int C = 512, D = 128;
  const int b = blockIdx.y;
  if (blockIdx.x == 0) {  // the new token's block (its test needs no argument load)
    if (store_new) store_new_token(a, b);
    return;
  }
  // every argument of the scoring path in the first batch of argument loads; the
  // request's three words go out together, and the query words (their addresses
  // need only b) before the wait for them: one round trip before the page loads
  // instead of a chain of three
  __asm__ volatile("" ::"s"(a.top_k), "s"(a.k_sel), "s"(a.R), "s"(a.MP), "s"(a.bounds_layer), "s"(a.scores));
  const int64_t s = a.seq[b];
  const int limit = a.limit[b];
  const int64_t req = a.rpi[b];
  const int G = a.H / (C / D);
  // channel pair (2t, 2t + 1) = head t >> 6, channels 2 (t & 63) .. +1
  const int tid = threadIdx.x;
  const uint32_t* qp = reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_bstride +
                                                         (int64_t)(tid >> 6) * G * D) + (tid & 63);
  uint32_t qw[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) qw[g] = qp[(int64_t)min(g, G - 1) * (D / 2)];
  __asm__ volatile("" ::"s"(s), "s"(limit), "s"(req) : "memory");
  const int lim = min(limit, a.MP);
  const int p0 = (blockIdx.x - 1) * kPagesPerBlock4;
  if (s <= a.top_k || a.k_sel == 0 || p0 >= lim || req < 0 || req >= a.R) return;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int pw = p0 + wave * 4;  // this wave's 4 pages
  uint4 w[4][2];
  {
    const char* rb = reinterpret_cast<const char*>(a.bounds_layer + req * a.MP * C) + 16 * lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const char* page = rb + (int64_t)min(pw + i, lim - 1) * (C * 4);
      w[i][0] = *reinterpret_cast<const uint4*>(page);
      w[i][1] = *reinterpret_cast<const uint4*>(page + C * 2);
    }
  }
  __shared__ __align__(16) float s_q[C];
  {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      if (g < G) {
        a0 = __fadd_rn(a0, bf2f((uint16_t)(qw[g] & 0xFFFFu)));
        a1 = __fadd_rn(a1, bf2f((uint16_t)(qw[g] >> 16)));
      }
    }
    s_q[2 * tid] = bf2f(f2bf(a0 / (float)G));
    s_q[2 * tid + 1] = bf2f(f2bf(a1 / (float)G));
  }
  lds_barrier();  // s_q is written; the page loads stay in flight
  if (pw >= lim) return;
  float4 q[2];
  q[0] = *reinterpret_cast<const float4*>(&s_q[4 * lane]);
  q[1] = *reinterpret_cast<const float4*>(&s_q[C / 2 + 4 * lane]);
  float u[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) u[i] = half_pages_partial(w[i], q);
  // tree levels 16 .. 1 over odd lanes, the 4 pages interleaved: after level 16 the
  // lower half of the wave holds pages 0, 1 and the upper half pages 2, 3; after
  // level 8 each 16-lane row holds one page
  const bool up32 = lane & 32, up16 = lane & 16;
  float v2[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float send = up32 ? u[j] : u[2 + j];
    const float keep = up32 ? u[2 + j] : u[j];
    v2[j] = __fadd_rn(keep, lane_xor32(send, lane));
  }
  float v;
  {
    const float send = up16 ? v2[0] : v2[1];
    const float keep = up16 ? v2[1] : v2[0];
    v = __fadd_rn(keep, lane_xor16(send, lane));
  }
  v = __fadd_rn(v, lane_xor8(v));  // lanes 2m+1 and 2m+9 of the row
  v = __fadd_rn(v, lane_up4(v));   // 2m+1 and 2m+5
  v = __fadd_rn(v, lane_xor2(v));  // 1 and 3
  const int p = pw + (lane >> 4);
  if ((lane & 15) == 1 && p < lim) a.scores[(int64_t)b * a.MP + p] = v;
}

// One block per request: top k_sel pages (quest.py:450-452) + token layout (453-460).
__global__ __launch_bounds__(kThreads) void select_layout_kernel(SelectArgs a) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  store_new_token(a, b);
  const int64_t s = a.seq[b];
  int32_t* pos = a.positions + (int64_t)b * a.top_k;
  if (s <= a.top_k) {  // dense layout, quest.py:339-342 / 460
    write_dense(pos, s, a.top_k);
    return;
  }
  const int k = a.k_sel;
  if (k == 0) {  // top_k == P: the recent window is the whole layout (quest.py:457-458)
    write_recent(pos, s, a.P);
    return;
  }
  const int64_t req = a.rpi[b];
  const int lim = (req >= 0 && req < a.R) ? min(a.limit[b], a.MP) : 0;
  const int n_eff = max(lim, k);
  const float* sc = a.scores + (int64_t)b * a.MP;

  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_prefix, s_mask;
  __shared__ int s_remaining;
  __shared__ uint32_t s_sel_key[kMaxSel];
  __shared__ int s_sel_idx[kMaxSel];
  __shared__ int s_order[kMaxSel];
  __shared__ int s_eq[256];
  __shared__ int s_gt;
  auto key_of = [&](int p) -> uint32_t {
    return p < lim ? orderable(sc[p]) : kNegInfKey;
  };
  if (tid == 0) {
    s_prefix = 0;
    s_mask = 0;
    s_remaining = k;
    s_gt = 0;
  }
  for (int shift = 24; shift >= 0; shift -= 8) {
    __syncthreads();
    const uint32_t prefix = s_prefix, mask = s_mask;
    const int remaining = s_remaining;
    s_hist[tid] = 0;
    __syncthreads();
    for (int p = tid; p < n_eff; p += kThreads) {
      const uint32_t key = key_of(p);
      if ((key & mask) == prefix) atomicAdd(&s_hist[(key >> shift) & 255u], 1u);
    }
    suffix_sum_256(s_hist);
    const uint32_t here = s_hist[tid];
    const uint32_t above = tid < 255 ? s_hist[tid + 1] : 0u;
    __syncthreads();
    if (here >= (uint32_t)remaining && above < (uint32_t)remaining) {
      s_prefix = prefix | ((uint32_t)tid << shift);
      s_mask = mask | (255u << shift);
      s_remaining = remaining - (int)above;
    }
  }
  __syncthreads();
  const uint32_t thr = s_prefix;
  const int ties = s_remaining;  // how many pages with key == thr to take
  const int gt = k - ties;

  // keys above the threshold (any order; ranked below), ties by lowest index
  const int chunk = (n_eff + kThreads - 1) / kThreads;
  const int lo = min(tid * chunk, n_eff), hi = min(lo + chunk, n_eff);
  int eq = 0;
  for (int p = lo; p < hi; ++p) {
    const uint32_t key = key_of(p);
    if (key > thr) {
      const int slot = atomicAdd(&s_gt, 1);
      s_sel_key[slot] = key;
      s_sel_idx[slot] = p;
    } else if (key == thr) {
      ++eq;
    }
  }
  s_eq[tid] = eq;
  prefix_sum_256_exclusive(s_eq);
  int rank = s_eq[tid];
  for (int p = lo; p < hi && rank < ties; ++p) {
    if (key_of(p) == thr) {
      s_sel_key[gt + rank] = thr;
      s_sel_idx[gt + rank] = p;
      ++rank;
    }
  }
  __syncthreads();
  for (int i = tid; i < k; i += kThreads) {
    const uint32_t ki = s_sel_key[i];
    const int ii = s_sel_idx[i];
    int r = 0;
    for (int j = 0; j < k; ++j) {
      const uint32_t kj = s_sel_key[j];
      r += (kj > ki) || (kj == ki && s_sel_idx[j] < ii);
    }
    s_order[r] = ii;
  }
  __syncthreads();
  const int P = a.P;
  for (int slot = tid; slot < k * P; slot += kThreads) {
    const int r = slot / P;
    pos[slot] = s_order[r] * P + (slot - r * P);
  }
  write_recent(pos + (int64_t)k * P, s, P);
}

// Top k <= 64 pages of n_eff <= 256*KPT keys, one block per request
// (select_topk_block), then the layout.
template <int KPT>
__global__ __launch_bounds__(kThreads) void select_filter_kernel(SelectArgs a) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  // Every load of the selection is issued up front: the request words and all
  // of the request's score slots (those past the candidate limit are masked
  // below), so the block waits for one memory round trip, not three.
  const int64_t s = a.seq[b];
  const int64_t req = a.rpi[b];
  const int lim_raw = a.limit[b];
  const float* sc = a.scores + (int64_t)b * a.MP;
  float sv[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int p = tid + kThreads * i;
    sv[i] = p < a.MP ? sc[p] : 0.0f;
  }
  int32_t* pos = a.positions + (int64_t)b * a.top_k;
  const int k = a.k_sel;
  if (s <= a.top_k || k == 0) {
    store_new_token(a, b);
    if (s <= a.top_k)
      write_dense(pos, s, a.top_k);
    else
      write_recent(pos, s, a.P);
    return;
  }
  const int lim = (req >= 0 && req < a.R) ? min(lim_raw, a.MP) : 0;
  __shared__ SelectSmem<KPT> sm;
  select_topk_block<KPT>(sv, lim, max(lim, k), k, sm);
  const int P = a.P;
  for (int slot = tid; slot < k * P; slot += kThreads) {
    const int r = slot / P;
    pos[slot] = sm.order[r] * P + (slot - r * P);
  }
  write_recent(pos + (int64_t)k * P, s, P);
  store_new_token(a, b);  // the attention launch that reads the pool comes after this one
}

// group_queries (quest.py:366-391) as its own kernel: out [bs, C] in q's dtype.
__global__ __launch_bounds__(kThreads) void group_queries_kernel(const void* q, int dtype,
                                                               int64_t bstride, int G, int D, int C,
                                                               void* out) {
  const int b = blockIdx.y;
  for (int c = blockIdx.x * kThreads + threadIdx.x; c < C; c += gridDim.x * kThreads) {
    const float v = gqa_mean(q, dtype, (int64_t)b * bstride, G, D, c);
    if (dtype == QQ_DTYPE_BF16)
      static_cast<uint16_t*>(out)[(int64_t)b * C + c] = f2bf(v);
    else
      static_cast<float*>(out)[(int64_t)b * C + c] = v;
  }
}

// page_scores (quest.py:393-405) over every page slot [0, MP), canonical order.
template <int M>
__global__ __launch_bounds__(kThreads) void page_scores_kernel(const void* qbar, int dtype,
                                                             int64_t bstride,
                                                             const uint32_t* bounds_layer,
                                                             const int64_t* rpi, int R, int MP,
                                                             int C, int m, float* scores) {
  const int b = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t req = rpi[b];
  if (req < 0 || req >= R) return;
  const int pw = blockIdx.x * kPagesPerBlock + wave * 8;
  if (pw >= MP) return;
  float qreg[M];
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const int c = lane * m + j;
    qreg[j] = (j < m && c < C) ? load_as_float(qbar, (int64_t)b * bstride + c, dtype) : 0.0f;
  }
  const uint32_t* pbase = bounds_layer + req * (int64_t)MP * C;
  uint32_t w[8][M];
#pragma unroll
  for (int i = 0; i < 8; ++i) load_lane_words<M>(w[i], pbase + (int64_t)(pw + i) * C, lane, m, C, pw + i < MP);
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = lane_partial<M>(w[i], qreg, lane, m, C);
  const float v = reduce8_pages(acc, lane);
  const int p = pw + (lane >> 3);
  if ((lane & 7) == 0 && p < MP) scores[(int64_t)b * MP + p] = v;
}

}  // namespace

void launch_select(const SelectArgs& a, int bs, int max_pages, int k_sel, hipStream_t s) {
  const int n_max = max(max_pages, k_sel);
  if (k_sel <= 64 && n_max <= 4 * kThreads)
    select_filter_kernel<4><<<bs, kThreads, 0, s>>>(a);
  else if (k_sel <= 64 && n_max <= 8 * kThreads)
    select_filter_kernel<8><<<bs, kThreads, 0, s>>>(a);
  else if (k_sel <= 64 && n_max <= 12 * kThreads)
    select_filter_kernel<12><<<bs, kThreads, 0, s>>>(a);
  else if (k_sel <= 64 && n_max <= 16 * kThreads)
    select_filter_kernel<16><<<bs, kThreads, 0, s>>>(a);
  else
    select_layout_kernel<<<bs, kThreads, 0, s>>>(a);
}

int launch_score(const SelectArgs& a, int bs, bool store_new, hipStream_t s) {
  dim3 grid(max(1, ceil_div(a.MP, kPagesPerBlock)), bs);
  const int M = (a.C + 63) / 64;
  const int st = store_new ? 1 : 0;
  const int G = a.KV > 0 ? a.H / a.KV : 0;
  if (a.C == 512 && a.D == 128 && a.q_dtype == QQ_DTYPE_BF16 && G >= 2 && G <= 8 && a.H == G * a.KV) {
    const int tiles = max(1, ceil_div(a.MP, kPagesPerBlock4));
    score_pages_fast4_kernel<<<dim3(tiles + 1, bs), kThreads, 0, s>>>(a, st);
  } else if (a.C == 512)
    score_pages_fast_kernel<8><<<grid, kThreads, 0, s>>>(a, st);
  else if (a.C == 1024)
    score_pages_fast_kernel<16><<<grid, kThreads, 0, s>>>(a, st);
  else if (a.C == 256)
    score_pages_fast_kernel<4><<<grid, kThreads, 0, s>>>(a, st);
  else if (M <= 1)
    score_candidates_kernel<1><<<grid, kThreads, 0, s>>>(a, st);
  else if (M <= 2)
    score_candidates_kernel<2><<<grid, kThreads, 0, s>>>(a, st);
  else if (M <= 4)
    score_candidates_kernel<4><<<grid, kThreads, 0, s>>>(a, st);
  else if (M <= 8)
    score_candidates_kernel<8><<<grid, kThreads, 0, s>>>(a, st);
  else
    score_candidates_kernel<16><<<grid, kThreads, 0, s>>>(a, st);
  return check_launch("quest page scores");
}

int launch_retrieve(const SelectArgs& a, int bs, hipStream_t s) {
  const int st = launch_score(a, bs, false, s);
  if (st != QQ_OK) return st;
  launch_select(a, bs, a.MP, a.k_sel, s);
  return check_launch("quest retrieve");
}

}  // namespace qq

using namespace qq;

extern "C" int qq_quest_group_queries(const void* q, int q_dtype, int64_t q_batch_stride,
                                      int num_q_heads, int kv_heads, int head_dim, int bs,
                                      void* out, void* stream) {
  QQ_REQUIRE(dtype_ok(q_dtype), "qq_quest_group_queries: unsupported dtype %d", q_dtype);
  QQ_REQUIRE(kv_heads > 0 && head_dim > 0 && num_q_heads > 0, "qq_quest_group_queries: bad heads");
  QQ_REQUIRE(num_q_heads % kv_heads == 0, "q_heads %d not divisible by kv_heads %d", num_q_heads,
             kv_heads);
  if (bs == 0) return QQ_OK;
  const int C = kv_heads * head_dim;
  dim3 grid(ceil_div(C, kThreads), bs);
  group_queries_kernel<<<grid, kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      q, q_dtype, q_batch_stride, num_q_heads / kv_heads, head_dim, C, out);
  return check_launch("qq_quest_group_queries");
}

extern "C" int qq_quest_page_scores(const void* grouped_q, int q_dtype, int64_t q_batch_stride,
                                    const uint16_t* page_k_bounds, int layer,
                                    const int64_t* req_pool_indices, int bs, int max_reqs,
                                    int max_pages, int kv_heads, int head_dim, float* scores,
                                    void* stream) {
  QQ_REQUIRE(dtype_ok(q_dtype), "qq_quest_page_scores: unsupported dtype %d", q_dtype);
  const int C = kv_heads * head_dim;
  QQ_REQUIRE(C > 0 && C <= kMaxC, "qq_quest_page_scores: kv_heads*head_dim %d unsupported", C);
  if (bs == 0 || max_pages == 0) return QQ_OK;
  const uint32_t* bl =
      reinterpret_cast<const uint32_t*>(page_k_bounds) + (int64_t)layer * max_reqs * max_pages * C;
  dim3 grid(ceil_div(max_pages, kPagesPerBlock), bs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int m = (C + 63) / 64;
  if (m <= 1)
    page_scores_kernel<1><<<grid, kThreads, 0, s>>>(grouped_q, q_dtype, q_batch_stride, bl,
                                                    req_pool_indices, max_reqs, max_pages, C, m, scores);
  else if (m <= 2)
    page_scores_kernel<2><<<grid, kThreads, 0, s>>>(grouped_q, q_dtype, q_batch_stride, bl,
                                                    req_pool_indices, max_reqs, max_pages, C, m, scores);
  else if (m <= 4)
    page_scores_kernel<4><<<grid, kThreads, 0, s>>>(grouped_q, q_dtype, q_batch_stride, bl,
                                                    req_pool_indices, max_reqs, max_pages, C, m, scores);
  else if (m <= 8)
    page_scores_kernel<8><<<grid, kThreads, 0, s>>>(grouped_q, q_dtype, q_batch_stride, bl,
                                                    req_pool_indices, max_reqs, max_pages, C, m, scores);
  else
    page_scores_kernel<16><<<grid, kThreads, 0, s>>>(grouped_q, q_dtype, q_batch_stride, bl,
                                                     req_pool_indices, max_reqs, max_pages, C, m, scores);
  return check_launch("qq_quest_page_scores");
}

extern "C" int qq_quest_retrieve_topk(const void* q, int q_dtype, int64_t q_batch_stride,
                                      int num_q_heads, const uint16_t* page_k_bounds, int layer,
                                      const int64_t* req_pool_indices, const int64_t* seq_lens,
                                      const int32_t* candidate_limit, int bs, int max_reqs,
                                      int max_pages, int kv_heads, int head_dim, int page_size,
                                      int top_k, float* scores_ws,
                                      int32_t* positions, void* stream) {
  QQ_REQUIRE(dtype_ok(q_dtype), "qq_quest_retrieve_topk: unsupported query dtype %d", q_dtype);
  QQ_REQUIRE(kv_heads > 0 && head_dim > 0 && num_q_heads > 0, "qq_quest_retrieve_topk: bad heads");
  QQ_REQUIRE(num_q_heads % kv_heads == 0, "q_heads %d not divisible by kv_heads %d", num_q_heads,
             kv_heads);
  QQ_REQUIRE(page_size > 0 && top_k > 0 && top_k % page_size == 0,
             "qq_quest_retrieve_topk: top_k %d must be a positive multiple of page_size %d", top_k,
             page_size);
  const int C = kv_heads * head_dim;
  const int k_sel = top_k / page_size - 1;
  QQ_REQUIRE(C <= kMaxC, "qq_quest_retrieve_topk: kv_heads*head_dim %d exceeds %d", C, kMaxC);
  QQ_REQUIRE(k_sel <= kMaxSel, "qq_quest_retrieve_topk: %d selected pages exceed %d", k_sel, kMaxSel);
  QQ_REQUIRE(bs >= 0 && layer >= 0 && max_pages >= 0, "qq_quest_retrieve_topk: bad sizes");
  if (bs == 0) return QQ_OK;
  SelectArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_bstride = q_batch_stride;
  a.H = num_q_heads;
  a.bounds_layer =
      reinterpret_cast<const uint32_t*>(page_k_bounds) + (int64_t)layer * max_reqs * max_pages * C;
  a.rpi = req_pool_indices;
  a.seq = seq_lens;
  a.limit = candidate_limit;
  a.R = max_reqs;
  a.MP = max_pages;
  a.KV = kv_heads;
  a.D = head_dim;
  a.C = C;
  a.m = (C + 63) / 64;
  a.P = page_size;
  a.top_k = top_k;
  a.k_sel = k_sel;
  a.ppb = kPagesPerBlock;
  a.scores = scores_ws;
  a.positions = positions;
  a.new_k = nullptr;
  const int st = launch_retrieve(a, bs, static_cast<hipStream_t>(stream));
  if (st != QQ_OK) return st;
  return check_launch("qq_quest_retrieve_topk");
}
