// Device building blocks shared by the Quest kernels: GQA mean, 8-page score
// reduction, the filter-based top-k page selection, the new-token store and
// the MFMA attention of one wave over 64 rows.  Reference formulas:
// src/qwenquest/quest.py:366-464 (group_queries, page_scores, retrieve_topk),
// src/qwenquest/attention/ops.py:48-66 (decode_attention),
// src/qwenquest/memory.py:114-120 (set_kv_buffer).
#pragma once

#include "qq_kernels.h"

namespace qq {

constexpr int kBlock = 256;  // threads of every Quest block (4 waves)
constexpr int kBlockWaves = kBlock / 64;
constexpr int kMaxC = 1024;  // KV * D

// ---------------------------------------------------------------- agent-scope
// Loads and stores at agent scope are coherent across the chip's L2 caches
// (they bypass the non-coherent cache levels), so data handed from one block
// to another inside a launch goes through them; s_waitcnt(0) before the
// hand-off's counter update makes the stores complete first.  No L2
// write-back is needed, unlike a release fence.
__device__ inline void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int32_t ld_agent(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t add_agent(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t ld_agent(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until every vector memory operation this wave issued has completed;
// the memory clobber keeps the compiler from moving memory accesses across it.
__device__ inline void wait_memory() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Block barrier for LDS hand-offs only: waits for this wave's LDS operations,
// not for its global loads and stores (which __syncthreads waits for), so they
// stay in flight across it; uses of their results get their own waits.
__device__ inline void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16-byte agent-scope loads and stores through a buffer resource (cache policy
// sc1, as the agent-scope accesses above use); offsets past `bytes` read zeros
// (and are not written).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kCachePolicyAgent = 16;  // sc1
__device__ inline __amdgpu_buffer_rsrc_t agent_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ inline float4 ld_agent_x4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const u32x4_t u = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, kCachePolicyAgent);
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}
__device__ inline void st_agent_x4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float4 v) {
  const u32x4_t u = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
  __builtin_amdgcn_raw_buffer_store_b128(u, r, (int)byte_off, 0, kCachePolicyAgent);
}

// ------------------------------------------------------------------ new token

// k_pool[new_locs[b]] = new_k[b] (and V), one row of C elements, converted to the pool dtype.
__device__ inline void store_new_token(const SelectArgs& a, int b) {
  if (!a.new_k) return;
  const int64_t loc = a.new_locs[b];
  if (loc < 0 || loc >= a.pool_rows) return;
  const int C = a.C;
  if (a.new_dtype == QQ_DTYPE_BF16 && a.pool_dtype == QQ_DTYPE_BF16 && C % 8 == 0) {
    const uint4* ks = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.new_k) + (int64_t)b * C);
    const uint4* vs = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.new_v) + (int64_t)b * C);
    uint4* kd = reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.k_pool) + loc * C);
    uint4* vd = reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.v_pool) + loc * C);
    for (int e = threadIdx.x; e < C / 8; e += blockDim.x) {
      kd[e] = ks[e];
      vd[e] = vs[e];
    }
    return;
  }
  for (int e = threadIdx.x; e < C; e += blockDim.x) {
    const float kv = load_as_float(a.new_k, (int64_t)b * C + e, a.new_dtype);
    const float vv = load_as_float(a.new_v, (int64_t)b * C + e, a.new_dtype);
    if (a.pool_dtype == QQ_DTYPE_BF16) {
      static_cast<uint16_t*>(a.k_pool)[loc * C + e] = f2bf(kv);
      static_cast<uint16_t*>(a.v_pool)[loc * C + e] = f2bf(vv);
    } else {
      static_cast<float*>(a.k_pool)[loc * C + e] = kv;
      static_cast<float*>(a.v_pool)[loc * C + e] = vv;
    }
  }
}

// --------------------------------------------------------------------- layout

// recent window (quest.py:333-336): min(max(s - P, 0) + j, s - 1), j < P
__device__ inline void write_recent(int32_t* pos, int64_t s, int P) {
  const int64_t start = max(s - P, (int64_t)0);
  for (int j = threadIdx.x; j < P; j += blockDim.x) pos[j] = (int32_t)min(start + j, s - 1);
}

// dense layout of a short request (quest.py:339-342): min(j, s - 1), j < top_k
__device__ inline void write_dense(int32_t* pos, int64_t s, int top_k) {
  for (int j = threadIdx.x; j < top_k; j += blockDim.x) pos[j] = (int32_t)min((int64_t)j, max(s - 1, (int64_t)0));
}

// ------------------------------------------------------------------- scoring

// GQA mean of channel c = h*D + d (quest.py:385-391): fp32 sum over the G query
// heads of KV head h in head order, divided by G, rounded once to the query
// dtype.  G == 1 returns the query unchanged.
__device__ inline float gqa_mean(const void* q, int dtype, int64_t qb, int G, int D, int c) {
  if (G == 1) return load_as_float(q, qb + c, dtype);
  const int h = c / D, d = c - h * D;
  float acc = 0.0f;
  for (int g = 0; g < G; ++g)
    acc = __fadd_rn(acc, load_as_float(q, qb + (int64_t)(h * G + g) * D + d, dtype));
  acc = acc / (float)G;
  return dtype == QQ_DTYPE_BF16 ? bf2f(f2bf(acc)) : acc;
}

// q-bar of channels [0, C) into LDS, computed once per block (each thread a
// channel pair when the query is bf16 and D is even: G 4-byte loads).
__device__ inline void block_qbar(float* s_q, const SelectArgs& a, int b) {
  const int G = a.H / a.KV;
  const int64_t qb = (int64_t)b * a.q_bstride;
  constexpr int kMaxG = 16;
  if (a.q_dtype == QQ_DTYPE_BF16 && a.D % 2 == 0 && G > 1 && G <= kMaxG) {
    for (int c = threadIdx.x * 2; c < a.C; c += kBlock * 2) {
      const int h = c / a.D, d = c - h * a.D;
      const uint32_t* qp =
          reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.q) + qb + (int64_t)h * G * a.D + d);
      uint32_t u[kMaxG];
#pragma unroll
      for (int g = 0; g < kMaxG; ++g) u[g] = g < G ? qp[(int64_t)g * (a.D / 2)] : 0u;  // all in flight
      float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
      for (int g = 0; g < kMaxG; ++g) {
        if (g < G) {
          a0 = __fadd_rn(a0, bf2f((uint16_t)(u[g] & 0xFFFFu)));
          a1 = __fadd_rn(a1, bf2f((uint16_t)(u[g] >> 16)));
        }
      }
      s_q[c] = bf2f(f2bf(a0 / (float)G));
      s_q[c + 1] = bf2f(f2bf(a1 / (float)G));
    }
    return;
  }
  for (int c = threadIdx.x; c < a.C; c += kBlock) s_q[c] = gqa_mean(a.q, a.q_dtype, qb, G, a.D, c);
}

// Lane exchanges without the LDS: gfx950's permlane swaps across rows and DPP
// moves within a row.  lane_xor32/16/8/2/1(v) = v of lane l ^ 32/16/8/2/1;
// lane_up4(v) = v of lane l + 4 in the row, which is lane l ^ 4 for lanes with
// bit 2 clear.  A permlane swap of (v, v) gives every lane the pair
// {v of the lower row or half, v of the upper one}.
__device__ inline float lane_xor32(float v, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((lane & 32) ? r[0] : r[1]);
}
__device__ inline float lane_xor16(float v, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((lane & 16) ? r[0] : r[1]);
}
template <int CTRL>
__device__ inline float dpp_f32(float v) {
  return __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), CTRL, 0xF, 0xF, false));
}
__device__ inline float lane_xor8(float v) { return dpp_f32<0x128>(v); }  // row_ror:8
__device__ inline float lane_up4(float v) { return dpp_f32<0x104>(v); }   // row_shl:4
__device__ inline float lane_xor2(float v) { return dpp_f32<0x4E>(v); }   // quad_perm [2, 3, 0, 1]
__device__ inline float lane_xor1(float v) { return dpp_f32<0xB1>(v); }   // quad_perm [1, 0, 3, 2]

// Lane partials of 8 pages at once.  acc[p] is this lane's partial of page p
// (its m channels, summed in order).  The 8 halving trees are interleaved: at
// level w = 32, 16, 8 each lane keeps half of its pages and adds the partner's
// (lane l ^ w) partial of them - the pairs are exactly the tree's (i, i + w) -
// then levels 4, 2, 1 run on one value.  Lane l ends with page l >> 3.
__device__ inline float reduce8_pages(float (&acc)[8], int lane) {
  const bool up32 = lane & 32, up16 = lane & 16, up8 = lane & 8;
  float v4[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float send = up32 ? acc[j] : acc[4 + j];
    const float keep = up32 ? acc[4 + j] : acc[j];
    v4[j] = __fadd_rn(keep, lane_xor32(send, lane));
  }
  float v2[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float send = up16 ? v4[j] : v4[2 + j];
    const float keep = up16 ? v4[2 + j] : v4[j];
    v2[j] = __fadd_rn(keep, lane_xor16(send, lane));
  }
  float v;
  {
    const float send = up8 ? v2[0] : v2[1];
    const float keep = up8 ? v2[1] : v2[0];
    v = __fadd_rn(keep, lane_xor8(send));
  }
  // levels 4, 2, 1: only lanes with bits 2..0 clear (one per page) return a
  // result, and their chain reads lanes l ^ 4 with bit 2 clear, so lane l + 4
  // stands in for l ^ 4
  v = __fadd_rn(v, lane_up4(v));
  v = __fadd_rn(v, lane_xor2(v));
  v = __fadd_rn(v, lane_xor1(v));
  return v;
}

// Bounds words of 8 pages for KV*D == 64*M (M a multiple of 4): lane l holds
// channels [l*M, l*M + M) as M/4 16-byte loads; pages at or past `lim` re-read
// page lim - 1 (their scores are not stored), so every load is unconditional.
template <int M>
__device__ inline void load_8pages(uint32_t (&w)[8][M], const uint32_t* req_bounds, int pw, int lim, int lane) {
  static_assert(M % 4 == 0, "16-byte lane loads");
  constexpr int C = 64 * M;
  const uint32_t lane_bytes = (uint32_t)lane * (M * 4);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const char* page = reinterpret_cast<const char*>(req_bounds + (int64_t)min(pw + i, lim - 1) * C);
#pragma unroll
    for (int j = 0; j < M / 4; ++j) {
      const uint4 v = *reinterpret_cast<const uint4*>(page + lane_bytes + 16 * j);
      w[i][4 * j] = v.x;
      w[i][4 * j + 1] = v.y;
      w[i][4 * j + 2] = v.z;
      w[i][4 * j + 3] = v.w;
    }
  }
}

// Scores of the 8 pages in w (quest.py:393-405): min or max picked by q-bar's
// sign with one byte permute per channel, fp32 products summed in channel
// order, then the halving tree.  Lane l returns page l >> 3.
template <int M>
__device__ inline float score_8pages(const uint32_t (&w)[8][M], const float* s_q, int lane) {
  float qreg[M];
  uint32_t sel[M];  // v_perm selector: max (high half) for q >= 0, else min, into bits 31:16
#pragma unroll
  for (int j = 0; j < M; ++j) {
    qreg[j] = s_q[lane * M + j];
    sel[j] = qreg[j] >= 0.0f ? 0x03020C0Cu : 0x01000C0Cu;
  }
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float t = __fmul_rn(qreg[0], __uint_as_float(__builtin_amdgcn_perm(w[i][0], w[i][0], sel[0])));
#pragma unroll
    for (int j = 1; j < M; ++j)
      t = __fadd_rn(t, __fmul_rn(qreg[j], __uint_as_float(__builtin_amdgcn_perm(w[i][j], w[i][j], sel[j]))));
    acc[i] = t;
  }
  return reduce8_pages(acc, lane);
}

// ----------------------------------------------------------------- selection

constexpr uint32_t kNegInfKey = 0x007FFFFFu;  // orderable(-inf): masked pages (quest.py:451)

// DPP lane moves (data-parallel primitives, VALU only) of a 64-bit value, as two
// 32-bit moves; every lane must be active.
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfRowMirror = 0x141; // lane i of each 8 -> lane 7 - i
template <int CTRL>
__device__ inline uint64_t dpp64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}

// The page whose score thread `tid` of an NT-thread selection holds in slot i.
// The scores arrive in page blocks (page tid + NT i: coalesced loads).  The
// selections take their threshold from the maxima of 64 groups of NT/64
// consecutive threads; with fewer candidates than threads, page blocks leave
// groups empty (127 candidates fill 16 of 64 groups at NT = 512), every key then
// passes the threshold and the ranking takes its quadratic path.  Such a block
// spreads its pages first: slot 0 moves through the LDS so that group g holds
// pages g, g + 64, ... and the k-th largest group maximum stays a tight bound
// (the other slots hold pages >= NT, past every candidate).
template <int NT>
__device__ inline int sel_page(int tid, int i, bool spread) {
  constexpr int GS = NT / 64;
  return spread ? NT * i + tid / GS + 64 * (tid % GS) : tid + NT * i;
}

// Slot 0's score after the spread (block-uniform `spread`; tmp: NT floats of LDS
// that nothing reads or writes until the next block barrier).
template <int NT>
__device__ inline float spread_slot0(float v, bool spread, float* tmp) {
  if (!spread) return v;
  tmp[threadIdx.x] = v;
  lds_barrier();
  return tmp[sel_page<NT>(threadIdx.x, 0, true)];
}

template <int KPT, int NT = kBlock>
struct SelectSmem {
  uint64_t cand[NT * KPT + 64];  // survivors, flattened (zero-padded up to 64)
  uint64_t gmax[64];             // maxima of the 64 groups of NT/64 threads
  int grank[64];                 // number of group maxima above each group's
  int crank[64];                 // number of survivors above each survivor (<= 64 of them)
  int wcnt[NT / 64];
  uint64_t tau;
  int order[64];
};

// Top k <= 64 pages of n_eff <= NT*KPT keys (quest.py:450-452), whole block of
// NT threads: sv[i] is the score of page tid + NT i (pages >= lim rank as
// -inf); a block with fewer candidates than threads spreads them first
// (sel_page).  Keys are (order-preserving score, ~page), so "larger" = higher
// score, then lower page, and all keys differ.
//   1. tau = the k-th largest of the maxima of 64 groups of NT/64 threads (1
//      when fewer than k groups hold keys).  The k largest group maxima are k
//      distinct keys >= tau, so every top-k key is >= tau;
//   2. the keys >= tau (at least k; about 40 of 2048 for distinct scores) are
//      compacted into one LDS array (ballot + mbcnt within a wave, wave counts
//      give the offsets);
//   3. each survivor's rank = number of survivors above it (split over the
//      waves when there are at most 64); ranks < k give the pages in
//      (score desc, page asc) order in s.order[0, k).
template <int KPT, int NT = kBlock>
__device__ inline void select_topk_block(const float (&sv)[KPT], int lim, int n_eff, int k,
                                         SelectSmem<KPT, NT>& s) {
  static_assert(NT == 256 || NT == 512, "64 groups of whole quads or octets");  // GS = 4 or 8
  constexpr int NW = NT / 64, GS = NT / 64, SHARE = 64 / NW;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const bool spread = lim < NT;  // block-uniform
  const float s0 = spread_slot0<NT>(sv[0], spread, reinterpret_cast<float*>(s.cand));
  uint64_t key[KPT];
  uint64_t tmax = 0ull;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int p = sel_page<NT>(tid, i, spread);
    key[i] = p < n_eff ? sel_key(p < lim ? orderable(i == 0 ? s0 : sv[i]) : kNegInfKey, p) : 0ull;
    tmax = key[i] > tmax ? key[i] : tmax;
  }
  // group maximum over GS consecutive lanes with DPP moves (no LDS round trips):
  // the other lane of each pair, the other pair of each quad, then (GS = 8)
  // the other quad of each half row
  uint64_t g = tmax;
  uint64_t o = dpp64<kDppQuadXor1>(g);
  g = o > g ? o : g;
  o = dpp64<kDppQuadXor2>(g);
  g = o > g ? o : g;
  if (GS == 8) {
    o = dpp64<kDppHalfRowMirror>(g);
    g = o > g ? o : g;
  }
  if (tid % GS == 0) s.gmax[tid / GS] = g;
  if (tid < 64) {
    s.grank[tid] = 0;
    s.crank[tid] = 0;
  }
  if (tid == 0) s.tau = 1ull;
  __syncthreads();
  // group i's rank, 1/NW of the comparisons per wave
  const uint64_t gi = s.gmax[lane];
  int part = 0;
#pragma unroll
  for (int j = 0; j < SHARE; ++j) part += s.gmax[wave * SHARE + j] > gi;
  atomicAdd(&s.grank[lane], part);
  __syncthreads();
  if (tid < 64 && gi != 0ull && s.grank[tid] == k - 1) s.tau = gi;  // unique: nonzero keys differ
  __syncthreads();
  const uint64_t tau = s.tau;
  uint64_t mask[KPT];
  int wave_total = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    mask[i] = __ballot(key[i] >= tau);
    wave_total += __popcll(mask[i]);
  }
  if (lane == 0) s.wcnt[wave] = wave_total;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int c = s.wcnt[w];
    base += w < wave ? c : 0;
    total += c;
  }
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    if (key[i] >= tau)
      s.cand[base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask[i] >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask[i], 0u))] = key[i];
    base += __popcll(mask[i]);
  }
  if (tid >= total && tid < 64) s.cand[tid] = 0ull;  // a zero key ranks above nothing
  __syncthreads();
  if (total <= 64) {
    // survivor `lane`'s rank, 1/NW of the comparisons per wave
    const uint64_t ci = s.cand[lane];
    int part = 0;
#pragma unroll
    for (int j = 0; j < SHARE; ++j) part += s.cand[wave * SHARE + j] > ci;
    atomicAdd(&s.crank[lane], part);
    __syncthreads();
    if (tid < total) {
      const int r = s.crank[tid];
      if (r < k) s.order[r] = (int)(~(uint32_t)s.cand[tid]);
    }
  } else {
    for (int i = tid; i < total; i += NT) {
      const uint64_t ci = s.cand[i];
      int r = 0;
      for (int j = 0; j < total; ++j) r += s.cand[j] > ci;
      if (r < k) s.order[r] = (int)(~(uint32_t)ci);
    }
  }
  __syncthreads();
}

// Lane exchanges of 32-bit words inside a wave without the LDS: lane l gets the
// word of lane l ^ J (DPP moves within a row of 16, permlane swaps across rows).
template <int J>
__device__ inline uint32_t lane_xor_u32(uint32_t v, int lane) {
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppQuadXor1, 0xF, 0xF, false);
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppQuadXor2, 0xF, 0xF, false);
  } else if constexpr (J == 4) {  // row_shl:4 gives lane l + 4, row_shr:4 lane l - 4
    const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x104, 0xF, 0xF, false);
    const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);
    return (lane & 4) ? dn : up;
  } else if constexpr (J == 8) {  // row_ror:8
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
  } else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else {
    static_assert(J == 32, "lane distance");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}

template <int J>
__device__ inline uint64_t lane_xor_u64(uint64_t v, int lane) {
  const uint32_t lo = lane_xor_u32<J>((uint32_t)v, lane);
  const uint32_t hi = lane_xor_u32<J>((uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

__device__ inline uint64_t readlane_u64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

template <int KPT, int NT>
struct RankSelectSmem {
  uint32_t gmax[64];             // 32-bit score keys: maxima of the 64 groups of NT/64 threads
  int gcnt[NT / 64][64];         // partial counts of group maxima >= each one, one row per wave
  uint64_t cand[NT * KPT + 64];  // survivors (score key, ~page), in arrival order
  int crank[NT / 64][64];        // partial ranks of the survivors (at most 64)
  int count;
  int order[64];                 // page of each rank (many-survivor path)
};

// Maximum of a 32-bit value over the wave (DPP / permlane exchanges, no LDS).
__device__ inline uint32_t wave_max_u32(uint32_t v, int lane) {
  v = max(v, lane_xor_u32<1>(v, lane));
  v = max(v, lane_xor_u32<2>(v, lane));
  v = max(v, lane_xor_u32<4>(v, lane));
  v = max(v, lane_xor_u32<8>(v, lane));
  v = max(v, lane_xor_u32<16>(v, lane));
  v = max(v, lane_xor_u32<32>(v, lane));
  return v;
}

// Top k <= 64 pages of n_eff <= NT*KPT pages (quest.py:450-452) with an NT-thread
// block (NT = 256 or 512): sv[i] is the score of page tid + NT i (pages >= lim
// rank as -inf), spread first when there are fewer candidates than threads
// (sel_page).  The order is (score desc, page asc): 64-bit keys (order-preserving
// score, ~page), all distinct.  Every comparison pass is split over the block's
// waves and handed over through LDS, 4 barriers in all:
//   A. per thread the largest 32-bit score key of its pages, per group of NT/64
//      consecutive threads the maximum (DPP lane moves);
//   B. for each group maximum the number of group maxima >= it; tau = the largest
//      group maximum that at least k group maxima reach (the k-th largest).  At
//      least k groups hold a page scoring >= tau, so every top-k page does;
//   C. the pages scoring >= tau (about 40 of 2048 for distinct scores) gathered
//      into one LDS array as 64-bit keys, each wave at an offset from one LDS
//      atomic;
//   D. up to 64 survivors: their ranks (the number of survivor keys above), each
//      wave's lane s ending with survivor s's rank, page and (when `page_rows` is
//      given) the page's first pool row, loaded while the ranks are counted.  More
//      survivors (ties): every thread ranks its share by counting, then lane r
//      takes rank r.
// The page of rank u is the lane whose rank is u (one ballot and a readlane).
template <int KPT, int NT>
__device__ inline void select_ranked(const float (&sv)[KPT], int lim, int n_eff, int k,
                                     RankSelectSmem<KPT, NT>& s, const int32_t* page_rows, int max_pages,
                                     int& my_rank, int& my_page, int& my_row0) {
  static_assert(NT == 256 || NT == 512, "64 groups of whole quads or octets");
  constexpr int NW = NT / 64, SHARE = 64 / NW;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const bool spread = lim < NT;  // block-uniform
  const float s0 = spread_slot0<NT>(sv[0], spread, reinterpret_cast<float*>(s.cand));
  uint32_t key[KPT];
  uint32_t tmax = 0u;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int p = sel_page<NT>(tid, i, spread);
    const uint32_t o = orderable(i == 0 ? s0 : sv[i]);
    key[i] = p < lim ? o : (p < n_eff ? kNegInfKey : 0u);  // 0: not a page (below every key)
    tmax = max(tmax, key[i]);
  }
  uint32_t g = max(tmax, lane_xor_u32<1>(tmax, lane));
  g = max(g, lane_xor_u32<2>(g, lane));
  if (NT == 512) g = max(g, lane_xor_u32<4>(g, lane));
  if ((tid & (NT / 64 - 1)) == 0) s.gmax[tid / (NT / 64)] = g;
  if (tid == 0) s.count = 0;
  lds_barrier();  // A
  const uint32_t gl = s.gmax[lane];
  {
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < SHARE; ++j) cnt += s.gmax[w * SHARE + j] >= gl ? 1 : 0;
    s.gcnt[w][lane] = cnt;
  }
  lds_barrier();  // B
  int ge = 0;
#pragma unroll
  for (int j = 0; j < NW; ++j) ge += s.gcnt[j][lane];
  // the k-th largest group maximum; a zero (no page) never survives
  const uint32_t tau = max(wave_max_u32(ge >= k ? gl : 0u, lane), 1u);
  uint64_t mask[KPT];
  int wave_total = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    mask[i] = __ballot(key[i] >= tau);
    wave_total += __popcll(mask[i]);
  }
  int base = 0;
  if (lane == 0) base = atomicAdd(&s.count, wave_total);
  base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    if (key[i] >= tau)
      s.cand[base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask[i] >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask[i], 0u))] =
          sel_key(key[i], sel_page<NT>(tid, i, spread));
    base += __popcll(mask[i]);
  }
  lds_barrier();  // C
  const int total = s.count;
  if (total <= 64) {  // block-uniform
    const uint64_t ci = lane < total ? s.cand[lane] : 0ull;
    const int page = (int)(~(uint32_t)ci);
    my_row0 = (page_rows && lane < total && page >= 0 && page < max_pages) ? page_rows[page] : -1;
    // every slot below 64 is read (past `total` it holds stale words, whose
    // comparisons are masked), so that the SHARE reads go out together instead of
    // one round trip each behind a branch
    const int wu = __builtin_amdgcn_readfirstlane(w);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < SHARE; ++j) {
      const int jj = wu * SHARE + j;
      const uint64_t cj = s.cand[jj];
      cnt += (int)(cj > ci) & (int)(jj < total);
    }
    s.crank[w][lane] = cnt;
    lds_barrier();  // D
    int r = 0;
#pragma unroll
    for (int j = 0; j < NW; ++j) r += s.crank[j][lane];
    my_rank = lane < total ? r : -1;
    my_page = page;
    return;
  }
  for (int i = tid; i < total; i += NT) {
    const uint64_t ci = s.cand[i];
    int r = 0;
    for (int j = 0; j < total; ++j) r += s.cand[j] > ci;
    if (r < k) s.order[r] = (int)(~(uint32_t)ci);
  }
  lds_barrier();
  my_rank = lane < k ? lane : -1;
  my_page = lane < k ? s.order[lane] : -1;
  my_row0 = (page_rows && my_page >= 0 && my_page < max_pages) ? page_rows[my_page] : -1;
}

// ----------------------------------------------------------------- attention

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kMfmaDim = 128;

// One wave: G <= 16 query heads (qh: G rows of 128 bf16) against 64 rows of
// one KV head.  krow/vrow[i] point at the 128 channels of row i's KV head
// (rows i >= cnt are masked and may point at any readable row).
//   S^T = K Q^T with v_mfma_f32_16x16x32_bf16: K rows are the A operand, 16
//   bytes per lane straight from memory, Q^T the B operand (query heads on N,
//   padded to 16).  The S^T accumulator gives each lane one head and 4
//   consecutive tokens, which is exactly the A-operand layout of
//   v_mfma_f32_16x16x16bf16_1k, so P = exp(S - m) (bf16) feeds O = P V without
//   an LDS round trip; V comes in 16-byte row slices (8 channels) transposed
//   4x8 in registers, channel d = 8*(lane % 16) + e.
// Returns, per lane, for head lo = lane % 16: mx (the row max of s*scale in
// log2 units) and sum = sum of the bf16-rounded exp2(s - mx); and
// o[e][i] = sum_t p[head 4*hi + i][t] v[t][8*lo + e] (hi = lane / 16).
__device__ inline void attn_wave64(const uint16_t* const* krow, const uint16_t* const* vrow,
                                   const uint16_t* qh, int G, int cnt, float sl2, float& mx_out,
                                   float& sum_out, float4_t (&o)[8]) {
  const int l = threadIdx.x & 63;
  const int lo = l & 15, hi = l >> 4;
  // K as the A operand: tile t (16 tokens) x k-step ks (32 channels): 16 bytes per lane.
  bf16x8_t ka[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint16_t* kp = krow[t * 16 + lo] + hi * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) ka[t][ks] = *reinterpret_cast<const bf16x8_t*>(kp + ks * 32);
  }
  // V row slices for P V: k-step s (16 tokens), token j of the lane's 4; 16 bytes =
  // channels 8*lo .. 8*lo + 7 of this KV head (16 lanes cover the 256-byte slice).
  uint4 vr[4][4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) vr[s][j] = *reinterpret_cast<const uint4*>(vrow[s * 16 + hi * 4 + j] + lo * 8);
  // Q^T as the B operand: query head lo (zero past G), channels 8*hi + 32*ks.
  bf16x8_t qb[4];
  {
    const uint16_t* qp = qh + (int64_t)lo * kMfmaDim + hi * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (lo < G) {
        qb[ks] = *reinterpret_cast<const bf16x8_t*>(qp + ks * 32);
      } else {
        qb[ks] = __builtin_bit_cast(bf16x8_t, u32x4_t{0u, 0u, 0u, 0u});
      }
    }
  }

  // S^T[token t*16 + 4*hi + i][head lo] in acc[t][i]
  float4_t acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[t][ks], qb[ks], acc[t], 0, 0, 0);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = t * 16 + hi * 4 + i;
      const float x = tok < cnt ? acc[t][i] * sl2 : -INFINITY;
      acc[t][i] = x;
      mx = fmaxf(mx, x);
    }
  mx = fmaxf(mx, lane_xor16(mx, l));
  mx = fmaxf(mx, lane_xor32(mx, l));
  float sum = 0.0f;
  short4_t pa[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t pb = cnt > 0 ? f2bf(exp2f(acc[t][i] - mx)) : (uint16_t)0;
      sum += bf2f(pb);
      pa[t][i] = (short)pb;
    }
  sum += lane_xor16(sum, l);
  sum += lane_xor32(sum, l);

#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    short4_t vb[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 u = vr[s][j];
      const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        vb[2 * x][j] = (short)(wv[x] & 0xFFFFu);
        vb[2 * x + 1][j] = (short)(wv[x] >> 16);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa[s], vb[e], o[e], 0, 0, 0);
  }
  mx_out = mx;
  sum_out = sum;
}

}  // namespace qq
