// One Quest decode layer for a batch, as QuestOnlyBackend.forward_decode does it
// (reference src/qwenquest/attention/quest_only.py:132-159): store the new
// token's K/V, select the positions, gather through req_to_token and attend.
//
// Fused path (bf16, KV*D = 4*128, page 64, at most 64 selected pages, at most
// 8192 pages per request, top_k <= 4096, and a zeroed sync buffer from the
// caller): two launches.
//   1. page scores of every long request (score_pages_fast_kernel in select.hip,
//      one 256-thread block per (request, 32 candidate pages), all resident at
//      once) and the new token's K/V (set_kv_buffer, memory.py:114-120).
//   2. attention (quest_attend_unit_kernel): the layout's slots come in units of
//      64 (a selected page, the recent window, or 64 slots of the dense layout).
//      One block of W waves per (request, KV head, part); unit_shape sizes the
//      grid to one round of resident blocks (batch 16 x top_k 2048: 8-wave blocks,
//      4 parts per (request, KV head), 256 blocks, one unit per wave).  Every
//      block first selects its request's pages from the scores (select_ranked in
//      qq_quest_dev.h; the blocks of a request compute the same list, so no block
//      waits on another).  Each wave then resolves its unit's 64 rows itself
//      (lane l: slot -> position -> req_to_token; the KV-head-0 blocks store the
//      positions), issues all 32 16-byte loads of the unit's K and V slices at
//      once (32 KiB per wave, 216 VGPRs, two waves per SIMD), computes
//      S^T = K Q^T (v_mfma_f32_16x16x32_bf16), one softmax over the 64 rows folded
//      into its running (M, L), and P V (v_mfma_f32_16x16x16bf16_1k, V transposed
//      in registers).  The W waves combine in LDS; the parts' (m, l, o) partials go
//      out with agent-scope stores, and the block that completes a (request, KV
//      head) count merges them into the output.
// The counters return to zero before the launch ends, so the next call (or a
// graph replay) starts clean.  quest_hisparse's attention over its hot-buffer
// rows runs the same kernel (its rows mode), in the same unit order, so both
// backends compute the same partials in the same order.
//
// Other shapes: four launches on one stream, each consuming the previous one's
// output: score (all CUs) -> select + new-token store (one block per request)
// -> chunk attention (MFMA) -> merge.
#include <algorithm>
#include <mutex>

#include "qq_quest_dev.h"

namespace qq {
namespace {

constexpr int kStepKV = 4;            // KV heads of the fused path (KV*D = 512)
constexpr int kStepMaxG = 16;
constexpr int kMaxSelFused = 64;
constexpr int kStepMaxTopK = 4096;
constexpr int kHeadWaves = 8;        // dense decode: 8-wave blocks (two waves per SIMD)
constexpr int kHeadTiles = 2;        // 16-row tiles per step (32 rows)
constexpr int kHeadDepth = 2;        // steps in flight per wave
constexpr int kMaxParts = 8;         // dense decode: parts merged in one pass
// The Quest step's attention (quest_attend_unit_kernel): up to kUnitParts blocks
// per (request, KV head), merged in one pass; the selection of a 4-wave block
// holds up to 32 scores per thread (8192 pages; its LDS, 68 KiB, still lets two
// blocks share a CU).
constexpr int kUnitParts = 8;
constexpr int kUnitMinWaves = 4;

struct StepArgs {
  SelectArgs s;            // scoring, selection, positions, new token
  const uint16_t* k;       // this layer's pool [kv_rows, KV, 128]
  const uint16_t* v;
  int64_t kv_rows;
  const int32_t* r2t;
  int64_t r2t_stride, r2t_rows;
  float sl2;               // scale * log2(e)
  uint16_t* out;           // [bs, H * 128] bf16
  float* part_o;           // [bs, KV, parts, G, 128] attention partials (workspace)
  float* part_ml;          // [bs, KV, parts, G, 2] (m in log2 units, l)
  uint32_t* sync;
  int bs, G;
  int parts, per_wave;     // attention blocks per (request, KV head); rows per wave
  const int64_t* rows_in;  // rows given [bs, rows_stride] (attention over given rows)
  int64_t rows_stride;
  const int32_t* actual;   // [bs] attended slots (attention over given rows)
};

// sync: one counter per (request, KV head), each on its own 128-byte line.
__device__ inline uint32_t* attn_count(const StepArgs& a, int bh) { return a.sync + bh * 32; }

__device__ inline bool needs_selection(const SelectArgs& sa, int64_t s) { return s > sa.top_k && sa.k_sel > 0; }

// One wave's step: the K and V slices of 16T layout rows of one KV head
// (lane layouts of attn_wave64: K tile t = tokens 16t .. 16t+15, V k-step u =
// tokens 16u .. 16u+15).
template <int T>
struct StepRegs {
  bf16x8_t ka[T][4];
  uint4 vr[T][4];
};

template <int T>
__device__ inline void load_step(StepRegs<T>& r, const int32_t* rows, int t0, const uint16_t* kb, const uint16_t* vb,
                                 int lo, int hi) {
  constexpr int kRow = kStepKV * kMfmaDim;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint16_t* kp = kb + (int64_t)rows[t0 + t * 16 + lo] * kRow + hi * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) r.ka[t][ks] = *reinterpret_cast<const bf16x8_t*>(kp + ks * 32);
  }
#pragma unroll
  for (int u = 0; u < T; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      r.vr[u][j] = *reinterpret_cast<const uint4*>(vb + (int64_t)rows[t0 + u * 16 + hi * 4 + j] * kRow + lo * 8);
}

// Online-softmax update with one step (tokens t0 .. t0+16T-1, the first
// `valid` of them real): M, L per head lo (log2 units), o[e][i] per (head
// 4hi+i, channel 8lo+e).
template <int T>
__device__ inline void attend_step(const StepRegs<T>& r, const bf16x8_t (&qb)[4], int valid, float sl2, float& M,
                                   float& L, float4_t (&o)[8], int lo, int hi) {
  float4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(r.ka[t][ks], qb[ks], acc[t], 0, 0, 0);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = (t * 16 + hi * 4 + i) < valid ? acc[t][i] * sl2 : -INFINITY;
      acc[t][i] = x;
      mx = fmaxf(mx, x);
    }
  const int lane = threadIdx.x & 63;
  mx = fmaxf(mx, lane_xor16(mx, lane));
  mx = fmaxf(mx, lane_xor32(mx, lane));
  const float Mn = fmaxf(M, mx);
  const float alpha = M == -INFINITY ? 0.0f : exp2f(M - Mn);  // rescale of the running sums
  float sum = 0.0f;
  short4_t pa[T];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t pb = Mn == -INFINITY ? (uint16_t)0 : f2bf(exp2f(acc[t][i] - Mn));
      sum += bf2f(pb);
      pa[t][i] = (short)pb;
    }
  sum += lane_xor16(sum, lane);
  sum += lane_xor32(sum, lane);
  L = L * alpha + sum;
  M = Mn;
  // o rows are heads 4hi + i: their scale factors live in lanes 4hi + i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float ai = __shfl(alpha, hi * 4 + i, 64);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e][i] *= ai;
  }
#pragma unroll
  for (int u = 0; u < T; ++u) {
    short4_t vbv[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 w = r.vr[u][j];
      const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        vbv[2 * x][j] = (short)(wv[x] & 0xFFFFu);
        vbv[2 * x + 1][j] = (short)(wv[x] >> 16);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa[u], vbv[e], o[e], 0, 0, 0);
  }
}

template <int W, int ROWCAP>
struct HeadSmem {
  int32_t rows[ROWCAP];  // this block's layout slots -> pool rows
  float m[W][kStepMaxG];
  float l[W][kStepMaxG];
  float o[W][kStepMaxG][kMfmaDim];
};

// The end of an attention block: its W waves' (M, L, o) (o[e][i]: head 4hi + i,
// channel 8lo + e) combined in LDS; with one part the block writes the output,
// else an (m, l, o) partial (agent scope) and the block that completes the
// (request, KV head) count merges the parts (up to MG at once; GROUPED: more in
// groups of MG, maximum first).  poison: the output becomes NaN.
template <int W, int MG, bool GROUPED>
__device__ inline void finish_block(const StepArgs& a, int bh, int part, float M, float L, const float4_t (&o)[8],
                                    bool poison, float (*sm_m)[kStepMaxG], float (*sm_l)[kStepMaxG],
                                    float (*sm_o)[kStepMaxG][kMfmaDim], uint32_t* s_last) {
  const SelectArgs& sa = a.s;
  constexpr int kThreads = 64 * W;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lo = lane & 15, hi = lane >> 4;
  const int parts = a.parts;
  const int b = bh / kStepKV, h = bh - b * kStepKV;
  const int G = a.G;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int head = hi * 4 + i;
    if (head < G) {
      float* dst = &sm_o[wave][head][lo * 8];
      *reinterpret_cast<float4*>(dst) = make_float4(o[0][i], o[1][i], o[2][i], o[3][i]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4][i], o[5][i], o[6][i], o[7][i]);
    }
  }
  if (hi == 0 && lo < G) {
    sm_m[wave][lo] = M;
    sm_l[wave][lo] = poison ? __builtin_nanf("") : L;  // NaN survives every weight of the merge
  }
  __syncthreads();
  uint16_t* outp = a.out + (int64_t)b * sa.H * kMfmaDim + (int64_t)h * G * kMfmaDim;
  const int64_t part_idx = (int64_t)bh * parts + part;
  const __amdgpu_buffer_rsrc_t po =
      agent_rsrc(a.part_o + part_idx * G * kMfmaDim, (uint32_t)(G * kMfmaDim * sizeof(float)));
  // each thread one head x 4 channels: the waves' (m, l, o) weighted in wave order
  for (int grp = tid; grp < G * (kMfmaDim / 4); grp += kThreads) {
    const int head = grp >> 5, d4 = (grp & 31) * 4;
    // every LDS read first (one wait instead of a chain of them), then the sums
    float mw[W], lw[W];
    float4 ov[W];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      mw[w] = sm_m[w][head];
      lw[w] = sm_l[w][head];
      ov[w] = *reinterpret_cast<const float4*>(&sm_o[w][head][d4]);
    }
    float Mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) Mx = fmaxf(Mx, mw[w]);
    float Ls = 0.0f;
    float4 Os = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float wgt = mw[w] == -INFINITY ? 0.0f : exp2f(mw[w] - Mx);
      Ls += wgt * lw[w];
      Os.x += wgt * ov[w].x;
      Os.y += wgt * ov[w].y;
      Os.z += wgt * ov[w].z;
      Os.w += wgt * ov[w].w;
    }
    if (parts == 1) {
      const bool any = !(Ls <= 0.0f);  // NaN (a poisoned part) stays NaN
      const uint32_t lo2 = (uint32_t)f2bf(any ? Os.x / Ls : 0.0f) | ((uint32_t)f2bf(any ? Os.y / Ls : 0.0f) << 16);
      const uint32_t hi2 = (uint32_t)f2bf(any ? Os.z / Ls : 0.0f) | ((uint32_t)f2bf(any ? Os.w / Ls : 0.0f) << 16);
      *reinterpret_cast<uint2*>(outp + head * kMfmaDim + d4) = make_uint2(lo2, hi2);
    } else {
      st_agent_x4(po, (uint32_t)((head * kMfmaDim + d4) * sizeof(float)), Os);
      if (d4 == 0) {
        st_agent(a.part_ml + (part_idx * G + head) * 2, Mx);
        st_agent(a.part_ml + (part_idx * G + head) * 2 + 1, Ls);
      }
    }
  }
  if (parts == 1) return;
  wait_memory();
  __syncthreads();
  if (tid == 0) *s_last = add_agent(attn_count(a, bh), 1u) == (uint32_t)(parts - 1);
  __syncthreads();
  if (!*s_last) return;
  if (tid == 0) st_agent(attn_count(a, bh), 0u);
  // merge the parts (in part order: the maximum of the parts' m first, then the
  // weighted sums): each thread one head x 4 channels; up to MG parts all loads
  // in flight at once, more parts (dense decode) in two passes of groups
  const int64_t part0 = (int64_t)bh * parts;
  const __amdgpu_buffer_rsrc_t ro =
      agent_rsrc(a.part_o + part0 * G * kMfmaDim, (uint32_t)(parts * G * kMfmaDim * sizeof(float)));
  const uint64_t* ml64 = reinterpret_cast<const uint64_t*>(a.part_ml) + part0 * G;
  for (int grp = tid; grp < G * (kMfmaDim / 4); grp += kThreads) {
    const int head = grp >> 5, d4 = (grp & 31) * 4;
    float Mx = -INFINITY;
    float Ls = 0.0f;
    float4 Os = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!GROUPED || parts <= MG) {
      float4 ov[MG];
      uint64_t mlv[MG];
#pragma unroll
      for (int j = 0; j < MG; ++j) {
        if (j < parts) {
          ov[j] = ld_agent_x4(ro, (uint32_t)(((j * G + head) * kMfmaDim + d4) * sizeof(float)));
          mlv[j] = ld_agent(ml64 + j * G + head);
        }
      }
#pragma unroll
      for (int j = 0; j < MG; ++j)
        if (j < parts) Mx = fmaxf(Mx, __uint_as_float((uint32_t)mlv[j]));
#pragma unroll
      for (int j = 0; j < MG; ++j) {
        if (j < parts) {
          const float mj = __uint_as_float((uint32_t)mlv[j]);
          const float wgt = mj == -INFINITY ? 0.0f : exp2f(mj - Mx);
          Ls += wgt * __uint_as_float((uint32_t)(mlv[j] >> 32));
          Os.x += wgt * ov[j].x;
          Os.y += wgt * ov[j].y;
          Os.z += wgt * ov[j].z;
          Os.w += wgt * ov[j].w;
        }
      }
    } else {
      for (int j0 = 0; j0 < parts; j0 += MG) {
        uint64_t mlv[MG];
#pragma unroll
        for (int j = 0; j < MG; ++j)
          if (j0 + j < parts) mlv[j] = ld_agent(ml64 + (j0 + j) * G + head);
#pragma unroll
        for (int j = 0; j < MG; ++j)
          if (j0 + j < parts) Mx = fmaxf(Mx, __uint_as_float((uint32_t)mlv[j]));
      }
      for (int j0 = 0; j0 < parts; j0 += MG) {
        float4 ov[MG];
        uint64_t mlv[MG];
#pragma unroll
        for (int j = 0; j < MG; ++j) {
          if (j0 + j < parts) {
            ov[j] = ld_agent_x4(ro, (uint32_t)((((j0 + j) * G + head) * kMfmaDim + d4) * sizeof(float)));
            mlv[j] = ld_agent(ml64 + (j0 + j) * G + head);
          }
        }
#pragma unroll
        for (int j = 0; j < MG; ++j) {
          if (j0 + j < parts) {
            const float mj = __uint_as_float((uint32_t)mlv[j]);
            const float wgt = mj == -INFINITY ? 0.0f : exp2f(mj - Mx);
            Ls += wgt * __uint_as_float((uint32_t)(mlv[j] >> 32));
            Os.x += wgt * ov[j].x;
            Os.y += wgt * ov[j].y;
            Os.z += wgt * ov[j].z;
            Os.w += wgt * ov[j].w;
          }
        }
      }
    }
    const bool any = !(Ls <= 0.0f);  // NaN (a poisoned part) stays NaN
    const uint32_t lo2 = (uint32_t)f2bf(any ? Os.x / Ls : 0.0f) | ((uint32_t)f2bf(any ? Os.y / Ls : 0.0f) << 16);
    const uint32_t hi2 = (uint32_t)f2bf(any ? Os.z / Ls : 0.0f) | ((uint32_t)f2bf(any ? Os.w / Ls : 0.0f) << 16);
    *reinterpret_cast<uint2*>(outp + head * kMfmaDim + d4) = make_uint2(lo2, hi2);
  }
}

// Dense decode's attention of one (request, KV head, part) by a block of W
// waves: the block's share of the dense layout's slots (positions 0 .. s - 1,
// attention/dense.py:26-42), per_wave rows per wave in steps of 16T rows
// (DEPTH steps in flight), the waves combined in LDS.  With one part the
// block writes the output; else it stores an (m, l, o) partial (agent scope)
// and the block that completes the (request, KV head) count merges the parts
// (up to MG at once; GROUPED: more in groups).
template <int W, int T, int DEPTH, int MG, bool GROUPED, int ROWCAP>
__device__ inline void attend_item(const StepArgs& a, int bh, int part, unsigned char* smem_raw, uint32_t* s_last) {
  using Smem = HeadSmem<W, ROWCAP>;
  Smem& sm = *reinterpret_cast<Smem*>(smem_raw);
  const SelectArgs& sa = a.s;
  constexpr int kThreads = 64 * W;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lo = lane & 15, hi = lane >> 4;
  const int b = bh / kStepKV, h = bh - b * kStepKV;
  const int64_t s = sa.seq[b];
  const int64_t req = sa.rpi[b];
  const int top_k = sa.top_k;  // the table's width: every context fits
  const int n = (int)min(max(s, (int64_t)0), (int64_t)top_k);
  const bool r2t_ok = req >= 0 && req < a.r2t_rows;
  // slots [slot_base, slot_base + per_block): per_wave rows per wave, a multiple of
  // the 32-row step; the row table is filled over the whole range (row 0 past n),
  // so every row a step reads is initialised and in range
  const int per_wave = a.per_wave;
  const int per_block = W * per_wave;  // <= ROWCAP
  const int slot_base = part * per_block;
  for (int i0 = 0; i0 < per_block; i0 += kThreads * 4) {
    int64_t rv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int slot = slot_base + i0 + tid + kThreads * u;
      const bool mine = i0 + tid + kThreads * u < per_block;  // only this block's share is read
      const int64_t p = min((int64_t)slot, max(s - 1, (int64_t)0));
      rv[u] = (mine && slot < n && r2t_ok && p < a.r2t_stride) ? a.r2t[req * a.r2t_stride + p] : 0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + tid + kThreads * u;
      const int slot = slot_base + i;
      if (i < per_block) {
        const int64_t row = rv[u];
        sm.rows[i] = (slot < n && row >= 0 && row < a.kv_rows) ? (int32_t)row : 0;
      }
    }
  }
  const int G = a.G;
  bf16x8_t qb[4];
  {
    const uint16_t* qp = static_cast<const uint16_t*>(sa.q) + (int64_t)b * sa.q_bstride +
                         (int64_t)(h * G + lo) * kMfmaDim + hi * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (lo < G) {
        qb[ks] = *reinterpret_cast<const bf16x8_t*>(qp + ks * 32);
      } else {
        qb[ks] = __builtin_bit_cast(bf16x8_t, u32x4_t{0u, 0u, 0u, 0u});
      }
    }
  }
  lds_barrier();  // the row table is in LDS; the query loads stay in flight
  // this wave's rows: local [r0, r0 + per_wave), real up to slot n
  constexpr int kStep = 16 * T;
  const int r0 = wave * per_wave;
  const int r_end = max(r0, min(r0 + per_wave, n - slot_base));
  const int nsteps = (r_end - r0 + kStep - 1) / kStep;
  const uint16_t* kb = a.k + h * kMfmaDim;
  const uint16_t* vb = a.v + h * kMfmaDim;
  float M = -INFINITY, L = 0.0f;
  float4_t o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = float4_t{0.f, 0.f, 0.f, 0.f};
  StepRegs<T> ring[DEPTH];
#pragma unroll
  for (int j = 0; j < DEPTH - 1; ++j)
    if (j < nsteps) load_step<T>(ring[j], sm.rows, r0 + kStep * j, kb, vb, lo, hi);
  for (int i0 = 0; i0 < nsteps; i0 += DEPTH) {
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) {
      const int i = i0 + j;
      if (i >= nsteps) break;
      const int ahead = i + DEPTH - 1;
      if (ahead < nsteps) load_step<T>(ring[(j + DEPTH - 1) % DEPTH], sm.rows, r0 + kStep * ahead, kb, vb, lo, hi);
      attend_step<T>(ring[j], qb, r_end - (r0 + kStep * i), a.sl2, M, L, o, lo, hi);
    }
  }
  finish_block<W, MG, GROUPED>(a, bh, part, M, L, o, false, sm.m, sm.l, sm.o, s_last);
}

using HeadSmemLaunch = HeadSmem<kHeadWaves, kStepMaxTopK>;

// Dense decode's attention launch: one 8-wave block per (request, KV head,
// part), blockIdx = (request, KV head) * parts + part.
__global__ __launch_bounds__(64 * kHeadWaves, 1) void quest_attend_part_kernel(StepArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ uint32_t s_last;
  const int bh = blockIdx.x / a.parts, part = blockIdx.x - bh * a.parts;
  attend_item<kHeadWaves, kHeadTiles, kHeadDepth, kMaxParts, true, kStepMaxTopK>(a, bh, part, smem_raw, &s_last);
}

// ------------------------------------------------------- per-page-unit attention
// The Quest step's attention (after the score launch; and over given rows for
// quest_hisparse, so that both compute the same partials in the same order):
// one 4-wave block per (request, KV head, part), blockIdx = (request, KV head) *
// parts + part.  The layout's slots come in units of 64 (a selected page, or the
// recent window, or 64 slots of the dense layout); wave w of part p takes units
// p*4 + w, p*4 + w + 4*parts, ...  (one unit per wave at top_k 2048).  Per unit a
// wave resolves its 64 rows itself (lane l: slot 64u + l -> position ->
// req_to_token), shuffles them into the MFMA lane layouts and issues all 32
// loads of the unit's K and V slices (32 KiB per wave) at once, then
// S^T = K Q^T (v_mfma_f32_16x16x32_bf16, K rows as the A operand, 16 B per
// lane), one softmax over the 64 rows folded into the wave's running (M, L),
// P (bf16) straight from the S^T accumulator into v_mfma_f32_16x16x16bf16_1k
// with V transposed in registers.  The block first selects its request's pages
// (select_pages_wave: every wave ends with the page list in its lanes).
template <int KPT, int W>
struct UnitSmem {
  union {
    RankSelectSmem<(KPT > 0 ? KPT : 1), 64 * W> sel;
    struct {
      float m[W][kStepMaxG];
      float l[W][kStepMaxG];
      float o[W][kStepMaxG][kMfmaDim];
    } comb;
  };
};

template <bool ROWS, int KPT, int W>
__global__ __launch_bounds__(64 * W, 8 / W) void quest_attend_unit_kernel(StepArgs a) {
  constexpr int NT = 64 * W;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ uint32_t s_last;
  UnitSmem<KPT, W>& sm = *reinterpret_cast<UnitSmem<KPT, W>*>(smem_raw);
  const SelectArgs& sa = a.s;
  int parts = a.parts;
  // the score buffer, its width and the limit array are read with the block's
  // coordinates (an empty asm ties them to `parts`), so that the score and limit
  // loads below go out with the request's words instead of one round trip after them
  if constexpr (!ROWS && KPT > 0) __asm__("" : "+s"(parts) : "s"(sa.scores), "s"(sa.MP), "s"(sa.limit));
  const int bh = blockIdx.x / parts, part = blockIdx.x - bh * parts;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lo = lane & 15, hi = lane >> 4;
  const int b = bh / kStepKV, h = bh - b * kStepKV;
  const int64_t s = ROWS ? 0 : sa.seq[b];
  const int64_t req = ROWS ? 0 : sa.rpi[b];
  const int top_k = sa.top_k, k = sa.k_sel;
  constexpr int P = 64;
  const int G = a.G;
  // Q^T as the B operand: query head lo (zero past G), channels 8hi + 32ks
  bf16x8_t qb[4];
  {
    const uint16_t* qp = static_cast<const uint16_t*>(sa.q) + (int64_t)b * sa.q_bstride +
                         (int64_t)(h * G + lo) * kMfmaDim + hi * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (lo < G) {
        qb[ks] = *reinterpret_cast<const bf16x8_t*>(qp + ks * 32);
      } else {
        qb[ks] = __builtin_bit_cast(bf16x8_t, u32x4_t{0u, 0u, 0u, 0u});
      }
    }
  }
  // the scores go out with the request's words (their addresses do not wait for
  // them): entries past the table re-read its last one and are masked below.  The
  // scheduling barrier keeps every use of the request's words after these loads, so
  // that the wait for the words does not come before them, and both branches below
  // read the scores, so that the loads are not moved into the selecting one
  float sv[KPT > 0 ? KPT : 1];
  int lim_raw = 0;
  if constexpr (KPT > 0) {
    const float* sc = sa.scores + (int64_t)b * sa.MP;
#pragma unroll
    for (int i = 0; i < KPT; ++i) sv[i] = sc[min(tid + NT * i, sa.MP - 1)];
    lim_raw = sa.limit[b];
    __builtin_amdgcn_sched_barrier(0);
  }
  const bool long_b = !ROWS && needs_selection(sa, s);
  // actual_lens (quest.py:345)
  const int n = ROWS ? min(max(a.actual[b], 0), top_k) : (int)min(max(s, (int64_t)0), (int64_t)top_k);
  const bool r2t_ok = !ROWS && req >= 0 && req < a.r2t_rows;
  int my_rank = -1, my_page = -1, my_row0 = -1;  // lane s: a survivor's rank, page, first pool row
  if constexpr (KPT > 0) {
    if (long_b) {  // block-uniform
      const int lim = (req >= 0 && req < sa.R) ? min(lim_raw, sa.MP) : 0;
      select_ranked<KPT, NT>(sv, lim, max(lim, k), k, sm.sel, nullptr, sa.MP, my_rank, my_page, my_row0);
    } else {
#pragma unroll
      for (int i = 0; i < KPT; ++i) __asm__ volatile("" ::"v"(sv[i]));
    }
  }
  const int units = top_k / P;
  const int stride_units = parts * W;
  const int64_t recent0 = max(s - P, (int64_t)0);
  int32_t* pos_out = !ROWS && h == 0 && sa.positions ? sa.positions + (int64_t)b * top_k : nullptr;
  const uint16_t* kb = a.k + h * kMfmaDim;
  const uint16_t* vb = a.v + h * kMfmaDim;
  constexpr int kRow = kStepKV * kMfmaDim;
  float M = -INFINITY, L = 0.0f;
  float4_t o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = float4_t{0.f, 0.f, 0.f, 0.f};
  bool bad = false;
  for (int u = part * W + wave; u < units; u += stride_units) {  // wave-uniform
    const int slot = u * P + lane;
    const int valid = min(n - u * P, P);  // real slots of this unit
    int64_t row = 0;
    if constexpr (ROWS) {
      if (lane < valid) {
        row = a.rows_in[(int64_t)b * a.rows_stride + slot];
        bad |= row < 0;
      }
    } else {
      int64_t p;
      if (!long_b)
        p = s <= top_k ? min((int64_t)slot, max(s - 1, (int64_t)0)) : min(recent0 + slot, s - 1);
      else if (u < k)
        p = (int64_t)__builtin_amdgcn_readlane(my_page, __builtin_ctzll(__ballot(my_rank == u))) * P + lane;
      else
        p = min(recent0 + (slot - k * P), s - 1);
      if (lane < valid && r2t_ok && p >= 0 && p < a.r2t_stride) row = a.r2t[req * a.r2t_stride + p];
      if (pos_out) pos_out[slot] = (int32_t)p;  // after the row load: waiting for the row does not wait for it
    }
    if (valid <= 0) continue;
    const int r32 = (row >= 0 && row < a.kv_rows) ? (int)row : 0;
    // every K and V load of the unit in flight at once
    bf16x8_t ka[4][4];
    uint4 vr[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint16_t* kp = kb + (int64_t)__shfl(r32, t * 16 + lo, 64) * kRow + hi * 8;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) ka[t][ks] = *reinterpret_cast<const bf16x8_t*>(kp + ks * 32);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        vr[t][j] = *reinterpret_cast<const uint4*>(vb + (int64_t)__shfl(r32, t * 16 + hi * 4 + j, 64) * kRow + lo * 8);
    __builtin_amdgcn_sched_barrier(0);  // all 32 loads go out before the first use of any
    // S^T[token 16t + 4hi + i][head lo] in acc[t][i]
    float4_t acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[t][ks], qb[ks], acc[t], 0, 0, 0);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = (t * 16 + hi * 4 + i) < valid ? acc[t][i] * a.sl2 : -INFINITY;
        acc[t][i] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, lane_xor16(mx, lane));
    mx = fmaxf(mx, lane_xor32(mx, lane));
    const float Mn = fmaxf(M, mx);
    const float alpha = M == -INFINITY ? 0.0f : exp2f(M - Mn);  // rescale of the running sums
    float sum = 0.0f;
    short4_t pa[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // v_exp_f32 as it is (exp2f adds a rescale for results below 2^-126, which only
        // the weights of rows 126 binary orders under the maximum reach) and the hardware's
        // round-to-nearest-even bf16 conversion, equal to f2bf for every value that is not NaN
        const uint16_t pbits = __builtin_bit_cast(uint16_t, (__bf16)__builtin_amdgcn_exp2f(acc[t][i] - Mn));
        sum += bf2f(pbits);
        pa[t][i] = (short)pbits;
      }
    sum += lane_xor16(sum, lane);
    sum += lane_xor32(sum, lane);
    L = L * alpha + sum;
    M = Mn;
    // o rows are heads 4hi + i: their scale factors live in lanes 4hi + i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ai = __shfl(alpha, hi * 4 + i, 64);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e][i] *= ai;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      short4_t vbv[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 w = vr[t][j];
        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          vbv[2 * x][j] = (short)(wv[x] & 0xFFFFu);
          vbv[2 * x + 1][j] = (short)(wv[x] >> 16);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa[t], vbv[e], o[e], 0, 0, 0);
    }
  }
  bool poison = false;
  if constexpr (ROWS) poison = __syncthreads_or(bad ? 1 : 0) != 0;  // a failed swap-in: NaN output
  else lds_barrier();  // the selection's LDS is free before the combine reuses it
  finish_block<W, kUnitParts, false>(a, bh, part, M, L, o, poison, sm.comb.m, sm.comb.l, sm.comb.o, &s_last);
}

}  // namespace
}  // namespace qq

using namespace qq;

extern "C" int64_t qq_quest_layer_step_sync_bytes(int bs, int kv_heads) {
  if (bs <= 0 || kv_heads <= 0) return 0;
  return (int64_t)bs * kv_heads * 32 * (int64_t)sizeof(uint32_t);
}

// Compute units of the current device (cached per device).
static int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// LDS of the dense attention kernel (above the 64 KiB default: opted in once per
// device).
static size_t head_smem_bytes() {
  static bool opted[64] = {false};
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !opted[dev]) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&quest_attend_part_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(HeadSmemLaunch));
    opted[dev] = true;
  }
  return sizeof(HeadSmemLaunch);
}

// LDS of a unit-attention instance: the wave combine, or the selection that
// aliases it (above the 64 KiB default for 8-wave blocks: opted in once per device).
template <bool ROWS, int KPT, int W>
static size_t unit_smem_bytes() {
  constexpr size_t kSmem = sizeof(UnitSmem<KPT, W>);
  static_assert(kSmem <= 160 * 1024, "within the CU's LDS");
  if constexpr (kSmem > 64 * 1024) {
    static bool opted[64] = {false};
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !opted[dev]) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&quest_attend_unit_kernel<ROWS, KPT, W>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSmem);
      opted[dev] = true;
    }
  }
  return kSmem;
}

template <bool ROWS, int KPT, int W>
static void launch_unit(const StepArgs& a, hipStream_t s) {
  const int blocks = a.bs * kStepKV * a.parts;
  quest_attend_unit_kernel<ROWS, KPT, W><<<blocks, 64 * W, unit_smem_bytes<ROWS, KPT, W>(), s>>>(a);
}

// The selection's scores per thread for n_max candidate pages (up to 8192: 32 per
// thread at W = 4, 16 at W = 8).
template <int W>
static void launch_attend_select(const StepArgs& a, int n_max, hipStream_t s) {
  constexpr int kT = 64 * W;
  constexpr int kMaxKpt = W == 4 ? 32 : 24;
  if (n_max <= 2 * kT) launch_unit<false, 2, W>(a, s);
  else if (n_max <= 4 * kT) launch_unit<false, 4, W>(a, s);
  else if (n_max <= 5 * kT) launch_unit<false, 5, W>(a, s);  // contexts up to 128K + a few pages at W = 8
  else if (n_max <= 6 * kT) launch_unit<false, 6, W>(a, s);
  else if (n_max <= 8 * kT) launch_unit<false, 8, W>(a, s);
  else if (n_max <= 9 * kT) launch_unit<false, 9, W>(a, s);  // contexts just past 128K at W = 4
  else if (n_max <= 12 * kT) launch_unit<false, 12, W>(a, s);
  else if (n_max <= 16 * kT) launch_unit<false, 16, W>(a, s);
  else if (n_max <= 24 * kT) launch_unit<false, 24, W>(a, s);
  else launch_unit<false, kMaxKpt, W>(a, s);  // contexts past 384K tokens at W = 4
}

// Shapes the fused layer step takes (bf16, KV*D = 4*128, G <= 16, page 64, at
// most 64 selected pages, top_k <= 4096, at most 8192 pages per request).
// new_dtype < 0: no new token.
static bool fused_shape(int q_dtype, int kv_dtype, int new_dtype, int num_q_heads, int kv_heads, int head_dim,
                        int page_size, int top_k, int max_pages) {
  if (kv_heads != kStepKV || head_dim != kMfmaDim || num_q_heads % kv_heads != 0 || page_size != 64 ||
      top_k <= 0 || top_k % page_size != 0)
    return false;
  return q_dtype == QQ_DTYPE_BF16 && kv_dtype == QQ_DTYPE_BF16 && (new_dtype < 0 || new_dtype == QQ_DTYPE_BF16) &&
         num_q_heads / kv_heads <= kStepMaxG && top_k / page_size - 1 <= kMaxSelFused && top_k <= kStepMaxTopK &&
         max_pages <= 32 * 64 * kUnitMinWaves;
}

// Launch shape of the unit attention: W waves per block, `parts` blocks per (request,
// KV head); a wave takes the units p*W + w, p*W + w + W*parts, ... one after the other.
// The grid is sized to one round of resident blocks, since each block pays its own
// selection, row lookups and merge before and after its streaming:
//  * fewer units than one 8-wave block per CU could take: 4-wave blocks, one unit per
//    wave (as many parts as that needs, up to kUnitParts);
//  * up to one (request, KV head) pair per CU: 8-wave blocks (one per CU), parts =
//    CUs / pairs (batch 16 x 2048 slots: 4 parts, one unit per wave; batch 32: 2 parts);
//  * more pairs: 4-wave blocks (two per CU), parts = ceil(2 CUs / pairs) (1 from 2 pairs
//    per CU on).
// Measured at 48 layers: batch 32 x 64K 51.3 -> 45.2 us per layer-step, batch 64 x 32K
// 83.5 -> 67.1, batch 96 x 21.8K 101.4 -> 93.0, batch 128 x 16K 147.6 -> 111.0 against
// one unit per wave throughout.
struct UnitShape {
  int W, parts;
};
static UnitShape unit_shape(int bs, int top_k) {
  const int64_t c = device_cu_count(), units = top_k / 64, pairs = (int64_t)bs * kStepKV;
  const int cap8 = std::max(1, std::min(kUnitParts, ceil_div(units, 8)));
  const int cap4 = std::max(1, std::min(kUnitParts, ceil_div(units, 4)));
  if (pairs * units < 8 * c) return {4, cap4};
  if (pairs <= c) return {8, (int)std::max<int64_t>(1, std::min<int64_t>(cap8, c / pairs))};
  return {4, std::max(1, std::min(cap4, ceil_div(2 * c, pairs)))};
}

extern "C" int qq_quest_fused_step(int q_dtype, int kv_dtype, int new_dtype, int num_q_heads, int kv_heads,
                                   int head_dim, int page_size, int top_k, int max_pages) {
  return fused_shape(q_dtype, kv_dtype, new_dtype, num_q_heads, kv_heads, head_dim, page_size, top_k, max_pages)
             ? 1
             : 0;
}

// The fused attention over given rows (one launch of quest_attend_unit_kernel in its rows mode);
// QQ_OK when launched, 1 when the shape or the buffers do not allow it.
int qq::attend_rows_fused(const void* q, int64_t q_bstride, int num_q_heads, const void* k_layer, const void* v_layer,
                      int64_t kv_rows, const int64_t* rows, int64_t slots, const int32_t* actual, int bs, float scale,
                      void* out, void* workspace, int64_t workspace_bytes, void* sync, int64_t sync_bytes,
                      hipStream_t s) {
  if (!sync || sync_bytes < qq_quest_layer_step_sync_bytes(bs, kStepKV) || slots <= 0 || slots > kStepMaxTopK ||
      slots % 64 != 0 || num_q_heads % kStepKV != 0 || num_q_heads / kStepKV > kStepMaxG || !workspace)
    return 1;
  const int top_k = (int)slots;
  const int G = num_q_heads / kStepKV;
  const UnitShape us = unit_shape(bs, top_k);
  const int W = us.W, parts = us.parts;
  const int64_t part_bytes = (int64_t)bs * kStepKV * parts * G * (kMfmaDim + 2) * (int64_t)sizeof(float);
  if (parts > 1 && workspace_bytes < part_bytes) return 1;
  StepArgs a{};
  a.s.q = q;
  a.s.q_dtype = QQ_DTYPE_BF16;
  a.s.q_bstride = q_bstride;
  a.s.H = num_q_heads;
  a.s.top_k = top_k;
  a.s.P = 64;
  a.k = static_cast<const uint16_t*>(k_layer);
  a.v = static_cast<const uint16_t*>(v_layer);
  a.kv_rows = kv_rows;
  a.sl2 = scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = a.part_o + (int64_t)bs * kStepKV * parts * G * kMfmaDim;
  a.parts = parts;
  a.sync = static_cast<uint32_t*>(sync);
  a.bs = bs;
  a.G = G;
  a.rows_in = rows;
  a.rows_stride = slots;
  a.actual = actual;
  if (W == 8)
    launch_unit<true, 0, 8>(a, s);
  else
    launch_unit<true, 0, 4>(a, s);
  return QQ_OK;
}

// Dense decode (attention/dense.py:26-42): every request attends
// req_to_token[req, 0 .. seq_len) - the fused attention kernel without a
// selection (its dense layout), at most kStepMaxTopK rows per block and as
// many parts per (request, KV head) as the longest context of the table needs.
static int dense_parts(int64_t max_rows) { return max(1, ceil_div(max_rows, kStepMaxTopK)); }

extern "C" int64_t qq_dense_decode_workspace_bytes(int bs, int64_t max_rows, int num_q_heads, int kv_heads) {
  if (bs <= 0 || max_rows <= 0 || kv_heads <= 0 || num_q_heads <= 0) return 0;
  const int parts = dense_parts(max_rows);
  return parts > 1 ? (int64_t)bs * kv_heads * parts * (num_q_heads / kv_heads) * (kMfmaDim + 2) *
                         (int64_t)sizeof(float)
                   : 0;
}

extern "C" int qq_dense_forward_decode(const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads,
                                       const void* k_new, const void* v_new, int new_dtype,
                                       const int64_t* out_cache_loc, void* k_layer, void* v_layer, int kv_dtype,
                                       int64_t kv_rows, int kv_heads, int head_dim, const int64_t* req_pool_indices,
                                       const int64_t* seq_lens, int bs, const int32_t* req_to_token,
                                       int64_t req_to_token_stride, int64_t req_to_token_rows, float scale,
                                       void* out, void* workspace, int64_t workspace_bytes, void* sync,
                                       int64_t sync_bytes, void* stream) {
  const char* what = "qq_dense_forward_decode";
  QQ_REQUIRE(q_dtype == QQ_DTYPE_BF16 && kv_dtype == QQ_DTYPE_BF16 && (!k_new || new_dtype == QQ_DTYPE_BF16) &&
                 kv_heads == kStepKV && head_dim == kMfmaDim && num_q_heads % kv_heads == 0 &&
                 num_q_heads / kv_heads <= kStepMaxG,
             "%s: the HIP dense decode takes bf16 queries and K/V, %d KV heads x %d, at most %d query heads "
             "per KV head", what, kStepKV, kMfmaDim, kStepMaxG);
  QQ_REQUIRE(bs >= 0 && req_to_token_stride > 0 && req_to_token_stride <= (int64_t)1 << 30, "%s: bad sizes", what);
  QQ_REQUIRE(!k_new || (v_new && out_cache_loc), "%s: new K without V or locations", what);
  if (bs == 0) return QQ_OK;
  QQ_REQUIRE(q && k_layer && v_layer && req_pool_indices && seq_lens && req_to_token && out, "%s: null pointer", what);
  QQ_REQUIRE(sync && sync_bytes >= qq_quest_layer_step_sync_bytes(bs, kv_heads), "%s: sync buffer too small", what);
  const int64_t need = qq_dense_decode_workspace_bytes(bs, req_to_token_stride, num_q_heads, kv_heads);
  QQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), "%s: workspace %lld bytes < %lld needed", what,
             (long long)workspace_bytes, (long long)need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (k_new) {  // set_kv_buffer (memory.py:114-120) before the attention reads the pool
    const int st = qq_kv_scatter(k_layer, v_layer, kv_dtype, kv_rows, k_new, v_new, new_dtype, out_cache_loc, bs,
                                 (int64_t)kv_heads * head_dim, stream);
    if (st != QQ_OK) return st;
  }
  const int top_k = (int)req_to_token_stride;  // every context fits: seq_len <= the table's width
  const int G = num_q_heads / kv_heads;
  const int parts = dense_parts(top_k);
  StepArgs a{};
  a.s.q = q;
  a.s.q_dtype = QQ_DTYPE_BF16;
  a.s.q_bstride = q_batch_stride;
  a.s.H = num_q_heads;
  a.s.rpi = req_pool_indices;
  a.s.seq = seq_lens;
  a.s.top_k = top_k;
  a.s.P = 64;
  a.s.k_sel = 0;  // no selection: positions 0 .. seq_len - 1
  a.k = static_cast<const uint16_t*>(k_layer);
  a.v = static_cast<const uint16_t*>(v_layer);
  a.kv_rows = kv_rows;
  a.r2t = req_to_token;
  a.r2t_stride = req_to_token_stride;
  a.r2t_rows = req_to_token_rows;
  a.sl2 = scale * kLog2e;
  a.out = static_cast<uint16_t*>(out);
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = a.part_o + (int64_t)bs * kStepKV * parts * G * kMfmaDim;
  a.sync = static_cast<uint32_t*>(sync);
  a.bs = bs;
  a.G = G;
  a.parts = parts;
  a.per_wave = ceil_div(top_k, parts * kHeadWaves * 32) * 32;
  quest_attend_part_kernel<<<bs * kStepKV * parts, 64 * kHeadWaves, head_smem_bytes(), s>>>(a);
  return check_launch(what);
}

static int forward_decode(
    const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads, const void* k_new,
    const void* v_new, int new_dtype, const int64_t* out_cache_loc, void* k_layer, void* v_layer,
    int kv_dtype, int64_t kv_rows, const uint16_t* page_k_bounds, int layer,
    const int64_t* req_pool_indices, const int64_t* seq_lens, const int32_t* candidate_limit,
    const int32_t* actual_lens, int bs, int max_reqs, int max_pages, int kv_heads, int head_dim,
    int page_size, int top_k, const int32_t* req_to_token, int64_t req_to_token_stride,
    int64_t req_to_token_rows, float scale, float* scores_ws, int32_t* positions, void* out,
    void* workspace, int64_t workspace_bytes, void* sync, int64_t sync_bytes, int phase, hipStream_t s, const char* what) {
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
  QQ_REQUIRE(phase >= 1 && phase <= 3, "%s: phase %d is not 1, 2 or 3", what, phase);
  if (bs == 0) return QQ_OK;

  SelectArgs sa{};
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
  const UnitShape us = unit_shape(bs, top_k);
  const int W = us.W, parts = us.parts;
  const int64_t part_bytes = (int64_t)bs * kv_heads * parts * G * (kMfmaDim + 2) * (int64_t)sizeof(float);
  const bool fused = sync && sync_bytes >= qq_quest_layer_step_sync_bytes(bs, kv_heads) &&
                     fused_shape(q_dtype, kv_dtype, k_new ? new_dtype : -1, num_q_heads, kv_heads, head_dim,
                                 page_size, top_k, max_pages) &&
                     workspace && workspace_bytes >= (parts > 1 ? part_bytes : 0);
  if (fused) {
    // 1. scores of the candidate pages (+ the new token's K/V), all CUs
    if (phase & 1) {
      const int st = launch_score(sa, bs, true, s);
      if (st != QQ_OK || !(phase & 2)) return st;
    }
    // 2. per (request, KV head, part): the request's selection, layout, attention, merge
    StepArgs a{};
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
    a.part_ml = a.part_o + (int64_t)bs * kv_heads * parts * G * kMfmaDim;
    a.parts = parts;
    a.sync = static_cast<uint32_t*>(sync);
    a.bs = bs;
    a.G = G;
    const int n_max = max(max_pages, k_sel);
    if (W == 8)
      launch_attend_select<8>(a, n_max, s);
    else
      launch_attend_select<4>(a, n_max, s);
    return check_launch(what);
  }

  if (phase & 1) {
    const int st = launch_retrieve(sa, bs, s);
    if (st != QQ_OK || !(phase & 2)) return st;
  }

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

extern "C" int qq_quest_forward_decode(
    const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads, const void* k_new,
    const void* v_new, int new_dtype, const int64_t* out_cache_loc, void* k_layer, void* v_layer,
    int kv_dtype, int64_t kv_rows, const uint16_t* page_k_bounds, int layer,
    const int64_t* req_pool_indices, const int64_t* seq_lens, const int32_t* candidate_limit,
    const int32_t* actual_lens, int bs, int max_reqs, int max_pages, int kv_heads, int head_dim,
    int page_size, int top_k, const int32_t* req_to_token, int64_t req_to_token_stride,
    int64_t req_to_token_rows, float scale, float* scores_ws, int32_t* positions, void* out,
    void* workspace, int64_t workspace_bytes, void* sync, int64_t sync_bytes, void* stream) {
  return forward_decode(q, q_dtype, q_batch_stride, num_q_heads, k_new, v_new, new_dtype, out_cache_loc, k_layer, v_layer,
      kv_dtype, kv_rows, page_k_bounds, layer, req_pool_indices, seq_lens, candidate_limit, actual_lens, bs,
      max_reqs, max_pages, kv_heads, head_dim, page_size, top_k, req_to_token, req_to_token_stride,
      req_to_token_rows, scale, scores_ws, positions, out, workspace, workspace_bytes, sync, sync_bytes, 3, static_cast<hipStream_t>(stream), "qq_quest_forward_decode");
}

extern "C" int qq_quest_forward_decode_phase(
    const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads, const void* k_new,
    const void* v_new, int new_dtype, const int64_t* out_cache_loc, void* k_layer, void* v_layer,
    int kv_dtype, int64_t kv_rows, const uint16_t* page_k_bounds, int layer,
    const int64_t* req_pool_indices, const int64_t* seq_lens, const int32_t* candidate_limit,
    const int32_t* actual_lens, int bs, int max_reqs, int max_pages, int kv_heads, int head_dim,
    int page_size, int top_k, const int32_t* req_to_token, int64_t req_to_token_stride,
    int64_t req_to_token_rows, float scale, float* scores_ws, int32_t* positions, void* out,
    void* workspace, int64_t workspace_bytes, void* sync, int64_t sync_bytes, int phase, void* stream) {
  return forward_decode(q, q_dtype, q_batch_stride, num_q_heads, k_new, v_new, new_dtype, out_cache_loc, k_layer, v_layer,
      kv_dtype, kv_rows, page_k_bounds, layer, req_pool_indices, seq_lens, candidate_limit, actual_lens, bs,
      max_reqs, max_pages, kv_heads, head_dim, page_size, top_k, req_to_token, req_to_token_stride,
      req_to_token_rows, scale, scores_ws, positions, out, workspace, workspace_bytes, sync, sync_bytes, phase, static_cast<hipStream_t>(stream), "qq_quest_forward_decode_phase");
}

// ------------------------------------------------------------ no allocation
// qq_quest_forward_decode_noalloc: the same layer with its scratch (page
// scores, attention partials, hand-off counters) in one file-scope device
// array instead of caller workspaces, for callers that cannot allocate.  Each
// device holds its own copy; its address is looked up once per device and the
// counter region is cleared there, after which every call leaves it cleared.
namespace {

constexpr int64_t kScratchBytes = 16ll << 20;
constexpr int64_t kScratchSyncBytes = 64ll << 10;             // [0, 64 KiB): counters
constexpr int64_t kScratchScoreBytes = (4ll << 20) - kScratchSyncBytes;  // [64 KiB, 4 MiB): page scores
constexpr int64_t kScratchWorkOffset = 4ll << 20;              // [4 MiB, 16 MiB): attention partials
constexpr int64_t kScratchWorkBytes = kScratchBytes - kScratchWorkOffset;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxDevices] = {nullptr};

__global__ void zero_words_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// The current device's scratch address (looked up, and its counters cleared
// on `s`, on the first call on that device); nullptr with the error recorded.
unsigned char* device_scratch(hipStream_t s) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error(QQ_EHIP, "qq_quest_forward_decode_noalloc: no current HIP device (or device id >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    set_error(QQ_EHIP, "qq_quest_forward_decode_noalloc: hipGetSymbolAddress(scratch) failed: %s",
              hipGetErrorString(e));
    return nullptr;
  }
  zero_words_kernel<<<64, 256, 0, s>>>(static_cast<uint32_t*>(p), kScratchSyncBytes / 4);
  if (check_launch("qq_quest_forward_decode_noalloc (scratch clear)") != QQ_OK) return nullptr;
  g_scratch_ptr[dev] = static_cast<unsigned char*>(p);
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int64_t qq_quest_forward_decode_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int qq_quest_forward_decode_noalloc(
    const void* q, int q_dtype, int64_t q_batch_stride, int num_q_heads, const void* k_new,
    const void* v_new, int new_dtype, const int64_t* out_cache_loc, void* k_layer, void* v_layer,
    int kv_dtype, int64_t kv_rows, const uint16_t* page_k_bounds, int layer,
    const int64_t* req_pool_indices, const int64_t* seq_lens, const int32_t* candidate_limit,
    const int32_t* actual_lens, int bs, int max_reqs, int max_pages, int kv_heads, int head_dim,
    int page_size, int top_k, const int32_t* req_to_token, int64_t req_to_token_stride,
    int64_t req_to_token_rows, float scale, int32_t* positions, void* out, void* stream) {
  const char* what = "qq_quest_forward_decode_noalloc";
  QQ_REQUIRE(bs >= 0 && max_pages > 0 && kv_heads > 0 && head_dim > 0 && num_q_heads > 0, "%s: bad sizes", what);
  if (bs == 0) return QQ_OK;
  // the hand-off counters are read only by the fused layer step; other shapes take the
  // four-launch path, which needs none
  const bool fused = fused_shape(q_dtype, kv_dtype, k_new ? new_dtype : -1, num_q_heads, kv_heads, head_dim,
                                 page_size, top_k, max_pages);
  const int64_t sync_need = fused ? qq_quest_layer_step_sync_bytes(bs, kv_heads) : 0;
  const int64_t score_need = (int64_t)bs * max_pages * (int64_t)sizeof(float);
  const int64_t work_need = qq_decode_attention_workspace_bytes(bs, top_k, num_q_heads, head_dim);
  QQ_REQUIRE(sync_need <= kScratchSyncBytes && score_need <= kScratchScoreBytes && work_need <= kScratchWorkBytes,
             "%s: batch %d x %d pages x top_k %d needs %lld B of counters, %lld B of scores and %lld B of "
             "partials; the fixed scratch holds %lld, %lld and %lld",
             what, bs, max_pages, top_k, (long long)sync_need, (long long)score_need, (long long)work_need,
             (long long)kScratchSyncBytes, (long long)kScratchScoreBytes, (long long)kScratchWorkBytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned char* base = device_scratch(s);
  if (!base) return QQ_EHIP;
  return forward_decode(q, q_dtype, q_batch_stride, num_q_heads, k_new, v_new, new_dtype, out_cache_loc, k_layer,
                        v_layer, kv_dtype, kv_rows, page_k_bounds, layer, req_pool_indices, seq_lens, candidate_limit,
                        actual_lens, bs, max_reqs, max_pages, kv_heads, head_dim, page_size, top_k, req_to_token,
                        req_to_token_stride, req_to_token_rows, scale,
                        reinterpret_cast<float*>(base + kScratchSyncBytes), positions, out, base + kScratchWorkOffset,
                        kScratchWorkBytes, base, kScratchSyncBytes, 3, s, what);
}
