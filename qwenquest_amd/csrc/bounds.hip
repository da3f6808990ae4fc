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
constexpr int kWaveFoldBatch = 32;  // rows in flight per wave of prefill_bounds_wave_kernel
constexpr int kWavePages = 1;      // pages per wave of prefill_bounds_wave_kernel
constexpr int kPfThreads = 128;  // 2 waves per block of prefill_bounds_wave_kernel

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

// bf16 keys with KV*D = C a power of two in [8, 2048]: the same fold with
// 16-byte loads.  L = C / 8 lanes cover a row (8 channels each), the block's
// kThreads / L row groups take contiguous runs of the chunk's rows, and the
// groups' results fold in group order - the rows are folded in their order,
// as above (ties and NaNs resolve as in a sequential fold).
template <int L>
__global__ __launch_bounds__(kThreads) void prefill_bounds_wide_kernel(PrefillArgs a) {
  constexpr int kGroups = kThreads / L;
  constexpr int C = L * 8;
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
  const uint4* kl = reinterpret_cast<const uint4*>(a.k_base + (int64_t)li * a.k_layer_stride_bytes);
  __shared__ int64_t s_rows[kRowChunk];
  __shared__ uint4 s_mn[kGroups][L], s_mx[kGroups][L];
  const int lane = threadIdx.x % L, grp = threadIdx.x / L;
  uint16_t mn[8], mx[8];  // the block's fold so far (kept by group 0)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    mn[e] = 0x7F80;
    mx[e] = 0xFF80;
  }
  for (int64_t t0 = begin; t0 < end; t0 += kRowChunk) {
    const int cnt = (int)min((int64_t)kRowChunk, end - t0);
    __syncthreads();
    for (int t = threadIdx.x; t < cnt; t += kThreads) {
      const int64_t row = load_index(a.idx, a.idx64, t0 + t);
      s_rows[t] = (row >= 0 && row < a.k_rows) ? row : -1;
    }
    __syncthreads();
    // group grp folds rows [r0, r1) of the chunk
    const int per = (cnt + kGroups - 1) / kGroups;
    const int r0 = min(cnt, grp * per), r1 = min(cnt, r0 + per);
    uint16_t gmn[8], gmx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      gmn[e] = 0x7F80;
      gmx[e] = 0xFF80;
    }
#pragma unroll 4
    for (int t = r0; t < r1; ++t) {
      const int64_t row = s_rows[t];
      if (row < 0) continue;
      const uint4 v = kl[row * (C / 8) + lane];
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint16_t x = (uint16_t)(w[e >> 1] >> ((e & 1) * 16));
        gmn[e] = bmin(gmn[e], x);
        gmx[e] = bmax(gmx[e], x);
      }
    }
    uint4 pm, px;
    pm.x = gmn[0] | ((uint32_t)gmn[1] << 16);
    pm.y = gmn[2] | ((uint32_t)gmn[3] << 16);
    pm.z = gmn[4] | ((uint32_t)gmn[5] << 16);
    pm.w = gmn[6] | ((uint32_t)gmn[7] << 16);
    px.x = gmx[0] | ((uint32_t)gmx[1] << 16);
    px.y = gmx[2] | ((uint32_t)gmx[3] << 16);
    px.z = gmx[4] | ((uint32_t)gmx[5] << 16);
    px.w = gmx[6] | ((uint32_t)gmx[7] << 16);
    s_mn[grp][lane] = pm;
    s_mx[grp][lane] = px;
    __syncthreads();
    if (grp == 0) {
#pragma unroll
      for (int g = 0; g < kGroups; ++g) {
        const uint4 qm = s_mn[g][lane], qx = s_mx[g][lane];
        const uint32_t wm[4] = {qm.x, qm.y, qm.z, qm.w}, wx[4] = {qx.x, qx.y, qx.z, qx.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          mn[e] = bmin(mn[e], (uint16_t)(wm[e >> 1] >> ((e & 1) * 16)));
          mx[e] = bmax(mx[e], (uint16_t)(wx[e >> 1] >> ((e & 1) * 16)));
        }
      }
    }
  }
  if (grp != 0) return;
  const int c0 = lane * 8;
  const int64_t rc = ((int64_t)layer * a.R + a.req) * C + c0;
  if (page < a.full_pages) {
    if (page < a.MP) {
      uint32_t* dst = a.bounds + (((int64_t)layer * a.R + a.req) * a.MP + page) * C + c0;
      uint4 lo, hi;
      lo.x = pack_pair(mn[0], mx[0]);
      lo.y = pack_pair(mn[1], mx[1]);
      lo.z = pack_pair(mn[2], mx[2]);
      lo.w = pack_pair(mn[3], mx[3]);
      hi.x = pack_pair(mn[4], mx[4]);
      hi.y = pack_pair(mn[5], mx[5]);
      hi.z = pack_pair(mn[6], mx[6]);
      hi.w = pack_pair(mn[7], mx[7]);
      reinterpret_cast<uint4*>(dst)[0] = lo;
      reinterpret_cast<uint4*>(dst)[1] = hi;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a.rmin[rc + e] = mn[e];
      a.rmax[rc + e] = mx[e];
    }
  }
}

// Two bf16 values (the halves of w) as 16-bit keys whose unsigned order is the values'
// order: x | 0x8000 for a clear sign bit, ~x for a set one.  Away from NaN and from
// zeros (-0 and +0 are equal values with different keys), equal keys are equal bit
// patterns, so the unsigned min / max of keys is torch.minimum / maximum of the values.
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t bf16x2_key(uint32_t w) { return w ^ ((((w >> 15) & 0x00010001u) * 0x7FFFu) | 0x80008000u); }
__device__ inline uint32_t bf16x2_unkey(uint32_t k) {
  return k ^ ((((~k >> 15) & 0x00010001u) * 0x7FFFu) | 0x80008000u);
}
__device__ inline uint32_t u16x2_min(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2_t, a), __builtin_bit_cast(u16x2_t, b)));
}
__device__ inline uint32_t u16x2_max(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, a), __builtin_bit_cast(u16x2_t, b)));
}
// max over the halves of (|x| - 1) mod 2^16: >= 0x7F80 exactly when a half is a NaN or a zero
__device__ inline uint32_t bf16x2_special(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2_t, w & 0x7FFF7FFFu) - (u16x2_t){1, 1});
}

// The wide fold for C = 512 (KV*D = 4 x 128, bf16): one wave per PPW consecutive pages
// of one layer, 4 waves per block, no LDS and no barrier.  Lane l holds channels 8l ..
// 8l + 7 of every row (one 1 KiB row per load instruction); a page's row indices come in
// with one load (lane r: row r of a 64-row chunk; the first chunk of every page of the
// wave is loaded up front) and reach the row loads through readlane, and the rows fold
// in order in batches of B loads in flight, so ties and NaNs resolve as in a sequential
// fold: a batch without NaNs and zeros folds as unsigned min / max of monotone 16-bit
// keys (two channels per instruction), any other batch element by element with
// torch.minimum / maximum semantics.  A row outside the buffer is not folded (its load
// reads row 0).
template <int B, int PPW>
__global__ __launch_bounds__(kPfThreads) void prefill_bounds_wave_kernel(PrefillArgs a) {
  constexpr int C = 512;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t page0 = ((int64_t)blockIdx.x * (kPfThreads / 64) + wave) * PPW;
  const int li = blockIdx.y;
  const int layer = a.layer_begin + li;
  if (a.set_counters && page0 == 0 && li == a.n_layers - 1 && lane == 0) {
    a.count[a.req] = (int32_t)(a.n - a.full_pages * a.P);
    a.page_idx[a.req] = (int32_t)a.full_pages;
  }
  if (page0 * a.P >= a.n) return;  // wave-uniform
  const uint4* kl = reinterpret_cast<const uint4*>(a.k_base + (int64_t)li * a.k_layer_stride_bytes);
  auto chunk_row = [&](int64_t t0, int cnt) -> int32_t {  // lane r: row t0 + r (-1: none)
    int64_t r = lane < cnt ? load_index(a.idx, a.idx64, t0 + lane) : -1;
    return (int32_t)((r >= 0 && r < a.k_rows) ? r : -1);  // rows < 2^31 (checked by the host)
  };
  int32_t first[PPW];
#pragma unroll
  for (int j = 0; j < PPW; ++j) {
    const int64_t begin = (page0 + j) * a.P;
    first[j] = chunk_row(begin, (int)max((int64_t)0, min((int64_t)min(a.P, 64), a.n - begin)));
  }
#pragma unroll
  for (int j = 0; j < PPW; ++j) {
    const int64_t page = page0 + j;
    const int64_t begin = page * a.P;
    const int64_t end = min(begin + (int64_t)a.P, a.n);
    if (begin >= end) break;  // wave-uniform
    // the fold so far as keys of channel pairs (8l + 2q, 8l + 2q + 1): +inf / -inf
    uint32_t kmn[4], kmx[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      kmn[q] = 0xFF80FF80u;
      kmx[q] = 0x007F007Fu;
    }
    for (int64_t t0 = begin; t0 < end && a.k_rows > 0; t0 += 64) {  // no rows: sentinels
      const int cnt = (int)min((int64_t)64, end - t0);
      const int32_t row32 = t0 == begin ? first[j] : chunk_row(t0, cnt);
      for (int tb = 0; tb < cnt; tb += B) {  // wave-uniform
        uint4 v[B];
        bool ok[B];
#pragma unroll
        for (int i = 0; i < B; ++i) {
          const int t = tb + i;
          const int r = t < cnt ? __builtin_amdgcn_readlane(row32, t) : -1;
          ok[i] = r >= 0;
          v[i] = kl[(int64_t)(ok[i] ? r : 0) * (C / 8) + lane];
        }
        uint32_t sp = 0;  // a NaN or a zero in the batch, or a NaN already folded (it must stay)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sp = u16x2_max(sp, u16x2_max(bf16x2_special(bf16x2_unkey(kmn[q])), bf16x2_special(bf16x2_unkey(kmx[q]))));
#pragma unroll
        for (int i = 0; i < B; ++i) {
          if (!ok[i]) continue;  // wave-uniform
          sp = u16x2_max(sp, u16x2_max(u16x2_max(bf16x2_special(v[i].x), bf16x2_special(v[i].y)),
                                       u16x2_max(bf16x2_special(v[i].z), bf16x2_special(v[i].w))));
        }
        const bool special = (sp & 0xFFFFu) >= 0x7F80u || (sp >> 16) >= 0x7F80u;
        if (!__builtin_amdgcn_ballot_w64(special)) {
          // no NaN and no zero in the batch or the fold so far: unsigned min / max of the keys
#pragma unroll
          for (int i = 0; i < B; ++i) {
            if (!ok[i]) continue;
            const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t kw = bf16x2_key(w[q]);
              kmn[q] = u16x2_min(kmn[q], kw);
              kmx[q] = u16x2_max(kmx[q], kw);
            }
          }
        } else {
          // NaNs or zeros: torch.minimum / maximum element by element, in row order
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t bmn = bf16x2_unkey(kmn[q]), bmx = bf16x2_unkey(kmx[q]);
            uint16_t mn0 = (uint16_t)bmn, mn1 = (uint16_t)(bmn >> 16);
            uint16_t mx0 = (uint16_t)bmx, mx1 = (uint16_t)(bmx >> 16);
#pragma unroll
            for (int i = 0; i < B; ++i) {
              if (!ok[i]) continue;
              const uint32_t w = q == 0 ? v[i].x : q == 1 ? v[i].y : q == 2 ? v[i].z : v[i].w;
              mn0 = bmin(mn0, (uint16_t)w);
              mn1 = bmin(mn1, (uint16_t)(w >> 16));
              mx0 = bmax(mx0, (uint16_t)w);
              mx1 = bmax(mx1, (uint16_t)(w >> 16));
            }
            kmn[q] = bf16x2_key((uint32_t)mn0 | ((uint32_t)mn1 << 16));
            kmx[q] = bf16x2_key((uint32_t)mx0 | ((uint32_t)mx1 << 16));
          }
        }
      }
    }
    uint16_t mn[8], mx[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t bmn = bf16x2_unkey(kmn[q]), bmx = bf16x2_unkey(kmx[q]);
      mn[2 * q] = (uint16_t)bmn;
      mn[2 * q + 1] = (uint16_t)(bmn >> 16);
      mx[2 * q] = (uint16_t)bmx;
      mx[2 * q + 1] = (uint16_t)(bmx >> 16);
    }
    const int c0 = lane * 8;
    if (page < a.full_pages) {
      if (page < a.MP) {
        uint32_t* dst = a.bounds + (((int64_t)layer * a.R + a.req) * a.MP + page) * C + c0;
        uint4 lo, hi;
        lo.x = pack_pair(mn[0], mx[0]);
        lo.y = pack_pair(mn[1], mx[1]);
        lo.z = pack_pair(mn[2], mx[2]);
        lo.w = pack_pair(mn[3], mx[3]);
        hi.x = pack_pair(mn[4], mx[4]);
        hi.y = pack_pair(mn[5], mx[5]);
        hi.z = pack_pair(mn[6], mx[6]);
        hi.w = pack_pair(mn[7], mx[7]);
        reinterpret_cast<uint4*>(dst)[0] = lo;
        reinterpret_cast<uint4*>(dst)[1] = hi;
      }
    } else {
      const int64_t rc = ((int64_t)layer * a.R + a.req) * C + c0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a.rmin[rc + e] = mn[e];
        a.rmax[rc + e] = mx[e];
      }
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

// quest_only.py:84-97: the previous token's pool row per listed request, -1 on a
// request's first decode step; the skip flags are cleared after every lookup.  One
// block, so the clears wait for all lookups.
__global__ __launch_bounds__(kThreads) void decode_step_locs_kernel(const int64_t* rpi, const int64_t* seq, int bs,
                                                                   uint8_t* skip, const int32_t* r2t,
                                                                   int64_t r2t_rows, int64_t r2t_cols,
                                                                   int64_t r2t_stride, int64_t* locs) {
  for (int i = threadIdx.x; i < bs; i += kThreads) {
    const int64_t r = rpi[i];
    int64_t loc = -1;
    if (r >= 0 && r < r2t_rows && !skip[r]) {
      const int64_t p = max(seq[i] - 2, (int64_t)0);
      if (p < r2t_cols) loc = r2t[r * r2t_stride + p];
    }
    locs[i] = loc;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < bs; i += kThreads) {
    const int64_t r = rpi[i];
    if (r >= 0 && r < r2t_rows) skip[r] = 0;
  }
}

// One decode step's bookkeeping in one launch (quest_only.py:84-97, quest.py:284-321
// and 325-362): blockIdx.x = batch entry, blockIdx.y = layer.  Every block looks up
// its entry's previous-token row itself (the lookup of decode_step_locs_kernel), folds
// that layer (decode_update_kernel with finalize) and counts itself done on the
// entry's counter; the entry's last block advances the page counters
// (advance_counters_kernel) and clears the first-step flag, after every block of the
// entry has read them.  The layer-0 block writes the step layout (prepare_step_kernel).
struct DecodeStepArgs {
  const int64_t *rpi, *seq;
  uint8_t* skip;
  const int32_t* r2t;
  int64_t r2t_rows, r2t_cols, r2t_stride;
  int64_t* locs_out;
  DecodeArgs d;
  int n_layers, top_k, avoid;
  int32_t *actual, *limit;
  int32_t *count, *page_idx;  // d's counters, advanced by the entry's last block
  uint32_t* sync;  // one counter per entry, each on its own 128-byte line
};

__global__ __launch_bounds__(kThreads) void decode_step_kernel(DecodeStepArgs a) {
  const int i = blockIdx.x;
  const int li = blockIdx.y;
  const DecodeArgs& d = a.d;
  const int64_t r = a.rpi[i];
  const int64_t s = a.seq[i];
  if (li == 0 && threadIdx.x == 0) {
    a.actual[i] = (int32_t)min(s, (int64_t)a.top_k);
    const int64_t full = s / d.P;
    a.limit[i] = (int32_t)(a.avoid ? max(full - 1, (int64_t)0) : full);
  }
  int64_t row = -1;
  if (r >= 0 && r < a.r2t_rows && !a.skip[r]) {
    const int64_t p = max(s - 2, (int64_t)0);
    if (p < a.r2t_cols) row = a.r2t[r * a.r2t_stride + p];
  }
  if (li == 0 && threadIdx.x == 0 && a.locs_out) a.locs_out[i] = row;
  const bool fold = r >= 0 && r < d.R && row >= 0;
  if (fold) {
    const bool row_ok = row < d.k_rows;
    const bool complete = d.count[r] == d.P - 1;
    const int64_t page = d.page_idx[r];
    const void* kl = d.k_base + (int64_t)li * d.k_layer_stride_bytes;
    for (int c = threadIdx.x; c < d.C; c += kThreads) {
      const int64_t rc = ((int64_t)li * d.R + r) * d.C + c;
      uint16_t mn = d.rmin[rc], mx = d.rmax[rc];
      if (row_ok) {
        const uint16_t v = load_as_bf16(kl, row * d.C + c, d.k_dtype);
        mn = bmin(mn, v);
        mx = bmax(mx, v);
      }
      if (complete) {
        if (page >= 0 && page < d.MP)
          d.bounds[(((int64_t)li * d.R + r) * d.MP + page) * d.C + c] = pack_pair(mn, mx);
        d.rmin[rc] = kBf16Max;
        d.rmax[rc] = kBf16Min;
      } else {
        d.rmin[rc] = mn;
        d.rmax[rc] = mx;
      }
    }
  }
  // this block's reads of the counters and the flag are done (their values were used)
  if (threadIdx.x == 0) {
    uint32_t* cnt = a.sync + (int64_t)i * 32;
    // agent scope: the entry's blocks run on any of the chip's L2 caches
    if (__hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)a.n_layers - 1) {
      __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (fold) {
        const int32_t c = a.count[r];
        if (c == d.P - 1) a.page_idx[r] += 1;
        a.count[r] = (c + 1) % d.P;
      }
      if (r >= 0 && r < a.r2t_rows) a.skip[r] = 0;
    }
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int C = a.C;
  const bool wide = k_dtype == QQ_DTYPE_BF16 && C >= 8 && C <= 8 * kThreads && (C & (C - 1)) == 0 &&
                    k_layer_stride % 8 == 0 && reinterpret_cast<uintptr_t>(k_base) % 16 == 0;
  if (!wide)
    prefill_bounds_kernel<<<grid, kThreads, 0, s>>>(a);
  else if (C == 512 && k_rows <= INT32_MAX)
    prefill_bounds_wave_kernel<kWaveFoldBatch, kWavePages>
        <<<dim3(ceil_div(pages, kPfThreads / 64 * kWavePages), n_layers), kPfThreads, 0, s>>>(a);
  else if (C == 512)
    prefill_bounds_wide_kernel<64><<<grid, kThreads, 0, s>>>(a);
  else if (C == 1024)
    prefill_bounds_wide_kernel<128><<<grid, kThreads, 0, s>>>(a);
  else if (C == 2048)
    prefill_bounds_wide_kernel<256><<<grid, kThreads, 0, s>>>(a);
  else if (C == 256)
    prefill_bounds_wide_kernel<32><<<grid, kThreads, 0, s>>>(a);
  else if (C == 128)
    prefill_bounds_wide_kernel<16><<<grid, kThreads, 0, s>>>(a);
  else if (C == 64)
    prefill_bounds_wide_kernel<8><<<grid, kThreads, 0, s>>>(a);
  else if (C == 32)
    prefill_bounds_wide_kernel<4><<<grid, kThreads, 0, s>>>(a);
  else if (C == 16)
    prefill_bounds_wide_kernel<2><<<grid, kThreads, 0, s>>>(a);
  else
    prefill_bounds_wide_kernel<1><<<grid, kThreads, 0, s>>>(a);
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

extern "C" int qq_quest_decode_step_locs(const int64_t* req_pool_indices, const int64_t* seq_lens, int bs,
                                         uint8_t* skip_first, const int32_t* req_to_token, int64_t r2t_rows,
                                         int64_t r2t_cols, int64_t r2t_stride, int64_t* device_locs_out,
                                         void* stream) {
  QQ_REQUIRE(bs >= 0 && r2t_rows >= 0 && r2t_cols >= 0 && r2t_stride >= r2t_cols,
             "qq_quest_decode_step_locs: bad arguments (rows %lld, columns %lld, stride %lld)", (long long)r2t_rows,
             (long long)r2t_cols, (long long)r2t_stride);
  if (bs == 0) return QQ_OK;
  decode_step_locs_kernel<<<1, kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      req_pool_indices, seq_lens, bs, skip_first, req_to_token, r2t_rows, r2t_cols, r2t_stride, device_locs_out);
  return check_launch("qq_quest_decode_step_locs");
}

extern "C" int64_t qq_quest_decode_step_sync_bytes(int bs) {
  return bs > 0 ? (int64_t)bs * 32 * (int64_t)sizeof(uint32_t) : 0;
}

extern "C" int qq_quest_decode_step(const int64_t* req_pool_indices, const int64_t* seq_lens, int bs,
                                    uint8_t* skip_first, const int32_t* req_to_token, int64_t r2t_rows,
                                    int64_t r2t_cols, int64_t r2t_stride, int64_t* device_locs_out,
                                    const void* k_base, int64_t k_layer_stride, int k_dtype, int64_t k_rows,
                                    uint16_t* page_k_bounds, uint16_t* running_k_min, uint16_t* running_k_max,
                                    int32_t* running_token_count, int32_t* running_page_idx, int num_layers,
                                    int max_reqs, int max_pages, int kv_heads, int head_dim, int page_size,
                                    int top_k, int avoid_recent_overlap, int32_t* actual_lens,
                                    int32_t* candidate_limit, void* sync, int64_t sync_bytes, void* stream) {
  const char* what = "qq_quest_decode_step";
  QQ_REQUIRE(dtype_ok(k_dtype), "%s: unsupported key dtype %d", what, k_dtype);
  QQ_REQUIRE(bs >= 0 && num_layers > 0 && page_size > 0 && top_k > 0 && r2t_rows >= 0 && r2t_cols >= 0 &&
                 r2t_stride >= r2t_cols,
             "%s: bad arguments (batch %d, layers %d, page %d, top_k %d, table %lld x %lld, stride %lld)", what,
             bs, num_layers, page_size, top_k, (long long)r2t_rows, (long long)r2t_cols, (long long)r2t_stride);
  if (bs == 0) return QQ_OK;
  QQ_REQUIRE(req_pool_indices && seq_lens && skip_first && req_to_token && k_base && page_k_bounds &&
                 running_k_min && running_k_max && running_token_count && running_page_idx && actual_lens &&
                 candidate_limit,
             "%s: null pointer", what);
  QQ_REQUIRE(sync && sync_bytes >= qq_quest_decode_step_sync_bytes(bs), "%s: sync buffer %lld bytes < %lld needed",
             what, (long long)sync_bytes, (long long)qq_quest_decode_step_sync_bytes(bs));
  DecodeStepArgs a;
  a.rpi = req_pool_indices;
  a.seq = seq_lens;
  a.skip = skip_first;
  a.r2t = req_to_token;
  a.r2t_rows = r2t_rows;
  a.r2t_cols = r2t_cols;
  a.r2t_stride = r2t_stride;
  a.locs_out = device_locs_out;
  a.d.k_base = static_cast<const char*>(k_base);
  a.d.k_layer_stride_bytes = k_layer_stride * dtype_size(k_dtype);
  a.d.k_dtype = k_dtype;
  a.d.k_rows = k_rows;
  a.d.reqs = nullptr;
  a.d.locs = nullptr;
  a.d.layer_begin = 0;
  a.d.finalize = 1;
  a.d.bounds = reinterpret_cast<uint32_t*>(page_k_bounds);
  a.d.rmin = running_k_min;
  a.d.rmax = running_k_max;
  a.d.count = running_token_count;
  a.d.page_idx = running_page_idx;
  a.d.R = max_reqs;
  a.d.MP = max_pages;
  a.d.C = kv_heads * head_dim;
  a.d.P = page_size;
  a.n_layers = num_layers;
  a.top_k = top_k;
  a.avoid = avoid_recent_overlap;
  a.actual = actual_lens;
  a.limit = candidate_limit;
  a.count = running_token_count;
  a.page_idx = running_page_idx;
  a.sync = static_cast<uint32_t*>(sync);
  decode_step_kernel<<<dim3(bs, num_layers), kThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
  return check_launch(what);
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
