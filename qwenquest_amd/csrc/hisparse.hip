// HiSparse hierarchical KV cache (Quest mode): pinned host tier + per-request
// LRU hot buffer on the GPU.
//
// Reference: src/qwenquest/hisparse/coordinator.py (HiSparseCoordinator).
// Layouts (reference coordinator.py:103-131):
//   device_k/v[layer]  [R*(buf+1), KV, D]; request r owns rows r*(buf+1) + slot,
//                      slot buf is the reserved newest-token slot
//   buffer_tokens      [L, R, buf] int64  position cached by each LRU slot (-1 none)
//   lru_slots          [L, R, buf] int64  slots, least -> most recently used
//   req_to_host_pool   [R, max_ctx] int64 host row of each position (-1 none)
//   host_k/v[layer]    [host_pool+1, KV, D] in pinned host memory, read and
//                      written by the kernels directly over PCIe (zero-copy)
//
// Swap-in, one block of 1024 threads per request (coordinator.py:232-304):
//   fast path seq <= buf: row = base + position;
//   otherwise the newest position maps to the reserved slot; the others are
//   deduplicated by first occurrence (LDS hash table, atomicMin of the entry
//   index); every LRU slot's token is looked up in the table (hits); misses =
//   first occurrences without a hit, ranked in entry order; evictable = LRU
//   entries that are not hits, ranked in LRU order; miss r goes to evictable r;
//   the LRU becomes [evictable[m:], victims, hits]; each entry (duplicates
//   included) reads its position's slot from the table.  Both error conditions
//   of the reference (too few victims, coordinator.py:278-279; a position
//   without host backup, :285-286) are detected before any state is written
//   and reported through a device error word.  A second kernel copies the missed
//   rows host -> device.
#include "qq_quest_dev.h"

namespace qq {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kMaxPerThread = 8;  // buf <= 8192, top_k <= 8192: entries per thread, general form
// the plan kernel's small form (top_k <= 2048, buf <= 4096): 2 entries and 4 LRU slots per
// thread, so that its per-thread state and the miss copy fit without spills
constexpr int kSmallEntries = 2;
constexpr int kSmallSlots = 4;
constexpr int kEmpty = -1;
constexpr int kErrVictims = 1;
constexpr int kErrHostRow = 2;
constexpr int kErrHostOom = 4;

struct SwapArgs {
  const int32_t* positions;
  int64_t pos_stride;
  const int32_t* actual;
  const int64_t* seq;
  const int64_t* rpi;
  int64_t* tokens;  // [R, buf] of this layer
  int64_t* lru;     // [R, buf] of this layer
  const int64_t* r2h;
  int64_t r2h_stride;
  int R, buf, top_k;
  int64_t* rows_out;
  int64_t rows_stride;
  int64_t* copy_dst;  // [bs, top_k]
  int64_t* copy_src;
  int32_t* copy_count;  // [bs]
  unsigned long long* stats;  // hits, misses, fast_path_calls
  int32_t* err;
  int32_t* err_mirror;  // host-mapped words set to 1 per error kind (may be null)
  int table_size;  // power of two >= 2 * top_k (4 * top_k when the LDS holds it)
  // the misses' copy (swap_copy_kernel): host tier rows -> hot buffer rows of this layer
  char* dev_k;
  char* dev_v;
  const char* host_k;
  const char* host_v;
  int64_t row_bytes, dev_rows, host_rows;
  // the step's new K / V rows ([bs] rows of row_bytes, the hot buffer's dtype), written to
  // each request's newest slot by the plan kernel; null: written elsewhere
  const char* new_k;
  const char* new_v;
};

__device__ inline uint32_t slot_hash(int p, int mask) {
  return ((uint32_t)p * 2654435761u >> 7) & (uint32_t)mask;
}

__device__ inline int table_find(const int* keys, int p, int mask) {
  uint32_t h = slot_hash(p, mask);
  for (int probe = 0; probe <= mask; ++probe) {
    const int k = keys[h];
    if (k == p) return (int)h;
    if (k == kEmpty) return -1;
    h = (h + 1) & (uint32_t)mask;
  }
  return -1;
}

// Exclusive block scan of one int per thread; returns the prefix, *total = sum.
__device__ inline int block_scan(int v, int* s_wave, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_wave[wave] = x;
  __syncthreads();
  int wave_base = 0, sum = 0;
  for (int w = 0; w < kPlanWaves; ++w) {
    const int t = s_wave[w];
    if (w < wave) wave_base += t;
    sum += t;
  }
  __syncthreads();
  *total = sum;
  return wave_base + x - v;
}

__device__ __forceinline__ int64_t wave_first(int64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// One round of the miss copy for 1 KiB rows (bf16, KV*D = 512): wave w copies misses
// base + w + NW*i, i < RPW, one 16-byte piece per lane and row.  Every row's indices are
// loaded first, then every row's K and V data, so that no data load waits for more than
// the index loads and all 2 * RPW loads of the wave are in flight at once.  The data
// loads go through a buffer resource per row whose size is 0 for a row that is not
// copied (past the count or out of its buffer): such a load reads zeros without touching
// memory, so every load is unconditional and the row data stays in registers.
template <int NW, int RPW>
__device__ __forceinline__ void copy_miss_round_1k(const SwapArgs& a, const int64_t* dsts, const int64_t* srcs,
                                                   int count, int base, int wave, int lane) {
  int64_t dst[RPW], src[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = base + wave + NW * i;
    dst[i] = r < count ? dsts[r] : -1;
    src[i] = r < count ? srcs[r] : -1;
  }
  bool ok[RPW];
  u32x4_t x[RPW], y[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    dst[i] = wave_first(dst[i]);  // one row per wave: every lane loaded the same index
    src[i] = wave_first(src[i]);
    ok[i] = dst[i] >= 0 && dst[i] < a.dev_rows && src[i] >= 0 && src[i] < a.host_rows;
    const int64_t row = ok[i] ? src[i] : 0;
    const int bytes = ok[i] ? 1024 : 0;
    x[i] = __builtin_amdgcn_raw_buffer_load_b128(
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(a.host_k + row * 1024), (short)0, bytes, 0x00020000),
        lane * 16, 0, 0);
    y[i] = __builtin_amdgcn_raw_buffer_load_b128(
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(a.host_v + row * 1024), (short)0, bytes, 0x00020000),
        lane * 16, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    if (ok[i]) {
      reinterpret_cast<u32x4_t*>(a.dev_k + dst[i] * 1024)[lane] = x[i];
      reinterpret_cast<u32x4_t*>(a.dev_v + dst[i] * 1024)[lane] = y[i];
    }
  }
}

// Exclusive block scan of one uint64 per thread (fields added without carries by the
// caller's choice of widths); returns the prefix, *total = sum.
__device__ inline uint64_t block_scan_u64(uint64_t v, uint64_t* s_wave, uint64_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)x, off, 64);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(x >> 32), off, 64);
    if (lane >= off) x += ((uint64_t)hi << 32) | lo;
  }
  if (lane == 63) s_wave[wave] = x;
  __syncthreads();
  uint64_t wave_base = 0, sum = 0;
  for (int w = 0; w < kPlanWaves; ++w) {
    const uint64_t t = s_wave[w];
    if (w < wave) wave_base += t;
    sum += t;
  }
  __syncthreads();
  *total = sum;
  return wave_base + x - v;
}

template <int KT, int KE>
__global__ __launch_bounds__(kPlanThreads) void swap_plan_kernel(SwapArgs a) {
  extern __shared__ __align__(16) int smem[];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int64_t req = a.rpi[b];
  const int64_t s = a.seq[b];
  const int buf = a.buf;
  const int n = (int)min((int64_t)a.actual[b], min(a.pos_stride, (int64_t)a.top_k));
  int64_t* rows = a.rows_out + (int64_t)b * a.rows_stride;
  const int32_t* pos = a.positions + (int64_t)b * a.pos_stride;
  if (req < 0 || req >= a.R) {
    for (int i = tid; i < a.top_k; i += kPlanThreads) rows[i] = -1;
    if (tid == 0) a.copy_count[b] = 0;
    return;
  }
  const int64_t base_row = req * (int64_t)(buf + 1);
  if (a.new_k && s >= 1) {  // the new token into its newest slot (coordinator.py:217-228)
    const int64_t loc = base_row + min(s - 1, (int64_t)buf);
    const int64_t units = a.row_bytes / 16;
    if (loc < a.dev_rows) {
      for (int64_t u = tid; u < 2 * units; u += kPlanThreads) {
        const bool v = u >= units;
        const int64_t w = v ? u - units : u;
        const uint4 x = reinterpret_cast<const uint4*>((v ? a.new_v : a.new_k) + (int64_t)b * a.row_bytes)[w];
        reinterpret_cast<uint4*>((v ? a.dev_v : a.dev_k) + loc * a.row_bytes)[w] = x;
      }
    }
  }
  if (s <= buf) {  // fast path: the whole sequence is resident, slot == position
    for (int i = tid; i < a.top_k; i += kPlanThreads) rows[i] = i < n ? base_row + pos[i] : -1;
    if (tid == 0) {
      a.copy_count[b] = 0;
      atomicAdd(&a.stats[2], 1ull);
    }
    return;
  }
  const int T = a.table_size, mask = T - 1;
  int* s_key = smem;                 // [T]
  int* s_val = s_key + T;            // [T] first entry index, later the slot
  int* s_vic = s_val + T;            // [top_k] victim slot of miss rank r
  int* s_tok = s_vic + a.top_k;      // [buf] position cached by each slot (-1 none)
  int* s_wave = s_tok + buf;         // [kPlanWaves]
  int* s_flag = s_wave + kPlanWaves; // [1] host-row error
  // [kPlanWaves] 64-bit scan totals, 8-byte aligned after the flag
  uint64_t* s_wave64 = reinterpret_cast<uint64_t*>(s_flag + 1 + ((buf + a.top_k + 1) & 1));
  int64_t* tok = a.tokens + req * (int64_t)buf;
  int64_t* lru = a.lru + req * (int64_t)buf;
  const int E = (buf + kPlanThreads - 1) / kPlanThreads;  // LRU entries per thread (a contiguous run)

  // Every global load that does not depend on another goes out first: the entries'
  // positions (i = tid + k*1024), the LRU order (j = tid*E + e) and every slot's token
  // (t = tid + e*1024); the entries' host rows follow as soon as their positions are in.
  int my_p[KT], my_slot[KE];
  int64_t my_tok[KE], my_host[KT];
#pragma unroll
  for (int k = 0; k < KT; ++k) {
    const int i = tid + k * kPlanThreads;
    my_p[k] = i < n ? pos[i] : -1;
  }
#pragma unroll
  for (int k = 0; k < KE; ++k) {
    const int j = tid * E + k;
    my_slot[k] = (k < E && j < buf) ? (int)lru[j] : -1;
    const int t = tid + k * kPlanThreads;
    my_tok[k] = t < buf ? tok[t] : -1;
  }
#pragma unroll
  for (int k = 0; k < KT; ++k) {
    const int64_t p = my_p[k];
    my_host[k] = (p >= 0 && p < a.r2h_stride) ? a.r2h[req * a.r2h_stride + p] : -1;
  }
  for (int h = tid; h < T; h += kPlanThreads) {
    s_key[h] = kEmpty;
    s_val[h] = 0x7FFFFFFF;
  }
  if (tid == 0) *s_flag = 0;
#pragma unroll
  for (int k = 0; k < KE; ++k) {
    const int t = tid + k * kPlanThreads;
    if (t < buf) s_tok[t] = (my_tok[k] >= 0 && my_tok[k] < 0x7FFFFFFF) ? (int)my_tok[k] : -1;
  }
  lds_barrier();  // LDS-only: the host-row loads stay in flight

  // dedup: insert every non-newest entry, keeping the smallest entry index (first occurrence)
  int my_h[KT];
  bool my_new[KT];
  const int64_t newest_pos = s - 1;
#pragma unroll
  for (int k = 0; k < KT; ++k) {
    const int i = tid + k * kPlanThreads;
    my_h[k] = -1;
    my_new[k] = false;
    if (i < n) {
      const int p = my_p[k];
      my_new[k] = (int64_t)p == newest_pos;
      if (!my_new[k]) {
        uint32_t h = slot_hash(p, mask);
        for (int probe = 0; probe <= mask; ++probe) {
          const int old = atomicCAS(&s_key[h], kEmpty, p);
          if (old == kEmpty || old == p) {
            atomicMin(&s_val[h], i);
            my_h[k] = (int)h;
            break;
          }
          h = (h + 1) & (uint32_t)mask;
        }
      }
    }
  }
  lds_barrier();
  bool my_first[KT];
#pragma unroll
  for (int k = 0; k < KT; ++k) {
    const int i = tid + k * kPlanThreads;
    my_first[k] = i < n && !my_new[k] && my_h[k] >= 0 && s_val[my_h[k]] == i;
  }
  lds_barrier();
  for (int h = tid; h < T; h += kPlanThreads) s_val[h] = -1;  // becomes position -> slot
  lds_barrier();

  // hits: the LRU run j = tid*E + e looks its slot's token up in the table
  bool my_hit[KE];
#pragma unroll
  for (int e = 0; e < KE; ++e) {
    my_hit[e] = false;
    const int slot = my_slot[e];
    const int t = (slot >= 0 && slot < buf) ? s_tok[slot] : -1;
    if (t >= 0) {
      const int h = table_find(s_key, t, mask);
      if (h >= 0) {
        s_val[h] = slot;
        my_hit[e] = true;
      }
    }
  }
  lds_barrier();

  // misses: first occurrences without a hit, ranked in entry order (entry i = tid + k*1024
  // is not contiguous per thread, so the ranks come from a scan per k-round); evictable
  // (non-hit) LRU entries ranked in LRU order; unique entries counted.  The first two
  // rounds, the evictable count and the unique count go through one scan of four 16-bit
  // counters (each total <= 8192, so no field carries into the next); rounds past the
  // second (top_k > 2048) take a scan each.
  const int rounds = (n + kPlanThreads - 1) / kPlanThreads;
  int uniq_local = 0;
  bool miss_k[KT];
#pragma unroll
  for (int k = 0; k < KT; ++k) {
    miss_k[k] = k < rounds && my_first[k] && s_val[my_h[k] >= 0 ? my_h[k] : 0] < 0;
    uniq_local += (k < rounds && my_first[k]) ? 1 : 0;
  }
  int ev_local = 0;
#pragma unroll
  for (int e = 0; e < KE; ++e)
    if (e < E && tid * E + e < buf && !my_hit[e]) ++ev_local;
  uint64_t packed_total;
  const uint64_t packed = block_scan_u64((uint64_t)(miss_k[0] ? 1 : 0) | ((uint64_t)(miss_k[1] ? 1 : 0) << 16) |
                                             ((uint64_t)ev_local << 32) | ((uint64_t)uniq_local << 48),
                                         s_wave64, &packed_total);
  int miss_rank[KT];
  miss_rank[0] = miss_k[0] ? (int)(packed & 0xFFFFu) : -1;
  int num_miss = (int)(packed_total & 0xFFFFu);
  miss_rank[1] = miss_k[1] ? num_miss + (int)((packed >> 16) & 0xFFFFu) : -1;
  num_miss += (int)((packed_total >> 16) & 0xFFFFu);
#pragma unroll
  for (int k = 2; k < KT; ++k) {
    miss_rank[k] = -1;
    if (k >= rounds) continue;  // block-uniform
    int tot;
    const int r = block_scan(miss_k[k] ? 1 : 0, s_wave, &tot);
    miss_rank[k] = miss_k[k] ? num_miss + r : -1;
    num_miss += tot;
  }
  const int ev_base = (int)((packed >> 32) & 0xFFFFu);
  const int n_ev = (int)((packed_total >> 32) & 0xFFFFu);
  const int uniq_total = (int)((packed_total >> 48) & 0xFFFFu);
  if (num_miss > n_ev) {  // coordinator.py:278-279
    if (tid == 0) {
      atomicOr(a.err, kErrVictims);
      if (a.err_mirror) a.err_mirror[0] = 1;
      a.copy_count[b] = 0;
    }
    for (int i = tid; i < a.top_k; i += kPlanThreads) rows[i] = -1;
    return;
  }
  {
    int e_rank = ev_base;
#pragma unroll
    for (int e = 0; e < KE; ++e) {
      if (e < E && tid * E + e < buf && !my_hit[e]) {
        if (e_rank < num_miss) s_vic[e_rank] = my_slot[e];
        ++e_rank;
      }
    }
  }
  lds_barrier();
  // victims: host rows must exist (coordinator.py:284-286), then record the copies
  int64_t* cdst = a.copy_dst + (int64_t)b * a.top_k;
  int64_t* csrc = a.copy_src + (int64_t)b * a.top_k;
#pragma unroll
  for (int k = 0; k < KT; ++k) {
    if (miss_rank[k] >= 0) {
      const int slot = s_vic[miss_rank[k]];
      const int64_t host = my_host[k];
      if (host < 0) atomicOr(s_flag, 1);
      s_val[my_h[k]] = slot;
      cdst[miss_rank[k]] = base_row + slot;
      csrc[miss_rank[k]] = host;
    }
  }
  lds_barrier();
  if (*s_flag) {
    if (tid == 0) {
      atomicOr(a.err, kErrHostRow);
      if (a.err_mirror) a.err_mirror[1] = 1;
      a.copy_count[b] = 0;
    }
    for (int i = tid; i < a.top_k; i += kPlanThreads) rows[i] = -1;
    return;
  }
  // commit: tokens of the victims, new LRU order (coordinator.py:291, 295)
#pragma unroll
  for (int k = 0; k < KT; ++k)
    if (miss_rank[k] >= 0) tok[s_vic[miss_rank[k]]] = my_p[k];
  {
    int e_rank = ev_base, h_rank = min(tid * E, buf) - ev_base;  // hits before this thread's run
#pragma unroll
    for (int e = 0; e < KE; ++e) {
      if (e < E && tid * E + e < buf) {
        int dst;
        if (!my_hit[e]) {
          dst = e_rank >= num_miss ? e_rank - num_miss : (n_ev - num_miss) + e_rank;
          ++e_rank;
        } else {
          dst = n_ev + h_rank;
          ++h_rank;
        }
        lru[dst] = my_slot[e];
      }
    }
  }
  // rows of every entry, duplicates included (coordinator.py:298-300)
#pragma unroll
  for (int k = 0; k < KT; ++k) {
    const int i = tid + k * kPlanThreads;
    if (i < n) rows[i] = my_new[k] ? base_row + buf : base_row + s_val[my_h[k]];
  }
  for (int i = n + tid; i < a.top_k; i += kPlanThreads) rows[i] = -1;
  if (tid == 0) {
    a.copy_count[b] = num_miss;
    atomicAdd(&a.stats[0], (unsigned long long)(uniq_total - num_miss));
    atomicAdd(&a.stats[1], (unsigned long long)num_miss);
  }
}

// Host -> device rows of the planned misses, read over PCIe by the kernel (zero-copy):
// grid (top_k / 64, bs), one block per 64 consecutive misses of a request.  Wave w copies
// misses w, w + 4, ..., w + 60 of its block: with 1 KiB rows all 32 16-byte loads of its
// 16 K and V rows are in flight at once, and the block's 4 waves read neighbouring host
// rows together (the misses of one page are consecutive host rows).  Other row sizes copy
// one row at a time per wave.  Rows outside their buffers are skipped.
constexpr int kCopyRowsPerBlock = 64;
constexpr int kCopyWaves = 4;

__global__ __launch_bounds__(kCopyWaves * 64) void swap_copy_kernel(SwapArgs a) {
  const int b = blockIdx.y;
  const int r0 = blockIdx.x * kCopyRowsPerBlock;
  const int count = min(a.copy_count[b], a.top_k);
  if (r0 >= count) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t* dsts = a.copy_dst + (int64_t)b * a.top_k;
  const int64_t* srcs = a.copy_src + (int64_t)b * a.top_k;
  if (a.row_bytes == 1024) {
    copy_miss_round_1k<kCopyWaves, kCopyRowsPerBlock / kCopyWaves>(a, dsts, srcs, count, r0, wave, lane);
    return;
  }
  const int64_t row_bytes = a.row_bytes, units = row_bytes / 16;
  const int r1 = min(count, r0 + kCopyRowsPerBlock);
  for (int r = r0 + wave; r < r1; r += kCopyWaves) {
    const int64_t d = dsts[r], src = srcs[r];
    if (d < 0 || d >= a.dev_rows || src < 0 || src >= a.host_rows) continue;
    const uint4* hk = reinterpret_cast<const uint4*>(a.host_k + src * row_bytes);
    const uint4* hv = reinterpret_cast<const uint4*>(a.host_v + src * row_bytes);
    uint4* dk = reinterpret_cast<uint4*>(a.dev_k + d * row_bytes);
    uint4* dv = reinterpret_cast<uint4*>(a.dev_v + d * row_bytes);
    for (int64_t u = lane; u < units; u += 64) {
      const uint4 xv = hk[u];
      const uint4 yv = hv[u];
      dk[u] = xv;
      dv[u] = yv;
    }
  }
}

// Row copies for every layer: dst[layer][dst_row(i)] = src[layer][src_row(i)].
// Rows whose index falls outside its buffer are skipped.  Grid-stride: each wave
// moves kCopyRowsPerWave rows of one layer at a time (lane l: 16-byte chunks l,
// l + 64, ... of each row), all their loads before their stores.
constexpr int kCopyRowsPerWave = 4;
__global__ __launch_bounds__(256) void copy_rows_kernel(const char* src, int64_t src_layer_stride,
                                                       int64_t src_rows, const int64_t* src_idx,
                                                       char* dst, int64_t dst_layer_stride,
                                                       int64_t dst_rows, const int64_t* dst_idx,
                                                       int n, int n_layers, int64_t row_bytes) {
  constexpr int R = kCopyRowsPerWave;
  const int lane = threadIdx.x & 63;
  const int64_t per_layer = ((int64_t)n + R - 1) / R;
  const int64_t groups = per_layer * n_layers;
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x / 64);
  const int64_t chunks = row_bytes / 16;
  for (int64_t g = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); g < groups; g += waves) {
    const int64_t layer = g / per_layer;
    const int i0 = (int)(g - layer * per_layer) * R;
    const uint4* sp[R];
    uint4* dp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = i0 + r;
      const int64_t s = i < n ? src_idx[i] : -1, d = i < n ? dst_idx[i] : -1;
      const bool ok = s >= 0 && s < src_rows && d >= 0 && d < dst_rows;
      sp[r] = ok ? reinterpret_cast<const uint4*>(src + layer * src_layer_stride + s * row_bytes) : nullptr;
      dp[r] = ok ? reinterpret_cast<uint4*>(dst + layer * dst_layer_stride + d * row_bytes) : nullptr;
    }
    for (int64_t c = lane; c < chunks; c += 64) {
      uint4 v[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (sp[r]) v[r] = sp[r][c];
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (dp[r]) dp[r][c] = v[r];
    }
  }
}

// Whether `p` is host memory (pinned, addressed by the device over PCIe).
static bool is_host_memory(const void* p) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();  // an unknown pointer: not host memory HIP knows of
    return false;
  }
  return attr.type == hipMemoryTypeHost;
}

// Per-request bookkeeping: mode 0 = admit (tokens[s] = s, lru[s] = s, host rows of
// positions [0, n)), mode 1 = release (tokens = -1, lru[s] = s, host rows = -1).
__global__ __launch_bounds__(256) void request_state_kernel(int64_t* tokens, int64_t* lru, int L, int R,
                                                          int buf, int64_t* r2h, int64_t r2h_stride,
                                                          int req, const int64_t* host_idx, int64_t n,
                                                          int mode) {
  const int layer = blockIdx.y;
  const int64_t off = ((int64_t)layer * R + req) * buf;
  for (int s = blockIdx.x * 256 + threadIdx.x; s < buf; s += gridDim.x * 256) {
    tokens[off + s] = mode == 0 ? (int64_t)s : -1;
    lru[off + s] = s;
  }
  if (layer == 0) {
    int64_t* row = r2h + (int64_t)req * r2h_stride;
    for (int64_t p = blockIdx.x * 256 + threadIdx.x; p < r2h_stride; p += gridDim.x * 256)
      row[p] = (mode == 0 && p < n) ? host_idx[p] : -1;
  }
}

// The host tier's free list on the device (TokenToKVPoolAllocator semantics,
// memory.py:47-70): ring[(head + i) % cap] for i < count are the free rows in
// order; alloc takes from the head, free appends at the tail.  state = {head, count}.

// alloc(n) for an admission: out[i] = the i-th free row; QQ_ERUNTIME-style error
// bit 4 (nothing taken) when fewer than n are free.
__global__ __launch_bounds__(256) void ring_alloc_kernel(const int64_t* ring, int64_t* state, int64_t cap,
                                                       int64_t n, int64_t* out, int32_t* err,
                                                       int32_t* err_mirror) {
  const int64_t head = state[0], count = state[1];
  __syncthreads();
  if (n > count) {
    if (threadIdx.x == 0) {
      atomicOr(err, kErrHostOom);
      if (err_mirror) err_mirror[2] = 1;
    }
    for (int64_t i = threadIdx.x; i < n; i += 256) out[i] = -1;
    return;
  }
  for (int64_t i = threadIdx.x; i < n; i += 256) out[i] = ring[(head + i) % cap];
  __syncthreads();
  if (threadIdx.x == 0) {
    state[0] = (head + n) % cap;
    state[1] = count - n;
  }
}

// free(rows): rows[i] > 0 are appended at the tail in order (one block; block scan).
__global__ __launch_bounds__(256) void ring_free_kernel(int64_t* ring, int64_t* state, int64_t cap,
                                                      const int64_t* rows, int64_t n) {
  __shared__ int s_wave[4];
  __shared__ int64_t s_base;  // free rows so far: the next one goes to ring[(head + s_base) % cap]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) s_base = state[1];
  const int64_t head = state[0];
  __syncthreads();
  for (int64_t i0 = 0; i0 < n; i0 += 256) {
    const int64_t i = i0 + tid;
    const int64_t r = i < n ? rows[i] : 0;
    const int keep = r > 0 ? 1 : 0;
    int x = keep;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    if (lane == 63) s_wave[wave] = x;
    __syncthreads();
    int wbase = 0, tot = 0;
    for (int w = 0; w < 4; ++w) {
      wbase += w < wave ? s_wave[w] : 0;
      tot += s_wave[w];
    }
    const int64_t base = s_base;
    const int64_t at = base + wbase + x - 1;
    if (keep && at < cap) ring[(head + at) % cap] = r;  // more rows than the pool holds: dropped
    __syncthreads();
    if (tid == 0) s_base = base + tot;
    __syncthreads();
  }
  if (tid == 0) state[1] = min(s_base, cap);
}

// The eager backup of one decode step (coordinator.py:183-212) without the host: for
// batch entry b (request rpi[b], previous position seq[b] - 2), skip and clear it when
// its request's skip flag is set (first step after admission); otherwise take the next
// free host row in batch order, record req_to_host_pool[req, seq - 2] and the device
// row of the previous token.  host_idx[b] / dev_rows[b] are -1 for skipped entries (the
// fold and the copies skip them).  Too few free rows: error bit 4, nothing taken
// (host_idx[b] = -1, so nothing is copied), while dev_rows[b] keeps the fold going.
__global__ __launch_bounds__(256) void backup_step_kernel(const int64_t* rpi, const int64_t* seq, int bs,
                                                        uint8_t* skip, int buf, int R, int64_t* r2h,
                                                        int64_t r2h_stride, const int64_t* ring, int64_t* state,
                                                        int64_t cap, int64_t* host_idx, int64_t* dev_rows,
                                                        int32_t* err, int32_t* err_mirror) {
  __shared__ int s_wave[4];
  __shared__ int s_total;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t head = state[0], count = state[1];
  // pass 1: which entries back up (the flags are read before any is cleared)
  int total = 0;
  for (int b0 = 0; b0 < bs; b0 += 256) {
    const int b = b0 + tid;
    int want = 0;
    if (b < bs) {
      const int64_t req = rpi[b];
      const int64_t prev = seq[b] - 2;
      want = req >= 0 && req < R && !skip[req] && prev >= 0 && prev < r2h_stride ? 1 : 0;
    }
    int x = want;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    if (lane == 63) s_wave[wave] = x;
    __syncthreads();
    for (int w = 0; w < 4; ++w) total += s_wave[w];
    __syncthreads();
  }
  if (tid == 0) s_total = total;
  __syncthreads();
  const bool oom = (int64_t)s_total > count;
  if (oom && tid == 0) {
    atomicOr(err, kErrHostOom);
    if (err_mirror) err_mirror[2] = 1;
  }
  // pass 2: ranks in batch order, rows, bookkeeping
  int base = 0;
  for (int b0 = 0; b0 < bs; b0 += 256) {
    const int b = b0 + tid;
    int want = 0;
    int64_t req = -1, prev = -1;
    if (b < bs) {
      req = rpi[b];
      prev = seq[b] - 2;
      want = req >= 0 && req < R && !skip[req] && prev >= 0 && prev < r2h_stride ? 1 : 0;
    }
    int x = want;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    if (lane == 63) s_wave[wave] = x;
    __syncthreads();
    int wbase = 0, tot = 0;
    for (int w = 0; w < 4; ++w) {
      wbase += w < wave ? s_wave[w] : 0;
      tot += s_wave[w];
    }
    if (b < bs) {
      // the fold takes every entry that wanted a backup, also when the host pool is
      // exhausted: the reference folds first and only then fails in alloc
      dev_rows[b] = want ? req * (int64_t)(buf + 1) + min(prev, (int64_t)buf) : -1;
      if (want && !oom) {
        const int64_t h = ring[(head + base + wbase + x - 1) % cap];
        host_idx[b] = h;
        r2h[req * r2h_stride + prev] = h;
      } else {
        host_idx[b] = -1;
      }
    }
    base += tot;
    __syncthreads();
  }
  // clear the skip flags of this batch's requests (after every read of them above)
  for (int b = tid; b < bs; b += 256) {
    const int64_t req = rpi[b];
    if (req >= 0 && req < R) skip[req] = 0;
  }
  if (tid == 0 && !oom) {
    state[0] = (head + s_total) % cap;
    state[1] = count - s_total;
  }
}

// write_new_token (coordinator.py:217-228): slot min(seq-1, buf) of each request.
template <typename Dst, typename Src>
__global__ __launch_bounds__(256) void write_new_kernel(Dst* k_dst, Dst* v_dst, const Src* k_src,
                                                      const Src* v_src, const int64_t* rpi,
                                                      const int64_t* seq, int buf, int R,
                                                      int64_t row_elems) {
  const int b = blockIdx.x;
  const int64_t req = rpi[b];
  if (req < 0 || req >= R) return;
  const int64_t loc = req * (int64_t)(buf + 1) + min(seq[b] - 1, (int64_t)buf);
  for (int64_t e = threadIdx.x; e < row_elems; e += 256) {
    if constexpr (sizeof(Dst) == sizeof(Src)) {
      k_dst[loc * row_elems + e] = k_src[(int64_t)b * row_elems + e];
      v_dst[loc * row_elems + e] = v_src[(int64_t)b * row_elems + e];
    } else if constexpr (sizeof(Dst) == 2) {
      k_dst[loc * row_elems + e] = f2bf((float)k_src[(int64_t)b * row_elems + e]);
      v_dst[loc * row_elems + e] = f2bf((float)v_src[(int64_t)b * row_elems + e]);
    } else {
      k_dst[loc * row_elems + e] = bf2f(k_src[(int64_t)b * row_elems + e]);
      v_dst[loc * row_elems + e] = bf2f(v_src[(int64_t)b * row_elems + e]);
    }
  }
}

}  // namespace
}  // namespace qq

using namespace qq;

// The plan kernel's LDS above the 64 KiB default (large buffers): opted in once per device.
static constexpr int kPlanMaxLds = 160 * 1024;
static int plan_lds_opt_in() {
  static bool opted[64] = {false};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return set_error(QQ_EHIP, "qq_hisparse_swap_in: no device");
  if (!opted[dev]) {
    const void* kernels[2] = {reinterpret_cast<const void*>(&swap_plan_kernel<kSmallEntries, kSmallSlots>),
                              reinterpret_cast<const void*>(&swap_plan_kernel<kMaxPerThread, kMaxPerThread>)};
    for (const void* k : kernels) {
      const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kPlanMaxLds);
      if (e != hipSuccess) return set_error(QQ_EHIP, "qq_hisparse_swap_in: LDS opt-in failed: %s", hipGetErrorString(e));
    }
    opted[dev] = true;
  }
  return QQ_OK;
}

// The swap-in of one layer: the plan, then (copy) the misses' host -> device copy.
static int swap_in(const char* what, bool copy, const int32_t* positions, int64_t positions_stride,
                   const int32_t* actual_lens, const int64_t* seq_lens, const int64_t* req_pool_indices, int bs,
                   int max_reqs, int device_buffer_size, int top_k, int64_t* buffer_tokens_layer,
                   int64_t* lru_slots_layer, const int64_t* req_to_host_pool, int64_t max_context_len,
                   void* device_k_layer, void* device_v_layer, const void* host_k_layer, const void* host_v_layer,
                   int64_t row_bytes, int64_t host_rows, int64_t* rows_out, int64_t* copy_dst, int64_t* copy_src,
                   int32_t* copy_count, uint64_t* stats, int32_t* error_flags, int32_t* error_mirror,
                   const void* new_k, const void* new_v, void* stream) {
  QQ_REQUIRE(bs >= 0 && max_reqs > 0 && device_buffer_size >= top_k && top_k > 0,
             "%s: bad sizes (buf %d, top_k %d)", what, device_buffer_size, top_k);
  QQ_REQUIRE(device_buffer_size <= kMaxPerThread * kPlanThreads && top_k <= kMaxPerThread * kPlanThreads,
             "%s: buffer %d / top_k %d exceed %d", what, device_buffer_size, top_k,
             kMaxPerThread * kPlanThreads);
  QQ_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0, "%s: row bytes %lld must be a multiple of 16",
             what, (long long)row_bytes);
  QQ_REQUIRE(positions_stride >= top_k, "%s: positions stride < top_k", what);
  if (bs == 0) return QQ_OK;
  // the dedup table: a power of two >= 4 * top_k when the LDS holds it (short probe
  // chains for the hit lookups), else >= 2 * top_k
  auto plan_smem = [&](int t) {
    return (size_t)(2 * t + top_k + device_buffer_size + kPlanWaves + 2) * sizeof(int) + kPlanWaves * sizeof(uint64_t);
  };
  int T = 1;
  while (T < 4 * top_k) T <<= 1;
  if (plan_smem(T) > (size_t)kPlanMaxLds) T >>= 1;
  const size_t smem = plan_smem(T);
  QQ_REQUIRE(smem <= kPlanMaxLds, "%s: top_k %d with a %d-slot buffer needs %zu bytes of LDS (at most %d)", what,
             top_k, device_buffer_size, smem, kPlanMaxLds);
  if (smem > 64 * 1024 && plan_lds_opt_in() != QQ_OK) return QQ_EHIP;
  SwapArgs a;
  a.positions = positions;
  a.pos_stride = positions_stride;
  a.actual = actual_lens;
  a.seq = seq_lens;
  a.rpi = req_pool_indices;
  a.tokens = buffer_tokens_layer;
  a.lru = lru_slots_layer;
  a.r2h = req_to_host_pool;
  a.r2h_stride = max_context_len;
  a.R = max_reqs;
  a.buf = device_buffer_size;
  a.top_k = top_k;
  a.rows_out = rows_out;
  a.rows_stride = top_k;
  a.copy_dst = copy_dst;
  a.copy_src = copy_src;
  a.copy_count = copy_count;
  a.stats = reinterpret_cast<unsigned long long*>(stats);
  a.err = error_flags;
  a.err_mirror = error_mirror;
  a.table_size = T;
  a.dev_k = static_cast<char*>(device_k_layer);
  a.dev_v = static_cast<char*>(device_v_layer);
  a.host_k = static_cast<const char*>(host_k_layer);
  a.host_v = static_cast<const char*>(host_v_layer);
  a.row_bytes = row_bytes;
  a.dev_rows = (int64_t)max_reqs * (device_buffer_size + 1);
  a.host_rows = host_rows;
  a.new_k = static_cast<const char*>(new_k);
  a.new_v = static_cast<const char*>(new_v);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (top_k <= kSmallEntries * kPlanThreads && device_buffer_size <= kSmallSlots * kPlanThreads)
    swap_plan_kernel<kSmallEntries, kSmallSlots><<<bs, kPlanThreads, smem, s>>>(a);
  else
    swap_plan_kernel<kMaxPerThread, kMaxPerThread><<<bs, kPlanThreads, smem, s>>>(a);
  if (copy)
    swap_copy_kernel<<<dim3((top_k + kCopyRowsPerBlock - 1) / kCopyRowsPerBlock, bs), kCopyWaves * 64, 0, s>>>(a);
  return check_launch(what);
}

extern "C" int qq_hisparse_swap_in(const int32_t* positions, int64_t positions_stride,
                                   const int32_t* actual_lens, const int64_t* seq_lens,
                                   const int64_t* req_pool_indices, int bs, int max_reqs,
                                   int device_buffer_size, int top_k, int64_t* buffer_tokens_layer,
                                   int64_t* lru_slots_layer, const int64_t* req_to_host_pool,
                                   int64_t max_context_len, void* device_k_layer,
                                   void* device_v_layer, const void* host_k_layer,
                                   const void* host_v_layer, int64_t row_bytes,
                                   int64_t host_rows, int64_t* rows_out, int64_t* copy_dst,
                                   int64_t* copy_src, int32_t* copy_count, uint64_t* stats,
                                   int32_t* error_flags, int32_t* error_mirror, const void* new_k,
                                   const void* new_v, void* stream) {
  QQ_REQUIRE((new_k == nullptr) == (new_v == nullptr), "qq_hisparse_swap_in: new_k and new_v go together");
  return swap_in("qq_hisparse_swap_in", true, positions, positions_stride, actual_lens, seq_lens, req_pool_indices,
                 bs, max_reqs, device_buffer_size, top_k, buffer_tokens_layer, lru_slots_layer, req_to_host_pool,
                 max_context_len, device_k_layer, device_v_layer, host_k_layer, host_v_layer, row_bytes, host_rows,
                 rows_out, copy_dst, copy_src, copy_count, stats, error_flags, error_mirror, new_k, new_v, stream);
}

extern "C" int qq_hisparse_swap_plan(const int32_t* positions, int64_t positions_stride,
                                     const int32_t* actual_lens, const int64_t* seq_lens,
                                     const int64_t* req_pool_indices, int bs, int max_reqs,
                                     int device_buffer_size, int top_k, int64_t* buffer_tokens_layer,
                                     int64_t* lru_slots_layer, const int64_t* req_to_host_pool,
                                     int64_t max_context_len, int64_t* rows_out, int64_t* copy_dst,
                                     int64_t* copy_src, int32_t* copy_count, uint64_t* stats,
                                     int32_t* error_flags, int32_t* error_mirror, void* stream) {
  return swap_in("qq_hisparse_swap_plan", false, positions, positions_stride, actual_lens, seq_lens,
                 req_pool_indices, bs, max_reqs, device_buffer_size, top_k, buffer_tokens_layer, lru_slots_layer,
                 req_to_host_pool, max_context_len, nullptr, nullptr, nullptr, nullptr, 16, 0, rows_out, copy_dst,
                 copy_src, copy_count, stats, error_flags, error_mirror, nullptr, nullptr, stream);
}

extern "C" int qq_copy_rows(const void* src, int64_t src_layer_stride_bytes, int64_t src_rows,
                            const int64_t* src_idx, void* dst, int64_t dst_layer_stride_bytes,
                            int64_t dst_rows, const int64_t* dst_idx, int n, int n_layers,
                            int64_t row_bytes, void* stream) {
  QQ_REQUIRE(n >= 0 && n_layers > 0 && row_bytes > 0 && row_bytes % 16 == 0,
             "qq_copy_rows: bad sizes");
  if (n == 0) return QQ_OK;
  // Device copies: up to 1024 blocks of 4 waves (every CU busy, the copy at HBM rate).
  // A large copy to or from pinned host memory is bound by PCIe, which 64 such blocks
  // saturate (measured device -> host: 55 GB/s with 64 blocks or more); it then stays
  // at 64 blocks, so kernels of other streams keep the rest of the chip while it runs.
  const int64_t groups = ((int64_t)n + kCopyRowsPerWave - 1) / kCopyRowsPerWave * n_layers;
  int64_t blocks = std::min<int64_t>((groups + 3) / 4, 1024);
  if (blocks > 64 && groups >= 4096 && (is_host_memory(dst) || is_host_memory(src))) blocks = 64;
  copy_rows_kernel<<<(int)blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const char*>(src), src_layer_stride_bytes, src_rows, src_idx,
      static_cast<char*>(dst), dst_layer_stride_bytes, dst_rows, dst_idx, n, n_layers, row_bytes);
  return check_launch("qq_copy_rows");
}

extern "C" int qq_hisparse_request_state(int64_t* buffer_tokens, int64_t* lru_slots, int num_layers,
                                         int max_reqs, int device_buffer_size,
                                         int64_t* req_to_host_pool, int64_t max_context_len,
                                         int req, const int64_t* host_idx, int64_t n, int release,
                                         void* stream) {
  QQ_REQUIRE(req >= 0 && req < max_reqs && num_layers > 0 && device_buffer_size > 0,
             "qq_hisparse_request_state: bad arguments");
  QQ_REQUIRE(release || n == 0 || host_idx, "qq_hisparse_request_state: host rows missing");
  QQ_REQUIRE(n <= max_context_len, "qq_hisparse_request_state: %lld positions exceed %lld",
             (long long)n, (long long)max_context_len);
  const int blocks = max(1, min(ceil_div(max((int64_t)device_buffer_size, max_context_len), 256), 512));
  request_state_kernel<<<dim3(blocks, num_layers), 256, 0, static_cast<hipStream_t>(stream)>>>(
      buffer_tokens, lru_slots, num_layers, max_reqs, device_buffer_size, req_to_host_pool,
      max_context_len, req, host_idx, n, release ? 1 : 0);
  return check_launch("qq_hisparse_request_state");
}

extern "C" int qq_hisparse_backup_step(const int64_t* req_pool_indices, const int64_t* seq_lens, int bs,
                                       uint8_t* skip_flags, int device_buffer_size, int max_reqs,
                                       int64_t* req_to_host_pool, int64_t max_context_len, const int64_t* free_ring,
                                       int64_t* free_state, int64_t free_cap, int64_t* host_idx,
                                       int64_t* device_rows, int32_t* error_flags, int32_t* error_mirror,
                                       void* stream) {
  QQ_REQUIRE(bs >= 0 && device_buffer_size > 0 && max_reqs > 0 && free_cap > 0,
             "qq_hisparse_backup_step: bad arguments");
  if (bs == 0) return QQ_OK;
  QQ_REQUIRE(req_pool_indices && seq_lens && skip_flags && req_to_host_pool && free_ring && free_state && host_idx &&
                 device_rows && error_flags,
             "qq_hisparse_backup_step: null pointer");
  backup_step_kernel<<<1, 256, 0, static_cast<hipStream_t>(stream)>>>(
      req_pool_indices, seq_lens, bs, skip_flags, device_buffer_size, max_reqs, req_to_host_pool, max_context_len,
      free_ring, free_state, free_cap, host_idx, device_rows, error_flags, error_mirror);
  return check_launch("qq_hisparse_backup_step");
}

extern "C" int qq_hisparse_ring_alloc(const int64_t* free_ring, int64_t* free_state, int64_t free_cap, int64_t n,
                                      int64_t* out, int32_t* error_flags, int32_t* error_mirror, void* stream) {
  QQ_REQUIRE(n >= 0 && free_cap > 0, "qq_hisparse_ring_alloc: bad sizes");
  if (n == 0) return QQ_OK;
  QQ_REQUIRE(free_ring && free_state && out && error_flags, "qq_hisparse_ring_alloc: null pointer");
  ring_alloc_kernel<<<1, 256, 0, static_cast<hipStream_t>(stream)>>>(free_ring, free_state, free_cap, n, out,
                                                                     error_flags, error_mirror);
  return check_launch("qq_hisparse_ring_alloc");
}

extern "C" int qq_hisparse_ring_free(int64_t* free_ring, int64_t* free_state, int64_t free_cap, const int64_t* rows,
                                     int64_t n, void* stream) {
  QQ_REQUIRE(n >= 0 && free_cap > 0, "qq_hisparse_ring_free: bad sizes");
  if (n == 0) return QQ_OK;
  QQ_REQUIRE(free_ring && free_state && rows, "qq_hisparse_ring_free: null pointer");
  ring_free_kernel<<<1, 256, 0, static_cast<hipStream_t>(stream)>>>(free_ring, free_state, free_cap, rows, n);
  return check_launch("qq_hisparse_ring_free");
}

extern "C" int qq_hisparse_write_new_token(void* device_k_layer, void* device_v_layer,
                                           int buf_dtype, const void* k, const void* v,
                                           int src_dtype, const int64_t* req_pool_indices,
                                           const int64_t* seq_lens, int bs,
                                           int device_buffer_size, int max_reqs,
                                           int64_t row_elems, void* stream) {
  QQ_REQUIRE(dtype_ok(buf_dtype) && dtype_ok(src_dtype), "qq_hisparse_write_new_token: dtype");
  QQ_REQUIRE(bs >= 0 && row_elems > 0, "qq_hisparse_write_new_token: bad sizes");
  if (bs == 0) return QQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (buf_dtype == QQ_DTYPE_BF16 && src_dtype == QQ_DTYPE_BF16)
    write_new_kernel<uint16_t, uint16_t><<<bs, 256, 0, s>>>(
        (uint16_t*)device_k_layer, (uint16_t*)device_v_layer, (const uint16_t*)k,
        (const uint16_t*)v, req_pool_indices, seq_lens, device_buffer_size, max_reqs, row_elems);
  else if (buf_dtype == QQ_DTYPE_F32 && src_dtype == QQ_DTYPE_F32)
    write_new_kernel<float, float><<<bs, 256, 0, s>>>(
        (float*)device_k_layer, (float*)device_v_layer, (const float*)k, (const float*)v,
        req_pool_indices, seq_lens, device_buffer_size, max_reqs, row_elems);
  else if (buf_dtype == QQ_DTYPE_BF16)
    write_new_kernel<uint16_t, float><<<bs, 256, 0, s>>>(
        (uint16_t*)device_k_layer, (uint16_t*)device_v_layer, (const float*)k, (const float*)v,
        req_pool_indices, seq_lens, device_buffer_size, max_reqs, row_elems);
  else
    write_new_kernel<float, uint16_t><<<bs, 256, 0, s>>>(
        (float*)device_k_layer, (float*)device_v_layer, (const uint16_t*)k, (const uint16_t*)v,
        req_pool_indices, seq_lens, device_buffer_size, max_reqs, row_elems);
  return check_launch("qq_hisparse_write_new_token");
}

// The host tier's pinned memory at its exact size (the reference's host_k / host_v,
// torch.zeros on the host device, coordinator.py:104-110): hipHostMalloc with the
// default flags (pinned, mapped into the device's address space), contents undefined.
extern "C" int qq_host_alloc(int64_t bytes, void** host_ptr) {
  QQ_REQUIRE(bytes > 0 && host_ptr, "qq_host_alloc: bad arguments");
  *host_ptr = nullptr;
  const hipError_t e = hipHostMalloc(host_ptr, (size_t)bytes, hipHostMallocDefault);
  if (e != hipSuccess || !*host_ptr) {
    (void)hipGetLastError();
    *host_ptr = nullptr;
    return set_error(QQ_EHIP, "qq_host_alloc: hipHostMalloc of %lld bytes failed: %s", (long long)bytes,
                     hipGetErrorString(e));
  }
  return QQ_OK;
}

extern "C" int qq_host_free(void* host_ptr) {
  if (!host_ptr) return QQ_OK;
  const hipError_t e = hipHostFree(host_ptr);
  if (e != hipSuccess) return set_error(QQ_EHIP, "qq_host_free: %s", hipGetErrorString(e));
  return QQ_OK;
}

extern "C" int qq_host_device_pointer(void* host_ptr, void** device_ptr) {
  QQ_REQUIRE(host_ptr && device_ptr, "qq_host_device_pointer: null pointer");
  const hipError_t e = hipHostGetDevicePointer(device_ptr, host_ptr, 0);
  if (e != hipSuccess)
    return set_error(QQ_EHIP, "hipHostGetDevicePointer: %s (is the memory pinned?)",
                     hipGetErrorString(e));
  return QQ_OK;
}
