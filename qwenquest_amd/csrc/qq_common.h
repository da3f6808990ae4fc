// Shared helpers for the qwenquest_amd HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/qwenquest_amd.h"

namespace qq {

constexpr uint16_t kBf16Max = 0x7F7F;  // +3.3895e38 (torch.finfo(bfloat16).max)
constexpr uint16_t kBf16Min = 0xFF7F;  // -3.3895e38
// (min, max) sentinel pair packed little-endian: min in the low half.
constexpr uint32_t kSentinelPair = (uint32_t)kBf16Max | ((uint32_t)kBf16Min << 16);

// Records a message for qq_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

__host__ __device__ inline float bf2f(uint16_t h) {
  return __uint_as_float((uint32_t)h << 16);
}

// float -> bf16, round to nearest even; NaN -> 0x7FC0 (torch's canonical NaN).
__host__ __device__ inline uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Load element `i` of a bf16 or fp32 array as float.
__device__ inline float load_as_float(const void* p, int64_t i, int dtype) {
  if (dtype == QQ_DTYPE_BF16) return bf2f(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

// Load element `i` as bf16 bits (fp32 input is rounded, as `.to(torch.bfloat16)` does).
__device__ inline uint16_t load_as_bf16(const void* p, int64_t i, int dtype) {
  if (dtype == QQ_DTYPE_BF16) return static_cast<const uint16_t*>(p)[i];
  return f2bf(static_cast<const float*>(p)[i]);
}

// torch.minimum / torch.maximum on bf16 values (NaN propagates, ties keep `a`).
__device__ inline uint16_t bmin(uint16_t a, uint16_t b) {
  float fa = bf2f(a), fb = bf2f(b);
  if (fa != fa) return a;
  if (fb != fb) return b;
  return fb < fa ? b : a;
}
__device__ inline uint16_t bmax(uint16_t a, uint16_t b) {
  float fa = bf2f(a), fb = bf2f(b);
  if (fa != fa) return a;
  if (fb != fb) return b;
  return fb > fa ? b : a;
}

// Monotone float -> uint32 key; -0 folds into +0, every NaN ranks highest.
__device__ inline uint32_t orderable(float f) {
  f = f + 0.0f;
  uint32_t u = __float_as_uint(f);
  if (f != f) return 0xFFFFFFFFu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// 64-bit selection key: order-preserving score in the high word, ~page in the
// low word, so "larger key" = higher score, then lower page index.
__device__ inline uint64_t sel_key(uint32_t score_key, int page) {
  return ((uint64_t)score_key << 32) | (uint32_t)(~(uint32_t)page);
}

inline int dtype_size(int dtype) { return dtype == QQ_DTYPE_BF16 ? 2 : 4; }
inline bool dtype_ok(int dtype) { return dtype == QQ_DTYPE_BF16 || dtype == QQ_DTYPE_F32; }

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

}  // namespace qq

#define QQ_REQUIRE(cond, ...)                                  \
  do {                                                         \
    if (!(cond)) return ::qq::set_error(QQ_EINVAL, __VA_ARGS__); \
  } while (0)
