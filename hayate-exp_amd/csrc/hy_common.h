// Shared device helpers and host-side error plumbing for libhayate_attn.
// Target: gfx950 (CDNA4), wave64.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hayate_attn.h"

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local message, negative return codes).
// ---------------------------------------------------------------------------
namespace hy {

void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Checks the launch status of the kernels just enqueued.
int launch_status(const char *what);

}  // namespace hy

#define HY_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      hy::set_error(__VA_ARGS__);      \
      return HY_EINVAL;                \
    }                                  \
  } while (0)

#define HY_REQUIRE_SUPPORTED(cond, ...) \
  do {                                  \
    if (!(cond)) {                      \
      hy::set_error(__VA_ARGS__);       \
      return HY_EUNSUPPORTED;           \
    }                                   \
  } while (0)

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
namespace hy {

constexpr int kHeadDim = 128;  // Qwen3 head_dim; the kernels are built for it.
constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// bf16 stored as raw uint16; widening is exact.
__device__ __forceinline__ float bf16_lo(uint32_t w) {
  return __uint_as_float(w << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t w) {
  return __uint_as_float(w & 0xffff0000u);
}

// fp32 -> bf16 round-to-nearest-even by gfx950's v_cvt_pk_bf16_f32. For
// every non-NaN input (all 2^32 fp32 patterns compared on MI355X) the result
// is the one torch's c10::BFloat16 conversion gives, subnormals and
// infinities included; a NaN becomes a quiet NaN that keeps its sign
// (torch: 0x7fc0 for both signs).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  const bf16x2_t h = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// 16-byte global load / store of 8 bf16 values.
__device__ __forceinline__ u32x4 load16(const void *p) {
  return *reinterpret_cast<const u32x4 *>(p);
}
__device__ __forceinline__ void store16(void *p, u32x4 v) {
  *reinterpret_cast<u32x4 *>(p) = v;
}
// Streaming 16-byte load (nontemporal: the line is not kept in the caches).
// For data read exactly once per launch, such as the K/V rows of a decode
// step; MI355X sustains about 10% more HBM read bandwidth with it.
__device__ __forceinline__ u32x4 load16_stream(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// Broadcast lane `src` of every 16-lane row to the whole row (DPP
// row_newbcast, gfx90a and later).
template <int src>
__device__ __forceinline__ float row_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      0, __float_as_int(x), 0x150 + src, 0xf, 0xf, false));
}

// Sum / max over the 16 lanes of a row (xor butterfly).
__device__ __forceinline__ float row16_sum(float x) {
  x += __shfl_xor(x, 8, 16);
  x += __shfl_xor(x, 4, 16);
  x += __shfl_xor(x, 2, 16);
  x += __shfl_xor(x, 1, 16);
  return x;
}

// Sequence and position of packed token `tok`: the sequence is the last
// index b with q_start[b] <= tok (cumulative query lengths q_start[0..n]),
// the position cache_lens[b] + tok - q_start[b]. tok is wave-uniform and
// below q_start[num_seqs]; every lane of the wave must be active (the
// search spreads candidates over the 64 lanes and reads the result with a
// ballot). Each round narrows [lo, lo + n) to one of 64 buckets with one
// vector load, so up to 64 sequences take a single round trip, where a
// binary search on scalar loads waits for log2(num_seqs) dependent ones.
// Indexes are clamped into [lo, lo + n), so every load stays in bounds.
struct TokenPos {
  int seq, pos;
};
__device__ __forceinline__ TokenPos locate_token(const int32_t *__restrict__ q_start,
                                                 const int32_t *__restrict__ cache_lens,
                                                 int num_seqs, int tok) {
  const int lane = static_cast<int>(threadIdx.x & (kWave - 1));
  int lo = 0, n = num_seqs;  // q_start[lo] <= tok < q_start[lo + n]
  while (n > kWave) {
    const int step = (n + kWave - 1) / kWave;
    const int idx = lo + lane * step;
    const bool ok = idx < lo + n && q_start[min(idx, lo + n - 1)] <= tok;
    const uint64_t m = __ballot(ok);  // lane 0 (idx = lo) always holds
    const int j = 63 - __clzll(static_cast<long long>(m));
    const int nlo = lo + j * step;
    n = min(step, lo + n - nlo);
    lo = nlo;
  }
  const int idx = lo + min(lane, n - 1);
  const int qs = q_start[idx];
  const int cl = cache_lens[idx];
  const uint64_t m = __ballot(lane < n && qs <= tok);
  const int j = 63 - __clzll(static_cast<long long>(m));
  const int q_row = __builtin_amdgcn_readlane(qs, j);
  const int cache = __builtin_amdgcn_readlane(cl, j);
  return {lo + j, cache + tok - q_row};
}

}  // namespace hy
