// Paged chunked-prefill causal attention on bf16 MFMA (gfx950).
//
// Grid: (kv head, prefill item); heads vary fastest, so the dispatcher walks
// items in the planner's longest-first order and, with 8 kv heads on the 8
// XCDs, every workgroup of one kv head lands on the same XCD (its L2 holds
// that head's K/V pages for all query tiles of the request). An item is a
// tile of kPrefillRows / G query tokens of one sequence; with its G query
// heads that is kPrefillRows (token, head) rows (prefill_shape.h), all
// reading the same K/V rows (GQA), over the key range [kv_begin, kv_end) of
// one split. Two 128-row workgroups share a CU, so one's prologue and
// epilogue overlap the other's main loop.
//
// Eight waves of 32 rows, two waves per SIMD: while one wave of a SIMD runs
// its softmax on the VALU the other one keeps the matrix core busy (a wave
// cannot overlap its own exp/fma work with its MFMAs). Row r = 32 w + c is
// token q_begin + r / G, head kv_head * G + r % G, so a wave spans 32 / G
// consecutive tokens and the causal diagonal cuts few of its key blocks.
//
// v_mfma_f32_32x32x16_bf16, transposed formulation (lane l, c = l % 32,
// h = l / 32):
//   S^T = K Q^T   A = K (32 keys x 16 dims) from LDS (one 16-byte read per
//                 lane, 272-byte rows: conflict-free); B = Q^T held in
//                 registers. Lane (c, h) ends with row c's scores for keys
//                 8 (i / 4) + 4 h + i % 4, i < 16, of the 32-key block.
//   softmax       per row: the two lanes of a row differ only in h; the
//                 row max and sum cross halves with v_permlane32_swap.
//   O^T += V^T P^T  B = P^T: the first (last) eight of the lane's scores
//                 are row c's probabilities for MFMA k index 8 h + j once k
//                 stands for key 16 kh + (j < 4 ? 4 h + j : 8 + 4 h + j - 4);
//                 A = V^T from LDS with ds_read_b64_tr_b16, which hands lane
//                 r of a 16-lane group four consecutive keys of dim r. One
//                 read instruction serves 32 lanes (four rows x 64 bytes)
//                 per LDS cycle; a 320-byte row pitch (80 dwords, 16 mod 64
//                 banks) puts those four rows on disjoint banks.
// K/V tiles of KEYS keys are double buffered in LDS: the next tile is loaded
// into registers while the current one is computed, then stored, then one
// barrier. The softmax rescales lazily: the exponent base of a row only
// moves when its max grows by more than 2^8, so the accumulators are rarely
// touched by VALU. Key blocks past the causal limit of every row of a wave
// are skipped by that wave.
// Rows at or past kv_end are filled from the last valid key, so masked
// scores never meet NaN bits of unwritten rows.
//
// A split whose item has slot >= 0 writes an fp32 partial (unnormalised
// O^T, row max in the exp2 domain, row sum) to the workspace;
// prefill_merge_kernel (hy_paged_prefill_merge) combines the splits of a
// query tile afterwards.
//
// Item key ranges start at multiples of 32 keys (hy_plan_tick cuts at
// multiples of the tile size), so each 32-key row group of a tile lies in
// one page and its page-table entry is a scalar load.

#include <type_traits>

#include "hy_common.h"
#include "prefill_shape.h"

namespace hy {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kRows = kPrefillRows;  // (token, head) rows per workgroup
constexpr int kThreads = 2 * kRows;  // one wave per 32 rows
constexpr int kKRow = 136;     // u16 per K row in LDS (272 bytes)
constexpr int kVRow = 160;     // u16 per V row in LDS (320 bytes)
constexpr float kLazy = 8.0f;  // rescale threshold, exp2 domain
constexpr int kTileKeys = kPrefillTileKeys;  // keys per LDS stage

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ bf16x8 pack8(const f32x16 &s, int base) {
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = static_cast<__bf16>(s[base + j]);
  return r;
}

__device__ __forceinline__ s16x4 tr_read(const uint16_t *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(const_cast<uint16_t *>(p)));
}

// v_permlane32_swap with both operands x: the first result holds, in every
// lane, x of lane l % 32 and the second x of lane 32 + l % 32, so combining
// the two gives the same value in both lanes of a row.
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int G, int KEYS>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(kPrefillWgPerCu * kThreads / 256, kPrefillWgPerCu * kThreads / 256)))
void prefill_kernel(
    const uint16_t *__restrict__ q, int64_t q_ss, int64_t q_st, int64_t q_sh,
    uint16_t *__restrict__ out, int64_t o_ss, int64_t o_st, int64_t o_sh,
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool,
    int64_t pool_hs, const int32_t *__restrict__ page_table, int64_t pt_stride,
    const int32_t *__restrict__ q_start, const int32_t *__restrict__ kv_lens,
    const int32_t *__restrict__ items, float *__restrict__ ws_acc, float *__restrict__ ws_ml,
    int num_kv_heads, int page_shift, float scale_log2) {
  static_assert(KEYS % 32 == 0 && KEYS >= 32, "tiles are whole 32-key blocks");
  constexpr int kChunks = KEYS * 16 / kThreads;  // 16-byte K (and V) chunks per thread
  constexpr int kPass = kThreads / 16;            // tile rows one chunk index covers
  static_assert(KEYS * 16 % kThreads == 0 && kPass % 16 == 0, "staging covers whole rows");
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][KEYS * kKRow];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][KEYS * kVRow];

  const int32_t *it = items + 8 * blockIdx.y;
  const int kvh = blockIdx.x;
  const int seq = it[0];
  const int q_begin = it[1];
  const int q_end = it[2];
  const int kv_begin = it[3];
  const int kv_end = it[4];
  const int slot = it[5];
  const int h0 = kvh * G;
  const int qs = q_start[seq];
  const int q_len = q_start[seq + 1] - qs;
  const int cache_len = kv_lens[seq] - q_len;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int c = lane & 31;
  const int h = lane >> 5;

  // This lane's row and its Q^T operand (zeros for rows past the chunk).
  const int r = 32 * wave + c;
  const int row_tok = q_begin + r / G;
  const bool live = row_tok < q_end;
  bf16x8 qop[8];
  {
    const uint16_t *src = q + seq * q_ss +
                          static_cast<int64_t>(qs + (live ? row_tok : q_begin)) * q_st +
                          (h0 + r % G) * q_sh;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (live) w = load16(src + 16 * kk + 8 * h);
      qop[kk] = __builtin_bit_cast(bf16x8, w);
      // Scores come out of the MFMA in exp2 units: q * scale * log2(e),
      // rounded to bf16 once here.
#pragma unroll
      for (int e = 0; e < 8; ++e)
        qop[kk][e] = static_cast<__bf16>(static_cast<float>(qop[kk][e]) * scale_log2);
    }
  }

  f32x16 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  // Exponent base of this lane's row, in exp2 units (fp32); -inf until the
  // row has seen a key. The QK^T chain subtracts it (as r_mma, 0 while
  // unset) with one more MFMA: A = 1 in k indices 0-2 (a constant), B = the
  // three bf16 parts of -r_mma (hi + mid + lo hold its 24 bits exactly) in
  // k indices 0-2 of this row, so the scores come out shifted by the exact
  // base and the probabilities are plain exp2 of them. With an exact base
  // the row max's probability is exactly 1 when the base is set, so its
  // bf16 rounding for the P V product matches the fp32 row sum.
  float base = -INFINITY;
  float r_mma = 0.f;
  float l_run = 0.f;
  bf16x8 shift_a, shift_b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    shift_a[e] = static_cast<__bf16>(e < 3 && h == 0 ? 1.0f : 0.0f);
    shift_b[e] = static_cast<__bf16>(0.0f);
  }

  // Causal limits: this row sees keys <= limit; every live row of the wave
  // sees keys <= wave_lo; no live row of the wave sees a key > wave_hi.
  const int last_key = kv_end - 1;
  const int limit = min(cache_len + row_tok, last_key);
  const int tw0 = q_begin + (32 * wave) / G;
  const int tw1 = min(q_end - 1, q_begin + (32 * wave + 31) / G);
  const bool wave_live = tw0 < q_end;
  const int wave_lo = min(cache_len + tw0, last_key);
  const int wave_hi = min(cache_len + tw1, last_key);

  const uint16_t *kh = k_pool + kvh * pool_hs;
  const uint16_t *vh = v_pool + kvh * pool_hs;
  const int32_t *pt = page_table + seq * pt_stride;
  const int page_mask = (1 << page_shift) - 1;

  // Staging: thread t moves chunk j < kChunks of the K and of the V tile:
  // row kPass j + t / 16, dims 8 (t % 16) .. +7. A 32-row group lies in one
  // page: one wave-uniform page lookup per chunk. Rows at or past kv_end
  // read the last valid key instead (any finite data: their scores are
  // masked), so the loads need no branch.
  const int srow = tid >> 4;
  const int scol = (tid & 15) * 8;
  // Page ids of a tile's chunks (scalar loads), fetched one tile before the
  // tile's loads so that no wave waits for them.
  struct Pages {
    int32_t id[kChunks];
  };
  auto fetch_pages = [&](int kt) __attribute__((always_inline)) {
    Pages pg;
#pragma unroll
    for (int j = 0; j < kChunks; ++j)
      pg.id[j] = pt[min(kt + ((kPass * j) & ~31), last_key) >> page_shift];
    return pg;
  };
  auto load_tile = [&](int kt, const Pages &pg, u32x4(&kr)[kChunks], u32x4(&vr)[kChunks])
                       __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int key = min(kt + kPass * j + srow, last_key);
      const int64_t p = (static_cast<int64_t>(pg.id[j]) << page_shift) + (key & page_mask);
      kr[j] = load16(kh + p * kHeadDim + scol);
      vr[j] = load16(vh + p * kHeadDim + scol);
    }
  };
  auto store_tile = [&](int b, const u32x4(&kr)[kChunks], const u32x4(&vr)[kChunks])
                        __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      *reinterpret_cast<u32x4 *>(&sK[b][(kPass * j + srow) * kKRow + scol]) = kr[j];
      *reinterpret_cast<u32x4 *>(&sV[b][(kPass * j + srow) * kVRow + scol]) = vr[j];
    }
  };

  // Per-lane LDS bases: K operand row c, dims 8 h; V^T transposed read: row
  // 4 (q16 / 2) + r16 / 4 of the key quad, dims 16 (q16 % 2) + 4 (r16 % 4).
  const int r16 = lane & 15;
  const int q16 = lane >> 4;
  const int k_base = c * kKRow + 8 * h;
  const int v_base = (4 * (q16 >> 1) + (r16 >> 2)) * kVRow + 16 * (q16 & 1) + 4 * (r16 & 3);

  // One 32-key block starting at key kb0, K/V rows at Kb/Vb in LDS.
  auto block = [&](auto masked, const uint16_t *Kb, const uint16_t *Vb, int kb0)
                   __attribute__((always_inline)) {
    constexpr bool kMasked = decltype(masked)::value;
    f32x16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const bf16x8 kop = *reinterpret_cast<const bf16x8 *>(Kb + k_base + 16 * kk);
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, qop[kk], s, 0, 0, 0);
    }
    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(shift_a, shift_b, s, 0, 0, 0);
    if constexpr (kMasked) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb0 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (key > limit) s[i] = -INFINITY;
      }
    }
    float mx = fmaxf(s[0], s[1]);
#pragma unroll
    for (int i = 2; i < 16; ++i) mx = fmaxf(mx, s[i]);
    mx = halves_max(mx);  // row max relative to r_mma
    // The base only moves when the row max exceeds it by more than kLazy
    // (from -inf: at the first visible key), so probabilities stay below
    // 2^kLazy; the new base is the row max.
    const bool need = base == -INFINITY ? mx != -INFINITY : mx > kLazy;
    if (__builtin_expect(__any(need), 0)) {
      const float r_new = need ? mx + r_mma : r_mma;
      const float delta = r_new - r_mma;
      const float alpha = base == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(-delta);
      if (need) {
        base = r_new;
        r_mma = r_new;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i] -= delta;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
      const float hi = __uint_as_float(f32_to_bf16_rne(r_mma) << 16);
      const float mid = __uint_as_float(f32_to_bf16_rne(r_mma - hi) << 16);
      const float lo = r_mma - hi - mid;  // at most 8 significant bits left
      shift_b[0] = static_cast<__bf16>(h == 0 ? -hi : 0.0f);
      shift_b[1] = static_cast<__bf16>(h == 0 ? -mid : 0.0f);
      shift_b[2] = static_cast<__bf16>(h == 0 ? -lo : 0.0f);
    }
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = __builtin_amdgcn_exp2f(s[i]);
      s[i] = p;
      psum += p;
    }
    l_run += psum;
    const bf16x8 pop0 = pack8(s, 0);
    const bf16x8 pop1 = pack8(s, 8);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int kh2 = 0; kh2 < 2; ++kh2) {
        const uint16_t *vp = Vb + v_base + 16 * kh2 * kVRow + 32 * db;
        const s16x4 lo = tr_read(vp);
        const s16x4 hi = tr_read(vp + 8 * kVRow);
        const s16x8 v8 = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, v8),
                                                          kh2 ? pop1 : pop0, acc[db], 0, 0, 0);
      }
  };

  const int n_tiles = (kv_end - kv_begin + KEYS - 1) / KEYS;
  {
    u32x4 kr[kChunks], vr[kChunks];
    load_tile(kv_begin, fetch_pages(kv_begin), kr, vr);
    store_tile(0, kr, vr);
  }
  Pages pg_next = {};
  if (n_tiles > 1) pg_next = fetch_pages(kv_begin + KEYS);
  __syncthreads();

  // Tiles whose keys every live row of the workgroup sees need no mask
  // (they come first); the rest decide per wave and 32-key block whether to
  // skip, compute plainly or mask.
  int n_plain = (min(cache_len + q_begin, last_key) + 1 - kv_begin) / KEYS;
  n_plain = n_plain < 0 ? 0 : (n_plain > n_tiles ? n_tiles : n_plain);
  auto iterate = [&](auto diag, int t) __attribute__((always_inline)) {
    constexpr bool kDiag = decltype(diag)::value;
    const int kt = kv_begin + KEYS * t;
    const int b = t & 1;
    const bool has_next = t + 1 < n_tiles;
    u32x4 kr[kChunks], vr[kChunks];
    if (has_next) {
      load_tile(kt + KEYS, pg_next, kr, vr);
      if (t + 2 < n_tiles) pg_next = fetch_pages(kt + 2 * KEYS);
    }
    if (wave_live) {
#pragma unroll
      for (int kb = 0; kb < KEYS / 32; ++kb) {
        const uint16_t *Kb = sK[b] + 32 * kb * kKRow;
        const uint16_t *Vb = sV[b] + 32 * kb * kVRow;
        const int kb0 = kt + 32 * kb;
        if constexpr (!kDiag) {
          block(std::false_type{}, Kb, Vb, kb0);
        } else {
          if (kb0 <= wave_hi) {
            if (kb0 + 31 <= wave_lo)
              block(std::false_type{}, Kb, Vb, kb0);
            else
              block(std::true_type{}, Kb, Vb, kb0);
          }
        }
      }
    }
    if (has_next) {
      store_tile(b ^ 1, kr, vr);
      __syncthreads();
    }
  };
  for (int t = 0; t < n_plain; ++t) iterate(std::false_type{}, t);
  for (int t = n_plain; t < n_tiles; ++t) iterate(std::true_type{}, t);

  // Epilogue: full row sums, then the output or the split's partial.
  const float lsum = halves_sum(l_run);
  if (slot < 0) {
    if (!live) return;
    const float inv = 1.0f / lsum;
    uint16_t *dst = out + seq * o_ss + static_cast<int64_t>(qs + row_tok) * o_st +
                    (h0 + r % G) * o_sh;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d = 32 * db + 8 * i4 + 4 * h;
        const uint32_t w0 = pack_bf16x2_rne(acc[db][4 * i4] * inv, acc[db][4 * i4 + 1] * inv);
        const uint32_t w1 =
            pack_bf16x2_rne(acc[db][4 * i4 + 2] * inv, acc[db][4 * i4 + 3] * inv);
        *reinterpret_cast<uint2 *>(dst + d) = make_uint2(w0, w1);
      }
  } else {
    const int64_t pr = (static_cast<int64_t>(slot) * num_kv_heads + kvh) * kRows + r;
    float *dst = ws_acc + pr * kHeadDim;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d = 32 * db + 8 * i4 + 4 * h;
        *reinterpret_cast<f32x4 *>(dst + d) =
            f32x4{acc[db][4 * i4], acc[db][4 * i4 + 1], acc[db][4 * i4 + 2],
                  acc[db][4 * i4 + 3]};
      }
    if (h == 0) {
      ws_ml[pr * 2 + 0] = base;
      ws_ml[pr * 2 + 1] = lsum;
    }
  }
}

// Combines the splits of a query tile: grid (kv head, merge item, kRows /
// 32 row groups), 512 threads = 32 rows x 16 lanes x 8 dims. Item = {seq,
// q_begin, q_end, first_slot, num_splits, q_row = q_start[seq], 0, 0}. Up
// to four splits are loaded in one round of independent loads: every load
// reads a real split (the index is clamped to the last one; a partial holds
// all kRows rows, so rows past q_end are in bounds too) and the ones past
// num_splits are then replaced by the empty partial, so no load sits behind
// a branch. Rows past q_end are computed and not stored.
template <int G>
__global__ __launch_bounds__(512) void prefill_merge_kernel(
    uint16_t *__restrict__ out, int64_t o_ss, int64_t o_st, int64_t o_sh,
    const int32_t *__restrict__ q_start, const int32_t *__restrict__ items,
    const float *__restrict__ ws_acc, const float *__restrict__ ws_ml, int num_kv_heads) {
  const int4 it0 = *reinterpret_cast<const int4 *>(items + 8 * blockIdx.y);
  const int4 it1 = *reinterpret_cast<const int4 *>(items + 8 * blockIdx.y + 4);
  const int kvh = blockIdx.x;
  const int seq = it0.x;
  const int q_begin = it0.y;
  const int q_end = it0.z;
  const int first = it0.w;
  const int nsplit = it1.x;
  const int r = 32 * blockIdx.z + (threadIdx.x >> 4);
  const int d = (threadIdx.x & 15) * 8;
  const int i = q_begin + r / G;
  const int64_t qs = it1.y;  // q_start[seq], carried by the item
  float mx = -INFINITY, lsum = 0.f;
  f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsplit; s0 += 4) {
    float m[4], l[4];
    f32x4 x0[4], x1[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t pr =
          (static_cast<int64_t>(first + min(s0 + j, nsplit - 1)) * num_kv_heads + kvh) * kRows + r;
      const float2 ml = *reinterpret_cast<const float2 *>(ws_ml + pr * 2);
      m[j] = ml.x;
      l[j] = ml.y;
      x0[j] = *reinterpret_cast<const f32x4 *>(ws_acc + pr * kHeadDim + d);
      x1[j] = *reinterpret_cast<const f32x4 *>(ws_acc + pr * kHeadDim + d + 4);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool live = s0 + j < nsplit;
      m[j] = live ? m[j] : -INFINITY;
      l[j] = live ? l[j] : 0.f;
      x0[j] = live ? x0[j] : f32x4{0.f, 0.f, 0.f, 0.f};
      x1[j] = live ? x1[j] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float cmx = mx;
#pragma unroll
    for (int j = 0; j < 4; ++j) cmx = fmaxf(cmx, m[j]);
    // All maxima -inf: both factors below are 0 and every term adds +0.
    const float f_old = mx == -INFINITY ? 0.f : exp2f(mx - cmx);
    lsum *= f_old;
    a0 *= f_old;
    a1 *= f_old;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float f = m[j] == -INFINITY ? 0.f : exp2f(m[j] - cmx);
      lsum += f * l[j];
      a0 += f * x0[j];
      a1 += f * x1[j];
    }
    mx = cmx;
  }
  if (i >= q_end) return;
  uint16_t *dst = out + seq * o_ss + (qs + i) * o_st + (kvh * G + r % G) * o_sh + d;
  *reinterpret_cast<u32x4 *>(dst) =
      u32x4{pack_bf16x2_rne(a0[0] / lsum, a0[1] / lsum), pack_bf16x2_rne(a0[2] / lsum, a0[3] / lsum),
            pack_bf16x2_rne(a1[0] / lsum, a1[1] / lsum), pack_bf16x2_rne(a1[2] / lsum, a1[3] / lsum)};
}

template <int G>
void launch_prefill(hipStream_t st, int num_kv_heads, int n_items, const uint16_t *q,
                    int64_t q_ss, int64_t q_st, int64_t q_sh, uint16_t *out, int64_t o_ss,
                    int64_t o_st, int64_t o_sh, const uint16_t *k_pool, const uint16_t *v_pool,
                    int64_t pool_hs, const int32_t *page_table, int64_t pt_stride,
                    const int32_t *q_start, const int32_t *kv_lens, const int32_t *items,
                    float *ws_acc, float *ws_ml, int page_shift, float scale_log2) {
  hipLaunchKernelGGL((prefill_kernel<G, kTileKeys>), dim3(num_kv_heads, n_items), dim3(kThreads), 0,
                     st, q, q_ss,
                     q_st, q_sh, out, o_ss, o_st, o_sh, k_pool, v_pool, pool_hs, page_table,
                     pt_stride, q_start, kv_lens, items, ws_acc, ws_ml, num_kv_heads, page_shift,
                     scale_log2);
}

template <int G>
void launch_prefill_merge(hipStream_t st, int num_kv_heads, int n_merge, uint16_t *out,
                          int64_t o_ss, int64_t o_st, int64_t o_sh, const int32_t *q_start,
                          const int32_t *merge_items, const float *ws_acc, const float *ws_ml) {
  hipLaunchKernelGGL(prefill_merge_kernel<G>, dim3(num_kv_heads, n_merge, kRows / 32), dim3(512),
                     0, st, out, o_ss, o_st, o_sh, q_start, merge_items, ws_acc, ws_ml,
                     num_kv_heads);
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace
}  // namespace hy

using hy::kHeadDim;

extern "C" int32_t hy_prefill_tile_rows(void) { return hy::kRows; }

extern "C" int64_t hy_prefill_workspace_bytes(int32_t n_slots, int32_t num_kv_heads,
                                              int32_t head_dim) {
  if (n_slots <= 0) return 0;
  const int64_t rows = static_cast<int64_t>(n_slots) * num_kv_heads * hy::kRows;
  return hy::align256(rows * head_dim * 4) + hy::align256(rows * 2 * 4);
}

extern "C" int hy_paged_prefill(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok, int64_t q_stride_head,
    void *out, int64_t o_stride_seq, int64_t o_stride_tok, int64_t o_stride_head,
    const void *k_pool, const void *v_pool, int64_t pool_head_stride,
    const int32_t *page_table, int64_t page_table_stride, const int32_t *q_start,
    const int32_t *kv_lens, const int32_t *prefill_items, int32_t n_prefill, int32_t n_slots,
    void *workspace, int64_t workspace_bytes, int32_t num_seqs, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t page_size, float scale, void *stream) {
  hy::clear_error();
  HY_REQUIRE(num_seqs >= 1, "num_seqs must be positive");
  HY_REQUIRE(scale > 0.f, "softmax scale must be positive");
  HY_REQUIRE(num_kv_heads >= 1 && num_q_heads >= num_kv_heads &&
                 num_q_heads % num_kv_heads == 0,
             "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)",
             num_q_heads, num_kv_heads);
  HY_REQUIRE_SUPPORTED(head_dim == kHeadDim, "head_dim %d unsupported (need %d)", head_dim,
                       kHeadDim);
  HY_REQUIRE_SUPPORTED(page_size >= 32 && (page_size & (page_size - 1)) == 0,
                       "page_size %d unsupported (power of two >= 32 required)", page_size);
  HY_REQUIRE(n_prefill >= 0 && n_slots >= 0, "item counts must be non-negative");
  if (n_prefill == 0) return HY_OK;
  HY_REQUIRE(n_prefill <= 65535, "%d prefill items exceed the grid limit of 65535", n_prefill);
  HY_REQUIRE(q && out && k_pool && v_pool && page_table && q_start && kv_lens && prefill_items,
             "hy_paged_prefill: null pointer argument");
  const int64_t need = hy_prefill_workspace_bytes(n_slots, num_kv_heads, head_dim);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    hy::set_error("workspace too small: need %lld bytes, got %lld",
                  static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    return HY_ENOSPACE;
  }
  float *ws_acc = nullptr, *ws_ml = nullptr;
  if (need > 0) {
    const int64_t rows = static_cast<int64_t>(n_slots) * num_kv_heads * hy::kRows;
    ws_acc = static_cast<float *>(workspace);
    ws_ml = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                      hy::align256(rows * head_dim * 4));
  }
  const int G = num_q_heads / num_kv_heads;
  const float scale_log2 = scale * hy::kLog2e;
  const int page_shift = __builtin_ctz(static_cast<unsigned>(page_size));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t *qq = static_cast<const uint16_t *>(q);
  uint16_t *oo = static_cast<uint16_t *>(out);
  const uint16_t *kp = static_cast<const uint16_t *>(k_pool);
  const uint16_t *vp = static_cast<const uint16_t *>(v_pool);
#define HY_PREFILL_CASE(GG)                                                                   \
  case GG:                                                                                    \
    hy::launch_prefill<GG>(st, num_kv_heads, n_prefill, qq, q_stride_seq, q_stride_tok,       \
                           q_stride_head, oo, o_stride_seq, o_stride_tok, o_stride_head, kp,  \
                           vp, pool_head_stride, page_table, page_table_stride, q_start,      \
                           kv_lens, prefill_items, ws_acc, ws_ml, page_shift, scale_log2);    \
    break;
  switch (G) {
    HY_PREFILL_CASE(1)
    HY_PREFILL_CASE(2)
    HY_PREFILL_CASE(4)
    HY_PREFILL_CASE(8)
    HY_PREFILL_CASE(16)
    default:
      hy::set_error("GQA group size %d unsupported (1, 2, 4, 8, 16)", G);
      return HY_EUNSUPPORTED;
  }
#undef HY_PREFILL_CASE
  return hy::launch_status("hy_paged_prefill");
}

extern "C" int hy_paged_prefill_merge(void *out, int64_t o_stride_seq, int64_t o_stride_tok,
                                      int64_t o_stride_head, const int32_t *q_start,
                                      const int32_t *merge_items, int32_t n_merge,
                                      int32_t n_slots, const void *workspace,
                                      int64_t workspace_bytes, int32_t num_q_heads,
                                      int32_t num_kv_heads, int32_t head_dim, void *stream) {
  hy::clear_error();
  HY_REQUIRE(n_merge >= 0 && n_slots >= 0, "item counts must be non-negative");
  if (n_merge == 0) return HY_OK;
  HY_REQUIRE(n_merge <= 65535, "%d merge items exceed the grid limit of 65535", n_merge);
  HY_REQUIRE(num_kv_heads >= 1 && num_q_heads >= num_kv_heads &&
                 num_q_heads % num_kv_heads == 0,
             "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)",
             num_q_heads, num_kv_heads);
  HY_REQUIRE_SUPPORTED(head_dim == kHeadDim, "head_dim %d unsupported (need %d)", head_dim,
                       kHeadDim);
  HY_REQUIRE(out && q_start && merge_items && workspace,
             "hy_paged_prefill_merge: null pointer argument");
  const int64_t need = hy_prefill_workspace_bytes(n_slots, num_kv_heads, head_dim);
  if (workspace_bytes < need) {
    hy::set_error("workspace too small: need %lld bytes, got %lld",
                  static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    return HY_ENOSPACE;
  }
  const int64_t rows = static_cast<int64_t>(n_slots) * num_kv_heads * hy::kRows;
  const float *ws_acc = static_cast<const float *>(workspace);
  const float *ws_ml = reinterpret_cast<const float *>(static_cast<const char *>(workspace) +
                                                       hy::align256(rows * head_dim * 4));
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint16_t *oo = static_cast<uint16_t *>(out);
  switch (num_q_heads / num_kv_heads) {
    case 1: hy::launch_prefill_merge<1>(st, num_kv_heads, n_merge, oo, o_stride_seq, o_stride_tok, o_stride_head, q_start, merge_items, ws_acc, ws_ml); break;
    case 2: hy::launch_prefill_merge<2>(st, num_kv_heads, n_merge, oo, o_stride_seq, o_stride_tok, o_stride_head, q_start, merge_items, ws_acc, ws_ml); break;
    case 4: hy::launch_prefill_merge<4>(st, num_kv_heads, n_merge, oo, o_stride_seq, o_stride_tok, o_stride_head, q_start, merge_items, ws_acc, ws_ml); break;
    case 8: hy::launch_prefill_merge<8>(st, num_kv_heads, n_merge, oo, o_stride_seq, o_stride_tok, o_stride_head, q_start, merge_items, ws_acc, ws_ml); break;
    case 16: hy::launch_prefill_merge<16>(st, num_kv_heads, n_merge, oo, o_stride_seq, o_stride_tok, o_stride_head, q_start, merge_items, ws_acc, ws_ml); break;
    default:
      hy::set_error("GQA group size %d unsupported (1, 2, 4, 8, 16)", num_q_heads / num_kv_heads);
      return HY_EUNSUPPORTED;
  }
  return hy::launch_status("hy_paged_prefill_merge");
}
