// Paged chunked-prefill causal attention on bf16 MFMA (gfx950).
//
// Grid: (kv head, prefill item); heads vary fastest, so the dispatcher walks
// items in the planner's longest-first order and, with 8 kv heads on the 8
// XCDs, every workgroup of one kv head lands on the same XCD (its L2 holds
// that head's K/V pages for all query tiles of the request). An item is a
// tile of kPrefillRows / G query tokens of one sequence; with its G query
// heads that is kPrefillRows (token, head) rows (prefill_shape.h), all
// reading the same K/V rows (GQA), over the key range [kv_begin, kv_end) of
// one split. One 512-thread workgroup per CU (128 KiB of LDS).
//
// Eight waves of 32 rows, two waves per SIMD. Row r = 32 w + c is token
// q_begin + r / G, head kv_head * G + r % G, so a wave spans 32 / G
// consecutive tokens and the causal diagonal cuts few of its key blocks.
//
// v_mfma_f32_32x32x16_bf16, transposed formulation (lane l, c = l % 32,
// h = l / 32):
//   S^T = K Q^T   A = K (32 keys x 16 dims) from LDS (one 16-byte read per
//                 lane); B = Q^T held in registers. Lane (c, h) ends with
//                 row c's scores for keys 8 (i / 4) + 4 h + i % 4, i < 16,
//                 of the 32-key block.
//   softmax       per row: p = exp2(fma(s, scale * log2(e), -base)), the
//                 score scaling in fp32 as the reference's; the two lanes
//                 of a row differ only in h; the row max and sum cross
//                 halves with v_permlane32_swap.
//   O^T += V^T P^T  B = P^T: the first (last) eight of the lane's scores
//                 are row c's probabilities for MFMA k index 8 h + j once k
//                 stands for key 16 kh + (j < 4 ? 4 h + j : 8 + 4 h + j - 4);
//                 A = V^T from LDS with ds_read_b64_tr_b16, which hands lane
//                 r of a 16-lane group four consecutive keys of dim r.
// K/V tiles of kTile keys sit in a ring of four LDS stages filled by
// gfx950's 16-byte direct-to-LDS loads (global_load_lds_dwordx4), two tiles
// ahead of the one being consumed, without passing through registers; one
// wait and one barrier per tile. The fourth stage keeps a tile's V rows in
// place while the next tile's first block runs their P V (below). A load
// instruction writes 64 lanes x 16 bytes to consecutive LDS addresses, so
// the bank-conflict-free layouts are
// lane permutations instead of padded rows (16-byte units, "chunk" = 8
// dims):
//   K: unit(row, chunk) = (row / 16) * 256 + chunk * 16 + row % 16. The
//      K-operand read (16 lanes = 16 rows, one chunk) touches 16
//      consecutive units; one load instruction = 16 rows x 4 chunks
//      (64-byte runs of each row).
//   V: unit(row, chunk) = (row / 4) * 64 + chunk * 4 + row % 4. The
//      transposing read (32 lanes = 4 rows x 32 dims) touches 16
//      consecutive units; one load instruction = 4 whole rows.
// Both give per-lane base addresses with compile-time offsets for every
// block, dim slice and row group. The block loop is software-pipelined: a
// wave computes block j + 1's scores on the matrix core while its VALU
// turns block j's scores into probabilities (see the block body below).
// The softmax rescales lazily: the exponent base of a row only moves when
// its max grows by more than 2^8, so the accumulators are rarely touched by
// VALU. Key blocks past the causal limit of every row of a wave are
// skipped by that wave.
// Rows at or past kv_end are loaded from the last valid key, so masked
// scores never meet NaN bits of unwritten rows.
//
// A split whose item has slot >= 0 writes an fp32 partial (unnormalised
// O^T, row max in the exp2 domain, row sum) to the workspace;
// prefill_merge_kernel (hy_paged_prefill_merge) combines the splits of a
// query tile afterwards.
//
// Item key ranges start at multiples of 64 keys (hy_plan_tick cuts at
// multiples of the 64-key tile), so the rows one wave loads of a tile lie
// in one page (pages hold at least 32 keys) and their page-table entry is a
// scalar load.

#include <type_traits>

#include "hy_common.h"
#include "prefill_shape.h"

namespace hy {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kRows = kPrefillRows;  // (token, head) rows per workgroup
constexpr int kThreads = 2 * kRows;  // one wave per 32 rows
constexpr float kLazy = 8.0f;  // rescale threshold, exp2 domain
constexpr float kLazyP = 256.0f;  // 2^kLazy

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ bf16x8 pack8(const f32x16 &s, int base) {
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = static_cast<__bf16>(s[base + j]);
  return r;
}

__device__ __forceinline__ float tree_sum16(const float (&p)[16]) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = p[2 * i] + p[2 * i + 1];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = a[2 * i] + a[2 * i + 1];
  return (a[0] + a[1]) + (a[2] + a[3]);
}

__device__ __forceinline__ float tree_max16(const f32x16 &s) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = fmaxf(s[2 * i], s[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = fmaxf(a[2 * i], a[2 * i + 1]);
  return fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3]));
}

__device__ __forceinline__ s16x4 tr_read(const uint16_t *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(const_cast<uint16_t *>(p)));
}

// 16 bytes from global memory straight into LDS: lane l's bytes land at
// lds + 16 l (lds is wave-uniform and goes to M0). Inline assembly, so the
// compiler neither orders LDS reads behind these writes nor waits for them:
// the kernel waits explicitly (wait_tile_loads) before the barrier that
// publishes a tile, and never reads a buffer that loads are filling.
__device__ __forceinline__ void load_to_lds(const uint16_t *g, const uint16_t *lds) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) uint16_t *)lds));
  // M0 has no other user in this kernel (no LDS-DMA builtins, no indexed
  // register access), so setting it here disturbs nothing.
  __asm__ volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                   :
                   : "v"(g), "s"(__builtin_amdgcn_readfirstlane(m0))
                   : "memory");
}

// Waits until this wave's outstanding vector-memory loads (the direct-to-LDS
// tile loads), LDS reads and scalar loads (the page-table lookups) have all
// completed: s_waitcnt vmcnt(0) lgkmcnt(0), expcnt left alone (simm16 0x0070).
// Issued through the builtin, the compiler's own wait tracking sees it, so
// it knows no scalar load is pending in the block loop that follows and can
// wait there for single LDS reads (a pending scalar load, which may return
// out of order, would force it to wait for every LDS read).
__device__ __forceinline__ void wait_tile_loads() {
  __builtin_amdgcn_s_waitcnt(0x0070);
  __asm__ volatile("" ::: "memory");
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

constexpr int kTile = 64;                        // keys per LDS stage (two blocks)
constexpr int kStage = 2 * kTile * kHeadDim;     // halfs per stage: K tile, then V tile
constexpr int kStages = 4;                       // ring of stages (128 KiB)

// Instruction classes for __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedValu = 0x002 | 0x400;  // VALU incl. transcendentals
constexpr int kSchedDsRead = 0x100;

template <int G>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_kernel(
    const uint16_t *__restrict__ q, int64_t q_ss, int64_t q_st, int64_t q_sh,
    uint16_t *__restrict__ out, int64_t o_ss, int64_t o_st, int64_t o_sh,
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool,
    int64_t pool_hs, const int32_t *__restrict__ page_table, int64_t pt_stride,
    const int32_t *__restrict__ items, float *__restrict__ ws_acc, float *__restrict__ ws_ml,
    int num_kv_heads, int page_shift, float scale_log2) {
  static_assert(kThreads == 512, "eight waves");
  __shared__ __attribute__((aligned(1024))) uint16_t smem[kStages * kStage];

  const int32_t *it = items + 8 * blockIdx.y;
  const int kvh = blockIdx.x;
  const int seq = it[0];
  const int q_begin = it[1];
  const int q_end = it[2];
  const int kv_begin = it[3];
  const int kv_end = it[4];
  const int slot = it[5];
  // the sequence's packed query row and cached length travel in the item,
  // so the Q loads and page-table reads issue one dependent read after
  // the kernel starts
  const int qs = it[6];
  const int cache_len = it[7];
  const int h0 = kvh * G;
  // an empty record (q_end <= q_begin) pads a list to a fixed launch size
  if (q_end <= q_begin) return;

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
    // rows past the chunk read the chunk's first row (in bounds) and are
    // zeroed, so the eight loads issue together without a branch
    const uint16_t *src = q + seq * q_ss +
                          static_cast<int64_t>(qs + (live ? row_tok : q_begin)) * q_st +
                          (h0 + r % G) * q_sh;
    u32x4 raw[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) raw[kk] = load16(src + 16 * kk + 8 * h);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      u32x4 w = raw[kk];
      if (!live) w = u32x4{0u, 0u, 0u, 0u};
      qop[kk] = __builtin_bit_cast(bf16x8, w);
    }
  }

  f32x16 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[db][i] = 0.f;
  // Scores come out of the MFMA unscaled (q and k as stored). A row's
  // probabilities are exp2(fma(s, scale * log2(e), -shift)): the fp32 score
  // scaling, in exp2 units, and the subtraction of the row's exponent base
  // rounded once. base is that exponent base, -inf until the row has seen a
  // key; shift is the value subtracted (0 while base is unset). The base is
  // set to the rounded scaled row max, so the max's own argument is within
  // an ulp of 0 and its probability rounds to 1 in bf16 for the P V product
  // as in the fp32 row sum.
  float base = -INFINITY;
  float shift = 0.f;
  float l_run = 0.f;

  // Causal limits: this row sees keys <= limit; every live row of the wave
  // sees keys <= wave_lo; no live row of the wave sees a key > wave_hi.
  const int last_key = kv_end - 1;
  const int limit = min(cache_len + row_tok, last_key);
  const int tw0 = q_begin + (32 * wave) / G;
  const int tw1 = min(q_end - 1, q_begin + (32 * wave + 31) / G);
  const bool wave_live = tw0 < q_end;
  const int wave_lo = min(cache_len + tw0, last_key);
  const int wave_hi = min(cache_len + tw1, last_key);
  // This wave computes the item's 32-key blocks [0, nb); blocks from jm on
  // cross its rows' diagonal and are masked.
  const int nb = wave_live && wave_hi >= kv_begin ? (wave_hi - kv_begin) / 32 + 1 : 0;
  const int jm = wave_lo >= kv_begin ? (wave_lo - kv_begin + 1) / 32 : 0;

  const uint16_t *kh = k_pool + kvh * pool_hs;
  const uint16_t *vh = v_pool + kvh * pool_hs;
  const int32_t *pt = page_table + seq * pt_stride;
  const int page_mask = (1 << page_shift) - 1;
  const int n_tiles = (kv_end - kv_begin + kTile - 1) / kTile;

  // Tile loads: wave w issues K instructions 2w, 2w + 1 (rows 16 (w / 2) +
  // lane % 16, chunks 4 (i % 4) + lane / 16) and V instructions 2w, 2w + 1
  // (rows 4 i + lane % 4, chunk lane / 4). A wave's rows lie in one page
  // (pages hold >= 32 keys), so each tensor needs one page id per tile;
  // they are fetched a tile ahead. Rows at or past kv_end load the last
  // valid key (any finite data: their scores are masked).
  // Page ids are non-negative (the host rejects others); held unsigned, they
  // widen to 64 bits without a sign extension that would make the compiler
  // wait for each id as soon as it is read. Keys are clamped to
  // [0, last_key], so every read stays inside the sequence's row.
  struct Pages {
    uint32_t k, v;
  };
  auto fetch_pages = [&](int kt) __attribute__((always_inline)) {
    Pages pg;
    pg.k = static_cast<uint32_t>(pt[max(min(kt + 16 * (wave >> 1), last_key), 0) >> page_shift]);
    pg.v = static_cast<uint32_t>(pt[max(min(kt + 8 * wave, last_key), 0) >> page_shift]);
    return pg;
  };
  auto issue_tile = [&](int kt, const Pages &pg, uint16_t *dst) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = 2 * wave + j;
      {
        const int key = min(kt + 16 * (i >> 2) + (lane & 15), last_key);
        const int64_t p = (static_cast<int64_t>(pg.k) << page_shift) + (key & page_mask);
        load_to_lds(kh + p * kHeadDim + 8 * (4 * (i & 3) + (lane >> 4)), dst + i * 512);
      }
      {
        const int key = min(kt + 4 * i + (lane & 3), last_key);
        const int64_t p = (static_cast<int64_t>(pg.v) << page_shift) + (key & page_mask);
        load_to_lds(vh + p * kHeadDim + 8 * (lane >> 2), dst + kTile * kHeadDim + i * 512);
      }
    }
  };

  // Per-lane LDS read bases (u16 units). K operand of row c, dims 16 kk +
  // 8 h: unit (c / 16) * 256 + (2 kk + h) * 16 + c % 16, i.e. base + 256 kk.
  // V^T transposed read of lane (q16, r16): row 4 (q16 / 2) + r16 / 4 (+ 8
  // for the second half, + 16 kh2, + 32 kb), dims 16 (q16 % 2) + 4 (r16 % 4)
  // (+ 32 db), i.e. base + 1024 hi + 2048 kh2 + 128 db.
  const int r16 = lane & 15;
  const int q16 = lane >> 4;
  const int k_base = (c >> 4) * 2048 + h * 128 + (c & 15) * 8;
  const int v_base = 512 * (q16 >> 1) + 64 * (q16 & 1) + 32 * ((r16 & 3) >> 1) + 8 * (r16 >> 2) +
                     4 * (r16 & 1);
  // Block j's K and V rows in the ring: stage (j / 2) % kStages, half j % 2.
  auto k_block = [&](int j) -> const uint16_t * {
    return smem + ((j >> 1) % kStages) * kStage + 4096 * (j & 1) + k_base;
  };
  auto v_block = [&](int j) -> const uint16_t * {
    return smem + ((j >> 1) % kStages) * kStage + kTile * kHeadDim + 4096 * (j & 1) + v_base;
  };

  // Software pipeline over this wave's blocks. Block j's body runs the
  // QK^T MFMAs of block j + 1 while the VALU does block j's softmax (the
  // two are independent), then block j - 1's P V MFMAs, so a block's
  // probabilities are used one body after they are made; K operands are
  // read two blocks ahead and V operands at the start of the body that
  // uses them, so no LDS read is waited for right after it is issued. The
  // scores are raw, so a block's softmax applies the base as it stands when
  // the softmax runs; block j - 1's P V goes in before block j's rebase,
  // which then scales it with the rest of the accumulator. Measured against
  // P V in the block's own body: 0.5 % less on prefill_4x512 and 0.7 % on
  // the mixed tick (graph steps, alternating runs).
  bf16x8 kop[8];
  auto read_k = [&](int j) __attribute__((always_inline)) {
    const uint16_t *kb = k_block(j);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) kop[kk] = *reinterpret_cast<const bf16x8 *>(kb + 256 * kk);
  };
  auto qk = [&]() __attribute__((always_inline)) {
    f32x16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[kk], qop[kk], s, 0, 0, 0);
    return s;
  };

  // Softmax of one block's raw scores s: lane (c, h) holds row c's scores
  // for keys 8 (i / 4) + 4 h + i % 4 of the block.
  // probs(): the common case, straight-line code the scheduler can
  // interleave with the next block's QK^T MFMAs: probabilities against the
  // current base, packed to bf16, and their sum (pairwise tree: four
  // dependent steps instead of fifteen). rebase(): when some row's
  // max exceeds the base by more than kLazy (or a row sees its first key)
  // the base moves and the block's probabilities are redone (rare). The
  // row max is only computed when a lane's probabilities sum to more than
  // 2^kLazy: below that no score of the lane can exceed the base by more
  // than kLazy (each probability is at most the sum), so the common path
  // carries no max tree.
  auto mask = [&](f32x16 &s, int kb0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kb0 + 8 * (i >> 2) + 4 * h + (i & 3);
      s[i] = key > limit ? -INFINITY : s[i];
    }
  };
  auto probs = [&](const f32x16 &s, bf16x8 &pop0, bf16x8 &pop1, float &psum)
                   __attribute__((always_inline)) {
    float pp[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], scale_log2, -shift));
      pp[i] = p;
      if (i < 8)
        pop0[i] = static_cast<__bf16>(p);
      else
        pop1[i - 8] = static_cast<__bf16>(p);
    }
    psum = tree_sum16(pp);
  };
  auto rebase = [&](const f32x16 &s, bf16x8 &pop0, bf16x8 &pop1, float &psum)
                    __attribute__((always_inline)) {
    // !(psum <= ...) also catches an overflowed (infinite) sum
    const bool check = base == -INFINITY || !(psum <= kLazyP);
    if (__builtin_expect(__any(check), 0)) {
      const float mraw = halves_max(tree_max16(s));  // raw row max
      const float mx = __builtin_fmaf(mraw, scale_log2, -shift);  // relative to shift
      const bool need = base == -INFINITY ? mraw != -INFINITY : mx > kLazy;
      if (__any(need)) {
        const float s_new = need ? mraw * scale_log2 : shift;
        const float delta = s_new - shift;
        const float alpha = base == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(-delta);
        if (need) {
          base = s_new;
          shift = s_new;
        }
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] *= alpha;
        float pp[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          pp[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], scale_log2, -shift));
          if (i < 8)
            pop0[i] = static_cast<__bf16>(pp[i]);
          else
            pop1[i - 8] = static_cast<__bf16>(pp[i]);
        }
        psum = tree_sum16(pp);
      }
    }
    l_run += psum;
  };
  // V^T operands of block j (eight 32-dim x 16-key slices), then P V.
  s16x8 vop[8];
  auto read_v = [&](int j, int half) __attribute__((always_inline)) {
    const uint16_t *vb = v_block(j);
#pragma unroll
    for (int db = 2 * half; db < 2 * half + 2; ++db)
#pragma unroll
      for (int kh2 = 0; kh2 < 2; ++kh2) {
        const s16x4 lo = tr_read(vb + 2048 * kh2 + 128 * db);
        const s16x4 hi = tr_read(vb + 2048 * kh2 + 128 * db + 1024);
        vop[2 * db + kh2] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
  };
  auto pv = [&](const bf16x8 &pop0, const bf16x8 &pop1) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int kh2 = 0; kh2 < 2; ++kh2)
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8, vop[2 * db + kh2]), kh2 ? pop1 : pop0, acc[db], 0, 0, 0);
  };

  // One block: half of block j - 1's V reads go out first (the LDS counter
  // holds at most 15 outstanding reads, so the first MFMA's wait for the K
  // operands cannot leave all 16 in flight); then QK^T of block j + 1 on the
  // matrix core, interleaved with the other V reads and block j's
  // probabilities (one MFMA, one LDS read, seven VALU instructions, eight
  // times); then block j - 1's P V, block j's rare rebase and the K reads of
  // block j + 2. The probabilities alternate between two register sets, as
  // the scores do.
  f32x16 s_a, s_b;
  bf16x8 pa0, pa1, pb0, pb1;
  auto body = [&](bool masked, int j, f32x16 &s_cur, f32x16 &s_nxt, bf16x8 &pop0, bf16x8 &pop1,
                  const bf16x8 &prev0, const bf16x8 &prev1) __attribute__((always_inline)) {
    float psum;
    if (masked) mask(s_cur, kv_begin + 32 * j);  // blocks on the diagonal
    // block j - 1's V (its P V runs in this body); for j = 0 block 0's
    // stage is read and the values are unused
    const int jv = j > 0 ? j - 1 : 0;
    read_v(jv, 0);
    __builtin_amdgcn_sched_barrier(0);
    // The two waves of a SIMD take turns: the one in this region (next
    // block's QK^T interleaved with this block's probabilities, the chain
    // that gates its next block) wins issue over the other wave's P V, K
    // reads and barrier wait. Measured on prefill_4x512: 4 % less kernel
    // time than without the priority (and than a priority on P V).
    __builtin_amdgcn_s_setprio(1);
    s_nxt = qk();
    read_v(jv, 1);
    probs(s_cur, pop0, pop1, psum);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedValu, 7, 0);
    }
    // the probabilities count as used here, so the compiler keeps them in
    // this straight-line region instead of sinking them past the rebase test
    __asm__ volatile("" ::"v"(psum), "v"(pop0), "v"(pop1));
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    if (j > 0) pv(prev0, prev1);  // block j - 1's P V, before block j's rebase
    rebase(s_cur, pop0, pop1, psum);
    read_k(j + 2);
  };

  // Prologue: the page ids of tiles 0-2 are read together (one round trip:
  // the tile loads below are inline assembly that no load may cross, so
  // reads placed after the first tile's loads would each wait for their
  // own), tiles 0 and 1 go in flight, then block 0's scores and block 1's
  // K operands.
  const Pages pg0 = fetch_pages(kv_begin);
  const Pages pg1 = fetch_pages(kv_begin + kTile);
  Pages pg_next = fetch_pages(kv_begin + 2 * kTile);
  if (n_tiles > 0) issue_tile(kv_begin, pg0, smem);
  if (n_tiles > 1) issue_tile(kv_begin + kTile, pg1, smem + kStage);
  wait_tile_loads();
  __syncthreads();
  read_k(0);
  s_a = qk();
  read_k(1);

  // Tile t: tile t + 2's loads go into the stage tile t - 1 used (every wave
  // left it before the last barrier), then this wave's blocks 2t, 2t + 1;
  // the barrier publishes tile t + 2, which the K reads two blocks ahead
  // need during tile t + 1. A block body always runs the next block's
  // QK^T and K reads (past the wave's last block they read stale LDS and
  // their results are dropped), so the body is one straight path.
  for (int t = 0; t < n_tiles; ++t) {
    if (t + 2 < n_tiles)
      issue_tile(kv_begin + (t + 2) * kTile, pg_next, smem + ((t + 2) % kStages) * kStage);
    // two bodies per tile with the score registers swapped, so the
    // next block's scores never have to be copied into place
    if (2 * t < nb) body(2 * t >= jm, 2 * t, s_a, s_b, pa0, pa1, pb0, pb1);
    if (2 * t + 1 < nb) body(2 * t + 1 >= jm, 2 * t + 1, s_b, s_a, pb0, pb1, pa0, pa1);
    if (t + 1 < n_tiles) {
      // tile t + 3's page ids; the wait below covers them too
      if (t + 3 < n_tiles) pg_next = fetch_pages(kv_begin + (t + 3) * kTile);
      wait_tile_loads();
      __syncthreads();
    }
  }

  // the last block's P V (its tile is still in the ring: nothing is issued
  // after the last barrier)
  if (nb > 0) {
    read_v(nb - 1, 0);
    read_v(nb - 1, 1);
    if ((nb - 1) & 1)
      pv(pb0, pb1);
    else
      pv(pa0, pa1);
  }
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
// q_begin, q_end, first_slot, num_splits, q_row = q_start[seq], 0, 0}.
// Splits are loaded kMergeRound at a time in rounds of independent loads:
// every load reads a real split (the index is clamped to the last one; a
// partial holds all kRows rows, so rows past q_end are in bounds too) and
// the ones past num_splits are then replaced by the empty partial, so no
// load sits behind a branch. Rounds of two match the planner's usual
// two-way split: rounds of four loaded its second partial three times and
// took 9.0 us against 7.3 us on prefill_4x512 (26 split tiles). Rows past q_end
// are computed and not stored.
constexpr int kMergeRound = 2;
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
  // an empty record pads a list to a fixed launch size
  if (q_end <= q_begin || nsplit <= 0) return;
  const int r = 32 * blockIdx.z + (threadIdx.x >> 4);
  const int d = (threadIdx.x & 15) * 8;
  const int i = q_begin + r / G;
  const int64_t qs = it1.y;  // q_start[seq], carried by the item
  float mx = -INFINITY, lsum = 0.f;
  f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsplit; s0 += kMergeRound) {
    float m[kMergeRound], l[kMergeRound];
    f32x4 x0[kMergeRound], x1[kMergeRound];
#pragma unroll
    for (int j = 0; j < kMergeRound; ++j) {
      const int64_t pr =
          (static_cast<int64_t>(first + min(s0 + j, nsplit - 1)) * num_kv_heads + kvh) * kRows + r;
      const float2 ml = *reinterpret_cast<const float2 *>(ws_ml + pr * 2);
      m[j] = ml.x;
      l[j] = ml.y;
      x0[j] = *reinterpret_cast<const f32x4 *>(ws_acc + pr * kHeadDim + d);
      x1[j] = *reinterpret_cast<const f32x4 *>(ws_acc + pr * kHeadDim + d + 4);
    }
#pragma unroll
    for (int j = 0; j < kMergeRound; ++j) {
      const bool live = s0 + j < nsplit;
      m[j] = live ? m[j] : -INFINITY;
      l[j] = live ? l[j] : 0.f;
      x0[j] = live ? x0[j] : f32x4{0.f, 0.f, 0.f, 0.f};
      x1[j] = live ? x1[j] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float cmx = mx;
#pragma unroll
    for (int j = 0; j < kMergeRound; ++j) cmx = fmaxf(cmx, m[j]);
    // All maxima -inf: both factors below are 0 and every term adds +0.
    const float f_old = mx == -INFINITY ? 0.f : exp2f(mx - cmx);
    lsum *= f_old;
    a0 *= f_old;
    a1 *= f_old;
#pragma unroll
    for (int j = 0; j < kMergeRound; ++j) {
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
                    const int32_t *items, float *ws_acc, float *ws_ml, int page_shift,
                    float scale_log2) {
  hipLaunchKernelGGL((prefill_kernel<G>), dim3(num_kv_heads, n_items), dim3(kThreads), 0,
                     st, q, q_ss,
                     q_st, q_sh, out, o_ss, o_st, o_sh, k_pool, v_pool, pool_hs, page_table,
                     pt_stride, items, ws_acc, ws_ml, num_kv_heads, page_shift, scale_log2);
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
                           vp, pool_head_stride, page_table, page_table_stride,               \
                           prefill_items, ws_acc, ws_ml, page_shift, scale_log2);             \
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
