// Tick planner: turns per-sequence (q_len, kv_len) into the work lists the
// decode and prefill kernels consume. Host-only code, no device access.
//
// Decode sequences (q_len == 1) are cut into token ranges ("splits") of equal
// size so that every workgroup streams about the same number of K/V bytes,
// whatever the spread of context lengths; a sequence with more than one
// split gets consecutive workspace slots and one merge group: the last of
// its workgroups to finish merges the partials inside the decode kernel.
// Prefill sequences (q_len > 1) are cut into query tiles of 128 / G tokens;
// tiles are ordered by the number of keys they read, longest first, so the
// short tiles fill in behind the long ones.

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

#include "../../include/hayate_attn.h"

namespace hy {
void set_error(const char *fmt, ...);
void clear_error();
}  // namespace hy

namespace {

constexpr int kSlice = 32;  // decode kernel's token slice
constexpr int kPrefillRows = 128;

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

}  // namespace

extern "C" int hy_plan_tick(const int32_t *q_lens, const int32_t *kv_lens,
                            int32_t num_seqs, int32_t num_q_heads,
                            int32_t num_kv_heads, int32_t page_size,
                            int32_t num_cus, int32_t target_tokens_per_split,
                            int32_t *decode_items, int32_t decode_capacity,
                            int32_t *prefill_items, int32_t prefill_capacity,
                            int32_t *counts_out) {
  hy::clear_error();
  if (num_seqs < 0 || (num_seqs > 0 && (q_lens == nullptr || kv_lens == nullptr)) ||
      counts_out == nullptr) {
    hy::set_error("hy_plan_tick: invalid sequence arrays");
    return HY_EINVAL;
  }
  if (num_kv_heads < 1 || num_q_heads < num_kv_heads || num_q_heads % num_kv_heads) {
    hy::set_error("hy_plan_tick: num_q_heads (%d) must be a multiple of num_kv_heads (%d)",
                  num_q_heads, num_kv_heads);
    return HY_EINVAL;
  }
  if (page_size < kSlice || page_size % kSlice) {
    hy::set_error("hy_plan_tick: page_size %d must be a multiple of %d", page_size, kSlice);
    return HY_EUNSUPPORTED;
  }
  const int G = num_q_heads / num_kv_heads;
  if (kPrefillRows % G) {
    hy::set_error("hy_plan_tick: GQA group size %d unsupported", G);
    return HY_EUNSUPPORTED;
  }
  int64_t decode_tokens = 0;
  for (int b = 0; b < num_seqs; ++b) {
    if (q_lens[b] < 0 || kv_lens[b] < q_lens[b]) {
      hy::set_error("hy_plan_tick: sequence %d has q_len %d, kv_len %d", b, q_lens[b],
                    kv_lens[b]);
      return HY_EINVAL;
    }
    if (q_lens[b] == 1) decode_tokens += kv_lens[b];
  }

  // Split length: about four workgroups per CU across all kv heads, in whole
  // 128-token units, at least 256 tokens so that each wave keeps two slices.
  int64_t split = target_tokens_per_split;
  if (split <= 0) {
    const int64_t cus = num_cus > 0 ? num_cus : 256;
    const int64_t want = (decode_tokens * num_kv_heads + 4 * cus - 1) / (4 * cus);
    split = std::max<int64_t>(256, round_up(std::max<int64_t>(want, 1), 128));
  } else {
    split = round_up(split, kSlice);
  }

  int32_t n_dec = 0, n_groups = 0, n_pre = 0, n_slots = 0;
  for (int b = 0; b < num_seqs; ++b) {
    if (q_lens[b] != 1) continue;
    const int64_t kv = kv_lens[b];
    // Equal-length splits (a multiple of 32 each) instead of a short tail.
    int64_t nsplit = (kv + split - 1) / split;
    const int64_t len = round_up((kv + nsplit - 1) / nsplit, kSlice);
    nsplit = (kv + len - 1) / len;
    const bool merged = nsplit > 1;
    if (n_dec + nsplit > decode_capacity) {
      hy::set_error("hy_plan_tick: decode capacity %d too small", decode_capacity);
      return HY_ENOSPACE;
    }
    for (int64_t s = 0; s < nsplit; ++s) {
      int32_t *it = decode_items + 8 * n_dec++;
      it[0] = b;
      it[1] = static_cast<int32_t>(s * len);
      it[2] = static_cast<int32_t>(std::min<int64_t>(kv, (s + 1) * len));
      it[3] = merged ? n_slots + static_cast<int32_t>(s) : -1;
      it[4] = merged ? n_groups : -1;
      it[5] = merged ? n_slots : -1;
      it[6] = static_cast<int32_t>(nsplit);
      it[7] = 0;
    }
    if (merged) {
      n_slots += static_cast<int32_t>(nsplit);
      ++n_groups;
    }
  }

  struct Tile {
    int32_t seq, q0, q1;
    int64_t keys;
  };
  std::vector<Tile> tiles;
  const int tile = kPrefillRows / G;
  for (int b = 0; b < num_seqs; ++b) {
    const int ql = q_lens[b];
    if (ql <= 1) continue;
    const int cache = kv_lens[b] - ql;
    for (int q0 = 0; q0 < ql; q0 += tile) {
      const int q1 = std::min(ql, q0 + tile);
      tiles.push_back({b, q0, q1, static_cast<int64_t>(cache) + q1});
    }
  }
  std::stable_sort(tiles.begin(), tiles.end(),
                   [](const Tile &a, const Tile &b) { return a.keys > b.keys; });
  if (static_cast<int64_t>(tiles.size()) > prefill_capacity) {
    hy::set_error("hy_plan_tick: prefill capacity %d too small (need %zu)",
                  prefill_capacity, tiles.size());
    return HY_ENOSPACE;
  }
  for (const Tile &t : tiles) {
    int32_t *pt = prefill_items + 4 * n_pre++;
    pt[0] = t.seq;
    pt[1] = t.q0;
    pt[2] = t.q1;
    pt[3] = 0;
  }
  counts_out[0] = n_dec;
  counts_out[1] = n_groups;
  counts_out[2] = n_pre;
  counts_out[3] = n_slots;
  return HY_OK;
}
