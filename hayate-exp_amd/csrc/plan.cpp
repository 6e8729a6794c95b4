// Tick planner: turns per-sequence (q_len, kv_len) into the work lists the
// decode and prefill kernels consume. Host-only code, no device access.
//
// Decode sequences (q_len == 1): their K/V rows, concatenated in sequence
// order, are cut into one chunk per CU and kv head, equal in cost (tokens
// plus a fixed charge for every piece after a chunk's first; cuts inside a
// sequence on multiples of 32 tokens); each piece of a sequence in
// a chunk gets W workspace slots (one per wave of the decode workgroup) and
// every decode sequence one merge item over its pieces' slots.
// Prefill sequences (q_len > 1) are cut into query tiles of kPrefillRows / G
// tokens (prefill_shape.h);
// the longest tiles are split along their key range when the simulated
// dispatch says so, and work is ordered longest first so the short items
// fill in behind the long ones.

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <functional>
#include <queue>
#include <vector>

#include "../../include/hayate_attn.h"
#include "decode_shape.h"
#include "prefill_shape.h"

namespace hy {
void set_error(const char *fmt, ...);
void clear_error();
}  // namespace hy

namespace {

constexpr int kSlice = 32;        // decode kernel's token slice
using hy::kPrefillRows;                          // rows of a prefill workgroup
constexpr int kPrefillKeys = hy::kPrefillTileKeys;  // keys per prefill step
// Prefill cost model, in units of one step (64 keys) of one workgroup,
// measured on MI355X from per-workgroup start/end stamps (s_memrealtime) on
// the 4 x 512 chunked prefill and the mixed tick: a workgroup takes 5.35 us
// + 1.86 us per step, so its fixed cost (Q load, first tiles, epilogue) is
// about 2.9 steps; a workgroup that follows another on the same CU starts
// 6.4 us (3.4 steps) after the previous one's last step; the merge launch
// costs about two steps and one split partial (write + read of its rows of
// fp32 O) a fortieth of a step.
constexpr double kPrefillFixed = 2.9;
constexpr double kPrefillGap = 3.4;
constexpr double kMergeLaunch = 2.0;
constexpr double kPartialCost = 0.025;
constexpr int kDecodeWgPerCu = 1;     // decode workgroups (chunks) per CU
using hy::kDecodeWaves;                // waves per decode workgroup: partials per piece
constexpr int64_t kMinChunk = 64;     // smallest decode chunk, in tokens (two slices)
// Cost of a decode piece after a chunk's first, in tokens: per-wave stamps
// (s_memrealtime) of the batch-32 decode on MI355X put a chunk at 43.4 /
// 45.0 / 45.7 / 46.5 us with 1 / 2 / 3 / 4 pieces for the same tokens
// (~1.1 us per piece: a partial flush, the next query rows and a partial
// last slice) at ~0.0192 us per token.
constexpr int64_t kDecodePieceCost = 64;

// How a prefill tile of `steps` key steps is cut into key ranges (parts).
// Even: the fewest parts of at most `len` steps, of equal length (+-1).
// Capped: parts of exactly `len` steps from the start and the remainder as a
// last, shorter part when it has at least `min_rest` steps (a short part
// fills the second slot of a CU whose first workgroup was short); a smaller
// remainder is spread over the full parts instead.
struct SplitRule {
  bool capped;
  int64_t len, min_rest;
};

void split_tile(int64_t steps, const SplitRule &r, std::vector<int64_t> &parts) {
  parts.clear();
  if (steps <= r.len) {
    parts.push_back(steps);
    return;
  }
  int64_t n = (steps + r.len - 1) / r.len;
  if (r.capped) {
    const int64_t full = steps / r.len;
    const int64_t rest = steps - full * r.len;
    if (rest == 0 || rest >= r.min_rest) {
      for (int64_t i = 0; i < full; ++i) parts.push_back(r.len);
      if (rest) parts.push_back(rest);
      return;
    }
    n = full;
  }
  for (int64_t i = 0; i < n; ++i) parts.push_back(steps / n + (i < steps % n ? 1 : 0));
}

// Makespan (in steps) of prefill tiles cut by `rule`, dispatched longest
// first onto `slots` workgroup slots (each kv head a separate workgroup),
// plus the merge launch and the merge traffic of the partials they create.
// With the slots a multiple of the kv heads, the copies of an item for the
// kv heads go to equally loaded slots, so one head on slots / heads slots
// gives the same makespan. The buffers are kept between calls, and a run
// stops as soon as it cannot end below `bound` (its value is then >= bound).
struct PrefillSim {
  std::vector<double> costs, free_at;
  std::vector<int64_t> parts;

  double cost(const std::vector<int64_t> &tile_steps, const SplitRule &rule, int num_kv_heads,
              int64_t slots, double bound) {
    costs.clear();
    int64_t partials = 0;
    double longest = 0.0, total = 0.0;
    for (int64_t st : tile_steps) {
      split_tile(st, rule, parts);
      for (int64_t p : parts) {
        costs.push_back(static_cast<double>(p) + kPrefillFixed);
        longest = std::max(longest, costs.back());
        total += costs.back();
      }
      if (parts.size() > 1) partials += static_cast<int64_t>(parts.size());
    }
    const double extra =
        (partials ? kMergeLaunch : 0.0) + kPartialCost * static_cast<double>(partials * num_kv_heads);
    int copies = num_kv_heads;
    if (slots % num_kv_heads == 0) {
      slots /= num_kv_heads;
      copies = 1;
    }
    // Lower bounds first: the longest part, and all the work spread evenly.
    const double lower = std::max(longest, total * copies / static_cast<double>(slots)) + extra;
    if (costs.empty() || lower >= bound) return lower;
    std::sort(costs.begin(), costs.end(), std::greater<double>());
    free_at.assign(static_cast<size_t>(slots), 0.0);  // a min-heap (all equal)
    double makespan = 0.0;
    for (double c : costs)
      for (int h = 0; h < copies; ++h) {
        std::pop_heap(free_at.begin(), free_at.end(), std::greater<double>());
        double &slot = free_at.back();
        slot += c + (slot > 0.0 ? kPrefillGap : 0.0);
        makespan = std::max(makespan, slot);
        std::push_heap(free_at.begin(), free_at.end(), std::greater<double>());
        if (makespan + extra >= bound) return makespan + extra;
      }
    return makespan + extra;
  }
};

}  // namespace

extern "C" int hy_plan_tick(const int32_t *q_lens, const int32_t *kv_lens,
                            int32_t num_seqs, int32_t num_q_heads,
                            int32_t num_kv_heads, int32_t page_size,
                            int32_t num_cus, int32_t target_tokens_per_split,
                            int32_t *decode_items, int32_t decode_capacity,
                            int32_t *merge_items, int32_t merge_capacity,
                            int32_t *prefill_items, int32_t prefill_capacity,
                            int32_t *prefill_merge_items, int32_t prefill_merge_capacity,
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
  if (page_size < kSlice || (page_size & (page_size - 1))) {
    hy::set_error("hy_plan_tick: page_size %d must be a power of two >= %d", page_size, kSlice);
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

  // Decode: the K/V rows of all decode sequences, concatenated in sequence
  // order, form one token stream per kv head that is cut into n_chunks
  // chunks of equal cost, one workgroup each. A cut inside a sequence
  // falls on a multiple of 32 tokens of that sequence. A chunk holds one or
  // more pieces (the part of one sequence inside the chunk); each wave of a
  // chunk's workgroup leaves one partial per piece, and the merge pass
  // combines all partials of a sequence.
  std::vector<int32_t> q_begin(static_cast<size_t>(num_seqs) + 1, 0);
  for (int b = 0; b < num_seqs; ++b) q_begin[b + 1] = q_begin[b] + q_lens[b];
  int64_t n_chunks = 0;
  if (decode_tokens > 0) {
    if (target_tokens_per_split > 0) {
      n_chunks = (decode_tokens + target_tokens_per_split - 1) / target_tokens_per_split;
    } else {
      const int64_t cus = num_cus > 0 ? num_cus : 256;
      n_chunks = std::max<int64_t>(1, (cus * kDecodeWgPerCu + num_kv_heads - 1) / num_kv_heads);
      n_chunks = std::min<int64_t>(n_chunks, std::max<int64_t>(1, decode_tokens / kMinChunk));
    }
  }
  struct PieceRec {
    int32_t seq, t0, t1, slice_begin;
  };
  struct ChunkRec {
    int32_t piece_begin, piece_end, n_slices;
  };
  struct DecodeCut {
    std::vector<PieceRec> pieces;
    std::vector<ChunkRec> chunks;
  };
  const int32_t max_pieces = hy::decode_max_pieces(G);
  // Cuts the decode stream into n_chunks chunks of equal cost, where a
  // chunk's cost is its tokens plus `piece_cost` for every piece after its
  // first, and `total` is the whole stream's cost.
  auto cut_stream = [&](int64_t total, int64_t piece_cost, DecodeCut &d) {
    d.pieces.clear();
    d.chunks.clear();
    int64_t pos = 0;          // stream cost before the next piece
    int64_t chunk = 0;        // index of the chunk being filled
    int64_t chunk_start = 0;  // stream cost where it began
    int32_t first = 0;        // its first piece
    int32_t slices = 0;       // its slices so far
    auto close_chunk = [&]() {
      if (static_cast<int32_t>(d.pieces.size()) > first)
        d.chunks.push_back({first, static_cast<int32_t>(d.pieces.size()), slices});
      first = static_cast<int32_t>(d.pieces.size());
      slices = 0;
      ++chunk;
      chunk_start = pos;
    };
    // Where the chunk being filled should end: the rest of the stream shared
    // evenly by the chunks still to fill. A chunk that the piece limit closed
    // early thus leaves its unfilled share to all later chunks instead of
    // moving every later cut one chunk ahead of the stream.
    auto chunk_target = [&]() -> int64_t {
      return chunk_start + (total - chunk_start) / (n_chunks - chunk);
    };
    for (int b = 0; b < num_seqs; ++b) {
      if (q_lens[b] != 1) continue;
      const int64_t kv = kv_lens[b];
      int64_t t = 0;
      while (t < kv) {
        // stream cost at token t once the piece's own cost is paid
        const int64_t at =
            pos + (static_cast<int32_t>(d.pieces.size()) > first ? piece_cost : 0);
        int64_t end = kv;
        bool cut = false;
        if (chunk < n_chunks - 1) {
          const int64_t chunk_end = chunk_target();
          if (chunk_end - at < kv - t) {
            end = std::min<int64_t>(
                kv, std::max<int64_t>(t, t + (chunk_end - at + kSlice / 2) / kSlice * kSlice));
            cut = true;
          }
        }
        if (end > t) {
          d.pieces.push_back({b, static_cast<int32_t>(t), static_cast<int32_t>(end), slices});
          slices += static_cast<int32_t>((end - t + kSlice - 1) / kSlice);
          pos = at + (end - t);
          t = end;
        }
        // A chunk also ends at the size of the kernel's query table.
        if (cut || static_cast<int32_t>(d.pieces.size()) - first >= max_pieces) close_chunk();
      }
    }
    if (static_cast<int32_t>(d.pieces.size()) > first)
      d.chunks.push_back({first, static_cast<int32_t>(d.pieces.size()), slices});
  };
  // The costliest chunk: its slices' tokens plus kDecodePieceCost for every
  // piece after its first.
  auto max_chunk_cost = [&](const DecodeCut &d) {
    int64_t worst = 0;
    for (const ChunkRec &c : d.chunks)
      worst = std::max<int64_t>(worst, static_cast<int64_t>(c.n_slices) * kSlice +
                                           kDecodePieceCost * (c.piece_end - c.piece_begin - 1));
    return worst;
  };
  // Equal tokens per chunk first; then cuts that price each extra piece,
  // the stream's total cost taken from the previous cut's piece count; the
  // cut with the cheapest costliest chunk is kept.
  DecodeCut best, trial;
  cut_stream(decode_tokens, 0, best);
  int64_t best_cost = max_chunk_cost(best);
  int64_t total = decode_tokens;
  for (int pass = 0; pass < 3 && n_chunks > 1; ++pass) {
    cut_stream(total, kDecodePieceCost, trial);
    const int64_t c = max_chunk_cost(trial);
    total = decode_tokens + kDecodePieceCost * static_cast<int64_t>(trial.pieces.size() -
                                                                    trial.chunks.size());
    if (c < best_cost) {
      best_cost = c;
      std::swap(best, trial);
    }
  }
  const std::vector<PieceRec> &pieces = best.pieces;
  const std::vector<ChunkRec> &chunks = best.chunks;
  // One merge item per decode sequence over its pieces' slots (its pieces
  // are consecutive).
  int32_t n_merge = 0, n_pre = 0;
  for (size_t i = 0; i < pieces.size();) {
    size_t j = i;
    while (j < pieces.size() && pieces[j].seq == pieces[i].seq) ++j;
    if (n_merge >= merge_capacity) {
      hy::set_error("hy_plan_tick: merge capacity %d too small", merge_capacity);
      return HY_ENOSPACE;
    }
    int32_t *mt = merge_items + 4 * n_merge++;
    mt[0] = pieces[i].seq;
    mt[1] = kDecodeWaves * static_cast<int32_t>(i);
    mt[2] = kDecodeWaves * static_cast<int32_t>(j - i);
    mt[3] = q_begin[pieces[i].seq];
    i = j;
  }
  const int32_t n_dec = static_cast<int32_t>(chunks.size());
  const int32_t n_pieces = static_cast<int32_t>(pieces.size());
  const int32_t n_slots = kDecodeWaves * n_pieces;
  if (static_cast<int64_t>(n_dec) + n_pieces > decode_capacity) {
    hy::set_error("hy_plan_tick: decode capacity %d too small (need %d)", decode_capacity,
                  n_dec + n_pieces);
    return HY_ENOSPACE;
  }
  // Chunk records carry their first piece so that a workgroup can issue its
  // first loads after one dependent read.
  for (int32_t i = 0; i < n_dec; ++i) {
    int32_t *it = decode_items + 8 * i;
    const PieceRec &f = pieces[chunks[i].piece_begin];
    it[0] = chunks[i].piece_begin;
    it[1] = chunks[i].piece_end;
    it[2] = chunks[i].n_slices;
    it[3] = f.seq;
    it[4] = f.t0;
    it[5] = f.t1;
    it[6] = kDecodeWaves * chunks[i].piece_begin;
    it[7] = q_begin[f.seq];
  }
  for (int32_t i = 0; i < n_pieces; ++i) {
    int32_t *it = decode_items + 8 * (n_dec + i);
    it[0] = pieces[i].seq;
    it[1] = pieces[i].t0;
    it[2] = pieces[i].t1;
    it[3] = kDecodeWaves * i;
    it[4] = pieces[i].slice_begin;
    it[5] = q_begin[pieces[i].seq];
    it[6] = kv_lens[pieces[i].seq] - 1;  // position of the sequence's query token
    it[7] = pieces[i].t1 == kv_lens[pieces[i].seq];  // the piece holds that token
  }

  // Prefill: query tiles of kPrefillRows / G tokens; the key range of a tile is
  // [0, cache_len + q_end). The longest tiles are split into key ranges by
  // the split rule whose simulated run is shortest.
  struct Tile {
    int32_t seq, q0, q1, kv_end;
    int64_t steps;
  };
  std::vector<Tile> tiles;
  const int tile = kPrefillRows / G;
  int64_t max_tile_steps = 0;
  for (int b = 0; b < num_seqs; ++b) {
    const int ql = q_lens[b];
    if (ql <= 1) continue;
    const int cache = kv_lens[b] - ql;
    for (int q0 = 0; q0 < ql; q0 += tile) {
      const int q1 = std::min(ql, q0 + tile);
      const int64_t st = (cache + q1 + kPrefillKeys - 1) / kPrefillKeys;
      tiles.push_back({b, q0, q1, cache + q1, st});
      max_tile_steps = std::max(max_tile_steps, st);
    }
  }
  SplitRule rule{false, std::max<int64_t>(max_tile_steps, 1), 0};
  if (!tiles.empty()) {
    std::vector<int64_t> tile_steps;
    for (const Tile &t : tiles) tile_steps.push_back(t.steps);
    const int64_t slots = static_cast<int64_t>(num_cus > 0 ? num_cus : 256) * hy::kPrefillWgPerCu;
    PrefillSim sim;
    double best = sim.cost(tile_steps, rule, num_kv_heads, slots, HUGE_VAL);
    // Candidates: every length down to 2 steps for short ranges, at most 32
    // evenly spaced ones for long ranges (the simulation is cheap), each cut
    // evenly and capped with a few remainder thresholds.
    const int64_t top = rule.len;
    const int64_t step = std::max<int64_t>(1, (top - 2) / 32);
    for (int64_t len = top - step; len >= 2; len -= step) {
      const SplitRule cands[] = {{false, len, 0}, {true, len, 1}, {true, len, 2},
                                 {true, len, 4}, {true, len, 8}, {true, len, len / 2}};
      for (const SplitRule &c : cands) {
        const double t = sim.cost(tile_steps, c, num_kv_heads, slots, best);
        if (t < best) {
          best = t;
          rule = c;
        }
      }
    }
  }
  struct PItem {
    int32_t seq, q0, q1, kv0, kv1, slot;
  };
  std::vector<PItem> pitems;
  int32_t n_pmerge = 0, n_pslots = 0;
  std::vector<int64_t> lens;
  for (const Tile &t : tiles) {
    split_tile(t.steps, rule, lens);
    const int64_t n = static_cast<int64_t>(lens.size());
    int64_t parts = 0, a = 0;
    for (int64_t len : lens) {
      const int32_t kv0 = static_cast<int32_t>(a * kPrefillKeys);
      const int32_t kv1 = static_cast<int32_t>(std::min<int64_t>(t.kv_end, (a + len) * kPrefillKeys));
      pitems.push_back({t.seq, t.q0, t.q1, kv0, kv1, n > 1 ? n_pslots + static_cast<int32_t>(parts) : -1});
      ++parts;
      a += len;
    }
    if (n > 1) {
      if (n_pmerge >= prefill_merge_capacity) {
        hy::set_error("hy_plan_tick: prefill merge capacity %d too small", prefill_merge_capacity);
        return HY_ENOSPACE;
      }
      int32_t *mt = prefill_merge_items + 8 * n_pmerge++;
      mt[0] = t.seq;
      mt[1] = t.q0;
      mt[2] = t.q1;
      mt[3] = n_pslots;
      mt[4] = static_cast<int32_t>(parts);
      mt[5] = q_begin[t.seq];
      mt[6] = mt[7] = 0;
      n_pslots += static_cast<int32_t>(parts);
    }
  }
  std::stable_sort(pitems.begin(), pitems.end(), [](const PItem &a, const PItem &b) {
    return a.kv1 - a.kv0 > b.kv1 - b.kv0;
  });
  if (static_cast<int64_t>(pitems.size()) > prefill_capacity) {
    hy::set_error("hy_plan_tick: prefill capacity %d too small (need %zu)", prefill_capacity,
                  pitems.size());
    return HY_ENOSPACE;
  }
  for (const PItem &p : pitems) {
    int32_t *pt = prefill_items + 8 * n_pre++;
    pt[0] = p.seq;
    pt[1] = p.q0;
    pt[2] = p.q1;
    pt[3] = p.kv0;
    pt[4] = p.kv1;
    pt[5] = p.slot;
    pt[6] = q_begin[p.seq];
    pt[7] = kv_lens[p.seq] - q_lens[p.seq];  // cached keys before the chunk
  }
  counts_out[0] = n_dec;
  counts_out[1] = n_merge;
  counts_out[2] = n_slots;
  counts_out[3] = n_pre;
  counts_out[4] = n_pmerge;
  counts_out[5] = n_pslots;
  counts_out[6] = n_pieces;
  return HY_OK;
}
