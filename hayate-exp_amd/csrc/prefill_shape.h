// Shape of a prefill work item, shared by the planner (host) and the prefill
// kernel: both must agree on it, and the split workspace is laid out by it.
#pragma once

namespace hy {

// (token, head) rows of one prefill workgroup: kPrefillRows / G query tokens
// times the G query heads of one kv head. Waves hold 32 rows each.
#ifndef HY_PREFILL_ROWS
#define HY_PREFILL_ROWS 256
#endif
constexpr int kPrefillRows = HY_PREFILL_ROWS;
// Keys per LDS tile of the prefill kernel; split key ranges start at
// multiples of it.
#ifndef HY_PREFILL_TILE_KEYS
#define HY_PREFILL_TILE_KEYS 64
#endif
constexpr int kPrefillTileKeys = HY_PREFILL_TILE_KEYS;
// Prefill workgroups resident per CU (registers and LDS allow this many).
constexpr int kPrefillWgPerCu = kPrefillRows <= 128 ? 2 : 1;

}  // namespace hy
