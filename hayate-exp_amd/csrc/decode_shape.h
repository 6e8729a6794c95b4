// Shape of the decode workgroup, shared by the kernel and the planner.
#pragma once

namespace hy {

// Waves per decode workgroup; every wave leaves one partial per piece. One
// workgroup per CU and two waves (32 KB of K/V loads in flight each) keep
// HBM busiest on MI355X; more waves per CU only add contention.
constexpr int kDecodeWaves = 2;

// LDS bytes holding the query rows (G heads x head_dim bf16) of the pieces
// of one chunk; the planner closes a chunk at decode_max_pieces(G) pieces
// (at most 32, the fused append's table of new K/V rows).
constexpr int kDecodeQTableBytes = 32768;

constexpr int decode_max_pieces(int group) {
  return kDecodeQTableBytes / (group * 128 * 2) < 32 ? kDecodeQTableBytes / (group * 128 * 2)
                                                      : 32;
}

}  // namespace hy
