// Split-K GQA paged decode attention (one query token per sequence).
//
// Grid: (decode item, kv head). A workgroup of 4 waves owns one token range
// [tok_begin, tok_end) of one sequence (a "split") and one kv head, and
// serves all G = num_q_heads / num_kv_heads query heads of that kv head from
// a single read of every K/V row (GQA sharing).
//
// The range is walked in 32-token slices (a slice never crosses a page since
// page_size is a multiple of 32); wave w takes slices w, w + 4, ... and keeps
// its own online-softmax state, so waves never synchronise until the end.
//
// Per slice and wave (lane l, n = l % 16, g = l / 16):
//   QK^T on MFMA  v_mfma_f32_16x16x32_bf16, A = K rows (16 tokens x 32 dims,
//                 loaded straight from HBM, lane n reads 16 B of row n),
//                 B = Q (32 dims x 16 columns; column n < G is query head n).
//                 C[token 4g + i][head n] lands in lane (n, g) register i.
//   softmax       exp2 domain, running max per head across the wave.
//   PV on VALU    lane (n, g) owns dims 8n..8n+7 and the tokens 16b + 4g + i
//                 whose scores already sit in row g, so p is broadcast within
//                 the 16-lane row with DPP row_newbcast (no LDS round trip).
// V rows are read as 4 whole 256-byte rows per instruction; K rows as 64-byte
// segments of 16 rows. The end of the split merges the four waves in LDS and
// either writes the bf16 output (single split) or an fp32 partial
// (acc, max, sum) to the workspace. In the second case the workgroup then
// bumps the arrival counter of its (sequence, kv head); the one that arrives
// last merges all partials of the sequence (log-sum-exp) and writes the
// output, then resets the counter, so a decode call is a single launch.

#include "hy_common.h"

namespace hy {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

template <int G>
__device__ __forceinline__ float bcast_head(float x, int h) {
  // h is a compile-time constant after unrolling.
  switch (h) {
    case 0: return row_bcast<0>(x);
    case 1: return row_bcast<1>(x);
    case 2: return row_bcast<2>(x);
    case 3: return row_bcast<3>(x);
    case 4: return row_bcast<4>(x);
    case 5: return row_bcast<5>(x);
    case 6: return row_bcast<6>(x);
    case 7: return row_bcast<7>(x);
    case 8: return row_bcast<8>(x);
    case 9: return row_bcast<9>(x);
    case 10: return row_bcast<10>(x);
    case 11: return row_bcast<11>(x);
    case 12: return row_bcast<12>(x);
    case 13: return row_bcast<13>(x);
    case 14: return row_bcast<14>(x);
    default: return row_bcast<15>(x);
  }
}

template <int G>
__global__ __launch_bounds__(256) void decode_kernel(
    const uint16_t *__restrict__ q, int64_t q_ss, int64_t q_st, int64_t q_sh,
    uint16_t *__restrict__ out, int64_t o_ss, int64_t o_st, int64_t o_sh,
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool,
    int64_t pool_hs, const int32_t *__restrict__ page_table, int64_t pt_stride,
    const int32_t *__restrict__ q_start, const int32_t *__restrict__ items,
    float *__restrict__ ws_acc, float *__restrict__ ws_ml,
    int32_t *__restrict__ counters, int num_q_heads, int num_kv_heads,
    int page_size, float scale_log2) {
  __shared__ float sm_acc[4][G][kHeadDim];
  __shared__ float sm_m[4][G];
  __shared__ float sm_l[4][G];
  __shared__ int sm_last;

  const int32_t *it = items + 8 * blockIdx.x;
  const int kvh = blockIdx.y;
  const int seq = it[0];
  const int tok_begin = it[1];
  const int tok_end = it[2];
  const int slot = it[3];

  const int wave = threadIdx.x >> 6;
  const int l = threadIdx.x & 63;
  const int n = l & 15;
  const int g = l >> 4;
  const int h0 = kvh * G;

  // Q operand: column n < G is query head h0 + n (token 0 of the sequence).
  const int64_t q_row = seq * q_ss + static_cast<int64_t>(q_start[seq]) * q_st;
  bf16x8 qop[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    u32x4 w = {0u, 0u, 0u, 0u};
    if (n < G) w = load16(q + q_row + (h0 + n) * q_sh + kk * 32 + g * 8);
    qop[kk] = __builtin_bit_cast(bf16x8, w);
  }

  float m_run = -INFINITY;  // per head n (lanes n < G meaningful)
  float l_run = 0.f;        // lane-partial sum for head n
  float acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;

  const uint16_t *kh = k_pool + kvh * pool_hs;
  const uint16_t *vh = v_pool + kvh * pool_hs;
  const int32_t *pt = page_table + seq * pt_stride;
  const int n_slices = (tok_end - tok_begin + 31) >> 5;

  for (int s = wave; s < n_slices; s += 4) {
    const int t0 = tok_begin + s * 32;
    const int64_t p0 = static_cast<int64_t>(pt[t0 / page_size]) * page_size + (t0 % page_size);
    const uint16_t *kb = kh + p0 * kHeadDim;
    const uint16_t *vb = vh + p0 * kHeadDim;

    u32x4 kreg[2][4];
    u32x4 vreg[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        kreg[b][kk] = load16(kb + (16 * b + n) * kHeadDim + kk * 32 + g * 8);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        vreg[b][i] = load16(vb + (16 * b + 4 * g + i) * kHeadDim + n * 8);

    f32x4 sc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      sc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, kreg[b][kk]), qop[kk], sc[b], 0, 0, 0);
    }

    const bool partial = t0 + 32 > tok_end;
    float mloc = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = sc[b][i] * scale_log2;
        if (partial && t0 + 16 * b + 4 * g + i >= tok_end) x = -INFINITY;
        sc[b][i] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = exp2f(sc[b][i] - m_new);
        sc[b][i] = p;
        psum += p;
      }
    l_run = l_run * alpha + psum;

    if (partial) {
      // Rows past the end may hold any bits (the pool is never cleared);
      // zero them so that p = 0 cannot meet a NaN.
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (t0 + 16 * b + 4 * g + i >= tok_end) vreg[b][i] = u32x4{0u, 0u, 0u, 0u};
    }

#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float a = bcast_head<G>(alpha, h);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] *= a;
    }
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float vf[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          vf[2 * j] = bf16_lo(vreg[b][i][j]);
          vf[2 * j + 1] = bf16_hi(vreg[b][i][j]);
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float p = bcast_head<G>(sc[b][i], h);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] += p * vf[e];
        }
      }
  }

  // Wave-level totals: sum the four 16-lane rows.
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = acc[h][e];
      x += __shfl_xor(x, 16);
      x += __shfl_xor(x, 32);
      acc[h][e] = x;
    }
  if (g == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) sm_acc[wave][h][n * 8 + e] = acc[h][e];
    if (n < G) {
      sm_m[wave][n] = m_run;
      sm_l[wave][n] = l_run;
    }
  }
  __syncthreads();

  // Merge the four waves; thread t handles (head, dim) pairs.
  const int64_t out_row = seq * o_ss + static_cast<int64_t>(q_start[seq]) * o_st;
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += 256) {
    const int h = idx / kHeadDim;
    const int d = idx % kHeadDim;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, sm_m[w][h]);
    float lsum = 0.f, a = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = sm_m[w][h] == -INFINITY ? 0.f : exp2f(sm_m[w][h] - mx);
      lsum += f * sm_l[w][h];
      a += f * sm_acc[w][h][d];
    }
    const int hq = h0 + h;
    if (slot < 0) {
      out[out_row + hq * o_sh + d] = static_cast<uint16_t>(f32_to_bf16_rne(a / lsum));
    } else {
      const int64_t base = static_cast<int64_t>(slot) * num_q_heads + hq;
      ws_acc[base * kHeadDim + d] = a;
      if (d == 0) {
        ws_ml[base * 2 + 0] = mx;
        ws_ml[base * 2 + 1] = lsum;
      }
    }
  }
  if (slot < 0) return;

  // Publish this split's partial, then count arrivals for the sequence.
  const int group = it[4];
  const int first = it[5];
  const int nsplit = it[6];
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&counters[group * num_kv_heads + kvh], 1);
    sm_last = prev == nsplit - 1;
  }
  __syncthreads();
  if (!sm_last) return;
  __threadfence();

  // Last arrival: merge every split of this sequence for the G heads.
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += 256) {
    const int hq = h0 + idx / kHeadDim;
    const int d = idx % kHeadDim;
    float mx = -INFINITY;
    for (int s = 0; s < nsplit; ++s)
      mx = fmaxf(mx, ws_ml[(static_cast<int64_t>(first + s) * num_q_heads + hq) * 2]);
    float lsum = 0.f, a = 0.f;
    for (int s = 0; s < nsplit; ++s) {
      const int64_t base = static_cast<int64_t>(first + s) * num_q_heads + hq;
      const float f = exp2f(ws_ml[base * 2] - mx);
      lsum += f * ws_ml[base * 2 + 1];
      a += f * ws_acc[base * kHeadDim + d];
    }
    out[out_row + hq * o_sh + d] = static_cast<uint16_t>(f32_to_bf16_rne(a / lsum));
  }
  if (threadIdx.x == 0) atomicExch(&counters[group * num_kv_heads + kvh], 0);
}

template <int G>
void launch_decode(hipStream_t st, dim3 grid, const uint16_t *q, int64_t q_ss,
                   int64_t q_st, int64_t q_sh, uint16_t *out, int64_t o_ss,
                   int64_t o_st, int64_t o_sh, const uint16_t *k_pool,
                   const uint16_t *v_pool, int64_t pool_hs,
                   const int32_t *page_table, int64_t pt_stride,
                   const int32_t *q_start, const int32_t *items, float *ws_acc,
                   float *ws_ml, int32_t *counters, int num_q_heads,
                   int num_kv_heads, int page_size, float scale_log2) {
  hipLaunchKernelGGL(decode_kernel<G>, grid, dim3(256), 0, st, q, q_ss, q_st,
                     q_sh, out, o_ss, o_st, o_sh, k_pool, v_pool, pool_hs,
                     page_table, pt_stride, q_start, items, ws_acc, ws_ml,
                     counters, num_q_heads, num_kv_heads, page_size,
                     scale_log2);
}

}  // namespace
}  // namespace hy

using hy::kHeadDim;

namespace {
// Workspace layout: [acc fp32 n_slots*Hq*D][max,sum fp32 n_slots*Hq*2]
// [counters int32 n_groups*Hkv], each part 256-byte aligned.
int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }
}  // namespace

extern "C" int64_t hy_decode_workspace_bytes(int32_t n_slots, int32_t n_groups,
                                             int32_t num_q_heads,
                                             int32_t num_kv_heads,
                                             int32_t head_dim) {
  if (n_slots <= 0 || n_groups <= 0) return 0;
  const int64_t acc = align256(static_cast<int64_t>(n_slots) * num_q_heads * head_dim * 4);
  const int64_t ml = align256(static_cast<int64_t>(n_slots) * num_q_heads * 2 * 4);
  const int64_t cnt = align256(static_cast<int64_t>(n_groups) * num_kv_heads * 4);
  return acc + ml + cnt;
}

extern "C" int hy_paged_decode(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok,
    int64_t q_stride_head, void *out, int64_t o_stride_seq,
    int64_t o_stride_tok, int64_t o_stride_head, const void *k_pool,
    const void *v_pool, int64_t pool_head_stride, const int32_t *page_table,
    int64_t page_table_stride, const int32_t *q_start,
    const int32_t *decode_items, int32_t n_decode, int32_t n_groups,
    int32_t n_slots, void *workspace, int64_t workspace_bytes,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t page_size, float scale, void *stream) {
  hy::clear_error();
  HY_REQUIRE(num_seqs >= 1, "num_seqs must be positive");
  HY_REQUIRE(num_kv_heads >= 1 && num_q_heads >= num_kv_heads &&
                 num_q_heads % num_kv_heads == 0,
             "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)",
             num_q_heads, num_kv_heads);
  HY_REQUIRE_SUPPORTED(head_dim == kHeadDim, "head_dim %d unsupported (need %d)",
                       head_dim, kHeadDim);
  HY_REQUIRE_SUPPORTED(page_size >= 32 && page_size % 32 == 0,
                       "page_size %d unsupported (multiple of 32 required)", page_size);
  HY_REQUIRE(n_decode >= 0 && n_groups >= 0 && n_slots >= 0,
             "item counts must be non-negative");
  HY_REQUIRE((n_groups == 0) == (n_slots == 0), "n_groups and n_slots must be both zero or both positive");
  if (n_decode == 0) return HY_OK;
  HY_REQUIRE(q && out && k_pool && v_pool && page_table && q_start && decode_items,
             "hy_paged_decode: null pointer argument");
  const int64_t need =
      hy_decode_workspace_bytes(n_slots, n_groups, num_q_heads, num_kv_heads, head_dim);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    hy::set_error("workspace too small: need %lld bytes, got %lld",
                  static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    return HY_ENOSPACE;
  }
  float *ws_acc = nullptr, *ws_ml = nullptr;
  int32_t *counters = nullptr;
  if (need > 0) {
    char *base = static_cast<char *>(workspace);
    const int64_t acc = align256(static_cast<int64_t>(n_slots) * num_q_heads * head_dim * 4);
    const int64_t ml = align256(static_cast<int64_t>(n_slots) * num_q_heads * 2 * 4);
    ws_acc = reinterpret_cast<float *>(base);
    ws_ml = reinterpret_cast<float *>(base + acc);
    counters = reinterpret_cast<int32_t *>(base + acc + ml);
  }
  const int G = num_q_heads / num_kv_heads;
  const float scale_log2 = scale * hy::kLog2e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(n_decode, num_kv_heads);
  const uint16_t *qq = static_cast<const uint16_t *>(q);
  uint16_t *oo = static_cast<uint16_t *>(out);
  const uint16_t *kp = static_cast<const uint16_t *>(k_pool);
  const uint16_t *vp = static_cast<const uint16_t *>(v_pool);
#define HY_DECODE_CASE(GG)                                                       \
  case GG:                                                                       \
    hy::launch_decode<GG>(st, grid, qq, q_stride_seq, q_stride_tok,              \
                          q_stride_head, oo, o_stride_seq, o_stride_tok,         \
                          o_stride_head, kp, vp, pool_head_stride, page_table,   \
                          page_table_stride, q_start, decode_items, ws_acc,      \
                          ws_ml, counters, num_q_heads, num_kv_heads, page_size, \
                          scale_log2);                                           \
    break;
  switch (G) {
    HY_DECODE_CASE(1)
    HY_DECODE_CASE(2)
    HY_DECODE_CASE(4)
    HY_DECODE_CASE(8)
    HY_DECODE_CASE(16)
    default:
      hy::set_error("GQA group size %d unsupported (1, 2, 4, 8, 16)", G);
      return HY_EUNSUPPORTED;
  }
#undef HY_DECODE_CASE
  return hy::launch_status("hy_paged_decode");
}
