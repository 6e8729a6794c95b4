// Split-K GQA paged decode attention (one query token per sequence).
//
// Grid: (kv head, decode item). A workgroup of 4 waves owns one token range
// [tok_begin, tok_end) of one sequence (a "split") and one kv head, and
// serves all G = num_q_heads / num_kv_heads query heads of that kv head from
// a single read of every K/V row (GQA sharing).
//
// The range is walked in 32-token slices (a slice never crosses a page since
// page_size is a power of two >= 32); wave w takes slices w, w + 4, ... and
// keeps its own online-softmax state, so waves never synchronise until the
// end. Both products run on v_mfma_f32_16x16x32_bf16 (lane l, n = l % 16,
// g = l / 16):
//
//   S = K Q^T   A = K rows (16 tokens x 32 dims), loaded from HBM straight
//               into registers (lane n reads 16 B of row n, a whole 256-byte
//               row per 16 lanes); B = Q^T, column n < G is query head n.
//               Lane (n, g) ends with the scores of head n for the slice
//               tokens 4g + i and 16 + 4g + i (i < 4).
//   O^T += V^T P^T  B = P^T must give lane (n, g) eight probabilities of
//               head n: exactly its own eight scores, once MFMA k index
//               8g + j stands for token (j < 4 ? 4g + j : 16 + 4g + j - 4).
//               A = V^T comes from LDS: V rows are loaded into registers
//               with whole-row 16-byte loads, written to a per-wave LDS
//               buffer and read back transposed with ds_read_b64_tr_b16,
//               which hands lane m of a 16-lane group four consecutive rows
//               of column m. (Streaming V with the direct HBM -> LDS load
//               makes the compiler wait for every outstanding load before
//               any LDS read, which serialises the prefetch below.)
//
// V rows sit in LDS with a 288-byte stride so that the four rows one
// transposed read touches start 8 banks apart. The K and V registers are double
// buffered: slice s + 4 is in flight while slice s is consumed. Rows past the
// end of the context may hold any bits; their scores are masked and their V
// values zeroed before the MFMA so that 0 * NaN never occurs.
//
// The end of a split merges the four waves in LDS and writes either the bf16
// output (single split) or an fp32 partial (acc, max, sum) to the workspace;
// decode_merge_kernel then combines the partials of each split sequence
// (log-sum-exp). The merge is a second launch (hy_paged_decode_merge) on the
// same stream: the kernel boundary publishes the partials without any
// device-scope fence.

#include "hy_common.h"

namespace hy {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWaves = 4;
constexpr int kSlice = 32;                       // tokens per slice
constexpr int kVRow = kHeadDim + 16;             // LDS V row stride (u16): 288 bytes
constexpr int kSliceElems = kSlice * kVRow;      // u16 per V transpose buffer

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Registers of one slice for one wave.
struct SliceRegs {
  u32x4 k[2][4];  // A operand of S = K Q^T: rows 16b + n, dims 32kk + 8g .. +7
  u32x4 v[8];     // V row 4i + g, dims 8n .. 8n + 7 (staged into LDS)
};

// Issues the 16 loads of the slice starting at logical token t0 (a multiple
// of 32, so the slice lies in one page) into registers. t0 and the page id
// are wave-uniform, so the page-table read is a scalar load. Every K/V row
// is read once per launch: the loads are nontemporal.
__device__ __forceinline__ void issue_slice(SliceRegs &r, const uint16_t *__restrict__ kh,
                                            const uint16_t *__restrict__ vh,
                                            const int32_t *__restrict__ pt, int t0,
                                            int page_shift, int lane) {
  const int page = pt[t0 >> page_shift];
  const int64_t p0 = (static_cast<int64_t>(page) << page_shift) + (t0 & ((1 << page_shift) - 1));
  const uint16_t *kb = kh + p0 * kHeadDim;
  const uint16_t *vb = vh + p0 * kHeadDim;
  const int n = lane & 15;
  const int g = lane >> 4;
  // V first: it is consumed (staged into LDS) before the K registers.
#pragma unroll
  for (int i = 0; i < 8; ++i) r.v[i] = load16_stream(vb + (4 * i + g) * kHeadDim + n * 8);
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      r.k[b][kk] = load16_stream(kb + (16 * b + n) * kHeadDim + kk * 32 + g * 8);
  // Keep the issue group together so that a consumer placed after it waits
  // only for the loads issued before the group.
  __builtin_amdgcn_sched_barrier(0);
}

// Writes the slice's V rows into the wave's LDS buffer (288-byte rows).
__device__ __forceinline__ void stage_v(const SliceRegs &r, uint16_t *vbuf, int lane) {
  const int n = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<u32x4 *>(vbuf + (4 * i + g) * kVRow + n * 8) = r.v[i];
}

// Transposed read of V^T for dims [16 db, 16 db + 16) and the four slice
// tokens key0 .. key0 + 3 (key0 a multiple of 4): lane m of the 16-lane
// group receives V[key0 + k][16 db + m], k < 4. Lane rho
// supplies row key0 + rho / 4, dims 16 db + 4 (rho % 4) .. +3; with 288-byte
// rows the four rows start 8 banks apart, so the read is conflict-free, and
// the address is a per-lane base plus a compile-time offset.
__device__ __forceinline__ s16x4 read_vt(const uint16_t *lane_base, int key0, int db) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4 *)(const_cast<uint16_t *>(lane_base) + key0 * kVRow + 16 * db));
}

// Scores, online softmax and PV for one slice whose V rows are already in
// `vbuf`. vt_base is this lane's transposed-read base in that buffer.
template <int G>
__device__ __forceinline__ void consume_slice(const SliceRegs &r, const uint16_t *vt_base,
                                              const bf16x8 (&qop)[4], int t0, int tok_end,
                                              int lane, float scale_log2, float &m_run,
                                              float &l_run, f32x4 (&acc)[8]) {
  const int g = lane >> 4;
  f32x4 sc[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    sc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, r.k[b][kk]), qop[kk], sc[b], 0, 0, 0);
  }

  // Online softmax in the exp2 domain on raw scores: max first, then
  // p = exp2(s * c - m * c) with c = scale * log2(e) > 0.
  const bool partial = t0 + kSlice > tok_end;
  float mloc = -INFINITY;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (partial && t0 + 16 * b + 4 * g + i >= tok_end) sc[b][i] = -INFINITY;
      mloc = fmaxf(mloc, sc[b][i]);
    }
  mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
  const float m_new = fmaxf(m_run, mloc);
  const float mc = m_new * scale_log2;
  const float alpha = __builtin_amdgcn_exp2f(m_run * scale_log2 - mc);
  m_run = m_new;
  float psum = 0.f;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[b][i], scale_log2, -mc));
      sc[b][i] = p;
      psum += p;
    }
  l_run = l_run * alpha + psum;

  bf16x8 pop;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    pop[i] = static_cast<__bf16>(sc[0][i]);
    pop[4 + i] = static_cast<__bf16>(sc[1][i]);
  }

  // Rescale the accumulator only when some head's running max moved.
  if (__any(alpha != 1.0f)) {
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[db] *= alpha;
  }

  if (!partial) {
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const s16x4 lo = read_vt(vt_base, 0, db);
      const s16x4 hi = read_vt(vt_base, 16, db);
      const s16x8 v8 = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, v8), pop,
                                                        acc[db], 0, 0, 0);
    }
  } else {
    // Keys past the end: zero their V values (the rows may hold any bits).
    s16x8 keep;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      keep[k] = t0 + 4 * g + k < tok_end ? -1 : 0;
      keep[4 + k] = t0 + 16 + 4 * g + k < tok_end ? -1 : 0;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const s16x4 lo = read_vt(vt_base, 0, db);
      const s16x4 hi = read_vt(vt_base, 16, db);
      const s16x8 v8 = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7) & keep;
      acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, v8), pop,
                                                        acc[db], 0, 0, 0);
    }
  }
}

// Two waves per SIMD (two workgroups per CU): the double-buffered slice
// registers need about 240 VGPRs.
template <int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_kernel(
    const uint16_t *__restrict__ q, int64_t q_ss, int64_t q_st, int64_t q_sh,
    uint16_t *__restrict__ out, int64_t o_ss, int64_t o_st, int64_t o_sh,
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool,
    int64_t pool_hs, const int32_t *__restrict__ page_table, int64_t pt_stride,
    const int32_t *__restrict__ q_start, const int32_t *__restrict__ items,
    float *__restrict__ ws_acc, float *__restrict__ ws_ml, int num_q_heads,
    int page_shift, float scale_log2) {
  // One V transpose buffer per wave; it also holds the cross-wave merge at
  // the end when that fits.
  __shared__ __attribute__((aligned(16))) uint16_t sV[kWaves][kSliceElems];
  constexpr int kMergeFloats = kWaves * G * kHeadDim + 2 * kWaves * G;
  constexpr bool kMergeInV = kMergeFloats * sizeof(float) <= sizeof(sV);
  __shared__ float sMergeExtra[kMergeInV ? 1 : kMergeFloats];

  // Grid (kv head, item): heads vary fastest so the dispatcher walks the
  // items in the planner's longest-first order.
  const int32_t *it = items + 4 * blockIdx.y;
  const int kvh = blockIdx.x;
  const int seq = it[0];
  const int tok_begin = it[1];
  const int tok_end = it[2];
  const int slot = it[3];

  // Wave index as a scalar: every per-slice address below is wave-uniform.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int h0 = kvh * G;

  // Q^T operand: column n < G is query head h0 + n (the sequence's token).
  const int64_t q_row = seq * q_ss + static_cast<int64_t>(q_start[seq]) * q_st;
  bf16x8 qop[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    u32x4 w = {0u, 0u, 0u, 0u};
    if (n < G) w = load16(q + q_row + (h0 + n) * q_sh + kk * 32 + g * 8);
    qop[kk] = __builtin_bit_cast(bf16x8, w);
  }

  float m_run = -INFINITY;  // running max of head n (raw scores)
  float l_run = 0.f;        // lane-partial sum of head n
  f32x4 acc[8];             // O^T[16 db + 4g + i][head n]
#pragma unroll
  for (int db = 0; db < 8; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint16_t *kh = k_pool + kvh * pool_hs;
  const uint16_t *vh = v_pool + kvh * pool_hs;
  const int32_t *pt = page_table + seq * pt_stride;
  const int n_slices = (tok_end - tok_begin + kSlice - 1) / kSlice;
  uint16_t *vbuf = sV[wave];
  const uint16_t *vt_base = vbuf + (4 * g + (n >> 2)) * kVRow + 4 * (n & 3);

  // Double-buffered slice loop: the loads of slice s + 4 are in flight
  // while slice s is consumed. A slice's V rows go to LDS before the next
  // slice is issued, so at most one slice's V registers are live with two
  // slices' K registers. The steady state issues unconditionally so that
  // every wait covers only earlier loads; the tail is peeled.
  if (wave < n_slices) {
    SliceRegs ra, rb;
    int s = wave;
    issue_slice(ra, kh, vh, pt, tok_begin + kSlice * s, page_shift, lane);
    while (s + 2 * kWaves < n_slices) {
      stage_v(ra, vbuf, lane);
      issue_slice(rb, kh, vh, pt, tok_begin + kSlice * (s + kWaves), page_shift, lane);
      consume_slice<G>(ra, vt_base, qop, tok_begin + kSlice * s, tok_end, lane, scale_log2,
                       m_run, l_run, acc);
      stage_v(rb, vbuf, lane);
      issue_slice(ra, kh, vh, pt, tok_begin + kSlice * (s + 2 * kWaves), page_shift, lane);
      consume_slice<G>(rb, vt_base, qop, tok_begin + kSlice * (s + kWaves), tok_end, lane,
                       scale_log2, m_run, l_run, acc);
      s += 2 * kWaves;
    }
    stage_v(ra, vbuf, lane);
    if (s + kWaves < n_slices) {
      issue_slice(rb, kh, vh, pt, tok_begin + kSlice * (s + kWaves), page_shift, lane);
      consume_slice<G>(ra, vt_base, qop, tok_begin + kSlice * s, tok_end, lane, scale_log2,
                       m_run, l_run, acc);
      stage_v(rb, vbuf, lane);
      consume_slice<G>(rb, vt_base, qop, tok_begin + kSlice * (s + kWaves), tok_end, lane,
                       scale_log2, m_run, l_run, acc);
    } else {
      consume_slice<G>(ra, vt_base, qop, tok_begin + kSlice * s, tok_end, lane, scale_log2,
                       m_run, l_run, acc);
    }
  }

  // Wave totals of the row sums (the four 16-lane rows hold disjoint tokens).
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  __syncthreads();  // every wave is done with its V buffer
  float *sm_acc = kMergeInV ? reinterpret_cast<float *>(&sV[0][0]) : sMergeExtra;
  float *sm_m = sm_acc + kWaves * G * kHeadDim;             // [wave][G]
  float *sm_l = sm_m + kWaves * G;                          // [wave][G]
  if (n < G) {
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sm_acc[(wave * G + n) * kHeadDim + 16 * db + 4 * g + i] = acc[db][i];
    if (g == 0) {
      sm_m[wave * G + n] = m_run;
      sm_l[wave * G + n] = l_run;
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
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, sm_m[w * G + h]);
    float lsum = 0.f, a = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = sm_m[w * G + h];
      const float f = mw == -INFINITY ? 0.f : exp2f((mw - mx) * scale_log2);
      lsum += f * sm_l[w * G + h];
      a += f * sm_acc[(w * G + h) * kHeadDim + d];
    }
    const int hq = h0 + h;
    if (slot < 0) {
      out[out_row + hq * o_sh + d] = static_cast<uint16_t>(f32_to_bf16_rne(a / lsum));
    } else {
      const int64_t base = static_cast<int64_t>(slot) * num_q_heads + hq;
      ws_acc[base * kHeadDim + d] = a;
      if (d == 0) {
        ws_ml[base * 2 + 0] = mx * scale_log2;  // max in the exp2 domain
        ws_ml[base * 2 + 1] = lsum;
      }
    }
  }
}

// Combines the partials of split sequences: grid (merge item, q head),
// 128 threads (dims). Item = {seq, first_slot, num_splits, 0}. Up to eight
// splits are loaded in one round of independent loads.
__global__ __launch_bounds__(128) void decode_merge_kernel(
    uint16_t *__restrict__ out, int64_t o_ss, int64_t o_st, int64_t o_sh,
    const int32_t *__restrict__ q_start, const int32_t *__restrict__ items,
    const float *__restrict__ ws_acc, const float *__restrict__ ws_ml, int num_q_heads) {
  const int32_t *it = items + 4 * blockIdx.x;
  const int seq = it[0];
  const int first = it[1];
  const int nsplit = it[2];
  const int hq = blockIdx.y;
  const int d = threadIdx.x;
  float mx = -INFINITY, lsum = 0.f, a = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += 8) {
    float m[8], l[8], x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t base = static_cast<int64_t>(first + s0 + j) * num_q_heads + hq;
      const bool live = s0 + j < nsplit;
      m[j] = live ? ws_ml[base * 2] : -INFINITY;
      l[j] = live ? ws_ml[base * 2 + 1] : 0.f;
      x[j] = live ? ws_acc[base * kHeadDim + d] : 0.f;
    }
    float cmx = mx;
#pragma unroll
    for (int j = 0; j < 8; ++j) cmx = fmaxf(cmx, m[j]);
    const float r = mx == -INFINITY ? 0.f : exp2f(mx - cmx);
    lsum *= r;
    a *= r;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = m[j] == -INFINITY ? 0.f : exp2f(m[j] - cmx);
      lsum += f * l[j];
      a += f * x[j];
    }
    mx = cmx;
  }
  out[seq * o_ss + static_cast<int64_t>(q_start[seq]) * o_st + hq * o_sh + d] =
      static_cast<uint16_t>(f32_to_bf16_rne(a / lsum));
}

template <int G>
void launch_decode(hipStream_t st, dim3 grid, const uint16_t *q, int64_t q_ss, int64_t q_st,
                   int64_t q_sh, uint16_t *out, int64_t o_ss, int64_t o_st, int64_t o_sh,
                   const uint16_t *k_pool, const uint16_t *v_pool, int64_t pool_hs,
                   const int32_t *page_table, int64_t pt_stride, const int32_t *q_start,
                   const int32_t *items, float *ws_acc, float *ws_ml, int num_q_heads,
                   int page_shift, float scale_log2) {
  hipLaunchKernelGGL(decode_kernel<G>, grid, dim3(256), 0, st, q, q_ss, q_st, q_sh, out, o_ss,
                     o_st, o_sh, k_pool, v_pool, pool_hs, page_table, pt_stride, q_start, items,
                     ws_acc, ws_ml, num_q_heads, page_shift, scale_log2);
}

// Workspace layout: [acc fp32 n_slots*Hq*D][max,sum fp32 n_slots*Hq*2],
// each part 256-byte aligned.
int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace
}  // namespace hy

using hy::kHeadDim;

extern "C" int64_t hy_decode_workspace_bytes(int32_t n_slots, int32_t num_q_heads,
                                             int32_t head_dim) {
  if (n_slots <= 0) return 0;
  return hy::align256(static_cast<int64_t>(n_slots) * num_q_heads * head_dim * 4) +
         hy::align256(static_cast<int64_t>(n_slots) * num_q_heads * 2 * 4);
}

extern "C" int hy_paged_decode(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok, int64_t q_stride_head,
    void *out, int64_t o_stride_seq, int64_t o_stride_tok, int64_t o_stride_head,
    const void *k_pool, const void *v_pool, int64_t pool_head_stride,
    const int32_t *page_table, int64_t page_table_stride, const int32_t *q_start,
    const int32_t *decode_items, int32_t n_decode, int32_t n_slots, void *workspace,
    int64_t workspace_bytes,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t page_size, float scale, void *stream) {
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
  HY_REQUIRE(n_decode >= 0 && n_slots >= 0, "item counts must be non-negative");
  if (n_decode == 0) return HY_OK;
  HY_REQUIRE(q && out && k_pool && v_pool && page_table && q_start && decode_items,
             "hy_paged_decode: null pointer argument");
  const int64_t need = hy_decode_workspace_bytes(n_slots, num_q_heads, head_dim);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    hy::set_error("workspace too small: need %lld bytes, got %lld",
                  static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    return HY_ENOSPACE;
  }
  float *ws_acc = nullptr, *ws_ml = nullptr;
  if (need > 0) {
    ws_acc = static_cast<float *>(workspace);
    ws_ml = reinterpret_cast<float *>(
        static_cast<char *>(workspace) +
        hy::align256(static_cast<int64_t>(n_slots) * num_q_heads * head_dim * 4));
  }
  const int G = num_q_heads / num_kv_heads;
  const float scale_log2 = scale * hy::kLog2e;
  const int page_shift = __builtin_ctz(static_cast<unsigned>(page_size));
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(num_kv_heads, n_decode);
  const uint16_t *qq = static_cast<const uint16_t *>(q);
  uint16_t *oo = static_cast<uint16_t *>(out);
  const uint16_t *kp = static_cast<const uint16_t *>(k_pool);
  const uint16_t *vp = static_cast<const uint16_t *>(v_pool);
#define HY_DECODE_CASE(GG)                                                                    \
  case GG:                                                                                    \
    hy::launch_decode<GG>(st, grid, qq, q_stride_seq, q_stride_tok, q_stride_head, oo,        \
                          o_stride_seq, o_stride_tok, o_stride_head, kp, vp, pool_head_stride, \
                          page_table, page_table_stride, q_start, decode_items, ws_acc, ws_ml, \
                          num_q_heads, page_shift, scale_log2);                               \
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

extern "C" int hy_paged_decode_merge(void *out, int64_t o_stride_seq, int64_t o_stride_tok,
                                     int64_t o_stride_head, const int32_t *q_start,
                                     const int32_t *merge_items, int32_t n_merge,
                                     int32_t n_slots, const void *workspace,
                                     int64_t workspace_bytes, int32_t num_q_heads,
                                     int32_t head_dim, void *stream) {
  hy::clear_error();
  HY_REQUIRE(n_merge >= 0 && n_slots >= 0, "item counts must be non-negative");
  if (n_merge == 0) return HY_OK;
  HY_REQUIRE_SUPPORTED(head_dim == kHeadDim, "head_dim %d unsupported (need %d)", head_dim,
                       kHeadDim);
  HY_REQUIRE(out && q_start && merge_items && workspace,
             "hy_paged_decode_merge: null pointer argument");
  const int64_t need = hy_decode_workspace_bytes(n_slots, num_q_heads, head_dim);
  if (workspace_bytes < need) {
    hy::set_error("workspace too small: need %lld bytes, got %lld",
                  static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    return HY_ENOSPACE;
  }
  const float *ws_acc = static_cast<const float *>(workspace);
  const float *ws_ml = reinterpret_cast<const float *>(
      static_cast<const char *>(workspace) +
      hy::align256(static_cast<int64_t>(n_slots) * num_q_heads * head_dim * 4));
  hipLaunchKernelGGL(hy::decode_merge_kernel, dim3(n_merge, num_q_heads), dim3(128), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint16_t *>(out),
                     o_stride_seq, o_stride_tok, o_stride_head, q_start, merge_items, ws_acc,
                     ws_ml, num_q_heads);
  return hy::launch_status("hy_paged_decode_merge");
}
