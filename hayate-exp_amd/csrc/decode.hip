// Stream-K GQA paged decode attention (one query token per sequence).
//
// Work split: the K/V rows of all decode sequences, in sequence order, form
// one token stream per kv head; the planner cuts it into chunks of equal
// cost (tokens plus a fixed charge per extra piece), one per CU and kv head,
// so every workgroup takes about the same time whatever the spread of
// context lengths. A chunk holds one or more pieces (the part of one
// sequence inside the chunk). Grid: (kv head, chunk); with 8 kv heads each
// XCD streams one head. A workgroup serves all
// G = num_q_heads / num_kv_heads query heads of its kv head from a single
// read of every K/V row (GQA sharing).
//
// The chunk is walked in 32-token slices (a slice never crosses a page since
// page_size is a power of two >= 32 and cuts fall on multiples of 32); wave
// w of W takes slices w, w + W, ... and keeps its own online-softmax state
// for the piece it is in, so waves never synchronise after the start. When
// a wave moves to a new piece it writes its partial (acc, max, sum) of the
// old one to the workspace, and decode_merge_kernel (a second launch on the
// same stream: the kernel boundary publishes the partials) combines the W
// partials of every piece of a sequence. One workgroup per CU with two waves
// keeps HBM busiest; more waves per CU only add contention.
//
// Both products run on v_mfma_f32_16x16x32_bf16 (lane l, n = l % 16,
// g = l / 16):
//
//   S = K Q^T   A = K rows (16 tokens x 32 dims), loaded from HBM straight
//               into registers (lane n reads 16 B of row n, a whole 256-byte
//               row per 16 lanes); B = Q^T, column n < G is query head n,
//               read from an LDS table of the chunk's query rows built at
//               the start. Lane (n, g) ends with the scores of head n for
//               the slice tokens 4g + i and 16 + 4g + i (i < 4).
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
// transposed read touches start 8 banks apart. The K and V registers are
// double buffered: slice k + W is in flight while slice k is consumed. Rows
// past the end of a context may hold any bits; their scores are masked and
// their V values zeroed before the MFMA so that 0 * NaN never occurs.

#include <mutex>

#include "decode_shape.h"
#include "hy_common.h"
#include "qknorm.h"

namespace hy {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWaves = kDecodeWaves;
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

// Token range of one piece (part of one sequence inside one chunk), as
// read from its record {seq, tok_begin, tok_end, slot_base, slice_begin,
// q_tok, 0, 0}.
struct Piece {
  int seq, t0, t1, slot, sb, qt, nsl, ends;
};

__device__ __forceinline__ Piece load_piece(const int32_t *pieces, int p) {
  const int32_t *r = pieces + 8 * p;
  Piece x;
  x.seq = r[0];
  x.t0 = r[1];
  x.t1 = r[2];
  x.slot = r[3];
  x.sb = r[4];
  x.qt = r[5];
  x.ends = r[7];
  x.nsl = (x.t1 - x.t0 + kSlice - 1) / kSlice;
  return x;
}

// Where an issued slice lies: its piece, first token and the piece's end;
// newrow is the slice row of its sequence's query token, or -1.
struct SliceMeta {
  int piece, t0, tend, newrow;
};

// Inputs of the fused append (hy_paged_decode_append): the raw q, k, v
// projections of the step's tokens, the norm weights and rope tables. The
// kernel's q then points at the raw q rows.
struct AppendArgs {
  uint16_t *q_out;
  int64_t qo_ss, qo_st, qo_sh;
  const uint16_t *k;
  int64_t k_ss, k_st, k_sh;
  const uint16_t *v;
  int64_t v_ss, v_st, v_sh;
  const uint16_t *q_w, *k_w;
  float q_eps, k_eps;
  const float *cos_t, *sin_t;
  int max_pos;  // rows of cos_t / sin_t
  const int32_t *cache_lens;
};

// Two waves per SIMD: the double-buffered slice registers need about 240
// VGPRs.
//
// kFused: the step's q/k RMSNorm + RoPE + K/V append happens here instead of
// in a separate launch. The prologue rotates the query rows of the chunk's
// pieces into the LDS table (the workgroup of a sequence's first piece also
// writes them to q_out), and for every piece that holds its sequence's new
// token it builds the new K and V rows of that position and writes them to
// their page; the workgroup's barrier publishes them before any wave loads
// that slice (only the one workgroup that owns the row reads it). The
// values are those of qknorm_rope_append_kernel, bit for bit.
template <int G, bool kFused>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_kernel(
    const uint16_t *__restrict__ q, int64_t q_ss, int64_t q_st, int64_t q_sh,
    uint16_t *__restrict__ k_pool, uint16_t *__restrict__ v_pool,
    int64_t pool_hs, const int32_t *__restrict__ page_table, int64_t pt_stride,
    const int32_t *__restrict__ items, int n_chunks, float *__restrict__ ws_acc,
    float *__restrict__ ws_ml, int num_q_heads, int page_shift, float scale_log2,
    AppendArgs ap) {
  // One V transpose buffer per wave and the query rows (G heads) of every
  // piece of the chunk.
  constexpr int kMaxPieces = decode_max_pieces(G);
  __shared__ __attribute__((aligned(16))) uint16_t sV[kWaves][kSliceElems];
  __shared__ __attribute__((aligned(16))) uint16_t sQ[kMaxPieces * G * kHeadDim];

  // Grid (kv head, chunk): heads vary fastest, so with 8 kv heads every
  // XCD streams one head.
  const int32_t *ch = items + 8 * blockIdx.y;
  const int32_t *pieces = items + 8 * n_chunks;
  const int kvh = blockIdx.x;
  const int pb = ch[0];
  const int pe = ch[1];
  const int n_sl = ch[2];
  // An empty chunk record (a fixed-size grid padded past the plan's chunks)
  // owns no piece and no partial slot: the whole workgroup leaves before
  // any barrier.
  if (pe <= pb) return;

  // Wave index as a scalar: every per-slice address below is wave-uniform.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int h0 = kvh * G;
  const uint16_t *kh = k_pool + kvh * pool_hs;
  const uint16_t *vh = v_pool + kvh * pool_hs;
  uint16_t *vbuf = sV[wave];
  const uint16_t *vt_base = vbuf + (4 * g + (n >> 2)) * kVRow + 4 * (n & 3);

  // Issue cursor: the piece holding the next slice to load (the chunk
  // record repeats its first piece).
  int ip = pb;
  Piece ipc;
  ipc.seq = ch[3];
  ipc.t0 = ch[4];
  ipc.t1 = ch[5];
  ipc.slot = ch[6];
  ipc.sb = 0;
  ipc.qt = ch[7];
  ipc.nsl = (ipc.t1 - ipc.t0 + kSlice - 1) / kSlice;
  ipc.ends = pieces[8 * pb + 7];
  // Loads slice k of the chunk (k-th 32-token slice in piece order) into r.
  // locate() moves the cursor to slice k and describes it; issue() also
  // loads it.
  auto locate = [&](SliceMeta &m, int k) {
    while (k >= ipc.sb + ipc.nsl) ipc = load_piece(pieces, ++ip);
    m.piece = ip;
    m.t0 = ipc.t0 + (k - ipc.sb) * kSlice;
    m.tend = ipc.t1;
    m.newrow = ipc.ends && m.t0 + kSlice >= ipc.t1 ? ipc.t1 - 1 - m.t0 : -1;
  };
  auto issue = [&](SliceRegs &r, SliceMeta &m, int k) {
    locate(m, k);
    issue_slice(r, kh, vh, page_table + ipc.seq * pt_stride, m.t0, page_shift, lane);
  };

  // Online-softmax state of the piece being accumulated (cp).
  int cp = pb;
  int c_slot = ipc.slot;
  float m_run = -INFINITY;  // running max of head n (raw scores)
  float l_run = 0.f;        // lane-partial sum of head n
  f32x4 acc[8];             // O^T[16 db + 4g + i][head n]
#pragma unroll
  for (int db = 0; db < 8; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Writes this wave's partial (acc, max in the exp2 domain, sum) of the
  // current piece to workspace slot `slot`; every wave owns one slot of
  // every piece of its chunk.
  auto flush = [&](int slot) {
    float l = l_run;
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (n < G) {
      const int64_t base = static_cast<int64_t>(slot) * num_q_heads + h0 + n;
      float *dst = ws_acc + base * kHeadDim + 4 * g;
#pragma unroll
      for (int db = 0; db < 8; ++db) *reinterpret_cast<f32x4 *>(dst + 16 * db) = acc[db];
      if (g == 0) {
        ws_ml[base * 2 + 0] = m_run * scale_log2;
        ws_ml[base * 2 + 1] = l;
      }
    }
  };
  auto reset = [&]() {
    m_run = -INFINITY;
    l_run = 0.f;
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  // Q^T operand of piece p: column n < G is query head h0 + n of its
  // sequence's token.
  bf16x8 qop[4];
  auto load_q = [&](int p) {
    const int j = p - pb;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (n < G && j < kMaxPieces)
        w = *reinterpret_cast<const u32x4 *>(sQ + (j * G + n) * kHeadDim + kk * 32 + g * 8);
      qop[kk] = __builtin_bit_cast(bf16x8, w);
    }
  };
  // Closes the current piece and every piece before p that this wave has
  // no slice of (their partials are empty), then starts piece p.
  auto move_to = [&](int p) {
    flush(c_slot + wave);
    reset();
    for (int x = cp + 1; x < p; ++x) flush(pieces[8 * x + 3] + wave);
    cp = p;
    c_slot = pieces[8 * p + 3];
    load_q(p);
  };

  // The first slice's loads go out before the query table is built: all
  // threads copy (fused: rotate) the query rows of the chunk's pieces into
  // LDS (the planner keeps a chunk within kMaxPieces pieces). Fused, a first
  // slice that holds a sequence's new token is loaded only after the
  // prologue has written that row and the barrier has published it.
  int k = wave;
  SliceRegs ra, rb;
  SliceMeta ma, mb;
  bool deferred = false;
  if (k < n_sl) {
    locate(ma, k);
    deferred = kFused && ma.newrow >= 0;
    if (!deferred)
      issue_slice(ra, kh, vh, page_table + ipc.seq * pt_stride, ma.t0, page_shift, lane);
  }
  const int n_p = min(pe - pb, kMaxPieces);
  if constexpr (!kFused) {
    for (int idx = threadIdx.x; idx < n_p * G * 16; idx += kWaves * 64) {
      const int j = idx / (G * 16);
      const int h = (idx / 16) % G;
      const int c = idx % 16;
      const int32_t *pr = pieces + 8 * (pb + j);
      const uint16_t *src = q + pr[0] * q_ss + static_cast<int64_t>(pr[5]) * q_st +
                            (h0 + h) * q_sh + c * 8;
      *reinterpret_cast<u32x4 *>(sQ + (j * G + h) * kHeadDim + c * 8) = load16(src);
    }
  } else {
    // One 16-lane group per head row: n_p * G query rows, then one new K/V
    // row pair per piece (kept only where the piece ends its sequence).
    const int l16 = threadIdx.x & 15;
    for (int row = threadIdx.x >> 4; row < n_p * (G + 1); row += kWaves * 4) {
      const int j = row < n_p * G ? row / G : row - n_p * G;
      const int32_t *pr = pieces + 8 * (pb + j);
      const int seq = pr[0];
      const int pos = pr[6];  // position of the step's token (its cache length)
      // pos < max_pos is the caller's contract; the clamp only keeps a call
      // that breaks it inside the tables.
      const int64_t trow = static_cast<int64_t>(min(pos, ap.max_pos - 1)) * kHeadDim;
      const float *cos_row = ap.cos_t ? ap.cos_t + trow : nullptr;
      const float *sin_row = ap.sin_t ? ap.sin_t + trow : nullptr;
      if (row < n_p * G) {
        const int hh = row % G;
        const int qt = pr[5];
        float x[8];
        unpack8(load16(q + seq * q_ss + static_cast<int64_t>(qt) * q_st + (h0 + hh) * q_sh +
                       l16 * 8),
                x);
        if (ap.q_w != nullptr) rms_norm8(x, ap.q_w, l16, ap.q_eps);
        if (cos_row != nullptr) rope8(x, cos_row, sin_row, l16);
        const u32x4 y = pack8_rne(x);
        *reinterpret_cast<u32x4 *>(sQ + (j * G + hh) * kHeadDim + l16 * 8) = y;
        if (pr[1] == 0)
          store16(ap.q_out + seq * ap.qo_ss + static_cast<int64_t>(qt) * ap.qo_st +
                      (h0 + hh) * ap.qo_sh + l16 * 8,
                  y);
      } else {
        if (pr[7]) {  // the piece holds position pos
          const int qt = pr[5];
          float x[8];
          unpack8(load16(ap.k + seq * ap.k_ss + static_cast<int64_t>(qt) * ap.k_st +
                         kvh * ap.k_sh + l16 * 8),
                  x);
          if (ap.k_w != nullptr) rms_norm8(x, ap.k_w, l16, ap.k_eps);
          if (cos_row != nullptr) rope8(x, cos_row, sin_row, l16);
          const u32x4 yk = pack8_rne(x);
          const u32x4 yv = load16(ap.v + seq * ap.v_ss + static_cast<int64_t>(qt) * ap.v_st +
                                  kvh * ap.v_sh + l16 * 8);
          const int page = page_table[seq * pt_stride + (pos >> page_shift)];
          const int64_t p = (static_cast<int64_t>(page) << page_shift) + (pos & ((1 << page_shift) - 1));
          store16(k_pool + kvh * pool_hs + p * kHeadDim + l16 * 8, yk);
          store16(v_pool + kvh * pool_hs + p * kHeadDim + l16 * 8, yv);
        }
      }
    }
  }
  __syncthreads();
  if (deferred) issue_slice(ra, kh, vh, page_table + ipc.seq * pt_stride, ma.t0, page_shift, lane);
  load_q(pb);

  // Wave w takes slices w, w + 4, ... of the chunk. Double-buffered: the
  // loads of slice k + 4 are in flight while slice k is consumed; a slice's
  // V rows go to LDS before the next slice is issued. The steady state
  // issues unconditionally so that every wait covers only earlier loads;
  // the tail is peeled.
  if (k < n_sl) {
    while (k + 2 * kWaves < n_sl) {
      stage_v(ra, vbuf, lane);
      issue(rb, mb, k + kWaves);
      if (ma.piece != cp) move_to(ma.piece);
      consume_slice<G>(ra, vt_base, qop, ma.t0, ma.tend, lane, scale_log2, m_run, l_run, acc);
      stage_v(rb, vbuf, lane);
      issue(ra, ma, k + 2 * kWaves);
      if (mb.piece != cp) move_to(mb.piece);
      consume_slice<G>(rb, vt_base, qop, mb.t0, mb.tend, lane, scale_log2, m_run, l_run, acc);
      k += 2 * kWaves;
    }
    stage_v(ra, vbuf, lane);
    if (k + kWaves < n_sl) {
      issue(rb, mb, k + kWaves);
      if (ma.piece != cp) move_to(ma.piece);
      consume_slice<G>(ra, vt_base, qop, ma.t0, ma.tend, lane, scale_log2, m_run, l_run, acc);
      stage_v(rb, vbuf, lane);
      if (mb.piece != cp) move_to(mb.piece);
      consume_slice<G>(rb, vt_base, qop, mb.t0, mb.tend, lane, scale_log2, m_run, l_run, acc);
    } else {
      if (ma.piece != cp) move_to(ma.piece);
      consume_slice<G>(ra, vt_base, qop, ma.t0, ma.tend, lane, scale_log2, m_run, l_run, acc);
    }
  }
  // Close the last piece and any later ones this wave had no slice of.
  flush(c_slot + wave);
  reset();
  for (int x = cp + 1; x < pe; ++x) flush(pieces[8 * x + 3] + wave);
}

// Combines the partials of every decode sequence: grid (merge item, q head
// group of 4), 128 threads = 4 heads x 32 lanes x 4 dims. Item = {seq,
// first_slot, num_partials, q_row = q_start[seq]}. Up to eight partials are
// loaded in one round of independent loads: every load reads a real
// partial (the split index is clamped to the last one) and the ones past
// num_partials are then replaced by the empty partial, so no load sits
// behind a branch. A lane whose head is past num_q_heads computes on a
// clamped head and does not store.
__global__ __launch_bounds__(128) void decode_merge_kernel(
    uint16_t *__restrict__ out, int64_t o_ss, int64_t o_st, int64_t o_sh,
    const int32_t *__restrict__ q_start, const int32_t *__restrict__ items,
    const float *__restrict__ ws_acc, const float *__restrict__ ws_ml, int num_q_heads) {
  const int4 it = *reinterpret_cast<const int4 *>(items + 4 * blockIdx.x);
  const int seq = it.x;
  const int first = it.y;
  const int nsplit = it.z;
  const int hq_lane = 4 * blockIdx.y + (threadIdx.x >> 5);
  const int hq = min(hq_lane, num_q_heads - 1);
  const int d = (threadIdx.x & 31) * 4;
  const int64_t qs = it.w;  // q_start[seq], carried by the item
  float mx = -INFINITY, lsum = 0.f;
  f32x4 a = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsplit; s0 += 8) {
    float m[8], l[8];
    f32x4 x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t base = static_cast<int64_t>(first + min(s0 + j, nsplit - 1)) * num_q_heads + hq;
      const float2 ml = *reinterpret_cast<const float2 *>(ws_ml + base * 2);
      m[j] = ml.x;
      l[j] = ml.y;
      x[j] = *reinterpret_cast<const f32x4 *>(ws_acc + base * kHeadDim + d);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool live = s0 + j < nsplit;
      m[j] = live ? m[j] : -INFINITY;
      l[j] = live ? l[j] : 0.f;
      x[j] = live ? x[j] : f32x4{0.f, 0.f, 0.f, 0.f};
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
  if (hq_lane >= num_q_heads) return;
  uint16_t *dst = out + seq * o_ss + qs * o_st + hq * o_sh + d;
  *reinterpret_cast<uint2 *>(dst) = make_uint2(pack_bf16x2_rne(a[0] / lsum, a[1] / lsum),
                                               pack_bf16x2_rne(a[2] / lsum, a[3] / lsum));
}

template <int G, bool kFused>
void launch_decode(hipStream_t st, dim3 grid, const uint16_t *q, int64_t q_ss, int64_t q_st,
                   int64_t q_sh, uint16_t *k_pool, uint16_t *v_pool, int64_t pool_hs,
                   const int32_t *page_table, int64_t pt_stride, const int32_t *items,
                   int n_chunks, float *ws_acc, float *ws_ml, int num_q_heads, int page_shift,
                   float scale_log2, const AppendArgs &ap) {
  hipLaunchKernelGGL((decode_kernel<G, kFused>), grid, dim3(kWaves * 64), 0, st, q, q_ss, q_st,
                     q_sh, k_pool, v_pool, pool_hs, page_table, pt_stride, items, n_chunks, ws_acc,
                     ws_ml, num_q_heads, page_shift, scale_log2, ap);
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

namespace {

// Shared by hy_paged_decode and hy_paged_decode_append: validation and the
// launch over the chunk grid.
int paged_decode_impl(const char *name, const void *q, int64_t q_stride_seq,
                      int64_t q_stride_tok, int64_t q_stride_head, void *out, const void *k_pool,
                      const void *v_pool, int64_t pool_head_stride, const int32_t *page_table,
                      int64_t page_table_stride, const int32_t *q_start,
                      const int32_t *decode_items, int32_t n_decode, int32_t n_slots,
                      void *workspace, int64_t workspace_bytes, int32_t num_seqs,
                      int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                      int32_t page_size, float scale, void *stream, const hy::AppendArgs *ap) {
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
  HY_REQUIRE(n_decode <= 65535, "%d decode chunks exceed the grid limit of 65535", n_decode);
  HY_REQUIRE(q && out && k_pool && v_pool && page_table && q_start && decode_items,
             "%s: null pointer argument", name);
  const int G = num_q_heads / num_kv_heads;
  HY_REQUIRE_SUPPORTED(G == 1 || G == 2 || G == 4 || G == 8 || G == 16,
                       "GQA group size %d unsupported (1, 2, 4, 8, 16)", G);
  HY_REQUIRE(n_slots > 0, "decode work needs workspace slots");
  const int64_t need = hy_decode_workspace_bytes(n_slots, num_q_heads, head_dim);
  if (workspace == nullptr || workspace_bytes < need) {
    hy::set_error("workspace too small: need %lld bytes, got %lld",
                  static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    return HY_ENOSPACE;
  }
  float *ws_acc = static_cast<float *>(workspace);
  float *ws_ml = reinterpret_cast<float *>(
      static_cast<char *>(workspace) +
      hy::align256(static_cast<int64_t>(n_slots) * num_q_heads * head_dim * 4));
  const float scale_log2 = scale * hy::kLog2e;
  const int page_shift = __builtin_ctz(static_cast<unsigned>(page_size));
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(num_kv_heads, n_decode);
  const uint16_t *qq = static_cast<const uint16_t *>(q);
  uint16_t *kp = static_cast<uint16_t *>(const_cast<void *>(k_pool));
  uint16_t *vp = static_cast<uint16_t *>(const_cast<void *>(v_pool));
  const hy::AppendArgs none{};
#define HY_DECODE_CASE(GG)                                                                     \
  case GG:                                                                                     \
    if (ap)                                                                                    \
      hy::launch_decode<GG, true>(st, grid, qq, q_stride_seq, q_stride_tok, q_stride_head, kp, \
                                  vp, pool_head_stride, page_table, page_table_stride,         \
                                  decode_items, n_decode, ws_acc, ws_ml, num_q_heads,          \
                                  page_shift, scale_log2, *ap);                                \
    else                                                                                       \
      hy::launch_decode<GG, false>(st, grid, qq, q_stride_seq, q_stride_tok, q_stride_head,    \
                                   kp, vp, pool_head_stride, page_table, page_table_stride,    \
                                   decode_items, n_decode, ws_acc, ws_ml, num_q_heads,         \
                                   page_shift, scale_log2, none);                              \
    break;
  switch (G) {
    HY_DECODE_CASE(1)
    HY_DECODE_CASE(2)
    HY_DECODE_CASE(4)
    HY_DECODE_CASE(8)
    HY_DECODE_CASE(16)
  }
#undef HY_DECODE_CASE
  return hy::launch_status(name);
}

}  // namespace

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
  (void)o_stride_seq;
  (void)o_stride_tok;
  (void)o_stride_head;
  return paged_decode_impl("hy_paged_decode", q, q_stride_seq, q_stride_tok, q_stride_head, out,
                           k_pool, v_pool, pool_head_stride, page_table, page_table_stride,
                           q_start, decode_items, n_decode, n_slots, workspace, workspace_bytes,
                           num_seqs, num_q_heads, num_kv_heads, head_dim, page_size, scale,
                           stream, nullptr);
}

namespace {

// Validates and packs the fused append's inputs (shared by
// hy_paged_decode_append and hy_paged_decode_append_noalloc).
int fill_append_args(const char *name, hy::AppendArgs &ap, void *q_out, int64_t qo_stride_seq,
                     int64_t qo_stride_tok, int64_t qo_stride_head, const void *k,
                     int64_t k_stride_seq, int64_t k_stride_tok, int64_t k_stride_head,
                     const void *v, int64_t v_stride_seq, int64_t v_stride_tok,
                     int64_t v_stride_head, const void *q_norm_weight,
                     const void *k_norm_weight, float q_eps, float k_eps,
                     const float *cos_table, const float *sin_table, int32_t max_positions,
                     const int32_t *cache_lens) {
  HY_REQUIRE(q_out && k && v && cache_lens, "%s: null pointer argument", name);
  HY_REQUIRE((cos_table == nullptr) == (sin_table == nullptr),
             "cos_table and sin_table must both be given or both be NULL");
  HY_REQUIRE(cos_table == nullptr || max_positions > 0,
             "max_positions must be positive when tables are given");
  ap.q_out = static_cast<uint16_t *>(q_out);
  ap.qo_ss = qo_stride_seq;
  ap.qo_st = qo_stride_tok;
  ap.qo_sh = qo_stride_head;
  ap.k = static_cast<const uint16_t *>(k);
  ap.k_ss = k_stride_seq;
  ap.k_st = k_stride_tok;
  ap.k_sh = k_stride_head;
  ap.v = static_cast<const uint16_t *>(v);
  ap.v_ss = v_stride_seq;
  ap.v_st = v_stride_tok;
  ap.v_sh = v_stride_head;
  ap.q_w = static_cast<const uint16_t *>(q_norm_weight);
  ap.k_w = static_cast<const uint16_t *>(k_norm_weight);
  ap.q_eps = q_eps;
  ap.k_eps = k_eps;
  ap.cos_t = cos_table;
  ap.sin_t = sin_table;
  ap.max_pos = max_positions;
  ap.cache_lens = cache_lens;
  return HY_OK;
}

// Validates and launches decode_merge_kernel over a workspace of n_slots
// partials (shared by hy_paged_decode_merge and
// hy_paged_decode_append_noalloc).
int decode_merge_impl(const char *name, void *out, int64_t o_stride_seq, int64_t o_stride_tok,
                      int64_t o_stride_head, const int32_t *q_start, const int32_t *merge_items,
                      int32_t n_merge, int32_t n_slots, const void *workspace,
                      int64_t workspace_bytes, int32_t num_q_heads, int32_t head_dim,
                      void *stream) {
  HY_REQUIRE(n_merge >= 0 && n_slots >= 0, "item counts must be non-negative");
  if (n_merge == 0) return HY_OK;
  HY_REQUIRE_SUPPORTED(head_dim == kHeadDim, "head_dim %d unsupported (need %d)", head_dim,
                       kHeadDim);
  HY_REQUIRE(num_q_heads >= 1 && (num_q_heads + 3) / 4 <= 65535, "num_q_heads %d out of range",
             num_q_heads);
  HY_REQUIRE(out && q_start && merge_items && workspace, "%s: null pointer argument", name);
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
  hipLaunchKernelGGL(hy::decode_merge_kernel, dim3(n_merge, (num_q_heads + 3) / 4), dim3(128), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint16_t *>(out),
                     o_stride_seq, o_stride_tok, o_stride_head, q_start, merge_items, ws_acc,
                     ws_ml, num_q_heads);
  return hy::launch_status(name);
}

}  // namespace

extern "C" int hy_paged_decode_append(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok, int64_t q_stride_head,
    void *q_out, int64_t qo_stride_seq, int64_t qo_stride_tok, int64_t qo_stride_head,
    const void *k, int64_t k_stride_seq, int64_t k_stride_tok, int64_t k_stride_head,
    const void *v, int64_t v_stride_seq, int64_t v_stride_tok, int64_t v_stride_head,
    const void *q_norm_weight, const void *k_norm_weight, float q_eps, float k_eps,
    const float *cos_table,
    const float *sin_table, int32_t max_positions, void *out, void *k_pool, void *v_pool,
    int64_t pool_head_stride, const int32_t *page_table, int64_t page_table_stride,
    const int32_t *q_start, const int32_t *cache_lens, const int32_t *decode_items,
    int32_t n_decode, int32_t n_slots, void *workspace, int64_t workspace_bytes,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t page_size, float scale, void *stream) {
  hy::clear_error();
  hy::AppendArgs ap;
  if (int rc = fill_append_args("hy_paged_decode_append", ap, q_out, qo_stride_seq,
                                qo_stride_tok, qo_stride_head, k, k_stride_seq, k_stride_tok,
                                k_stride_head, v, v_stride_seq, v_stride_tok, v_stride_head,
                                q_norm_weight, k_norm_weight, q_eps, k_eps, cos_table,
                                sin_table,
                                max_positions, cache_lens))
    return rc;
  return paged_decode_impl("hy_paged_decode_append", q, q_stride_seq, q_stride_tok,
                           q_stride_head, out, k_pool, v_pool, pool_head_stride, page_table,
                           page_table_stride, q_start, decode_items, n_decode, n_slots,
                           workspace, workspace_bytes, num_seqs, num_q_heads, num_kv_heads,
                           head_dim, page_size, scale, stream, &ap);
}

extern "C" int hy_paged_decode_merge(void *out, int64_t o_stride_seq, int64_t o_stride_tok,
                                     int64_t o_stride_head, const int32_t *q_start,
                                     const int32_t *merge_items, int32_t n_merge,
                                     int32_t n_slots, const void *workspace,
                                     int64_t workspace_bytes, int32_t num_q_heads,
                                     int32_t head_dim, void *stream) {
  hy::clear_error();
  return decode_merge_impl("hy_paged_decode_merge", out, o_stride_seq, o_stride_tok,
                           o_stride_head, q_start, merge_items, n_merge, n_slots, workspace,
                           workspace_bytes, num_q_heads, head_dim, stream);
}

// ---------------------------------------------------------------------------
// hy_paged_decode_append_noalloc: the fused decode step (decode kernel +
// merge) with its fp32 partials in a file-scope device array instead of a
// caller workspace, for callers that cannot allocate device memory.
//
// The array is HY_NOALLOC_SCRATCH_BYTES (8 MiB) per GPU, held for the life of
// the process. Host code never passes the array's name to a kernel (on the
// host it is a stand-in, not a device address): the first call on each
// device, with that device current, resolves its address with
// hipGetSymbolAddress and keeps it per device. Every call on one GPU shares
// its array, so calls that overlap on one GPU (two streams, two threads)
// race. Nothing in it needs clearing: the decode kernel writes every slot the
// merge reads (each wave flushes a partial for every piece of its chunk,
// empty ones included) before the merge, on the same stream, reads it.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[HY_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, or nullptr (the error
// message is set).
void *scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    hy::set_error("hy_paged_decode_append_noalloc: no usable current HIP device (%d)", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      hy::set_error("hy_paged_decode_append_noalloc: hipGetSymbolAddress failed on device %d: %s",
                    dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int hy_paged_decode_append_noalloc(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok, int64_t q_stride_head,
    void *q_out, int64_t qo_stride_seq, int64_t qo_stride_tok, int64_t qo_stride_head,
    const void *k, int64_t k_stride_seq, int64_t k_stride_tok, int64_t k_stride_head,
    const void *v, int64_t v_stride_seq, int64_t v_stride_tok, int64_t v_stride_head,
    const void *q_norm_weight, const void *k_norm_weight, float q_eps, float k_eps,
    const float *cos_table,
    const float *sin_table, int32_t max_positions, void *out, int64_t o_stride_seq,
    int64_t o_stride_tok, int64_t o_stride_head, void *k_pool, void *v_pool,
    int64_t pool_head_stride, const int32_t *page_table, int64_t page_table_stride,
    const int32_t *q_start, const int32_t *cache_lens, const int32_t *decode_items,
    int32_t n_decode, const int32_t *merge_items, int32_t n_merge, int32_t n_slots,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t page_size, float scale, void *stream) {
  hy::clear_error();
  HY_REQUIRE(n_slots >= 0 && num_q_heads >= 1, "item counts must be non-negative");
  // The scratch keeps whatever the previous call left; a merge is only
  // meaningful over partials this same call's decode launch wrote.
  HY_REQUIRE(!(n_decode == 0 && n_merge > 0),
             "merge items without decode items would merge stale scratch partials");
  const int64_t need = hy_decode_workspace_bytes(n_slots, num_q_heads, head_dim);
  if (need > HY_NOALLOC_SCRATCH_BYTES) {
    hy::set_error("hy_paged_decode_append_noalloc: %d partial slots x %d heads need %lld bytes, "
                  "more than the %lld-byte static scratch; use hy_paged_decode_append with a "
                  "caller workspace",
                  n_slots, num_q_heads, static_cast<long long>(need),
                  static_cast<long long>(HY_NOALLOC_SCRATCH_BYTES));
    return HY_ENOSPACE;
  }
  hy::AppendArgs ap;
  if (int rc = fill_append_args("hy_paged_decode_append_noalloc", ap, q_out, qo_stride_seq,
                                qo_stride_tok, qo_stride_head, k, k_stride_seq, k_stride_tok,
                                k_stride_head, v, v_stride_seq, v_stride_tok, v_stride_head,
                                q_norm_weight, k_norm_weight, q_eps, k_eps, cos_table,
                                sin_table,
                                max_positions, cache_lens))
    return rc;
  if (n_decode == 0 && n_merge == 0) return HY_OK;
  void *ws = scratch_on_current_device();
  if (ws == nullptr) return HY_ELAUNCH;
  if (int rc = paged_decode_impl("hy_paged_decode_append_noalloc", q, q_stride_seq, q_stride_tok,
                                 q_stride_head, out, k_pool, v_pool, pool_head_stride,
                                 page_table, page_table_stride, q_start, decode_items, n_decode,
                                 n_slots, ws, HY_NOALLOC_SCRATCH_BYTES, num_seqs, num_q_heads,
                                 num_kv_heads, head_dim, page_size, scale, stream, &ap))
    return rc;
  return decode_merge_impl("hy_paged_decode_append_noalloc", out, o_stride_seq, o_stride_tok,
                           o_stride_head, q_start, merge_items, n_merge, n_slots, ws,
                           HY_NOALLOC_SCRATCH_BYTES, num_q_heads, head_dim, stream);
}
