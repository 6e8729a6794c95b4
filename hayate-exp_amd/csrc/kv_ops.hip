// Paged KV append, fused QK-RMSNorm + RoPE + append, page gather/scatter.
//
// Work decomposition: the copies (plain append, gather, scatter) give one
// 16-lane row group to each 128-element head row, every lane moving 8 bf16
// (16 bytes), so a wave covers four head rows with fully coalesced 256-byte
// row segments. The fused norm + rotation + append gives 8 lanes to a row
// (two 128-byte halves per lane group; see qknorm.h). Both appends take one
// token per wave; its sequence and position come from one wave-wide search
// round (locate_token) and its page from a scalar load.
//
// Built with -ffp-contract=off: the norm and rotation must round each fp32
// product and sum separately, as the reference's chain of elementwise torch
// ops does (hayate/model/rope.py:44-47), so no FMA contraction is allowed.

#include <stdarg.h>
#include <stdio.h>

#include "hy_common.h"
#include "qknorm.h"

namespace hy {

namespace {

constexpr int kRowsPerBlock = 16;   // copies: 256 threads = 16 head rows
constexpr int kTokensPerBlock = 4;  // appends: one token per wave

// Physical token index of logical position t of sequence b.
__device__ __forceinline__ int64_t phys_token(const int32_t *__restrict__ pt,
                                              int64_t pt_stride, int b, int t,
                                              int page_size) {
  const int page = pt[static_cast<int64_t>(b) * pt_stride + t / page_size];
  return static_cast<int64_t>(page) * page_size + (t % page_size);
}

// ---------------------------------------------------------------------------
// Plain append: pool[h, phys(b, c_b + i)] = src[b, i, h]  (K and V).
// One token per wave and 8 kv heads per grid row (blockIdx.y): the wave's 16
// rows (8 K, 8 V) go in four 16-lane row loads per lane. The token is
// wave-uniform: its sequence and position take one search round and its
// page a scalar load; without a per-sequence stride the row loads are
// issued before them.
// ---------------------------------------------------------------------------
template <bool kSeqStride>
__global__ __launch_bounds__(256) void kv_append_kernel(
    uint16_t *__restrict__ k_pool, uint16_t *__restrict__ v_pool,
    int64_t pool_hs, const uint16_t *__restrict__ k, int64_t k_ss,
    int64_t k_st, int64_t k_sh, const uint16_t *__restrict__ v, int64_t v_ss,
    int64_t v_st, int64_t v_sh, const int32_t *__restrict__ q_start,
    const int32_t *__restrict__ cache_lens,
    const int32_t *__restrict__ page_table, int64_t pt_stride, int num_seqs,
    int total_tokens, int num_kv_heads, int page_size) {
  const int tok = __builtin_amdgcn_readfirstlane(blockIdx.x * kTokensPerBlock + (threadIdx.x >> 6));
  if (tok >= total_tokens) return;
  const int lane = threadIdx.x & 15;
  const int grp = (threadIdx.x >> 4) & 3;  // row within one four-row load
  // Row 4 j + grp of the wave: K head h0 + r for r < 8, else V head h0 + r - 8.
  const int h0 = blockIdx.y * 8;
  u32x4 raw[4];
  auto issue_loads = [&](int b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 4 * j + grp;
      const int h = h0 + (r & 7);
      if (h >= num_kv_heads) continue;
      raw[j] = load16(r < 8 ? k + b * k_ss + static_cast<int64_t>(tok) * k_st + h * k_sh + lane * 8
                            : v + b * v_ss + static_cast<int64_t>(tok) * v_st + h * v_sh + lane * 8);
    }
  };
  if (!kSeqStride) issue_loads(0);
  const TokenPos tp = locate_token(q_start, cache_lens, num_seqs, tok);
  const int b = tp.seq;
  if (kSeqStride) issue_loads(b);
  const int64_t p = phys_token(page_table, pt_stride, b, tp.pos, page_size);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * j + grp;
    const int h = h0 + (r & 7);
    if (h >= num_kv_heads) continue;
    store16((r < 8 ? k_pool : v_pool) + h * pool_hs + p * kHeadDim + lane * 8, raw[j]);
  }
}

// ---------------------------------------------------------------------------
// Fused q/k RMSNorm + RoPE + K/V append.
// Rows in the paired-half layout (qknorm.h): 8 lanes per head row, eight
// rows side by side in a wave. A wave takes one token and either up to 32
// of its q heads (four rows per 8-lane group) or up to 8 of its kv heads
// (the k row normed and rotated into the K pool, the v row copied into the
// V pool). Grid (token blocks of 4, ceil(Hq / 32) q chunks then
// ceil(Hkv / 8) kv chunks). The token's sequence, position and page, the
// norm weights and the cos/sin row are looked up once per wave; the token is
// uniform over the wave, so the sequence and position take one wave-wide
// search round and the page a scalar load. Without a per-sequence
// stride (packed or contiguous batches) a row's address needs only the
// token index, so the row loads are issued first and stay in flight through
// the search.
// The kernel moves each row once and spends about 200 VALU instructions per
// row and lane group on the exact norm and rotation. Measured on MI355X,
// four q rows per lane group beat two (8 % slower on a 2,048-token prefill)
// and one (7 %): the cos/sin row and the weights are then loaded and held
// for four rows at a time.
// ---------------------------------------------------------------------------
constexpr int kQRows = 4;           // q rows per 8-lane group
constexpr int kQChunk = 8 * kQRows; // q heads per wave
constexpr int kKvChunk = 8;         // kv heads per wave

__device__ __forceinline__ void load_half_rows(const float *__restrict__ row, int lane,
                                               float (&lo)[8], float (&hi)[8]) {
  load_row8(row, lane, lo);
  load_row8(row + 64, lane, hi);
}

template <bool kSeqStride>
__global__ __launch_bounds__(256) void qknorm_rope_append_kernel(
    const uint16_t *__restrict__ q, int64_t q_ss, int64_t q_st, int64_t q_sh,
    uint16_t *__restrict__ q_out, int64_t qo_ss, int64_t qo_st, int64_t qo_sh,
    const uint16_t *__restrict__ k, int64_t k_ss, int64_t k_st, int64_t k_sh,
    const uint16_t *__restrict__ v, int64_t v_ss, int64_t v_st, int64_t v_sh,
    const uint16_t *__restrict__ q_w, const uint16_t *__restrict__ k_w,
    float q_eps, float k_eps, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, uint16_t *__restrict__ k_pool,
    uint16_t *__restrict__ v_pool, int64_t pool_hs,
    const int32_t *__restrict__ q_start, const int32_t *__restrict__ cache_lens,
    const int32_t *__restrict__ page_table, int64_t pt_stride, int num_seqs,
    int total_tokens, int num_q_heads, int num_kv_heads, int page_size,
    int max_positions) {
  const int lane = threadIdx.x & 7;          // position in the row's 8-lane group
  const int slot = (threadIdx.x >> 3) & 7;   // row group within the wave
  const int tok = __builtin_amdgcn_readfirstlane(blockIdx.x * kTokensPerBlock + (threadIdx.x >> 6));
  const int gq = (num_q_heads + kQChunk - 1) / kQChunk;
  const bool is_q = static_cast<int>(blockIdx.y) < gq;
  // q: heads h0 + 8 j, j < nrows; kv: k head h0 and v head h0.
  const int h0 = is_q ? blockIdx.y * kQChunk + slot : (blockIdx.y - gq) * kKvChunk + slot;
  const int nrows = is_q ? (h0 < num_q_heads ? min(kQRows, (num_q_heads - h0 + 7) / 8) : 0)
                         : (h0 < num_kv_heads ? 1 : 0);
  const bool live = nrows > 0;

  // raw[2 j], raw[2 j + 1]: lo and hi halves of q row j; for kv: k then v.
  u32x4 raw[2 * kQRows];
  auto issue_loads = [&](int b) {
    if (is_q) {
      const uint16_t *src = q + b * q_ss + static_cast<int64_t>(tok) * q_st + h0 * q_sh + lane * 8;
#pragma unroll
      for (int j = 0; j < kQRows; ++j) {
        if (j < nrows) {
          raw[2 * j] = load16(src + 8 * j * q_sh);
          raw[2 * j + 1] = load16(src + 8 * j * q_sh + 64);
        }
      }
    } else {
      const uint16_t *ks = k + b * k_ss + static_cast<int64_t>(tok) * k_st + h0 * k_sh + lane * 8;
      const uint16_t *vs = v + b * v_ss + static_cast<int64_t>(tok) * v_st + h0 * v_sh + lane * 8;
      raw[0] = load16(ks);
      raw[1] = load16(ks + 64);
      raw[2] = load16(vs);
      raw[3] = load16(vs + 64);
    }
  };
  if (tok >= total_tokens) return;  // the whole wave
  if (!kSeqStride && live) issue_loads(0);
  // Every load is issued before the first use of any: rows, weights, the
  // token's sequence and position (one search round), the cos/sin row and
  // the page (scalar).
  const uint16_t *w = is_q ? q_w : k_w;
  const float eps = is_q ? q_eps : k_eps;
  u32x4 w_lo, w_hi;
  if (live && w != nullptr) {
    w_lo = load16(w + lane * 8);
    w_hi = load16(w + 64 + lane * 8);
  }
  // every lane of the wave takes part in the search
  const TokenPos tp = locate_token(q_start, cache_lens, num_seqs, tok);
  // A whole 8-lane group leaves together, so the group's DPP reads below
  // only see active lanes.
  if (!live) return;
  const int b = tp.seq;
  const int pos = tp.pos;
  if (kSeqStride) issue_loads(b);
  const bool rot = cos_t != nullptr;
  float cl[8], ch[8], sl[8], sh[8];
  if (rot) {
    // Positions must be below max_positions (the caller's contract); the
    // clamp only keeps a call that breaks it inside the tables.
    const int64_t off = static_cast<int64_t>(min(pos, max_positions - 1)) * kHeadDim;
    load_half_rows(cos_t + off, lane, cl, ch);
    load_half_rows(sin_t + off, lane, sl, sh);
  }
  const int64_t p = is_q ? 0 : phys_token(page_table, pt_stride, b, pos, page_size);

  float wl[8], wh[8];
  if (w != nullptr) {
    unpack8(w_lo, wl);
    unpack8(w_hi, wh);
  }
  auto finish_row = [&](u32x4 lo, u32x4 hi, uint16_t *dst) {
    float xl[8], xh[8];
    unpack8(lo, xl);
    unpack8(hi, xh);
    if (w != nullptr) rms_norm16(xl, xh, wl, wh, eps);
    if (rot) rope16(xl, xh, cl, ch, sl, sh);
    store16(dst, pack8_rne(xl));
    store16(dst + 64, pack8_rne(xh));
  };
  if (is_q) {
    uint16_t *dst = q_out + b * qo_ss + static_cast<int64_t>(tok) * qo_st + h0 * qo_sh + lane * 8;
#pragma unroll
    for (int j = 0; j < kQRows; ++j)
      if (j < nrows) finish_row(raw[2 * j], raw[2 * j + 1], dst + 8 * j * qo_sh);
    return;
  }
  const int64_t row = h0 * pool_hs + p * kHeadDim + lane * 8;
  store16(v_pool + row, raw[2]);
  store16(v_pool + row + 64, raw[3]);
  finish_row(raw[0], raw[1], k_pool + row);
}

// ---------------------------------------------------------------------------
// Gather / scatter between pages and a (layer, head, token) tensor.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void page_gather_kernel(
    const uint16_t *__restrict__ pool, int64_t pool_ls, int64_t pool_hs,
    const int32_t *__restrict__ pages, int length, uint16_t *__restrict__ out,
    int num_layers, int num_kv_heads, int page_size) {
  const int lane = threadIdx.x & 15;
  const int64_t rows = static_cast<int64_t>(num_layers) * num_kv_heads * length;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 4);
       row < rows; row += static_cast<int64_t>(gridDim.x) * kRowsPerBlock) {
    const int t = static_cast<int>(row % length);
    const int64_t lh = row / length;
    const int h = static_cast<int>(lh % num_kv_heads);
    const int l = static_cast<int>(lh / num_kv_heads);
    const int64_t p = static_cast<int64_t>(pages[t / page_size]) * page_size + t % page_size;
    const uint16_t *src = pool + l * pool_ls + h * pool_hs + p * kHeadDim;
    store16(out + row * kHeadDim + lane * 8, load16(src + lane * 8));
  }
}

__global__ __launch_bounds__(256) void page_scatter_kernel(
    uint16_t *__restrict__ pool, int64_t pool_ls, int64_t pool_hs,
    const int32_t *__restrict__ pages, int length,
    const uint16_t *__restrict__ src, int64_t s_ls, int64_t s_hs, int64_t s_ts,
    int num_layers, int num_kv_heads, int page_size) {
  const int lane = threadIdx.x & 15;
  const int64_t rows = static_cast<int64_t>(num_layers) * num_kv_heads * length;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 4);
       row < rows; row += static_cast<int64_t>(gridDim.x) * kRowsPerBlock) {
    const int t = static_cast<int>(row % length);
    const int64_t lh = row / length;
    const int h = static_cast<int>(lh % num_kv_heads);
    const int l = static_cast<int>(lh / num_kv_heads);
    const int64_t p = static_cast<int64_t>(pages[t / page_size]) * page_size + t % page_size;
    uint16_t *dst = pool + l * pool_ls + h * pool_hs + p * kHeadDim;
    store16(dst + lane * 8, load16(src + l * s_ls + h * s_hs + t * s_ts + lane * 8));
  }
}

inline unsigned grid_for_rows(int64_t rows) {
  return static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock);
}

}  // namespace

// ---------------------------------------------------------------------------
// Error plumbing shared by every translation unit.
// ---------------------------------------------------------------------------
static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

int launch_status(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return HY_ELAUNCH;
  }
  return HY_OK;
}

const char *last_error() { return g_err; }

}  // namespace hy

using hy::kHeadDim;

extern "C" int hy_version(void) { return (0 << 16) | 1; }

extern "C" const char *hy_last_error(void) { return hy::last_error(); }

static int check_common(int32_t num_seqs, int32_t total_tokens,
                        int32_t num_kv_heads, int32_t head_dim,
                        int32_t page_size) {
  HY_REQUIRE(num_seqs >= 1, "num_seqs must be positive (got %d)", num_seqs);
  HY_REQUIRE(total_tokens >= 0, "total_tokens must be non-negative");
  HY_REQUIRE(num_kv_heads >= 1, "num_kv_heads must be positive");
  HY_REQUIRE_SUPPORTED(head_dim == kHeadDim,
                       "head_dim %d unsupported (kernels are built for %d)",
                       head_dim, kHeadDim);
  HY_REQUIRE_SUPPORTED(page_size >= 32 && page_size % 32 == 0,
                       "page_size %d unsupported (multiple of 32 required)",
                       page_size);
  return HY_OK;
}

extern "C" int hy_kv_append(void *k_pool, void *v_pool,
                            int64_t pool_head_stride, const void *k,
                            int64_t k_stride_seq, int64_t k_stride_tok,
                            int64_t k_stride_head, const void *v,
                            int64_t v_stride_seq, int64_t v_stride_tok,
                            int64_t v_stride_head, const int32_t *q_start,
                            const int32_t *cache_lens,
                            const int32_t *page_table,
                            int64_t page_table_stride, int32_t num_seqs,
                            int32_t total_tokens, int32_t num_kv_heads,
                            int32_t head_dim, int32_t page_size,
                            void *stream) {
  hy::clear_error();
  if (int rc = check_common(num_seqs, total_tokens, num_kv_heads, head_dim, page_size))
    return rc;
  HY_REQUIRE(k_pool && v_pool && k && v && q_start && cache_lens && page_table,
             "hy_kv_append: null pointer argument");
  if (total_tokens == 0) return HY_OK;
  HY_REQUIRE((num_kv_heads + 7) / 8 <= 65535, "num_kv_heads (%d) too large", num_kv_heads);
  const bool seq_stride = k_stride_seq || v_stride_seq;
  auto kernel = seq_stride ? hy::kv_append_kernel<true> : hy::kv_append_kernel<false>;
  hipLaunchKernelGGL(kernel,
                     dim3((total_tokens + hy::kTokensPerBlock - 1) / hy::kTokensPerBlock,
                          (num_kv_heads + 7) / 8),
                     dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint16_t *>(k_pool),
                     static_cast<uint16_t *>(v_pool), pool_head_stride,
                     static_cast<const uint16_t *>(k), k_stride_seq,
                     k_stride_tok, k_stride_head,
                     static_cast<const uint16_t *>(v), v_stride_seq,
                     v_stride_tok, v_stride_head, q_start, cache_lens,
                     page_table, page_table_stride, num_seqs, total_tokens,
                     num_kv_heads, page_size);
  return hy::launch_status("hy_kv_append");
}

extern "C" int hy_qknorm_rope_append(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok,
    int64_t q_stride_head, void *q_out, int64_t qo_stride_seq,
    int64_t qo_stride_tok, int64_t qo_stride_head, const void *k,
    int64_t k_stride_seq, int64_t k_stride_tok, int64_t k_stride_head,
    const void *v, int64_t v_stride_seq, int64_t v_stride_tok,
    int64_t v_stride_head, const void *q_norm_weight,
    const void *k_norm_weight, float q_eps, float k_eps, const float *cos_table,
    const float *sin_table, int32_t max_positions, void *k_pool, void *v_pool,
    int64_t pool_head_stride, const int32_t *q_start,
    const int32_t *cache_lens, const int32_t *page_table,
    int64_t page_table_stride, int32_t num_seqs, int32_t total_tokens,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t page_size, void *stream) {
  hy::clear_error();
  if (int rc = check_common(num_seqs, total_tokens, num_kv_heads, head_dim, page_size))
    return rc;
  HY_REQUIRE(num_q_heads >= 1, "num_q_heads must be positive");
  HY_REQUIRE(q && q_out && k && v && k_pool && v_pool && q_start &&
                 cache_lens && page_table,
             "hy_qknorm_rope_append: null pointer argument");
  HY_REQUIRE((cos_table == nullptr) == (sin_table == nullptr),
             "cos_table and sin_table must both be given or both be NULL");
  HY_REQUIRE(cos_table == nullptr || max_positions > 0,
             "max_positions must be positive when tables are given");
  if (total_tokens == 0) return HY_OK;
  HY_REQUIRE(num_q_heads + 2 * num_kv_heads <= 65535, "too many heads (%d q, %d kv)",
             num_q_heads, num_kv_heads);
  const int gq = (num_q_heads + hy::kQChunk - 1) / hy::kQChunk;
  const int gkv = (num_kv_heads + hy::kKvChunk - 1) / hy::kKvChunk;
  // Row addresses that need no sequence index let the kernel load rows
  // before it searches for the token's sequence.
  const bool seq_stride = q_stride_seq || qo_stride_seq || k_stride_seq || v_stride_seq;
  auto kernel = seq_stride ? hy::qknorm_rope_append_kernel<true>
                           : hy::qknorm_rope_append_kernel<false>;
  hipLaunchKernelGGL(
      kernel, dim3((total_tokens + hy::kTokensPerBlock - 1) / hy::kTokensPerBlock, gq + gkv),
      dim3(256), 0, static_cast<hipStream_t>(stream), static_cast<const uint16_t *>(q),
      q_stride_seq, q_stride_tok, q_stride_head, static_cast<uint16_t *>(q_out),
      qo_stride_seq, qo_stride_tok, qo_stride_head,
      static_cast<const uint16_t *>(k), k_stride_seq, k_stride_tok,
      k_stride_head, static_cast<const uint16_t *>(v), v_stride_seq,
      v_stride_tok, v_stride_head,
      static_cast<const uint16_t *>(q_norm_weight),
      static_cast<const uint16_t *>(k_norm_weight), q_eps, k_eps, cos_table, sin_table,
      static_cast<uint16_t *>(k_pool), static_cast<uint16_t *>(v_pool),
      pool_head_stride, q_start, cache_lens, page_table, page_table_stride,
      num_seqs, total_tokens, num_q_heads, num_kv_heads, page_size, max_positions);
  return hy::launch_status("hy_qknorm_rope_append");
}

extern "C" int hy_page_gather(const void *pool, int64_t pool_layer_stride,
                              int64_t pool_head_stride, const int32_t *pages,
                              int32_t length, void *out, int32_t num_layers,
                              int32_t num_kv_heads, int32_t head_dim,
                              int32_t page_size, void *stream) {
  hy::clear_error();
  if (int rc = check_common(1, 0, num_kv_heads, head_dim, page_size)) return rc;
  HY_REQUIRE(length >= 0, "length must be non-negative");
  HY_REQUIRE(num_layers >= 1, "num_layers must be positive");
  if (length == 0) return HY_OK;
  HY_REQUIRE(pool && pages && out, "hy_page_gather: null pointer argument");
  const int64_t rows = static_cast<int64_t>(num_layers) * num_kv_heads * length;
  const int64_t blocks = (rows + 15) / 16;
  const unsigned grid = static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
  hipLaunchKernelGGL(hy::page_gather_kernel, dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t *>(pool), pool_layer_stride,
                     pool_head_stride, pages, length,
                     static_cast<uint16_t *>(out), num_layers, num_kv_heads,
                     page_size);
  return hy::launch_status("hy_page_gather");
}

extern "C" int hy_page_scatter(void *pool, int64_t pool_layer_stride,
                               int64_t pool_head_stride, const int32_t *pages,
                               int32_t length, const void *src,
                               int64_t src_stride_layer,
                               int64_t src_stride_head, int64_t src_stride_tok,
                               int32_t num_layers, int32_t num_kv_heads,
                               int32_t head_dim, int32_t page_size,
                               void *stream) {
  hy::clear_error();
  if (int rc = check_common(1, 0, num_kv_heads, head_dim, page_size)) return rc;
  HY_REQUIRE(length >= 0, "length must be non-negative");
  HY_REQUIRE(num_layers >= 1, "num_layers must be positive");
  if (length == 0) return HY_OK;
  HY_REQUIRE(pool && pages && src, "hy_page_scatter: null pointer argument");
  const int64_t rows = static_cast<int64_t>(num_layers) * num_kv_heads * length;
  const int64_t blocks = (rows + 15) / 16;
  const unsigned grid = static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
  hipLaunchKernelGGL(hy::page_scatter_kernel, dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<uint16_t *>(pool), pool_layer_stride,
                     pool_head_stride, pages, length,
                     static_cast<const uint16_t *>(src), src_stride_layer,
                     src_stride_head, src_stride_tok, num_layers,
                     num_kv_heads, page_size);
  return hy::launch_status("hy_page_scatter");
}
