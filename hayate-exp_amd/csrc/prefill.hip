// Paged chunked-prefill causal attention on bf16 MFMA (gfx950).
//
// Grid: (prefill item, kv head). An item is a tile of 128 / G query tokens of
// one sequence; with its G query heads that is 128 (token, head) rows, which
// all read the same K/V (GQA). Four waves, 32 rows each (two 16-row blocks).
//
// Per 64-key tile the workgroup stages K (row-major, 272-byte padded rows)
// and V transposed (Vt[dim][key], 136-byte rows) in LDS; each thread moves
// four 16-byte rows of V and writes them back as eight 8-byte key quads.
//
// Transposed formulation with v_mfma_f32_16x16x32_bf16 (lane l, m = l % 16,
// g = l / 16):
//   S^T = K Q^T  A = K (16 keys x 32 dims) from LDS, B = Q^T (32 dims x 16
//                rows) held in registers; lane (m, g) ends with the scores of
//                row m for keys 4g..4g+3 (+16 for the second key block).
//   softmax      per row, lanes of one row differ only in g (xor 16 / 32).
//   O^T += V^T P^T  B = P^T needs lane (m, g) to hold row m's probabilities
//                for 8 keys: exactly its own 8 scores once the MFMA k index
//                8g + j is mapped to key (j < 4 ? 4g + j : 16 + 4g + j - 4);
//                A = V^T uses the same key map, two 8-byte LDS reads.
// The accumulator O^T[dim 16db + 4g + i][row m] keeps each row in one lane
// group, so rescaling by the running max is a per-lane multiply.

#include "hy_common.h"

namespace hy {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kRows = 128;       // (token, head) rows per workgroup
constexpr int kKeys = 64;        // keys per LDS tile
constexpr int kKStride = 136;    // u16 per K row in LDS (256 B + 16 B pad)
constexpr int kVtStride = 68;    // u16 per Vt row in LDS (128 B + 8 B pad)

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 pack_p(const f32x4 a, const f32x4 b) {
  bf16x8 r;
  r[0] = static_cast<__bf16>(a[0]);
  r[1] = static_cast<__bf16>(a[1]);
  r[2] = static_cast<__bf16>(a[2]);
  r[3] = static_cast<__bf16>(a[3]);
  r[4] = static_cast<__bf16>(b[0]);
  r[5] = static_cast<__bf16>(b[1]);
  r[6] = static_cast<__bf16>(b[2]);
  r[7] = static_cast<__bf16>(b[3]);
  return r;
}

template <int G>
__global__ __launch_bounds__(256) void prefill_kernel(
    const uint16_t *__restrict__ q, int64_t q_ss, int64_t q_st, int64_t q_sh,
    uint16_t *__restrict__ out, int64_t o_ss, int64_t o_st, int64_t o_sh,
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool,
    int64_t pool_hs, const int32_t *__restrict__ page_table, int64_t pt_stride,
    const int32_t *__restrict__ q_start, const int32_t *__restrict__ kv_lens,
    const int32_t *__restrict__ items, int page_size, float scale_log2) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[kKeys * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[kHeadDim * kVtStride];

  const int seq = items[blockIdx.x * 4 + 0];
  const int q_begin = items[blockIdx.x * 4 + 1];
  const int q_end = items[blockIdx.x * 4 + 2];
  const int kvh = blockIdx.y;
  const int h0 = kvh * G;
  const int qs = q_start[seq];
  const int q_len = q_start[seq + 1] - qs;
  const int cache_len = kv_lens[seq] - q_len;
  const int kv_end = cache_len + q_end;  // keys any row of this tile may see

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int l = tid & 63;
  const int m = l & 15;
  const int g = l >> 4;

  // Q^T operand per row block: row r = 32 * wave + 16 * rb + m.
  bf16x8 qop[2][4];
  int row_tok[2];  // query index within the sequence for this lane's row
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int r = 32 * wave + 16 * rb + m;
    const int i = q_begin + r / G;
    const int h = h0 + r % G;
    row_tok[rb] = i;
    const bool live = i < q_end;
    const uint16_t *src = q + seq * q_ss + static_cast<int64_t>(qs + (live ? i : q_begin)) * q_st + h * q_sh;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (live) w = load16(src + kk * 32 + g * 8);
      qop[rb][kk] = __builtin_bit_cast(bf16x8, w);
    }
  }

  f32x4 acc[2][8];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};

  const uint16_t *kh = k_pool + kvh * pool_hs;
  const uint16_t *vh = v_pool + kvh * pool_hs;
  const int32_t *pt = page_table + seq * pt_stride;
  // First key that is masked for at least one row of this tile.
  const int diag_begin = cache_len + q_begin;

  // Staging assignment: K chunk c = tid + 256 j -> (row c / 16, col c % 16);
  // V: thread owns dims 8 * (tid % 16) .. +7 of keys 4 * (tid / 16) .. +3.
  const int vd = (tid & 15) * 8;
  const int vk = (tid >> 4) * 4;

  for (int kt = 0; kt < kv_end; kt += kKeys) {
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + 256 * j;
      const int row = c >> 4;
      const int col = c & 15;
      const int key = kt + row;
      u32x4 w = {0u, 0u, 0u, 0u};
      if (key < kv_end) {
        const int64_t p = static_cast<int64_t>(pt[key / page_size]) * page_size + key % page_size;
        w = load16(kh + p * kHeadDim + col * 8);
      }
      *reinterpret_cast<u32x4 *>(&sK[row * kKStride + col * 8]) = w;
    }
    {
      u32x4 vr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kt + vk + i;
        vr[i] = u32x4{0u, 0u, 0u, 0u};
        if (key < kv_end) {
          const int64_t p = static_cast<int64_t>(pt[key / page_size]) * page_size + key % page_size;
          vr[i] = load16(vh + p * kHeadDim + vd);
        }
      }
      // Transpose 4 keys x 8 dims into 8 dims x 4 keys.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo01 = (vr[0][j] & 0xffffu) | (vr[1][j] << 16);
        const uint32_t lo23 = (vr[2][j] & 0xffffu) | (vr[3][j] << 16);
        const uint32_t hi01 = (vr[0][j] >> 16) | (vr[1][j] & 0xffff0000u);
        const uint32_t hi23 = (vr[2][j] >> 16) | (vr[3][j] & 0xffff0000u);
        uint32_t *d0 = reinterpret_cast<uint32_t *>(&sVt[(vd + 2 * j) * kVtStride + vk]);
        uint32_t *d1 = reinterpret_cast<uint32_t *>(&sVt[(vd + 2 * j + 1) * kVtStride + vk]);
        d0[0] = lo01;
        d0[1] = lo23;
        d1[0] = hi01;
        d1[1] = hi23;
      }
    }
    __syncthreads();

    const bool need_mask = kt + kKeys > diag_begin;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      // S^T for both row blocks and both 16-key blocks of this 32-key step.
      f32x4 s[2][2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) s[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8 kop = *reinterpret_cast<const bf16x8 *>(
              &sK[(32 * ks + 16 * kb + m) * kKStride + kk * 32 + g * 8]);
#pragma unroll
          for (int rb = 0; rb < 2; ++rb)
            s[rb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[rb][kk], s[rb][kb], 0, 0, 0);
        }

      bf16x8 pop[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const int limit = cache_len + row_tok[rb];  // last visible key
        float mloc = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float x = s[rb][kb][i] * scale_log2;
            if (need_mask) {
              const int key = kt + 32 * ks + 16 * kb + 4 * g + i;
              if (key > limit) x = -INFINITY;
            }
            s[rb][kb][i] = x;
            mloc = fmaxf(mloc, x);
          }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float m_new = fmaxf(m_run[rb], mloc);
        // A row whose keys so far are all masked keeps m = -inf; guard the
        // exponent so that it contributes exact zeros.
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m_run[rb] - m_use);
        m_run[rb] = m_new;
        float psum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = exp2f(s[rb][kb][i] - m_use);
            s[rb][kb][i] = p;
            psum += p;
          }
        l_run[rb] = l_run[rb] * alpha + psum;
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[rb][db] *= alpha;
        pop[rb] = pack_p(s[rb][0], s[rb][1]);
      }

#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const uint16_t *vrow = &sVt[(16 * db + m) * kVtStride + 32 * ks + 4 * g];
        const s16x4 a0 = *reinterpret_cast<const s16x4 *>(vrow);
        const s16x4 a1 = *reinterpret_cast<const s16x4 *>(vrow + 16);
        const bf16x8 vop = __builtin_bit_cast(
            bf16x8, (__attribute__((ext_vector_type(8))) short){a0[0], a0[1], a0[2], a0[3],
                                                                a1[0], a1[1], a1[2], a1[3]});
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          acc[rb][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[rb], acc[rb][db], 0, 0, 0);
      }
    }
  }

  // Row sums across the four key groups, then normalise and store.
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    float lsum = l_run[rb];
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    const float inv = 1.0f / lsum;
    const int r = 32 * wave + 16 * rb + m;
    const int i = row_tok[rb];
    if (i >= q_end) continue;
    const int h = h0 + r % G;
    uint16_t *dst = out + seq * o_ss + static_cast<int64_t>(qs + i) * o_st + h * o_sh;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const uint32_t w0 = f32_to_bf16_rne(acc[rb][db][0] * inv) |
                          (f32_to_bf16_rne(acc[rb][db][1] * inv) << 16);
      const uint32_t w1 = f32_to_bf16_rne(acc[rb][db][2] * inv) |
                          (f32_to_bf16_rne(acc[rb][db][3] * inv) << 16);
      uint32_t *d = reinterpret_cast<uint32_t *>(dst + 16 * db + 4 * g);
      d[0] = w0;
      d[1] = w1;
    }
  }
}

template <int G>
void launch_prefill(hipStream_t st, dim3 grid, const uint16_t *q, int64_t q_ss,
                    int64_t q_st, int64_t q_sh, uint16_t *out, int64_t o_ss,
                    int64_t o_st, int64_t o_sh, const uint16_t *k_pool,
                    const uint16_t *v_pool, int64_t pool_hs,
                    const int32_t *page_table, int64_t pt_stride,
                    const int32_t *q_start, const int32_t *kv_lens,
                    const int32_t *items, int page_size, float scale_log2) {
  hipLaunchKernelGGL(prefill_kernel<G>, grid, dim3(256), 0, st, q, q_ss, q_st,
                     q_sh, out, o_ss, o_st, o_sh, k_pool, v_pool, pool_hs,
                     page_table, pt_stride, q_start, kv_lens, items,
                     page_size, scale_log2);
}

}  // namespace
}  // namespace hy

using hy::kHeadDim;

extern "C" int hy_paged_prefill(
    const void *q, int64_t q_stride_seq, int64_t q_stride_tok,
    int64_t q_stride_head, void *out, int64_t o_stride_seq,
    int64_t o_stride_tok, int64_t o_stride_head, const void *k_pool,
    const void *v_pool, int64_t pool_head_stride, const int32_t *page_table,
    int64_t page_table_stride, const int32_t *q_start, const int32_t *kv_lens,
    const int32_t *prefill_items, int32_t n_prefill, int32_t num_seqs,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t page_size, float scale, void *stream) {
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
  HY_REQUIRE(n_prefill >= 0, "n_prefill must be non-negative");
  if (n_prefill == 0) return HY_OK;
  HY_REQUIRE(q && out && k_pool && v_pool && page_table && q_start && kv_lens &&
                 prefill_items,
             "hy_paged_prefill: null pointer argument");
  const int G = num_q_heads / num_kv_heads;
  const float scale_log2 = scale * hy::kLog2e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(n_prefill, num_kv_heads);
  const uint16_t *qq = static_cast<const uint16_t *>(q);
  uint16_t *oo = static_cast<uint16_t *>(out);
  const uint16_t *kp = static_cast<const uint16_t *>(k_pool);
  const uint16_t *vp = static_cast<const uint16_t *>(v_pool);
#define HY_PREFILL_CASE(GG)                                                     \
  case GG:                                                                      \
    hy::launch_prefill<GG>(st, grid, qq, q_stride_seq, q_stride_tok,            \
                           q_stride_head, oo, o_stride_seq, o_stride_tok,       \
                           o_stride_head, kp, vp, pool_head_stride, page_table, \
                           page_table_stride, q_start, kv_lens, prefill_items,  \
                           page_size, scale_log2);                              \
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
