"""The reference's CPU attention path, restated on torch's FlexAttention.

TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times this on the
host's cores as the reported CPU baseline, and tests may check it; the
product path never imports it.

What the reference runs for one paged layer when its tensors live on the
CPU (hayate/engine/paged_cache.py):
* the K/V append: write_layer's index_put into the pool (:44-60);
* the block mask: a logical causal BlockMask over the batch
  (create_block_mask with the page size as block size, :266-281), converted
  to physical pages by mapping its kv block indices through the page table
  and re-expressing the mask and a score_mod in physical key positions
  (:317-385);
* attention: flex_attention under torch.compile with enable_gqa over the
  whole layer pool (:20, :62-71; see compiled_flex_attention for the one
  compile option that differs).
The steps are the reference's because the baseline must be its algorithm;
the code is this module's own. It needs a uniform batch (one query length
for every request), as the reference's begin_batch does (:202-213).
"""

from __future__ import annotations

import torch
from torch.nn.attention.flex_attention import BlockMask, create_block_mask, flex_attention

_compiled = None


def compiled_flex_attention():
    """torch.compile(flex_attention), built once (paged_cache.py:20).

    The reference compiles with dynamic=True. On the CPU, torch 2.10's
    Inductor C++ template for flex attention with a score_mod fails to
    compile under dynamic shapes (C++ error: 'cur_qSplitSize0' was not
    declared), so the baseline compiles with static shapes (one compile per
    workload shape; the mask and score_mod are the reference's)."""
    global _compiled
    if _compiled is None:
        _compiled = torch.compile(flex_attention, dynamic=False)
    return _compiled


class FlexPagedBatch:
    """Per-forward metadata of a uniform batch: page table, cache lengths,
    and the physical-page BlockMask + score_mod (paged_cache.py:202-293,
    317-385)."""

    def __init__(self, page_lists, cache_lens, query_len, page_size, capacity_tokens):
        b = len(page_lists)
        num_pages = capacity_tokens // page_size
        self.page_size = page_size
        self.query_len = query_len
        table = torch.full((b, num_pages), -1, dtype=torch.long)
        phys_to_logical = torch.full((b, num_pages), -1, dtype=torch.long)
        for row, pages in enumerate(page_lists):
            ids = torch.tensor(pages, dtype=torch.long)
            table[row, : len(pages)] = ids
            phys_to_logical[row, ids] = torch.arange(len(pages), dtype=torch.long)
        self.page_table = table
        self.cache_lens = torch.tensor(cache_lens, dtype=torch.long)
        kv_lens = self.cache_lens + query_len
        cl = self.cache_lens

        def causal(bi, _h, qi, ki):
            return (ki >= 0) & (ki < kv_lens[bi]) & (ki <= cl[bi] + qi)

        logical = create_block_mask(causal, B=b, H=None, Q_LEN=query_len,
                                    KV_LEN=int(kv_lens.max()), device="cpu",
                                    BLOCK_SIZE=(page_size, page_size))

        def to_physical(indices):
            # logical kv block -> physical page, padded to the pool's page count
            mapped = torch.gather(table, 1, indices.reshape(b, -1).to(torch.long))
            out = torch.zeros((*indices.shape[:-1], num_pages), dtype=torch.int32)
            out[..., : indices.shape[-1]] = mapped.reshape(indices.shape).to(torch.int32)
            return out

        full_num = full_idx = None
        if logical.full_kv_num_blocks is not None:
            full_num = logical.full_kv_num_blocks.clone()
            full_idx = to_physical(logical.full_kv_indices)

        def logical_key(bi, pk):
            lp = phys_to_logical[bi, pk // page_size]
            lk = lp * page_size + pk % page_size
            return lk, (lp >= 0) & (lk >= 0) & (lk < kv_lens[bi])

        def physical_mask(bi, h, qi, pk):
            lk, valid = logical_key(bi, pk)
            return valid & logical.mask_mod(bi, h, qi, lk)

        def physical_score(score, bi, h, qi, pk):
            return torch.where(logical_key(bi, pk)[1], score, float("-inf"))

        self.block_mask = BlockMask.from_kv_blocks(
            logical.kv_num_blocks.clone(), to_physical(logical.kv_indices), full_num, full_idx,
            logical.BLOCK_SIZE, physical_mask, seq_lengths=(logical.seq_lengths[0],
                                                            capacity_tokens))
        self.score_mod = physical_score

    def write_layer(self, k_pool, v_pool, k, v):
        """pool[0, h, phys(b, c_b + t), :] = k[b, h, t, :] (paged_cache.py:44-60);
        pools (1, Hkv, capacity, D), k / v (B, Hkv, T, D)."""
        t = k.shape[2]
        logical = self.cache_lens[:, None] + torch.arange(t, dtype=torch.long)[None, :]
        phys = (torch.gather(self.page_table, 1, logical // self.page_size) * self.page_size
                + logical % self.page_size)
        k_pool[0, :, phys, :] = k.permute(1, 0, 2, 3)
        v_pool[0, :, phys, :] = v.permute(1, 0, 2, 3)

    def attend_layer(self, q, k_pool, v_pool):
        """Compiled flex_attention over the layer pool (paged_cache.py:62-71):
        q (B, Hq, T, D) -> (B, Hq, T, D)."""
        return compiled_flex_attention()(q, k_pool, v_pool, score_mod=self.score_mod,
                                         block_mask=self.block_mask, enable_gqa=True)
