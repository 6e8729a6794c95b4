"""hy_paged_decode_append_noalloc against hy_paged_decode_append +
hy_paged_decode_merge (through the C ABI, via PagedKVBatch.decode_layer).

The no-allocation entry point keeps the split partials in the library's
static device scratch. Two calls in a row on the same GPU — the batch-32
decode step, then a smaller one (batch 5) — must each match the
workspace path bit for bit (rotated q, K/V pools, attention output): the
second call runs over the first call's scratch contents. A tick whose
partials exceed the scratch is refused before any launch.
"""

import numpy as np
import pytest
import torch

from gpu_util import EPS, bits, layer_bits, say

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from hayate_amd import _native
    from hayate_amd.workloads import make_workload

DEV = "cuda"


def _pair(lengths):
    kw = {} if lengths is None else {"lengths": lengths}
    return (make_workload("decode_b32", device=DEV, **kw),
            make_workload("decode_b32", device=DEV, **kw))


def _check_call(w_static, w_ws, what):
    b_static = w_static.begin()
    q_s, out_s = b_static.decode_layer(0, w_static.q, w_static.k, w_static.v, w_static.q_norm_w,
                                       w_static.k_norm_w, EPS, w_static.cos, w_static.sin,
                                       no_alloc=True)
    b_ws = w_ws.begin()
    q_w, out_w = b_ws.decode_layer(0, w_ws.q, w_ws.k, w_ws.v, w_ws.q_norm_w, w_ws.k_norm_w, EPS,
                                   w_ws.cos, w_ws.sin)
    torch.cuda.synchronize()
    plan = b_static.plan(w_static.q.shape[1])
    need = _native.decode_workspace_bytes(plan.n_slots, w_static.q.shape[1], 128)
    say(f"  {what}: {w_static.manager.num_pages} pages, {plan.n_slots} slots, {need} B scratch")
    assert np.array_equal(bits(q_s), bits(q_w)), f"{what}: rotated q differs"
    ks, vs = layer_bits(w_static.manager)
    kw, vw = layer_bits(w_ws.manager)
    assert np.array_equal(ks, kw), f"{what}: K pool differs"
    assert np.array_equal(vs, vw), f"{what}: V pool differs"
    assert np.array_equal(bits(out_s), bits(out_w)), f"{what}: attention output differs"


def test_noalloc_decode_matches_workspace_path_on_two_calls():
    say("[no-alloc decode: batch 32 then batch 5]")
    w_a, w_b = _pair(None)
    _check_call(w_a, w_b, "batch 32")
    del w_a, w_b
    small = ([300, 4000, 17, 1023, 128], [1] * 5)
    w_a, w_b = _pair(small)
    _check_call(w_a, w_b, "batch 5")


def test_noalloc_refuses_partials_beyond_the_scratch():
    say("[no-alloc decode: oversize tick refused]")
    n = 400  # 400 pieces x 2 waves x 32 heads x 130 floats > 8 MiB
    w = make_workload("decode_b32", device=DEV, lengths=([40] * n, [1] * n), fill=False)
    batch = w.begin()
    plan = batch.plan(w.q.shape[1])
    assert _native.decode_workspace_bytes(plan.n_slots, 32, 128) > _native.NOALLOC_SCRATCH_BYTES
    with pytest.raises(MemoryError):
        batch.decode_layer(0, w.q, w.k, w.v, w.q_norm_w, w.k_norm_w, EPS, w.cos, w.sin,
                           no_alloc=True)
