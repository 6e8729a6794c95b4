"""Host-side pieces of the attention module and model that run without a
GPU: the fused q/k/v projection and the checkpoint name map."""

import torch

from hayate_amd.attention import GroupedQueryAttention
from hayate_amd.model import Qwen3Config, Qwen3Model, qwen_weight_map


def test_fused_qkv_projection_views_one_gemm():
    torch.manual_seed(0)
    mod = GroupedQueryAttention(64, 4, 2, 16, dtype=torch.float32)
    x = torch.randn(3, 5, 64)
    q, k, v = mod.project_qkv(x)
    torch.testing.assert_close(q, mod.q_proj(x).view(3, 5, 4, 16))
    torch.testing.assert_close(k, mod.k_proj(x).view(3, 5, 2, 16))
    torch.testing.assert_close(v, mod.v_proj(x).view(3, 5, 2, 16))
    # views of one buffer: no split copies, rows 16-byte aligned
    base = q.untyped_storage().data_ptr()
    assert k.untyped_storage().data_ptr() == base == v.untyped_storage().data_ptr()
    assert q.stride() == (5 * 128, 128, 16, 1) and k.stride(1) == 128
    # the fused weight follows in-place updates of the parameters
    with torch.no_grad():
        mod.k_proj.weight.mul_(2)
    _, k2, _ = mod.project_qkv(x)
    torch.testing.assert_close(k2, 2 * k)


def test_fused_qkv_weight_is_the_only_copy():
    """q/k/v_proj.weight are views of the one fused buffer (no second copy of
    the projection weights); in-place loads write through; the buffer is
    rebuilt, and the rebuild counter advances, only when a parameter is
    replaced rather than updated, and the first build under inference_mode
    still leaves trainable parameters."""
    import hayate_amd.attention as A

    torch.manual_seed(1)
    mod = GroupedQueryAttention(64, 4, 2, 16, dtype=torch.float32)
    x = torch.randn(2, 3, 64)
    ref = [lin.weight.detach().clone() for lin in (mod.q_proj, mod.k_proj, mod.v_proj)]
    n0 = A.qkv_rebuilds
    with torch.inference_mode():
        f = mod.fused_qkv_weight()
    assert A.qkv_rebuilds == n0 + 1
    assert torch.equal(f, torch.cat(ref))
    base = f.untyped_storage().data_ptr()
    for lin in (mod.q_proj, mod.k_proj, mod.v_proj):
        assert lin.weight.untyped_storage().data_ptr() == base
        assert isinstance(lin.weight, torch.nn.Parameter) and lin.weight.requires_grad
        assert not lin.weight.is_inference()
    assert mod.q_proj(x).requires_grad
    # a state-dict load copies into the views: same buffer, new values
    sd = {k: (2 * v if k.endswith("proj.weight") else v) for k, v in mod.state_dict().items()}
    mod.load_state_dict(sd)
    assert mod.fused_qkv_weight() is f and A.qkv_rebuilds == n0 + 1
    assert torch.equal(f, 2 * torch.cat(ref))
    # replacing a parameter rebuilds the buffer from the current weights
    mod.v_proj.weight = torch.nn.Parameter(torch.zeros_like(mod.v_proj.weight))
    f2 = mod.fused_qkv_weight()
    assert f2 is not f and A.qkv_rebuilds == n0 + 2
    assert torch.equal(f2[-32:], torch.zeros(32, 64)) and torch.equal(f2[:64], 2 * ref[0])


def test_checkpoint_name_map_covers_every_parameter():
    cfg = Qwen3Config(vocab_size=64, hidden_size=32, num_layers=2, num_heads=4,
                      num_kv_groups=2, head_dim=8, intermediate_size=48)
    with torch.device("meta"):
        model = Qwen3Model(cfg)
    names = qwen_weight_map(model)
    params = {id(p) for p in model.parameters()}
    assert {id(p) for p in names.values()} == params
    assert "model.layers.1.self_attn.q_norm.weight" in names
    assert len(names) == 3 + 11 * 2


def test_stop_ids_from_generation_config_and_tokenizer(tmp_path):
    """End-of-generation ids (engine.py:112-129 of the reference): the
    checkpoint's generation_config.json eos id or list, plus the
    tokenizer's eos id; a missing or broken config leaves the tokenizer's."""
    import json
    from types import SimpleNamespace

    from hayate_amd.engine import _stop_token_ids

    tok = SimpleNamespace(eos_token_id=7)
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": [1, 2]}))
    assert _stop_token_ids(str(tmp_path), tok) == {1, 2, 7}
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": 3}))
    assert _stop_token_ids(str(tmp_path), None) == {3}
    (tmp_path / "generation_config.json").write_text("{not json")
    assert _stop_token_ids(str(tmp_path), tok) == {7}
    assert _stop_token_ids(None, tok) == {7}
    assert _stop_token_ids(str(tmp_path / "missing"), None) == set()
