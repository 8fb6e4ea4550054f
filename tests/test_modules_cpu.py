"""EnhancedMultiHeadAttention and the interface's convenience wrappers on the
CPU: construction, the mask-to-bias conversion against the reference's
materialised formula (examples/basic_usage.py:232-251), argument forwarding
and the performance-mode context managers (interface.py:611-661)."""
import pytest
import torch

import flash_attention_v100 as fa
from flash_attention_v100 import interface
from flash_attention_v100.modules import EnhancedMultiHeadAttention, mask_to_bias


def _reference_bias(attn_mask, key_padding_mask, B, H, Sq, Sk):
    # examples/basic_usage.py:232-251: zeros (B, H, Sq, Sk), masked_fill -inf
    bias = torch.zeros(B, H, Sq, Sk)
    if attn_mask is not None:
        if attn_mask.dim() == 2:
            bias = bias.masked_fill(attn_mask.unsqueeze(0).unsqueeze(0), float("-inf"))
        elif attn_mask.dim() == 3:
            bias = bias.masked_fill(attn_mask.unsqueeze(1), float("-inf"))
    if key_padding_mask is not None:
        bias = bias.masked_fill(key_padding_mask.unsqueeze(1).unsqueeze(1), float("-inf"))
    return bias


@pytest.mark.parametrize("kind", ["2d", "3d", "pad", "2d+pad", "3d+pad"])
def test_mask_to_bias_matches_reference_formula(kind):
    g = torch.Generator().manual_seed(3)
    B, H, Sq, Sk = 3, 4, 5, 7
    am = None
    if kind.startswith("2d"):
        am = torch.rand(Sq, Sk, generator=g) < 0.3
    elif kind.startswith("3d"):
        am = torch.rand(B, Sq, Sk, generator=g) < 0.3
    kpm = torch.rand(B, Sk, generator=g) < 0.3 if "pad" in kind else None
    got = mask_to_bias(am, kpm, B, Sq, Sk, torch.float32, "cpu")
    assert got.dim() == 4 and got.shape[1] == 1  # broadcasts over heads, never materialised per head
    assert torch.equal(got.expand(B, H, Sq, Sk), _reference_bias(am, kpm, B, H, Sq, Sk))


def test_mask_to_bias_float_mask_and_errors():
    am = torch.randn(4, 6)
    got = mask_to_bias(am, None, 2, 4, 6, torch.float32, "cpu")
    assert torch.equal(got[0, 0], am)
    assert mask_to_bias(None, None, 2, 4, 6, torch.float32, "cpu") is None
    with pytest.raises(ValueError):
        mask_to_bias(torch.zeros(4, 5, dtype=torch.bool), None, 2, 4, 6, torch.float32, "cpu")
    with pytest.raises(ValueError):
        mask_to_bias(None, torch.zeros(2, 5, dtype=torch.bool), 2, 4, 6, torch.float32, "cpu")
    with pytest.raises(ValueError):
        mask_to_bias(torch.zeros(1, 1, 4, 6, dtype=torch.bool), None, 2, 4, 6, torch.float32, "cpu")


def test_module_construction_and_init():
    torch.manual_seed(0)
    m = EnhancedMultiHeadAttention(256, 4, dropout=0.1, bias=True, batch_first=False,
                                   optimization_strategy="speed", enable_gradient_checkpointing=True)
    assert (m.embed_dim, m.num_heads, m.head_dim, m.dropout) == (256, 4, 64, 0.1)
    for lin in (m.q_proj, m.k_proj, m.v_proj, m.out_proj):
        assert lin.weight.shape == (256, 256) and torch.equal(lin.bias, torch.zeros(256))
        bound = (6.0 / (256 + 256)) ** 0.5  # Xavier uniform
        assert lin.weight.abs().max() <= bound
    assert EnhancedMultiHeadAttention(64, 2, bias=False).q_proj.bias is None
    with pytest.raises(AssertionError):
        EnhancedMultiHeadAttention(100, 3)
    assert m.get_performance_stats() is None


def test_module_forwards_arguments(monkeypatch):
    # the module's call into flash_attention_v100, recorded on the CPU
    seen = {}

    def fake(q, k, v, **kw):
        seen.update(kw, q=q.shape, k=k.shape, v=v.shape)
        return q.clone()

    monkeypatch.setattr("flash_attention_v100.modules.flash_attention_v100", fake)
    m = EnhancedMultiHeadAttention(64, 4, dropout=0.2, batch_first=False)
    x = torch.randn(10, 2, 64)  # (S, B, E)
    kpm = torch.zeros(2, 10, dtype=torch.bool)
    kpm[1, 7:] = True
    out, w = m(x, key_padding_mask=kpm, is_causal=True)
    assert out.shape == (10, 2, 64) and w is None
    assert seen["q"] == (2, 10, 4, 16) and seen["causal"] is True and seen["dropout_p"] == 0.2
    assert seen["bias"].shape == (2, 1, 1, 10) and torch.isneginf(seen["bias"][1, 0, 0, 7:]).all()
    m.eval()
    with pytest.warns(UserWarning):
        out, w = m(x, need_weights=True)
    assert seen["dropout_p"] == 0.0 and seen["bias"] is None and w.shape == (2, 4, 10, 10)


def test_convenience_wrappers_and_modes(monkeypatch):
    seen = []
    monkeypatch.setattr(interface, "flash_attention_v100", lambda q, k, v, **kw: seen.append(kw) or q)
    t = torch.zeros(1)
    interface.flash_attention_v100_causal(t, t, t, scale=0.5)
    interface.flash_attention_v100_with_dropout(t, t, t, 0.3, causal=True)
    assert seen == [{"causal": True, "scale": 0.5}, {"dropout_p": 0.3, "causal": True}]
    assert fa.flash_attention_v100_causal is not None and fa.flash_attention_v100_with_dropout is not None
    assert interface.current_optimization_strategy() == "balanced"
    with fa.flash_attention_performance_mode("speed"):
        assert interface.current_optimization_strategy() == "speed"
        with fa.flash_attention_memory_mode():
            assert interface.current_optimization_strategy() == "memory"
        assert interface.current_optimization_strategy() == "speed"
    assert interface.current_optimization_strategy() == "balanced"
    with pytest.raises(ValueError):
        with fa.flash_attention_performance_mode("fastest"):
            pass
