"""EnhancedMultiHeadAttention (reference examples/basic_usage.py:48-255) on the
gfx950 kernels against the same layer evaluated in float64 on the CPU with the
oracle's attention: outputs and parameter gradients, with key-padding and
attention masks, causal masking, (S, B, E) inputs and gradient checkpointing.

Float32 layers run the kernels' fp32 path: tolerance 1e-5 of max|oracle| (the
projections add float32 GEMM rounding of the same order, so 2e-5 is used).
"""
import pytest
import torch

from flash_attention_v100 import EnhancedMultiHeadAttention
from flash_attention_v100.modules import mask_to_bias
from oracle import attention as oa

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(msg):
    print(msg, flush=True)


def reference_layer(m, query, key_padding_mask=None, attn_mask=None, is_causal=False):
    """The layer in float64 on the CPU: projections, oracle attention with the
    masks as an additive bias, output projection.  Returns (out, param grads fn)."""
    P = {n: p.detach().double().cpu().requires_grad_(True) for n, p in m.named_parameters()}
    x = query.detach().double().cpu()
    if not m.batch_first:
        x = x.transpose(0, 1)
    B, S, E = x.shape
    H, Dh = m.num_heads, m.head_dim

    def lin(name, t):
        return t @ P[name + ".weight"].T + P[name + ".bias"]

    q = lin("q_proj", x).view(B, S, H, Dh)
    k = lin("k_proj", x).view(B, S, H, Dh)
    v = lin("v_proj", x).view(B, S, H, Dh)
    bias = mask_to_bias(attn_mask.cpu() if attn_mask is not None else None,
                        key_padding_mask.cpu() if key_padding_mask is not None else None,
                        B, S, S, torch.float64, "cpu")
    o, _ = oa.attention_forward(q, k, v, is_causal, Dh ** -0.5, dtype=torch.float64, bias=bias)
    out = lin("out_proj", o.reshape(B, S, E))
    if not m.batch_first:
        out = out.transpose(0, 1)
    return out, P


CASES = [
    # (batch_first, causal, key padding, attn mask)
    (True, False, False, False),
    (True, True, True, False),
    (False, False, True, True),
    (True, False, False, True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"bf{int(c[0])}-causal{int(c[1])}-pad{int(c[2])}-mask{int(c[3])}")
def test_layer_matches_float64_reference(case):
    batch_first, causal, pad, mask = case
    say(f"case: EnhancedMultiHeadAttention fp32 {case}")
    torch.manual_seed(0)
    B, S, E, H = 2, 96, 256, 4
    m = EnhancedMultiHeadAttention(E, H, batch_first=batch_first).to(DEV)
    with torch.no_grad():  # non-zero projection biases so that they are checked too
        for lin in (m.q_proj, m.k_proj, m.v_proj, m.out_proj):
            lin.bias.normal_(0, 0.1)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, S, E, generator=g)
    if not batch_first:
        x = x.transpose(0, 1).contiguous()
    kpm = None
    if pad:
        kpm = torch.zeros(B, S, dtype=torch.bool)
        kpm[1, 70:] = True
    am = None
    if mask:
        am = torch.rand(S, S, generator=g) < 0.2
        am.fill_diagonal_(False)  # every query keeps a key
    xd = x.to(DEV).requires_grad_(True)
    out, w = m(xd, key_padding_mask=kpm.to(DEV) if pad else None, attn_mask=am.to(DEV) if mask else None,
               is_causal=causal)
    assert w is None
    dout = torch.randn(out.shape, generator=g)
    out.backward(dout.to(DEV))
    ref, P = reference_layer(m, x, kpm, am, causal)
    ref.backward(dout.double())
    tol = 2e-5 * ref.abs().max().item()
    err = (out.detach().cpu().double() - ref.detach()).abs().max().item()
    say(f"out err {err:.3e} tol {tol:.3e}")
    assert err <= tol
    # the key projection's bias gradient is exactly 0 in exact arithmetic (a
    # shift of every key moves all scores of a query alike): gradients get an
    # absolute floor of 1e-5 times the largest parameter-gradient magnitude
    floor = 1e-5 * max(P[n].grad.abs().max().item() for n in P)
    for n, p in m.named_parameters():
        rg = P[n].grad
        e = (p.grad.cpu().double() - rg).abs().max().item()
        t = max(2e-5 * rg.abs().max().item(), floor)
        say(f"grad {n} err {e:.3e} tol {t:.3e}")
        assert e <= t, n


def test_layer_bf16_close_to_reference_and_checkpointing():
    say("case: EnhancedMultiHeadAttention bf16, checkpointing on/off")
    torch.manual_seed(0)
    B, S, E, H = 2, 256, 512, 4
    m = EnhancedMultiHeadAttention(E, H).to(DEV).to(torch.bfloat16)
    x = torch.randn(B, S, E, device=DEV, dtype=torch.bfloat16)
    outs = []
    for ckpt in (False, True):
        m.enable_gradient_checkpointing = ckpt
        m.zero_grad()
        o, _ = m(x, is_causal=True)
        o.float().pow(2).sum().backward()
        outs.append((o.detach(), [p.grad.clone() for p in m.parameters()]))
    assert torch.equal(outs[0][0], outs[1][0])
    for a, b in zip(outs[0][1], outs[1][1]):
        assert torch.equal(a, b)
    ref, _ = reference_layer(m, x, is_causal=True)
    err = (outs[0][0].cpu().double() - ref.detach()).abs().max().item()
    assert err <= 3e-2 * ref.abs().max().item(), err


def test_layer_dropout_training_vs_eval_and_stats():
    say("case: EnhancedMultiHeadAttention dropout / eval / stats")
    torch.manual_seed(0)
    m = EnhancedMultiHeadAttention(256, 4, dropout=0.3, enable_performance_monitoring=True).to(DEV)
    x = torch.randn(2, 128, 256, device=DEV)
    torch.manual_seed(5)
    a, _ = m(x)
    torch.manual_seed(5)
    b, _ = m(x)
    assert torch.equal(a, b)  # the Philox seed comes from torch's CPU generator
    m.eval()
    c, _ = m(x)
    d, _ = m(x)
    assert torch.equal(c, d) and not torch.equal(a, c)
    st = m.get_performance_stats()
    assert st["forward_count"] == 4 and st["mean_ms"] > 0
