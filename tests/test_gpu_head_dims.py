"""Head dims between the compiled 32 / 64 / 128 (and 256 for fp16 / bf16 inputs
without a bias) run zero-padded to the next one (``_lib.padded_head_dim``):
zero columns of q, k and v add nothing to the
scores, the scale is the caller's D**-0.5, and the extra columns of O, dQ,
dK, dV are exactly zero, so results at D are those of the attention at D.
The dropout mask depends on (b, h, query, key) only: it is the C oracle's
mask for the same seed and offset.  O, LSE, dQ, dK, dV against the float64
oracle with the tolerance of the other parity tests (fp16/bf16 within 2x the
error of the reference math run in the inputs' dtype, fp32 within 1e-5)."""
import warnings

import pytest
import torch

import flash_attention_v100 as fa
from flash_attention_v100 import _lib
from helpers import assert_parity, c_keep_mask, compare, make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # dtype, B, S, H, Hkv, D, causal, p
    (torch.bfloat16, 2, 200, 4, 2, 80, True, 0.0),
    (torch.float16, 1, 333, 2, 2, 96, False, 0.1),
    (torch.bfloat16, 1, 128, 3, 1, 16, True, 0.0),
    (torch.float32, 1, 100, 2, 2, 48, False, 0.0),
    (torch.float16, 1, 257, 2, 2, 120, True, 0.0),
    # head dim 256 (fp16 / bf16 without a bias) and dims padded to it
    (torch.bfloat16, 2, 300, 4, 2, 256, True, 0.0),
    (torch.float16, 1, 257, 2, 2, 256, False, 0.1),
    (torch.float16, 1, 130, 3, 1, 200, True, 0.0),
    (torch.bfloat16, 1, 64, 2, 2, 129, False, 0.0),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-S{c[2]}-H{c[3]}-Hkv{c[4]}-D{c[5]}-{c[6]}-p{c[7]}" for c in CASES])
def test_padded_head_dim_parity(case):
    dt, B, S, H, Hkv, D, causal, p = case
    print(f"case: padded head dim {case}", flush=True)
    dp = _lib.padded_head_dim(D, dt)
    assert dp in _lib.HEAD_DIMS + (_lib.WIDE_HEAD_DIM,) and dp >= D
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dt, Hkv=Hkv, seed=31))
    scale = D ** -0.5
    seed, offset = 1234, 64
    o, lse, _ = _lib.fwd(q, k, v, causal, scale, p, seed, offset)
    dq, dk, dv = _lib.bwd(q, k, v, o, do, lse, causal, scale, p, seed, offset)
    torch.cuda.synchronize()
    assert o.shape == q.shape and dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    keep = torch.from_numpy(c_keep_mask(seed, offset, B, H, S, S, p)).to(DEV) if p > 0 else None
    res = compare(q, k, v, do, causal, scale, (o, lse, dq, dk, dv), keep=keep, p=p)
    assert_parity(res, dt, f"D={D}")


def test_padded_head_dim_through_the_interface():
    # no fallback warning: the kernels run; gradients through autograd equal the ABI's
    q, k, v, do = (t.to(DEV) for t in make_inputs(2, 150, 4, 72, torch.bfloat16, seed=32))
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        out = fa.flash_attention_v100(qq, kk, vv, causal=True)
    out.backward(do)
    o, lse, _ = _lib.fwd(q, k, v, True, 72 ** -0.5)
    dq, dk, dv = _lib.bwd(q, k, v, o, do, lse, True, 72 ** -0.5)
    assert torch.equal(out, o) and torch.equal(qq.grad, dq) and torch.equal(kk.grad, dk) and torch.equal(vv.grad, dv)


def test_head_dim_256_through_the_interface():
    # fp16 / bf16 at D = 256 run the kernels (no fallback warning), with
    # dropout through the autograd route (keep bits stored by the forward);
    # gradients equal the ABI's for the same seed and offset
    B, S, H, D = 1, 200, 2, 256
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.bfloat16, seed=33))
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        out = fa.flash_attention_v100(qq, kk, vv, causal=True, dropout_p=0.1, dropout_seed=7, dropout_offset=0)
    out.backward(do)
    o, lse, _ = _lib.fwd(q, k, v, True, D ** -0.5, 0.1, 7, 0)
    dq, dk, dv = _lib.bwd(q, k, v, o, do, lse, True, D ** -0.5, 0.1, 7, 0)
    assert torch.equal(out, o) and torch.equal(qq.grad, dq) and torch.equal(kk.grad, dk) and torch.equal(vv.grad, dv)


@pytest.mark.parametrize("what", ["bias", "fp32"])
def test_head_dim_256_without_kernel_falls_back(what):
    # a bias or float32 inputs at D = 256 have no kernel: NotImplementedError,
    # served by the on-device math with fallback_on_error=True
    B, S, H, D = 1, 96, 2, 256
    dt = torch.float32 if what == "fp32" else torch.bfloat16
    q, k, v, _ = (t.to(DEV) for t in make_inputs(B, S, H, D, dt, seed=34))
    bias = torch.randn(B, H, S, S, device=DEV).to(dt) if what == "bias" else None
    with pytest.warns(UserWarning, match="falling back"):
        out = fa.flash_attention_v100(q, k, v, causal=True, bias=bias)
    with pytest.raises(NotImplementedError):
        fa.flash_attention_v100(q, k, v, causal=True, bias=bias, fallback_on_error=False)
    s = torch.matmul(q.float().transpose(1, 2), k.float().transpose(1, 2).transpose(-2, -1).contiguous()) * D ** -0.5
    if bias is not None:
        s = s + bias.float()
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool, device=DEV).triu(1), float("-inf"))
    ref = torch.matmul(torch.softmax(s, -1), v.float().transpose(1, 2)).transpose(1, 2)
    assert (out.float() - ref).abs().max().item() < (2e-2 if dt != torch.float32 else 1e-5)


@pytest.mark.parametrize("causal", [True, False])
def test_head_dim_256_full_size(causal):
    # D = 256 at a full-size shape (4096 tokens, GQA 16 / 8 heads): O, LSE, dQ,
    # dK, dV against the float64 oracle within the 2x envelope, as the
    # BASELINE configs are checked
    B, S, H, Hkv, D = 2, 4096, 16, 8, 256
    print(f"case: D=256 full size ({B},{S},{H},{Hkv},{D}) bf16 causal={causal}", flush=True)
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.bfloat16, Hkv=Hkv, seed=35))
    scale = D ** -0.5
    o, lse, _ = _lib.fwd(q, k, v, causal, scale)
    dq, dk, dv = _lib.bwd(q, k, v, o, do, lse, causal, scale)
    torch.cuda.synchronize()
    res = compare(q, k, v, do, causal, scale, (o, lse, dq, dk, dv))
    assert_parity(res, torch.bfloat16, f"D=256 full size causal={causal}")
