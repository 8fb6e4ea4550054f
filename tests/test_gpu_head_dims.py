"""Head dims between the compiled 32 / 64 / 128 run zero-padded to the next
one (``_lib.padded_head_dim``): zero columns of q, k and v add nothing to the
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
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-S{c[2]}-H{c[3]}-Hkv{c[4]}-D{c[5]}-{c[6]}-p{c[7]}" for c in CASES])
def test_padded_head_dim_parity(case):
    dt, B, S, H, Hkv, D, causal, p = case
    print(f"case: padded head dim {case}", flush=True)
    assert _lib.padded_head_dim(D) in _lib.HEAD_DIMS and _lib.padded_head_dim(D) >= D
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
