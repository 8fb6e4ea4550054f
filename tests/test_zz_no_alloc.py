"""fa_bwd_static (the backward on the library's own device scratch, no
workspace argument, no allocation) against fa_bwd on the same inputs: the
kernels are the same, so dQ, dK and dV must be bit-identical.  Two calls in a
row, the second on a smaller problem (the scratch keeps the first call's
contents), then a third back at the first size."""
import pytest
import torch

from flash_attention_v100 import _lib
from helpers import make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(msg):
    print(msg, flush=True)


def _case(B, S, H, Hkv, D, dtype, causal, p=0.0, seed=21):
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dtype, Hkv=Hkv, seed=seed))
    scale = D ** -0.5
    kb = None
    if p > 0:
        kb = _lib.alloc_keep_bits(B, H, S, S, q.device)
    o, lse, _ = _lib.fwd(q, k, v, causal, scale, p, 5, 3, keep_bits=kb)
    ref = _lib.bwd(q, k, v, o, do, lse, causal, scale, p, 5, 3, keep_bits=kb)
    got = _lib.bwd_static(q, k, v, o, do, lse, causal, scale, p, 5, 3, keep_bits=kb)
    torch.cuda.synchronize()
    for n, a, b in zip(("dQ", "dK", "dV"), got, ref):
        assert torch.equal(a, b), n


def test_bwd_static_equals_bwd_on_consecutive_calls():
    shapes = [
        (2, 1024, 8, 8, 128, torch.bfloat16, True),
        (1, 300, 4, 2, 64, torch.float16, False),   # smaller, ragged, GQA
        (2, 1024, 8, 8, 128, torch.bfloat16, True),
    ]
    for sh in shapes:
        say(f"case: fa_bwd_static vs fa_bwd {sh}")
        _case(*sh)


def test_bwd_static_dropout_and_fp32():
    say("case: fa_bwd_static with dropout keep bits, fp32")
    _case(2, 500, 4, 4, 32, torch.float32, True, p=0.1)
    say("case: fa_bwd_static with regenerated dropout, fp16")
    _case(1, 257, 2, 2, 64, torch.float16, True, p=0.2, seed=22)


def test_bwd_static_rejects_oversized_problem():
    # 64 heads x 70000 queries need ~35 MiB of workspace rows: refused with
    # FA_ERR_SCRATCH before any launch (strided views keep the inputs small)
    q = torch.zeros(1, 70000, 1, 64, device=DEV, dtype=torch.bfloat16).expand(1, 70000, 64, 64)
    lse = torch.zeros(1, 64, 70000, device=DEV)
    with pytest.raises(_lib.FlashAttentionKernelError) as ei:
        _lib.bwd_static(q, q, q, q, q, lse, True, 0.125)
    assert ei.value.code == _lib.ERR_SCRATCH
