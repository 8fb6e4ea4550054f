"""Parity of the 8-wave ping-pong backward kernels (dkdv_pp_kernel,
dq_pp_kernel), called through the C ABI, against the float64 oracle and bit
for bit against dkdv_kernel / dq_kernel.

The library runs them for 16-bit inputs with D = 128, no bias and no dropout,
when their workgroups fill the chip: ceil(Sk / 256) * Hkv * B >= 256 (dK/dV,
256 keys per workgroup) and ceil(Sq / 256) * H * B >= 256 (dQ, 256 queries
per workgroup).  Every shape below meets both rules, with the edge cases of
their tile loops: Sq and Sk not multiples of the tiles or blocks, GQA (the
query heads of a KV group in one run of tiles), Sq != Sk in both directions
under causal masking (top-left aligned), strided views, fp16 and bf16.  Per
key (per query) they do the arithmetic of dkdv_kernel (dq_kernel) in the same
order, so a (batch, head) slice computed inside a grid that routes to them
equals, bit for bit, the same slice computed alone on a small grid, which the
other kernels run; so do dQ and the workspace rows of stage 3 (dQ with delta
computed in the kernel) and of stages 0 then 2 (delta pre-pass, then dQ).
"""
import pytest
import torch

from flash_attention_v100 import _lib
from helpers import assert_parity, compare, make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(msg):
    print(msg, flush=True)


def routes_to_dkdv_pp(B, Sk, Hkv, D, dtype):
    return dtype != torch.float32 and D == 128 and ((Sk + 255) // 256) * Hkv * B >= 256


def routes_to_dq_pp(B, Sq, H, D, dtype):
    return dtype != torch.float32 and D == 128 and ((Sq + 255) // 256) * H * B >= 256


CASES = [
    # dtype, B, Sq, Sk, H, Hkv, causal
    (torch.bfloat16, 2, 1000, 777, 256, 64, False),   # ragged Sq and Sk, GQA 4:1
    (torch.float16, 1, 1000, 1000, 256, 256, True),   # causal, ragged last tile and key block
    (torch.bfloat16, 4, 700, 1300, 64, 16, True),     # causal with Sq < Sk (keys past the last query)
    (torch.bfloat16, 2, 1500, 600, 128, 64, True),    # causal with Sq > Sk, GQA 2:1
    (torch.float16, 1, 64, 2048, 256, 32, False),     # one query tile, GQA 8:1
]


def _id(c):
    dt, B, Sq, Sk, H, Hkv, causal = c
    return f"{str(dt)[6:]}-B{B}-Sq{Sq}-Sk{Sk}-H{H}-Hkv{Hkv}-{'causal' if causal else 'full'}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_bwd_pp_parity(case):
    dt, B, Sq, Sk, H, Hkv, causal = case
    assert routes_to_dkdv_pp(B, Sk, Hkv, 128, dt) and routes_to_dq_pp(B, Sq, H, 128, dt)
    say(f"case: ping-pong backward {_id(case)}")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Sq, H, 128, dt, Sk=Sk, Hkv=Hkv, seed=31))
    scale = 128 ** -0.5
    o, lse, _ = _lib.fwd(q, k, v, causal, scale)
    dq, dk, dv = _lib.bwd(q, k, v, o, do, lse, causal, scale)
    torch.cuda.synchronize()
    res = compare(q, k, v, do, causal, scale, (o, lse, dq, dk, dv), hpc=8)
    assert_parity(res, dt, _id(case))


@pytest.mark.parametrize("causal", [False, True])
def test_bwd_pp_equals_other_kernels_bitwise(causal):
    """Batch 0 of a (16, 1100, 32) grid (routed to dkdv_pp_kernel and
    dq_pp_kernel) against the same batch run alone (160 workgroups of each:
    dkdv_kernel, dq_kernel), also through strided (B, H, S, D)-major views."""
    B, S, H, D = 16, 1100, 32, 128
    assert routes_to_dkdv_pp(B, S, H, D, torch.bfloat16) and not routes_to_dkdv_pp(1, S, H, D, torch.bfloat16)
    assert routes_to_dq_pp(B, S, H, D, torch.bfloat16) and not routes_to_dq_pp(1, S, H, D, torch.bfloat16)
    say(f"case: ping-pong backward vs dkdv_kernel / dq_kernel bitwise, ({B},{S},{H},{D}) bf16 causal={causal}")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.bfloat16, seed=32))
    scale = D ** -0.5
    o, lse, _ = _lib.fwd(q, k, v, causal, scale)
    dq, dk, dv = _lib.bwd(q, k, v, o, do, lse, causal, scale)
    one = [t[:1].contiguous() for t in (q, k, v, o, do)]
    dq1, dk1, dv1 = _lib.bwd(*one, lse[:1].contiguous(), causal, scale)
    qs, ks, vs, os_, dos = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v, o, do))
    dq2, dk2, dv2 = _lib.bwd(qs, ks, vs, os_, dos, lse, causal, scale)
    torch.cuda.synchronize()
    assert torch.equal(dk[:1], dk1) and torch.equal(dv[:1], dv1) and torch.equal(dq[:1], dq1)
    assert torch.equal(dk, dk2) and torch.equal(dv, dv2) and torch.equal(dq, dq2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_dq_pp_stage3_equals_prepass_then_dq(dt):
    """include/fa_abi.h: stage 3 (dQ computing delta itself) equals stage 0 then
    stage 2 (dQ reading delta from the workspace) bit for bit, rows and dQ,
    including the padding rows past Sq (Sq = 1100: 256-query workgroups reach
    past the 1152 workspace rows, which they must not write) and a row whose
    LSE is -inf."""
    import ctypes
    B, S, H, D = 2, 1100, 128, 128
    assert routes_to_dq_pp(B, S, H, D, dt)
    say(f"case: dq_pp stage 3 vs stages 0 + 2, ({B},{S},{H},{D}) {dt}")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dt, Hkv=32, seed=33))
    o, lse, _ = _lib.fwd(q, k, v, True, D ** -0.5)
    lse[0, 1, 5] = float("-inf")
    lib = _lib.load()
    outs = []
    for stages in ((0, 2), (3,)):
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        a = _lib.bwd_args(q, k, v, o, do, lse, dq, dk, dv, True, D ** -0.5, 0.0, 0, 0)
        nbytes = lib.fa_bwd_workspace_size(ctypes.byref(a))
        ws = torch.full((nbytes // 4,), 7.0, device=DEV)
        sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for st in stages:
            assert lib.fa_bwd_stage(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), nbytes, st, sp) == 0
        torch.cuda.synchronize()
        rows = B * H * 2 * ((S + 127) // 128 * 128)
        outs.append((ws.clone(), dq.clone(), rows))
    assert torch.equal(outs[0][0], outs[1][0])  # the whole workspace, past the rows included
    assert torch.equal(outs[0][1], outs[1][1])
    assert bool((outs[1][0][outs[1][2]:] == 7.0).all())
