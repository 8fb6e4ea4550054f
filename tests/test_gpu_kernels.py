"""Parity of the gfx950 kernels, called through the C ABI, against the oracle.

Tolerance: fp16/bf16 outputs within 2x the error of the
reference's own math run in the same dtype on the GPU (both against the
float64 oracle); fp32 within 1e-5 of max|oracle|; dropout masks bit-exact.
Small shapes use the CPU oracle; the benchmark configurations C1-C5 evaluate the same
oracle functions in float64 on the GPU, one head chunk at a time.
"""
import json
import os

import numpy as np
import pytest
import torch

from flash_attention_v100 import _lib
from helpers import assert_parity, c_keep_mask, compare, make_inputs

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DEV = "cuda"


def say(msg):
    print(msg, flush=True)


def run(q, k, v, do, causal, scale, p=0.0, seed=0, offset=0, bwd=True):
    o, lse, _ = _lib.fwd(q, k, v, causal, scale, p, seed, offset)
    if not bwd:
        torch.cuda.synchronize()
        return o, lse
    dq, dk, dv = _lib.bwd(q, k, v, o, do, lse, causal, scale, p, seed, offset)
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv


# ----------------------------------------------------------------------------- RNG

def test_rand_matches_triton_vectors():
    say("case: fa_rand vs triton_rand_vectors.json")
    with open(os.path.join(GOLDEN, "triton_rand_vectors.json")) as f:
        cases = json.load(f)["cases"]
    for c in cases:
        ctr = torch.tensor(np.array(c["counters"], dtype=np.uint64).view(np.int64), device=DEV)
        u = _lib.rand(c["seed"], ctr).cpu().numpy().view(np.uint32)
        assert np.array_equal(u, np.array(c["uniform_f32_bits"], dtype=np.uint32)), c["seed"]


@pytest.mark.parametrize("shape,seed,offset", [
    ((8, 16, 1000, 1000), 42, 0),          # C5 mask
    ((2, 3, 77, 129), 42, 2**32 - 5),      # counter crosses the 32-bit boundary
    ((1, 2, 33, 65), 2**63 + 5, 2**64 - 100),  # 64-bit wrap of the counter
])
def test_dropout_mask_bit_exact(shape, seed, offset):
    say(f"case: fa_dropout_mask {shape} seed={seed} offset={offset}")
    B, H, Sq, Sk = shape
    got = _lib.dropout_mask(seed, offset, B, H, Sq, Sk, 0.1).cpu().numpy()
    want = c_keep_mask(seed, offset, B, H, Sq, Sk, 0.1)
    assert np.array_equal(got, want)


# ----------------------------------------------------------------------------- small shapes, CPU oracle

SMALL = []
for dt in (torch.float16, torch.bfloat16, torch.float32):
    for D in (32, 64, 128):
        for causal in (False, True):
            SMALL.append((dt, 2, 200, 200, 3, 3, D, causal))
SMALL += [
    (torch.bfloat16, 1, 130, 257, 2, 2, 64, True),    # Sq < Sk
    (torch.bfloat16, 1, 300, 77, 2, 2, 64, True),     # Sq > Sk (top-left causal)
    (torch.float16, 1, 300, 77, 2, 2, 128, False),
    (torch.bfloat16, 2, 160, 160, 4, 2, 128, True),   # GQA 2:1
    (torch.float16, 1, 96, 96, 8, 1, 64, False),      # MQA
    (torch.float32, 1, 150, 150, 4, 2, 64, True),     # fp32 GQA
    (torch.bfloat16, 1, 1, 1, 2, 2, 64, True),        # single query / key
    (torch.float16, 3, 1, 50, 2, 2, 32, False),       # decode-like
    (torch.bfloat16, 1, 64, 1, 2, 2, 128, False),     # single key
    (torch.bfloat16, 2, 3, 8192, 4, 1, 128, False),   # decode against a long context (MQA)
    (torch.float16, 32, 64, 64, 16, 16, 64, True),    # many small (batch, head) slices
]


def _id(c):
    dt, B, Sq, Sk, H, Hkv, D, causal = c
    return f"{str(dt)[6:]}-B{B}-Sq{Sq}-Sk{Sk}-H{H}-Hkv{Hkv}-D{D}-{'causal' if causal else 'full'}"


@pytest.mark.parametrize("case", SMALL, ids=[_id(c) for c in SMALL])
def test_small_fwd_bwd(case):
    dt, B, Sq, Sk, H, Hkv, D, causal = case
    say(f"case: small {_id(case)}")
    q, k, v, do = make_inputs(B, Sq, H, D, dt, Sk=Sk, Hkv=Hkv, seed=7)
    scale = D ** -0.5
    outs = run(*(t.to(DEV) for t in (q, k, v, do)), causal, scale)
    res = compare(*(t.to(DEV) for t in (q, k, v, do)), causal, scale, outs, ref_device="cpu")
    assert_parity(res, dt, _id(case))


@pytest.mark.parametrize("D", [32, 64, 128])
def test_small_dropout(D):
    B, S, H, p = 2, 150, 3, 0.2
    say(f"case: small dropout D={D}")
    for dt in (torch.float16, torch.float32):
        q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dt, seed=11))
        outs = run(q, k, v, do, True, D ** -0.5, p, seed=123, offset=456)
        keep = torch.from_numpy(c_keep_mask(123, 456, B, H, S, S, p)).bool().to(DEV)
        res = compare(q, k, v, do, True, D ** -0.5, outs, keep=keep, p=p, ref_device="cpu")
        assert_parity(res, dt, f"dropout D={D} {dt}")


# ----------------------------------------------------------------------------- benchmark configs C1-C5

def test_c1_forward():
    say("case: C1 (2,1024,12,64) fp16 non-causal fwd")
    q, k, v, do = (t.to(DEV) for t in make_inputs(2, 1024, 12, 64, torch.float16))
    outs = run(q, k, v, do, False, 0.125, bwd=False)
    res = compare(q, k, v, do, False, 0.125, outs, ref_device="cpu", with_bwd=False)
    assert_parity(res, torch.float16, "C1")


def test_c2_fwd_bwd():
    say("case: C2 (2,1024,12,64) fp16 causal fwd+bwd")
    q, k, v, do = (t.to(DEV) for t in make_inputs(2, 1024, 12, 64, torch.float16))
    outs = run(q, k, v, do, True, 0.125)
    res = compare(q, k, v, do, True, 0.125, outs, ref_device="cpu")
    assert_parity(res, torch.float16, "C2")


def test_c3_fwd_bwd():
    say("case: C3 (4,4096,32,128) bf16 causal fwd+bwd")
    q, k, v, do = (t.to(DEV) for t in make_inputs(4, 4096, 32, 128, torch.bfloat16))
    scale = 128 ** -0.5
    outs = run(q, k, v, do, True, scale)
    res = compare(q, k, v, do, True, scale, outs, hpc=8)
    assert_parity(res, torch.bfloat16, "C3")


def test_c3_size_independent_invariants():
    # sum_j P_ij = 1 => sum_j dV_j = sum_i dO_i ; sum_j dS_ij = 0 => sum_j dK_j = 0
    say("case: C3 invariants")
    q, k, v, do = (t.to(DEV) for t in make_inputs(4, 4096, 32, 128, torch.bfloat16))
    o, lse, dq, dk, dv = run(q, k, v, do, True, 128 ** -0.5)
    s_dv = dv.double().sum(1)
    s_do = do.double().sum(1)
    assert (s_dv - s_do).abs().max().item() <= 2e-2 * s_do.abs().max().item()
    s_dk = dk.double().sum(1)
    assert s_dk.abs().max().item() <= 2e-2 * dk.double().abs().sum(1).max().item()
    assert torch.isfinite(o).all() and torch.isfinite(lse).all() and torch.isfinite(dq).all()


@pytest.mark.parametrize("causal", [True, False])
def test_c4_long_sequence(causal):
    say(f"case: C4 (1,16384,16,128) bf16 causal={causal} q,k~N(0,4)")
    q, k, v, do = (t.to(DEV) for t in make_inputs(1, 16384, 16, 128, torch.bfloat16, qk_scale=2.0))
    scale = 128 ** -0.5
    outs = run(q, k, v, do, causal, scale)
    res = compare(q, k, v, do, causal, scale, outs, hpc=1)
    assert_parity(res, torch.bfloat16, f"C4 causal={causal}")


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_c5_edge_sweep(D, dt):
    say(f"case: C5 (8,1000,16,{D}) {dt} causal dropout 0.1 seed 42 offset 0")
    B, S, H, p = 8, 1000, 16, 0.1
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dt))
    scale = D ** -0.5
    keep_dev = _lib.dropout_mask(42, 0, B, H, S, S, p).bool()
    keep = torch.from_numpy(c_keep_mask(42, 0, B, H, S, S, p)).bool().to(DEV)
    assert torch.equal(keep_dev, keep)
    outs = run(q, k, v, do, True, scale, p, seed=42, offset=0)
    res = compare(q, k, v, do, True, scale, outs, keep=keep, p=p, hpc=8)
    assert_parity(res, dt, f"C5 D={D}")


def test_deterministic():
    say("case: determinism (2,1024,8,128) bf16 causal, two runs")
    q, k, v, do = (t.to(DEV) for t in make_inputs(2, 1024, 8, 128, torch.bfloat16, seed=3))
    a = run(q, k, v, do, True, 128 ** -0.5)
    b = run(q, k, v, do, True, 128 ** -0.5)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_strided_inputs_match_contiguous():
    say("case: (B,H,S,D)-major storage viewed as (B,S,H,D)")
    q, k, v, do = (t.to(DEV) for t in make_inputs(2, 256, 4, 64, torch.bfloat16, seed=5))
    qs, ks, vs, dos = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v, do))
    assert qs.stride() != q.stride()
    a = run(q, k, v, do, True, 0.125)
    b = run(qs, ks, vs, dos, True, 0.125)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_slices_spanning_more_than_2_gib():
    # q, k, v, dO are one-head views into a (1, 16384, 1024, 128) bf16 buffer:
    # each (b, h) slice spans 4 GiB, beyond a 32-bit buffer range, while the
    # work stays that of one head.  The outputs must equal those of contiguous
    # copies bit for bit (same kernels, same values).
    S, HB, D = 16384, 1024, 128
    say(f"case: one head of a (1, {S}, {HB}, {D}) bf16 buffer, causal fwd+bwd")
    buf = torch.empty(1, S, HB, D, device=DEV, dtype=torch.bfloat16)
    src = make_inputs(1, S, 1, D, torch.bfloat16, seed=6)
    for i, t in enumerate(src):
        buf[:, :, i:i + 1] = t.to(DEV)
    views = [buf[:, :, i:i + 1] for i in range(4)]
    assert views[0].stride(1) * (S - 1) * 2 >= 2 ** 31
    a = run(*views, True, D ** -0.5)
    b = run(*(t.to(DEV) for t in src), True, D ** -0.5)
    for name, x, y in zip(("O", "LSE", "dQ", "dK", "dV"), a, b):
        assert torch.equal(x, y), name
    del buf, views


def test_empty_keys():
    say("case: Sk = 0")
    q = torch.randn(1, 5, 2, 64, device=DEV, dtype=torch.float16)
    k = torch.empty(1, 0, 2, 64, device=DEV, dtype=torch.float16)
    o, lse, _ = _lib.fwd(q, k, k, False, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(o, torch.zeros_like(o)) and bool((lse == float("-inf")).all())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_bwd_stage3_equals_prepass_then_dq(dt, D):
    # include/fa_abi.h: stage 3 writes the workspace rows and dQ in one pass
    # (16-bit: the dQ kernel computes delta itself, summing as the pre-pass
    # does); its rows and dQ equal stage 0 then stage 2 bit for bit, including
    # the padding rows past Sq and rows whose LSE is -inf
    import ctypes
    say(f"case: stage 3 vs stages 0 + 2, {dt} D={D}")
    B, S, H = 2, 300, 4
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dt, Hkv=2, seed=37))
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
        outs.append((ws[:rows].clone(), dq.clone()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("case", [
    # dtype, B, S, H, Hkv, D, causal: small grids (fewer dK/dV and dQ workgroups
    # than CUs each); the first three run as the delta pre-pass plus one launch
    # of both kinds of workgroups (causal, or both kinds fit the CUs at once)
    (torch.float16, 2, 1024, 12, 12, 64, True),    # C2
    (torch.bfloat16, 2, 777, 8, 8, 128, False),    # 112 + 112 workgroups
    (torch.bfloat16, 1, 1000, 8, 2, 64, True),     # GQA 4:1, ragged tiles
    (torch.float16, 2, 1024, 12, 12, 64, False),   # 384 workgroups, non-causal: two passes
])
def test_small_grid_bwd_equals_the_two_passes(case):
    # fa_bwd on a small grid equals stage 3 (dQ with the delta rows) followed by
    # stage 1 (dK/dV) bit for bit, whichever way it schedules the two passes
    import ctypes
    dt, B, S, H, Hkv, D, causal = case
    say(f"case: small-grid fa_bwd vs stages 3 + 1, {case}")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dt, Hkv=Hkv, seed=41))
    scale = D ** -0.5
    o, lse, _ = _lib.fwd(q, k, v, causal, scale)
    ref = _lib.bwd(q, k, v, o, do, lse, causal, scale)
    lib = _lib.load()
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    a = _lib.bwd_args(q, k, v, o, do, lse, dq, dk, dv, causal, scale, 0.0, 0, 0)
    ws = torch.empty(lib.fa_bwd_workspace_size(ctypes.byref(a)), device=DEV, dtype=torch.uint8)
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for st in (3, 1):
        assert lib.fa_bwd_stage(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(), st, sp) == 0
    torch.cuda.synchronize()
    assert torch.equal(dq, ref[0]) and torch.equal(dk, ref[1]) and torch.equal(dv, ref[2])
    res = compare(q, k, v, do, causal, scale, (o, lse) + tuple(ref), hpc=8)
    assert_parity(res, dt, str(case))


@pytest.mark.parametrize("with_bias", [False, True])
def test_bwd_stages_on_two_streams(with_bias):
    # include/fa_abi.h: after stage 0, stages 1 (dK/dV) and 2 (dQ) are
    # independent and may run on two streams when no bias gradient is asked
    # for (a bias alone included); with one, stage 1 writes the dS that stage 2
    # reads, so stage 2 follows stage 1.  Results equal fa_bwd's bit for bit.
    import ctypes
    say(f"case: fa_bwd_stage on two streams, bias={with_bias}")
    B, S, H, D = 2, 333, 4, 64
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.bfloat16, Hkv=2, seed=31))
    pb = None
    if with_bias:
        bias = torch.randn(1, H, S, S, device=DEV).to(torch.bfloat16)
        pb = _lib.prepare_bias(bias, B, H, S, S, torch.bfloat16)
    o, lse, _ = _lib.fwd(q, k, v, True, D ** -0.5, bias=pb)
    lib = _lib.load()
    for want_db in ((False, True) if with_bias else (False,)):
        ref = _lib.bwd(q, k, v, o, do, lse, True, D ** -0.5, bias=pb, want_dbias=want_db)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        # the gradient in the bias dtype, as _lib.bwd makes it (a float32 one
        # sums float32 parts, a bf16 one bf16 parts: not the same bits)
        db = torch.empty(1, H, S, 336, device=DEV, dtype=torch.bfloat16)[..., :S] if want_db else None
        a = _lib.bwd_args(q, k, v, o, do, lse, dq, dk, dv, True, D ** -0.5, 0.0, 0, 0, pb, db)
        ws = torch.empty(lib.fa_bwd_workspace_size(ctypes.byref(a)), device=DEV, dtype=torch.uint8)
        wsp = ctypes.c_void_p(ws.data_ptr())
        s0, s1, s2 = torch.cuda.current_stream(), torch.cuda.Stream(), torch.cuda.Stream()
        assert lib.fa_bwd_stage(ctypes.byref(a), wsp, ws.numel(), 0, ctypes.c_void_p(s0.cuda_stream)) == 0
        s1.wait_stream(s0)
        s2.wait_stream(s0)
        assert lib.fa_bwd_stage(ctypes.byref(a), wsp, ws.numel(), 1, ctypes.c_void_p(s1.cuda_stream)) == 0
        if want_db:
            s2.wait_stream(s1)  # dQ reads the dS stage 1 wrote
        assert lib.fa_bwd_stage(ctypes.byref(a), wsp, ws.numel(), 2, ctypes.c_void_p(s2.cuda_stream)) == 0
        s0.wait_stream(s1)
        s0.wait_stream(s2)
        torch.cuda.synchronize()
        assert torch.equal(dq, ref[0]) and torch.equal(dk, ref[1]) and torch.equal(dv, ref[2])
        if want_db:
            assert torch.equal(db, ref[3])
