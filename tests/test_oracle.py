"""Pins for the CPU oracle (no GPU).

Each oracle function is checked against something that does not share its
code: published known-answer vectors (Random123), Triton's own tl.rand
outputs (committed fixture), scalar brute force, torch's SDPA, closed forms and
invariants.  The last tests plant mistakes in the oracle and show the pins
catch them.
"""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import philox
from helpers import c_keep_mask, c_rand, oracle_clib

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _kat():
    with open(os.path.join(GOLDEN, "random123_philox4x32_10_kat.json")) as f:
        return json.load(f)["cases"]


def _triton():
    with open(os.path.join(GOLDEN, "triton_rand_vectors.json")) as f:
        return json.load(f)["cases"]


# ----------------------------------------------------------------------------- Philox

@pytest.mark.parametrize("case", _kat())
def test_philox_numpy_random123_kat(case):
    c = [np.uint32(int(x, 16)) for x in case["ctr"]]
    k = [np.uint32(int(x, 16)) for x in case["key"]]
    out = philox.philox4x32_10(*c, *k)
    assert [f"{int(x):08x}" for x in out] == case["out"]


@pytest.mark.parametrize("case", _kat())
def test_philox_c_random123_kat(case):
    ctr = np.array([int(x, 16) for x in case["ctr"]], dtype=np.uint32)
    key = np.array([int(x, 16) for x in case["key"]], dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    oracle_clib().oracle_philox4x32_10(ctr.ctypes.data, key.ctypes.data, out.ctypes.data)
    assert [f"{int(x):08x}" for x in out] == case["out"]


@pytest.mark.parametrize("case", _triton(), ids=lambda c: f"seed{c['seed']}")
def test_rand_matches_triton_interpreter(case):
    ctr = np.array(case["counters"], dtype=np.uint64)
    u_np = philox.rand(case["seed"], ctr)
    u_c = c_rand(case["seed"], ctr)
    want = np.array(case["uniform_f32_bits"], dtype=np.uint32)
    assert np.array_equal(u_np.view(np.uint32), want)
    assert np.array_equal(u_c.view(np.uint32), want)
    x, _, _, _ = philox.philox4x32_10((ctr & np.uint64(0xFFFFFFFF)).astype(np.uint32),
                                      (ctr >> np.uint64(32)).astype(np.uint32), 0, 0,
                                      np.uint32(case["seed"] & 0xFFFFFFFF), np.uint32(case["seed"] >> 32))
    assert np.array_equal(x, np.array(case["randint_u32"], dtype=np.uint32))


def test_uniform_mapping_edges():
    # x = 0 -> 0; int32 max -> just below 1; int32 min folds to int32 max
    u = philox.uint_to_uniform(np.array([0, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF], dtype=np.uint32))
    assert u[0] == 0.0
    assert u[1] < 1.0 and u[1] == u[2]
    assert u[3] == 0.0  # -1 folds to 0


@pytest.mark.parametrize("offset", [0, 12345, 2**32 - 5, 2**64 - 3])
def test_dropout_mask_numpy_equals_c(offset):
    B, H, Sq, Sk, p = 2, 3, 17, 23, 0.1
    a = philox.dropout_keep_mask(42, offset, B, H, Sq, Sk, p)
    b = c_keep_mask(42, offset, B, H, Sq, Sk, p).astype(bool)
    assert np.array_equal(a, b)


def test_dropout_counter_layout():
    # element (b, h, i, j) uses counter offset + ((b*H + h)*Sq + i)*Sk + j
    B, H, Sq, Sk = 2, 3, 5, 7
    c = philox.dropout_counters(100, B, H, Sq, Sk)
    b, h, i, j = 1, 2, 3, 4
    assert int(c[b, h, i, j]) == 100 + ((b * H + h) * Sq + i) * Sk + j
    # rows differ (the reference's counter dropped i, so all rows shared a mask)
    keep = philox.dropout_keep_mask(7, 0, 1, 1, 64, 64, 0.5)
    assert not all(np.array_equal(keep[0, 0, 0], keep[0, 0, r]) for r in range(1, 64))


def test_dropout_keep_rate():
    keep = philox.dropout_keep_mask(42, 0, 1, 4, 128, 128, 0.1)
    rate = keep.mean()
    assert abs(rate - 0.9) < 0.01


# ----------------------------------------------------------------------------- forward

def _rand(shape, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64).to(dtype)


SMALL = [
    # B, Sq, Sk, H, Hkv, D, causal
    (1, 5, 5, 2, 2, 4, False),
    (2, 6, 6, 2, 1, 8, True),
    (1, 7, 4, 3, 3, 4, True),   # Sq > Sk, top-left causal
    (1, 3, 9, 2, 2, 4, True),   # Sq < Sk
    (1, 4, 1, 1, 1, 4, False),  # Sk = 1
]


@pytest.mark.parametrize("B,Sq,Sk,H,Hkv,D,causal", SMALL)
def test_forward_vs_brute_force(B, Sq, Sk, H, Hkv, D, causal):
    q = _rand((B, Sq, H, D), 1)
    k = _rand((B, Sk, Hkv, D), 2)
    v = _rand((B, Sk, Hkv, D), 3)
    o, lse = oa.attention_forward(q, k, v, causal, 0.37)
    ob, lb = oa.brute_force_forward(q, k, v, causal, 0.37)
    assert torch.allclose(o, ob, atol=1e-12, rtol=0)
    assert torch.allclose(lse, lb, atol=1e-12, rtol=0)


def test_forward_dropout_vs_brute_force():
    B, S, H, D, p = 1, 6, 2, 4, 0.3
    q, k, v = _rand((B, S, H, D), 4), _rand((B, S, H, D), 5), _rand((B, S, H, D), 6)
    keep = torch.from_numpy(philox.dropout_keep_mask(9, 3, B, H, S, S, p))
    o, _ = oa.attention_forward(q, k, v, True, None, keep, p)
    ob, _ = oa.brute_force_forward(q, k, v, True, None, keep.tolist(), p)
    assert torch.allclose(o, ob, atol=1e-12, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
def test_forward_vs_sdpa(causal):
    q, k, v = _rand((2, 33, 3, 16), 7), _rand((2, 33, 3, 16), 8), _rand((2, 33, 3, 16), 9)
    o, _ = oa.attention_forward(q, k, v, causal, 0.25)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                         is_causal=causal, scale=0.25).transpose(1, 2)
    assert torch.allclose(o, ref, atol=1e-12, rtol=0)


def test_default_scale_is_rsqrt_d():
    q, k, v = _rand((1, 4, 1, 16), 1), _rand((1, 4, 1, 16), 2), _rand((1, 4, 1, 16), 3)
    a, _ = oa.attention_forward(q, k, v)
    b, _ = oa.attention_forward(q, k, v, scale=0.25)
    assert torch.equal(a, b)


def test_closed_forms():
    B, S, H, D = 1, 8, 2, 4
    v = _rand((B, S, H, D), 11)
    k = _rand((B, S, H, D), 12)
    zero_q = torch.zeros(B, S, H, D, dtype=torch.float64)
    # q = 0: non-causal -> mean of V; causal -> prefix means
    o, lse = oa.attention_forward(zero_q, k, v, False)
    assert torch.allclose(o, v.mean(1, keepdim=True).expand_as(o), atol=1e-14)
    assert torch.allclose(lse, torch.full_like(lse, math.log(S)), atol=1e-14)
    oc, lsec = oa.attention_forward(zero_q, k, v, True)
    prefix = torch.cumsum(v, 1) / torch.arange(1, S + 1, dtype=torch.float64).view(1, S, 1, 1)
    assert torch.allclose(oc, prefix, atol=1e-14)
    assert torch.allclose(lsec[0, 0], torch.log(torch.arange(1, S + 1, dtype=torch.float64)), atol=1e-14)
    # causal row 0 attends only to key 0
    q = _rand((B, S, H, D), 13)
    oc, _ = oa.attention_forward(q, k, v, True)
    assert torch.allclose(oc[:, 0], v[:, 0], atol=1e-14)
    # Sk = 1 -> O = V
    o1, _ = oa.attention_forward(q, k[:, :1], v[:, :1], False)
    assert torch.allclose(o1, v[:, :1].expand_as(o1), atol=1e-14)


def test_key_permutation_invariance():
    q, k, v = _rand((1, 9, 2, 8), 21), _rand((1, 9, 2, 8), 22), _rand((1, 9, 2, 8), 23)
    perm = torch.randperm(9, generator=torch.Generator().manual_seed(0))
    o1, l1 = oa.attention_forward(q, k, v, False)
    o2, l2 = oa.attention_forward(q, k[:, perm], v[:, perm], False)
    assert torch.allclose(o1, o2, atol=1e-13) and torch.allclose(l1, l2, atol=1e-13)


def test_gqa_equals_repeated_heads():
    q, k, v = _rand((1, 6, 4, 8), 31), _rand((1, 6, 2, 8), 32), _rand((1, 6, 2, 8), 33)
    o1, _ = oa.attention_forward(q, k, v, True)
    o2, _ = oa.attention_forward(q, k.repeat_interleave(2, 2), v.repeat_interleave(2, 2), True)
    assert torch.equal(o1, o2)


def test_empty_keys_give_zero_and_neg_inf():
    q = _rand((1, 3, 1, 4), 1)
    k = torch.zeros(1, 0, 1, 4, dtype=torch.float64)
    o, lse = oa.attention_forward(q, k, k, False)
    assert torch.equal(o, torch.zeros_like(o)) and torch.isinf(lse).all() and (lse < 0).all()


# ----------------------------------------------------------------------------- backward

@pytest.mark.parametrize("B,Sq,Sk,H,Hkv,D,causal", SMALL)
def test_backward_formulas_vs_autograd(B, Sq, Sk, H, Hkv, D, causal):
    q = _rand((B, Sq, H, D), 41)
    k = _rand((B, Sk, Hkv, D), 42)
    v = _rand((B, Sk, Hkv, D), 43)
    do = _rand((B, Sq, H, D), 44)
    o, lse, dq, dk, dv = oa.attention_autograd(q, k, v, do, causal, 0.4)
    dq2, dk2, dv2 = oa.attention_backward(q, k, v, o, do, lse, causal, 0.4)
    for a, b in ((dq, dq2), (dk, dk2), (dv, dv2)):
        assert torch.allclose(a, b, atol=1e-12, rtol=0)


def test_backward_dropout_formulas_vs_autograd():
    B, S, H, D, p = 1, 7, 2, 4, 0.25
    q, k, v, do = (_rand((B, S, H, D), s) for s in (51, 52, 53, 54))
    keep = torch.from_numpy(philox.dropout_keep_mask(5, 0, B, H, S, S, p))
    o, lse, dq, dk, dv = oa.attention_autograd(q, k, v, do, True, None, keep, p)
    dq2, dk2, dv2 = oa.attention_backward(q, k, v, o, do, lse, True, None, keep, p)
    for a, b in ((dq, dq2), (dk, dk2), (dv, dv2)):
        assert torch.allclose(a, b, atol=1e-12, rtol=0)


def test_gradcheck_tiny():
    q, k, v = (_rand((1, 4, 1, 3), s).requires_grad_(True) for s in (61, 62, 63))
    f = lambda a, b, c: oa.attention_forward(a, b, c, True, 0.7)[0]  # noqa: E731
    assert torch.autograd.gradcheck(f, (q, k, v))


def test_backward_invariants():
    # sum_j dS_ij = 0  =>  sum over keys of dK = 0;  sum_j P_ij = 1  =>  sum_j dV_j = sum_i dO_i
    B, S, H, D = 2, 12, 2, 8
    q, k, v, do = (_rand((B, S, H, D), s) for s in (71, 72, 73, 74))
    for causal in (False, True):
        o, lse, dq, dk, dv = oa.attention_autograd(q, k, v, do, causal)
        assert torch.allclose(dk.sum(1), torch.zeros_like(dk.sum(1)), atol=1e-12)
        assert torch.allclose(dv.sum(1), do.sum(1), atol=1e-12)


# ----------------------------------------------------------------------------- additive bias

# (B|1, H|1, Sq|1) with B = 2, H = 3; None = the full query dimension
BIAS_SHAPES = [(2, 3, None), (1, 3, None), (2, 1, None), (1, 1, None), (2, 1, 1)]


def _bias_shape(bshape, Sq, Sk):
    b, h, s = bshape
    return (b, h, Sq if s is None else s, Sk)


@pytest.mark.parametrize("bshape", BIAS_SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_bias_forward_vs_brute_force(bshape, causal):
    B, Sq, Sk, H, Hkv, D = 2, 6, 5, 3, 3, 4
    q, k, v = _rand((B, Sq, H, D), 111), _rand((B, Sk, Hkv, D), 112), _rand((B, Sk, Hkv, D), 113)
    bias = _rand(_bias_shape(bshape, Sq, Sk), 114)
    o, lse = oa.attention_forward(q, k, v, causal, 0.6, bias=bias)
    ob, lb = oa.brute_force_forward(q, k, v, causal, 0.6, bias=bias)
    assert torch.allclose(o, ob, atol=1e-12, rtol=0) and torch.allclose(lse, lb, atol=1e-12, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
def test_bias_forward_vs_sdpa_float_mask(causal):
    # SDPA adds a float attn_mask to the scaled scores: the same operation
    B, S, H, D = 2, 17, 3, 8
    q, k, v = _rand((B, S, H, D), 121), _rand((B, S, H, D), 122), _rand((B, S, H, D), 123)
    bias = _rand((1, H, S, S), 124)
    mask = bias.expand(B, H, S, S).clone()
    if causal:
        mask = mask.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    o, _ = oa.attention_forward(q, k, v, causal, 0.3, bias=bias)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                         attn_mask=mask, scale=0.3).transpose(1, 2)
    assert torch.allclose(o, ref, atol=1e-12, rtol=0)


def test_bias_closed_forms():
    B, S, H, D = 1, 9, 2, 4
    q, k, v = _rand((B, S, H, D), 131), _rand((B, S, H, D), 132), _rand((B, S, H, D), 133)
    o0, l0 = oa.attention_forward(q, k, v, False)
    # a bias constant along the keys shifts LSE and leaves O unchanged
    row = _rand((1, H, S, 1), 134)
    o1, l1 = oa.attention_forward(q, k, v, False, bias=row.expand(1, H, S, S))
    assert torch.allclose(o1, o0, atol=1e-13) and torch.allclose(l1, l0 + row[..., 0], atol=1e-13)
    # a -inf bias on key j is the same as removing key j
    bias = torch.zeros(1, 1, S, S, dtype=torch.float64)
    bias[..., 3] = float("-inf")
    keep = [j for j in range(S) if j != 3]
    o2, l2 = oa.attention_forward(q, k, v, False, bias=bias)
    o3, l3 = oa.attention_forward(q, k[:, keep], v[:, keep], False)
    assert torch.allclose(o2, o3, atol=1e-13) and torch.allclose(l2, l3, atol=1e-13)


@pytest.mark.parametrize("causal", [False, True])
def test_bias_row_without_visible_key(causal):
    # a query row whose bias is -inf on every key: O = 0, LSE = -inf and zero
    # gradients (FlashAttention-2's convention), the other rows unchanged
    B, S, H, D = 1, 7, 2, 4
    q, k, v, do = (_rand((B, S, H, D), s) for s in (171, 172, 173, 174))
    bias = _rand((1, H, S, S), 175)
    bias[0, 1, 4, :] = float("-inf")
    o, lse, dq, dk, dv, db = oa.attention_autograd(q, k, v, do, causal, 0.5, bias=bias)
    ob, lb = oa.brute_force_forward(q, k, v, causal, 0.5, bias=bias)
    assert torch.equal(o[0, 4, 1], torch.zeros(D, dtype=torch.float64)) and torch.isneginf(lse[0, 1, 4])
    assert torch.allclose(o, ob, atol=1e-12, rtol=0) and torch.equal(torch.isneginf(lb), torch.isneginf(lse))
    fin = ~torch.isneginf(lse)
    assert torch.allclose(lse[fin], lb[fin], atol=1e-12, rtol=0)
    for t in (dq, dk, dv, db):
        assert torch.isfinite(t).all()
    assert torch.equal(dq[0, 4, 1], torch.zeros(D, dtype=torch.float64))
    assert torch.equal(db[0, 1, 4], torch.zeros(S, dtype=torch.float64))
    dq2, dk2, dv2, db2 = oa.attention_backward(q, k, v, o, do, lse, causal, 0.5, bias=bias)
    for a, b in ((dq, dq2), (dk, dk2), (dv, dv2), (db, db2)):
        assert torch.allclose(a, b, atol=1e-12, rtol=0)
    # the remaining rows equal attention with the dead row's query removed
    # from the problem (rows are independent): compare against head 0, which
    # has no dead row, run alone
    o0, l0 = oa.attention_forward(q[:, :, :1], k[:, :, :1], v[:, :, :1], causal, 0.5, bias=bias[:, :1])
    assert torch.allclose(o[:, :, :1], o0, atol=1e-13) and torch.allclose(lse[:, :1], l0, atol=1e-13)


@pytest.mark.parametrize("bshape", BIAS_SHAPES)
def test_bias_backward_formulas_vs_autograd(bshape):
    B, Sq, Sk, H, Hkv, D = 2, 7, 6, 3, 3, 4
    q, k, v = _rand((B, Sq, H, D), 141), _rand((B, Sk, Hkv, D), 142), _rand((B, Sk, Hkv, D), 143)
    do = _rand((B, Sq, H, D), 144)
    bias = _rand(_bias_shape(bshape, Sq, Sk), 145)
    o, lse, dq, dk, dv, db = oa.attention_autograd(q, k, v, do, True, 0.5, bias=bias)
    dq2, dk2, dv2, db2 = oa.attention_backward(q, k, v, o, do, lse, True, 0.5, bias=bias)
    assert db.shape == bias.shape
    for a, b in ((dq, dq2), (dk, dk2), (dv, dv2), (db, db2)):
        assert torch.allclose(a, b, atol=1e-12, rtol=0)


def test_bias_gradient_invariants():
    # dBias = dS: its rows sum to zero (sum_j P_ij (dP_ij - delta_i) = 0), it is
    # zero where the causal mask removes a key, and a broadcast bias gets the
    # sum of the full-shape gradient over the broadcast dimensions
    B, S, H, D = 2, 8, 3, 4
    q, k, v, do = (_rand((B, S, H, D), s) for s in (151, 152, 153, 154))
    full = _rand((B, H, S, S), 155)
    *_, dfull = oa.attention_autograd(q, k, v, do, True, bias=full)
    assert torch.allclose(dfull.sum(-1), torch.zeros_like(dfull.sum(-1)), atol=1e-12)
    assert torch.equal(dfull.masked_select(torch.triu(torch.ones(S, S, dtype=torch.bool), 1).expand_as(dfull)),
                       torch.zeros(B * H * S * (S - 1) // 2, dtype=torch.float64))
    shared = full[:1, :1]
    *_, dshared = oa.attention_autograd(q, k, v, do, True, bias=shared)
    *_, dexp = oa.attention_autograd(q, k, v, do, True, bias=shared.expand(B, H, S, S).contiguous())
    assert torch.allclose(dshared, dexp.sum((0, 1), keepdim=True), atol=1e-12)


def test_planted_mistake_scaled_bias_is_caught(monkeypatch):
    # bias added before the scale (scale * (qk + bias)) instead of after it
    q, k, v = _rand((1, 5, 2, 4), 161), _rand((1, 5, 2, 4), 162), _rand((1, 5, 2, 4), 163)
    bias = _rand((1, 2, 5, 5), 164)
    ob, _ = oa.brute_force_forward(q, k, v, False, 0.5, bias=bias)
    orig = oa._scores
    monkeypatch.setattr(oa, "_scores", lambda q_, k_, c, s, d, b=None: orig(q_, k_, c, s, d, None if b is None else b * s))
    o, _ = oa.attention_forward(q, k, v, False, 0.5, bias=bias)
    assert not torch.allclose(o, ob, atol=1e-6)


# ----------------------------------------------------------------------------- planted mistakes

def test_planted_mistake_wrong_causal_diagonal_is_caught(monkeypatch):
    q, k, v = _rand((1, 5, 1, 4), 81), _rand((1, 5, 1, 4), 82), _rand((1, 5, 1, 4), 83)
    ob, _ = oa.brute_force_forward(q, k, v, True)
    monkeypatch.setattr(oa, "_causal_mask",
                        lambda sq, sk, device=None: torch.triu(torch.ones(sq, sk, dtype=torch.bool), diagonal=0))
    o, _ = oa.attention_forward(q, k, v, True)
    assert not torch.allclose(o, ob, atol=1e-6)


def test_planted_mistake_dropped_scale_is_caught(monkeypatch):
    q, k, v = _rand((1, 5, 1, 4), 91), _rand((1, 5, 1, 4), 92), _rand((1, 5, 1, 4), 93)
    ob, lb = oa.brute_force_forward(q, k, v, False, 0.5)
    orig = oa._scores
    monkeypatch.setattr(oa, "_scores", lambda q_, k_, c, s, d, b=None: orig(q_, k_, c, 1.0, d, b))
    o, lse = oa.attention_forward(q, k, v, False, 0.5)
    assert not torch.allclose(lse, lb, atol=1e-6)


def test_planted_mistake_transposed_operand_is_caught(monkeypatch):
    B, S, H, D = 1, 6, 1, 6
    q, k, v, do = (_rand((B, S, H, D), s) for s in (101, 102, 103, 104))
    o, lse, dq, dk, dv = oa.attention_autograd(q, k, v, do, False)
    orig_matmul = torch.matmul

    def bad_matmul(a, b):  # transposes the second operand of square products
        if a.shape[-1] == b.shape[-2] == b.shape[-1]:
            b = b.transpose(-2, -1)
        return orig_matmul(a, b)

    monkeypatch.setattr(torch, "matmul", bad_matmul)
    dq2, dk2, dv2 = oa.attention_backward(q, k, v, o, do, lse, False)
    monkeypatch.setattr(torch, "matmul", orig_matmul)
    assert not (torch.allclose(dq, dq2, atol=1e-6) and torch.allclose(dk, dk2, atol=1e-6)
                and torch.allclose(dv, dv2, atol=1e-6))


def test_planted_mistake_dropout_counter_without_row_is_caught(monkeypatch):
    # the reference's defect: counter without the row index -> every row of a
    # tile shares one mask; the committed layout test must reject it
    def bad_counters(offset, B, H, Sq, Sk):
        j = np.arange(Sk, dtype=np.uint64)
        return np.broadcast_to(j + np.uint64(offset), (B, H, Sq, Sk)).copy()

    monkeypatch.setattr(philox, "dropout_counters", bad_counters)
    keep = philox.dropout_keep_mask(7, 0, 1, 1, 64, 64, 0.5)
    assert all(np.array_equal(keep[0, 0, 0], keep[0, 0, r]) for r in range(1, 64))
    assert not np.array_equal(keep, c_keep_mask(7, 0, 1, 1, 64, 64, 0.5).astype(bool))
