"""Additive attention bias on the gfx950 kernels (through the C ABI and the
autograd wrapper) against the float64 oracle: O, LSE, dQ, dK, dV and dBias.

The bias is added to the scaled scores before the causal mask (reference
kernels/forward_kernel.py:166-182); dBias = dS summed over the broadcast
dimensions (the reference returned zeros, ops/attention.py:297-301).
Tolerance as for the other parity tests: fp16/bf16 within 2x the error of the
reference math run in the inputs' dtype (bias included) against the oracle;
fp32 within 1e-5 of max|oracle|.
"""
import pytest
import torch

import flash_attention_v100 as fa
from flash_attention_v100 import _lib
from helpers import assert_parity, c_keep_mask, lowp_math, make_inputs, maxabs, reduce_kv
from oracle import attention as oa

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("O", "LSE", "dQ", "dK", "dV", "dBias")


def say(msg):
    print(msg, flush=True)


def make_bias(shape, dtype, seed=7, mag=2.0):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * mag).to(dtype)


def run_kernels(q, k, v, do, causal, scale, bias, p=0.0, seed=0, offset=0):
    dev = [t.to(DEV) for t in (q, k, v, do)]
    b = bias.to(DEV)
    o, lse, _ = _lib.fwd(dev[0], dev[1], dev[2], causal, scale, p, seed, offset, bias=b)
    dq, dk, dv, db = _lib.bwd(dev[0], dev[1], dev[2], o, dev[3], lse, causal, scale, p, seed, offset,
                              bias=b, want_dbias=True)
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv, db


def check(q, k, v, do, causal, scale, bias, outs, keep=None, p=0.0, label="", names=NAMES):
    """Whole-problem comparison (small shapes): float64 oracle on the CPU, the
    envelope (lowp math in the inputs' dtype) on the GPU; ``outs`` holds the
    kernel outputs named by ``names`` (a prefix of NAMES)."""
    o, lse = oa.attention_forward(q, k, v, causal, scale, keep, p, torch.float64, bias=bias)
    refs = [o, lse] + list(oa.attention_backward(q, k, v, o, do, lse, causal, scale, keep, p, bias=bias))
    res = {}
    env = None
    if q.dtype != torch.float32:
        dev = [t.to(DEV) for t in (q, k, v, do)]
        env = list(lowp_math(*dev, causal, scale, keep.to(DEV) if keep is not None else None, p,
                             bias=bias.to(DEV)))
        env[3] = reduce_kv(env[3], k.shape[2])
        env[4] = reduce_kv(env[4], k.shape[2])
    for i, n in enumerate(names):
        rf = refs[i]
        ek = maxabs(outs[i].cpu(), rf)
        ee = maxabs(env[i].cpu(), rf) if env is not None else None
        res[n] = [ek, ee, rf.abs().max().item()]
    assert_parity(res, q.dtype, label)
    return res


CASES = []
for dt in (torch.float16, torch.bfloat16, torch.float32):
    for D in (32, 64, 128):
        for causal in (False, True):
            CASES.append((dt, 2, 200, 200, 3, 3, D, causal, (2, 3, 200, 200), None))
CASES += [
    # broadcast shapes of the reference's (B|1, H|1, Sq, Sk), plus a key-padding row
    (torch.bfloat16, 2, 160, 160, 4, 4, 64, True, (1, 4, 160, 160), None),
    (torch.bfloat16, 2, 160, 160, 4, 4, 64, False, (2, 1, 160, 160), None),
    (torch.float16, 2, 160, 160, 4, 4, 128, True, (1, 1, 160, 160), None),
    (torch.float16, 2, 160, 160, 4, 4, 64, False, (2, 1, 1, 160), None),
    # float32 bias with 16-bit inputs
    (torch.bfloat16, 1, 150, 150, 4, 4, 128, True, (1, 4, 150, 150), torch.float32),
    (torch.float16, 2, 100, 100, 2, 2, 64, False, (2, 2, 100, 100), torch.float32),
    # ragged and unaligned rows (Sk * 2 bytes not a multiple of 16: padded copy), Sq != Sk
    (torch.bfloat16, 1, 130, 77, 2, 2, 64, True, (1, 2, 130, 77), None),
    (torch.float16, 1, 77, 261, 2, 2, 128, False, (1, 1, 77, 261), None),
    (torch.float32, 1, 99, 13, 2, 2, 32, True, (1, 2, 99, 13), None),
    # grouped KV heads
    (torch.bfloat16, 2, 160, 160, 4, 2, 128, True, (2, 4, 160, 160), None),
    (torch.float16, 1, 96, 96, 8, 1, 64, False, (1, 8, 96, 96), None),
    # gradients summed by the library over batch and/or heads, ragged keys (Sk % 4 != 0)
    (torch.bfloat16, 2, 99, 150, 2, 2, 64, True, (1, 1, 99, 150), None),
    (torch.float16, 3, 70, 70, 4, 2, 128, True, (1, 4, 70, 70), None),
    (torch.float32, 2, 64, 93, 3, 3, 32, False, (2, 1, 64, 93), None),
    (torch.bfloat16, 2, 130, 131, 4, 1, 64, True, (2, 1, 1, 131), torch.float32),
    # single query / key
    (torch.bfloat16, 1, 1, 1, 2, 2, 64, True, (1, 2, 1, 1), None),
    (torch.float16, 3, 1, 50, 2, 2, 32, False, (3, 2, 1, 50), None),
]


def _id(c):
    dt, B, Sq, Sk, H, Hkv, D, causal, bshape, bdt = c
    tag = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}
    return (f"{tag[dt]}-B{B}-Sq{Sq}-Sk{Sk}-H{H}-Hkv{Hkv}-D{D}-{'causal' if causal else 'full'}"
            f"-bias{'x'.join(map(str, bshape))}{'-' + tag[bdt] if bdt else ''}")


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_bias_fwd_bwd(case):
    dt, B, Sq, Sk, H, Hkv, D, causal, bshape, bdt = case
    say(f"case: bias {_id(case)}")
    q, k, v, do = make_inputs(B, Sq, H, D, dt, Sk=Sk, Hkv=Hkv, seed=11)
    bias = make_bias(bshape, bdt or dt)
    scale = D ** -0.5
    outs = run_kernels(q, k, v, do, causal, scale, bias)
    assert outs[5].shape == bias.shape and outs[5].dtype == bias.dtype
    check(q, k, v, do, causal, scale, bias, outs, label=_id(case))


@pytest.mark.parametrize("causal", [False, True])
def test_bias_with_dropout(causal):
    B, S, H, D, p, seed, offset = 2, 180, 2, 64, 0.1, 1234, 77
    say(f"case: bias + dropout causal={causal}")
    q, k, v, do = make_inputs(B, S, H, D, torch.float32, seed=12)
    bias = make_bias((1, H, S, S), torch.float32)
    keep = torch.from_numpy(c_keep_mask(seed, offset, B, H, S, S, p)).bool()
    outs = run_kernels(q, k, v, do, causal, D ** -0.5, bias, p, seed, offset)
    check(q, k, v, do, causal, D ** -0.5, bias, outs, keep=keep, p=p, label="bias+dropout")


def test_bias_minus_inf_key_padding():
    # -inf entries remove keys (every row keeps some): same as dropping those keys
    B, S, H, D = 2, 200, 2, 64
    say("case: -inf key padding bias")
    q, k, v, do = make_inputs(B, S, H, D, torch.float16, seed=13)
    bias = torch.zeros(B, 1, 1, S, dtype=torch.float16)
    bias[0, ..., 150:] = float("-inf")
    bias[1, ..., 7::3] = float("-inf")
    outs = run_kernels(q, k, v, do, False, D ** -0.5, bias)
    for t in outs[:5]:
        assert torch.isfinite(t).all()
    check(q, k, v, do, False, D ** -0.5, bias, outs, label="-inf padding")
    # batch 0 equals attention over its first 150 keys
    o0, l0, _ = _lib.fwd(q[:1].to(DEV), k[:1, :150].to(DEV), v[:1, :150].to(DEV), False, D ** -0.5)
    assert maxabs(outs[0][:1], o0) < 2e-3 and maxabs(outs[1][:1], l0) < 1e-3


@pytest.mark.parametrize("causal", [False, True])
def test_bias_row_without_visible_key(causal):
    # HF-style 4-D masks with padded query rows: a row whose bias is -inf on
    # every key has O = 0, LSE = -inf, and contributes nothing to the
    # gradients (dK/dV stay finite; its dQ and dBias rows are 0)
    B, S, H, D = 2, 150, 2, 64
    say(f"case: bias row without a visible key causal={causal}")
    q, k, v, do = make_inputs(B, S, H, D, torch.bfloat16, seed=19)
    bias = make_bias((B, H, S, S), torch.bfloat16)
    bias[0, 1, 37, :] = float("-inf")
    bias[1, 0, 149, :] = float("-inf")
    outs = run_kernels(q, k, v, do, causal, D ** -0.5, bias)
    o, lse, dq, dk, dv, db = (t.cpu() for t in outs)
    for t in (o, dq, dk, dv, db):
        assert torch.isfinite(t).all()
    dead = ((0, 1, 37), (1, 0, 149))
    for b, h, i in dead:
        assert torch.isneginf(lse[b, h, i]) and not o[b, i, h].any()
        assert not dq[b, i, h].any() and not db[b, h, i].any()
    # The rest against the oracle: a dead row adds nothing to dK / dV, which is
    # what a row with dO = 0 adds, so the reference problem gives the dead rows
    # a finite bias and dO = 0 (the reference math's softmax would put NaN in
    # them); the dead rows' own O / LSE entries, checked above, take the
    # oracle's values so that they do not enter the comparison.
    bias2, do2 = bias.clone(), do.clone()
    for b, h, i in dead:
        bias2[b, h, i] = 0
        do2[b, i, h] = 0
    ro, rl = oa.attention_forward(q, k, v, causal, D ** -0.5, bias=bias2)
    outs2 = [t.double() for t in (o, lse, dq, dk, dv, db)]
    for b, h, i in dead:
        outs2[0][b, i, h] = ro[b, i, h]
        outs2[1][b, h, i] = rl[b, h, i]
    check(q, k, v, do2, causal, D ** -0.5, bias2, outs2, label="dead row")


def test_float32_bias_keeps_precision_with_bf16_inputs():
    # ALiBi-style bias with magnitudes in the hundreds: rounding it to bf16
    # moves logits by up to 0.5, reading it as float32 does not
    B, S, H, D = 1, 300, 2, 64
    say("case: float32 ALiBi bias, bf16 inputs")
    q, k, v, do = make_inputs(B, S, H, D, torch.bfloat16, seed=14)
    i = torch.arange(S, dtype=torch.float32)
    slopes = torch.tensor([0.5, 0.75]).view(1, H, 1, 1)
    bias = -(slopes * (i.view(S, 1) - i.view(1, S)).abs()) + 100.0
    ref, _ = oa.attention_forward(q, k, v, True, D ** -0.5, bias=bias)
    o32, _, _ = _lib.fwd(q.to(DEV), k.to(DEV), v.to(DEV), True, D ** -0.5, bias=bias.to(DEV))
    o16, _, _ = _lib.fwd(q.to(DEV), k.to(DEV), v.to(DEV), True, D ** -0.5, bias=bias.to(torch.bfloat16).to(DEV))
    e32, e16 = maxabs(o32.cpu(), ref), maxabs(o16.cpu(), ref)
    say(f"err fp32 bias {e32:.3e}  bf16-rounded bias {e16:.3e}")
    assert e32 * 10 < e16


def test_bias_max_vals_and_launchers():
    B, S, H, D = 1, 256, 2, 64
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.bfloat16, seed=15))
    bias = make_bias((1, H, S, S), torch.bfloat16).to(DEV)
    o, lse, mx = fa.flash_attention_forward_triton_enhanced(q, k, v, 0.125, True, bias=bias)
    s = torch.matmul(q.float().transpose(1, 2), k.float().transpose(1, 2).transpose(-2, -1).contiguous()) * 0.125
    s = s + bias.float()
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool, device=DEV), 1), float("-inf"))
    assert torch.allclose(mx, s.amax(-1), atol=1e-3)
    assert torch.allclose(lse, torch.logsumexp(s, -1), atol=1e-3)
    dq, dk, dv, db = fa.flash_attention_backward_triton_enhanced(q, k, v, o, do, lse, mx, 0.125, True,
                                                                 bias=bias, return_dbias=True)
    dq2, dk2, dv2, db2 = _lib.bwd(q, k, v, o, do, lse, True, 0.125, bias=bias, want_dbias=True)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2) and torch.equal(db, db2)


def test_bias_grad_through_interface():
    B, S, H, D = 2, 192, 4, 64
    say("case: bias grad via flash_attention_v100")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.float16, seed=16))
    bias = make_bias((1, H, S, S), torch.float16).to(DEV)
    qq, kk, vv, bb = (t.clone().requires_grad_(True) for t in (q, k, v, bias))
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # no fallback warning: the kernels ran
        o = fa.flash_attention_v100(qq, kk, vv, causal=True, bias=bb)
    o.backward(do)
    o2, lse2, _ = _lib.fwd(q, k, v, True, D ** -0.5, bias=bias)
    dq, dk, dv, db = _lib.bwd(q, k, v, o2, do, lse2, True, D ** -0.5, bias=bias, want_dbias=True)
    assert torch.equal(o, o2) and torch.equal(qq.grad, dq) and torch.equal(kk.grad, dk)
    assert torch.equal(vv.grad, dv) and torch.equal(bb.grad, db)
    # a bias without requires_grad gets no gradient and the same dK/dV; dQ is
    # then recomputed from S and dP instead of read back from the stored dS,
    # which sums the same rounded dS K terms in another order on small grids
    # (the key loop split in two): equal to within two units of the last place
    qq2, kk2 = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    fa.flash_attention_v100(qq2, kk2, v, causal=True, bias=bias).backward(do)
    assert torch.equal(kk2.grad, dk)
    ulp = 2.0 ** -10  # float16
    assert ((qq2.grad.float() - dq.float()).abs() <= 2 * ulp * dq.float().abs() + 1e-6).all()
    outs = (o2.cpu(), lse2.cpu(), dq.cpu(), dk.cpu(), dv.cpu(), db.cpu())
    check(*(t.cpu() for t in (q, k, v, do)), True, D ** -0.5, bias.cpu(), outs, label="interface bias")


def test_bias_deterministic():
    q, k, v, do = (t.to(DEV) for t in make_inputs(1, 333, 4, 128, torch.bfloat16, seed=17))
    bias = make_bias((1, 4, 333, 333), torch.bfloat16).to(DEV)
    a = run_kernels(q, k, v, do, True, 0.1, bias)
    b = run_kernels(q, k, v, do, True, 0.1, bias)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_bias_views():
    # expanded (stride-0) views, a slice of a wider row buffer, and a transposed
    # (non-unit key stride) view all give the result of the materialised bias
    B, S, H, D = 2, 96, 2, 64
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.bfloat16, seed=18))
    base = make_bias((1, 1, S, S), torch.bfloat16).to(DEV)
    wide = torch.zeros(B, H, S, S + 40, device=DEV, dtype=torch.bfloat16)
    wide[..., 8:8 + S] = base
    views = {
        "expanded": base.expand(B, H, S, S),
        "sliced": wide[..., 8:8 + S],
        "transposed": base.expand(B, H, S, S).transpose(-1, -2).contiguous().transpose(-1, -2),
    }
    ref = fa.flash_attention_v100(q, k, v, causal=True, bias=base.expand(B, H, S, S).contiguous())
    for name, bv in views.items():
        say(f"case: bias view {name} strides {bv.stride()}")
        out = fa.flash_attention_v100(q, k, v, causal=True, bias=bv)
        assert torch.equal(out, ref), name
    # gradients through an expanded view land on the (1, 1, S, S) leaf
    leaf = base.clone().requires_grad_(True)
    o = fa.flash_attention_v100(q, k, v, causal=True, bias=leaf.expand(B, H, S, S))
    o.backward(do)
    _, lse, _ = _lib.fwd(q, k, v, True, D ** -0.5, bias=base.expand(B, H, S, S).contiguous())
    *_, db = _lib.bwd(q, k, v, o.detach(), do, lse, True, D ** -0.5,
                      bias=base.expand(B, H, S, S).contiguous(), want_dbias=True)
    assert leaf.grad.shape == (1, 1, S, S)
    assert torch.allclose(leaf.grad.float(), db.float().sum((0, 1), keepdim=True), atol=2e-2, rtol=2e-2)


# The bias gradient through the C ABI into a buffer prefilled with NaN: every
# element must be written, the causal zeros included.  Routes: dS read back by
# the dQ pass (2-byte dS, float32 dS), and the recomputing dQ pass with the
# dK/dV kernel writing the zeros (rows of Sk * 2 bytes not a multiple of 16).
NAN_CASES = [
    (torch.bfloat16, 1, 384, 384, 2, 2, 128, None),
    (torch.float16, 2, 256, 256, 2, 1, 64, torch.float32),
    (torch.float16, 1, 200, 77, 2, 2, 64, None),
    (torch.bfloat16, 1, 130, 304, 2, 2, 32, None),
]


@pytest.mark.parametrize("case", NAN_CASES, ids=[f"{c[0]}-Sq{c[2]}-Sk{c[3]}-D{c[6]}-{c[7]}" for c in NAN_CASES])
def test_dbias_every_element_written(case):
    import ctypes
    dt, B, Sq, Sk, H, Hkv, D, bdt = case
    say(f"case: dbias over NaN {case}")
    q, k, v, do = make_inputs(B, Sq, H, D, dt, Sk=Sk, Hkv=Hkv, seed=21)
    bias = make_bias((B, H, Sq, Sk), bdt or dt)
    scale = D ** -0.5
    dev = [t.to(DEV) for t in (q, k, v, do)]
    o, lse, _ = _lib.fwd(dev[0], dev[1], dev[2], True, scale, bias=bias.to(DEV))
    pb = _lib.prepare_bias(bias.to(DEV), B, H, Sq, Sk, dt)
    dq, dk, dv = (torch.full_like(t, float("nan")) for t in dev[:3])
    db = torch.full((B, H, Sq, Sk), float("nan"), device=DEV, dtype=bias.dtype)
    lib = _lib.load()
    a = _lib.bwd_args(dev[0], dev[1], dev[2], o, dev[3], lse, dq, dk, dv, True, scale, 0.0, 0, 0, pb, db)
    ws = torch.empty(max(int(lib.fa_bwd_workspace_size(ctypes.byref(a))), 256), device=DEV, dtype=torch.uint8)
    st = lib.fa_bwd(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, _lib.strerror(st)
    torch.cuda.synchronize()
    assert not torch.isnan(db).any() and not torch.isnan(dq).any()
    assert torch.equal(db.tril(), db)  # causal: zeros above the diagonal (key > query)
    check(q, k, v, do, True, scale, bias, [t.cpu() for t in (o, lse, dq, dk, dv, db)], label=str(case))


@pytest.mark.parametrize("causal,dt,D", [(True, torch.bfloat16, 128), (False, torch.float16, 64),
                                         (True, torch.float16, 32)])
def test_bias_without_dbias(causal, dt, D):
    # a bias with no gradient requested: dQ recomputes dS, dK/dV run without stores
    B, S, H = 1, 300, 2
    say(f"case: bias without dbias causal={causal} {dt} D={D}")
    q, k, v, do = make_inputs(B, S, H, D, dt, seed=22)
    bias = make_bias((1, H, S, S), dt)
    scale = D ** -0.5
    dev = [t.to(DEV) for t in (q, k, v, do)]
    o, lse, _ = _lib.fwd(dev[0], dev[1], dev[2], causal, scale, bias=bias.to(DEV))
    dq, dk, dv = _lib.bwd(dev[0], dev[1], dev[2], o, dev[3], lse, causal, scale, bias=bias.to(DEV))
    torch.cuda.synchronize()
    check(q, k, v, do, causal, scale, bias, [t.cpu() for t in (o, lse, dq, dk, dv)],
          label=f"no dbias D={D}", names=NAMES[:5])


def test_bias_long_causal():
    # many key blocks and query tiles: the bias prefetch across tiles, dS read
    # back by the dQ pass, and the zeros of whole row tails
    B, S, H, D = 1, 1024, 2, 128
    say("case: bias long causal bf16 S=1024 D=128")
    q, k, v, do = make_inputs(B, S, H, D, torch.bfloat16, seed=23)
    bias = make_bias((1, H, S, S), torch.bfloat16)
    outs = run_kernels(q, k, v, do, True, D ** -0.5, bias)
    check(q, k, v, do, True, D ** -0.5, bias, [t.cpu() for t in outs], label="long causal")



@pytest.mark.parametrize("kind", ["full", "heads"])
def test_bias_dbias_full_size(kind):
    # The benchmark's bias workloads, B=4, S=4096, H=32, D=128 bf16 causal with
    # a (B, H, S, S) bias ("full") or a (1, H, S, S) one whose gradient sums
    # the batch ("heads", through per-batch parts), and their gradients: a
    # race between the tile copies and the waits that guard them shows at
    # this size and not at the small ones.  No output may be non-finite; dK /
    # dV equal those of the backward without a gradient bit for bit (the dS
    # stores change no arithmetic) and dQ (from the stored dS) theirs within 2
    # bf16 ulp; dBias of two heads against float32 torch math from the
    # kernel's own O and LSE (within 1% of its largest magnitude; exactly 0
    # above the diagonal).
    B, S, H, D = 4, 4096, 32, 128
    say(f"case: bias + dbias full size B=4 S=4096 H=32 D=128 bf16 causal, {kind}")
    g = torch.Generator(DEV).manual_seed(31)
    q, k, v, do = (torch.randn(B, S, H, D, generator=g, device=DEV).to(torch.bfloat16) for _ in range(4))
    bias = (torch.randn(B if kind == "full" else 1, H, S, S, generator=g, device=DEV) * 2.0).to(torch.bfloat16)
    scale = D ** -0.5
    o, lse, _ = _lib.fwd(q, k, v, True, scale, bias=bias)
    dq, dk, dv, db = _lib.bwd(q, k, v, o, do, lse, True, scale, bias=bias, want_dbias=True)
    dq2, dk2, dv2 = _lib.bwd(q, k, v, o, do, lse, True, scale, bias=bias)
    torch.cuda.synchronize()
    assert db.shape == bias.shape
    for n, t in (("O", o), ("LSE", lse), ("dQ", dq), ("dK", dk), ("dV", dv), ("dBias", db)):
        assert torch.isfinite(t.float()).all(), n
    assert torch.equal(dk, dk2) and torch.equal(dv, dv2)
    ulp = 2.0 ** -7  # bfloat16
    assert ((dq.float() - dq2.float()).abs() <= 2 * ulp * dq2.float().abs() + 1e-6).all()
    mask = torch.ones(S, S, dtype=torch.bool, device=DEV).triu(1)
    for b, h in ((0, 0), (3, 31)):
        ref = torch.zeros(S, S, device=DEV)
        for bb in ((b,) if kind == "full" else range(B)):
            qs, ks, vs, dos, os_ = (t[bb, :, h].float() for t in (q, k, v, do, o))
            st = qs @ ks.T * scale + bias[bb if kind == "full" else 0, h].float()
            st.masked_fill_(mask, -float("inf"))
            pm = torch.exp(st - lse[bb, h].float()[:, None])
            ref += pm * (dos @ vs.T - (dos * os_).sum(1, keepdim=True))
        bo = b if kind == "full" else 0
        got = db[bo, h].float()
        assert torch.equal(got[mask], torch.zeros_like(got[mask])), (bo, h)
        err = (got - ref).abs().max().item()
        say(f"  dBias[{bo},{h}] max err {err:.3g} of max {ref.abs().max().item():.3g}")
        assert err <= 0.01 * ref.abs().max().item(), (bo, h, err)

# Grids of at least 256 workgroups of 256 queries with a 16-bit bias and no
# dropout take the forward whose waves stage their bias rows through LDS; the
# small cases above do not.  O and LSE of a subset of heads against the
# oracle and the envelope.
STAGED = [
    # dtype, B, Sq, Sk, H, Hkv, D, causal, bias shape (None: (B, H, Sq, Sk))
    (torch.bfloat16, 1, 512, 512, 128, 128, 64, True, None),
    (torch.float16, 2, 500, 504, 64, 16, 128, False, None),
    (torch.bfloat16, 1, 300, 1024, 256, 256, 32, True, None),
    (torch.bfloat16, 2, 520, 520, 64, 64, 128, True, None),
    # broadcast biases (zero batch / head / query strides)
    (torch.bfloat16, 2, 512, 512, 64, 64, 128, True, (1, 64, 512, 512)),
    (torch.float16, 2, 512, 520, 64, 32, 64, False, (2, 1, 1, 520)),
]


@pytest.mark.parametrize("case", STAGED, ids=[f"{c[0]}-B{c[1]}-Sq{c[2]}-Sk{c[3]}-H{c[4]}-D{c[6]}-{c[7]}-{c[8]}" for c in STAGED])
def test_bias_staged_forward(case):
    dt, B, Sq, Sk, H, Hkv, D, causal, bshape = case
    say(f"case: staged-bias forward {case}")
    q, k, v, _ = make_inputs(B, Sq, H, D, dt, Sk=Sk, Hkv=Hkv, seed=24)
    bias = make_bias(bshape or (B, H, Sq, Sk), dt)
    scale = D ** -0.5
    o, lse, _ = _lib.fwd(q.to(DEV), k.to(DEV), v.to(DEV), causal, scale, bias=bias.to(DEV))
    torch.cuda.synchronize()
    g = H // Hkv
    for hh in (0, H // 2 + 1, H - 1):
        kh = hh // g
        bh = bias[:, hh:hh + 1] if bias.shape[1] > 1 else bias
        qs, ks, vs, bs = q[:, :, hh:hh + 1], k[:, :, kh:kh + 1], v[:, :, kh:kh + 1], bh
        ro, rl = oa.attention_forward(qs, ks, vs, causal, scale, None, 0.0, torch.float64, bias=bs)
        eo, el = lowp_math(qs.to(DEV), ks.to(DEV), vs.to(DEV), None, causal, scale, with_bwd=False, bias=bs.to(DEV))
        res = {"O": [maxabs(o[:, :, hh:hh + 1].cpu(), ro), maxabs(eo.cpu(), ro), ro.abs().max().item()],
               "LSE": [maxabs(lse[:, hh:hh + 1].cpu(), rl), maxabs(el.cpu(), rl), rl.abs().max().item()]}
        assert_parity(res, dt, f"staged head {hh}")


@pytest.mark.parametrize("side", [False, True])
def test_dbias_zero_tails_beside_dkdv_equal_staged(side, monkeypatch):
    """The whole backward with a causal bias gradient written in place writes
    the gradient's zero row tails in its dQ pass, or (FA_DBIAS_SIDE_STREAM=1)
    on the library's side stream, beside the dK/dV pass, joined back to the
    caller's stream; run stage by stage the dQ pass writes them.  All must give
    the same bits, every element written, from a non-default stream, on two
    calls in a row (the second smaller)."""
    import ctypes
    if side:
        monkeypatch.setenv("FA_DBIAS_SIDE_STREAM", "1")
    else:
        monkeypatch.delenv("FA_DBIAS_SIDE_STREAM", raising=False)
    lib = _lib.load()
    side = torch.cuda.Stream()
    for B, S, H, D, dt in ((2, 640, 2, 128, torch.bfloat16), (1, 384, 3, 64, torch.float16)):
        say(f"case: dbias zero tails on the side stream B={B} S={S} H={H} D={D} {dt}")
        q, k, v, do = make_inputs(B, S, H, D, dt, seed=23)
        bias = make_bias((B, H, S, S), dt)
        scale = D ** -0.5
        dev = [t.to(DEV) for t in (q, k, v, do)]
        o, lse, _ = _lib.fwd(dev[0], dev[1], dev[2], True, scale, bias=bias.to(DEV))
        pb = _lib.prepare_bias(bias.to(DEV), B, H, S, S, dt)
        outs = []
        for staged in (False, True):
            dq, dk, dv = (torch.full_like(t, float("nan")) for t in dev[:3])
            db = torch.full((B, H, S, S), float("nan"), device=DEV, dtype=dt)
            a = _lib.bwd_args(dev[0], dev[1], dev[2], o, dev[3], lse, dq, dk, dv, True, scale, 0.0, 0, 0, pb, db)
            nws = int(lib.fa_bwd_workspace_size(ctypes.byref(a)))
            ws = torch.empty(max(nws, 256), device=DEV, dtype=torch.uint8)
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                sp = ctypes.c_void_p(side.cuda_stream)
                wsp = ctypes.c_void_p(ws.data_ptr())
                if staged:
                    for stage in (0, 1, 2):
                        st = lib.fa_bwd_stage(ctypes.byref(a), wsp, ws.numel(), stage, sp)
                        assert st == 0, _lib.strerror(st)
                else:
                    st = lib.fa_bwd(ctypes.byref(a), wsp, ws.numel(), sp)
                    assert st == 0, _lib.strerror(st)
                # stream order: a reader on the caller's stream sees every zero
                flat = db.view(-1)[: db.numel()].float().isnan().sum()
            side.synchronize()
            assert flat.item() == 0
            outs.append((dq, dk, dv, db))
        for x, y in zip(*outs):
            assert torch.equal(x, y)
        assert torch.equal(outs[0][3].tril(), outs[0][3])


def test_dbias_side_stream_from_two_threads(monkeypatch):
    """Two host threads, each on its own stream, run the whole backward with a
    causal bias gradient (FA_DBIAS_SIDE_STREAM=1: zero tails forked onto the
    library's one side stream per GPU and joined back) several times at once;
    every result equals the single-threaded one bit for bit."""
    import ctypes
    import threading
    monkeypatch.setenv("FA_DBIAS_SIDE_STREAM", "1")
    lib = _lib.load()
    say("case: dbias zero tails on the side stream from two threads")
    B, S, H, D, dt = 1, 512, 2, 64, torch.bfloat16
    probs, refs = [], []
    for seed in (41, 42):
        q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dt, seed=seed))
        bias = make_bias((B, H, S, S), dt, seed=seed).to(DEV)
        o, lse, _ = _lib.fwd(q, k, v, True, D ** -0.5, bias=bias)
        pb = _lib.prepare_bias(bias, B, H, S, S, dt)
        refs.append(_lib.bwd(q, k, v, o, do, lse, True, D ** -0.5, bias=pb, want_dbias=True))
        probs.append((q, k, v, o, do, lse, pb))
    torch.cuda.synchronize()
    errors = []

    def worker(i):
        try:
            q, k, v, o, do, lse, pb = probs[i]
            st = torch.cuda.Stream()
            st.wait_stream(torch.cuda.default_stream())
            with torch.cuda.stream(st):
                for rep in range(4):
                    dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
                    db = torch.full((B, H, S, S), float("nan"), device=DEV, dtype=dt)
                    a = _lib.bwd_args(q, k, v, o, do, lse, dq, dk, dv, True, D ** -0.5, 0.0, 0, 0, pb, db)
                    ws = torch.empty(max(int(lib.fa_bwd_workspace_size(ctypes.byref(a))), 256), device=DEV,
                                     dtype=torch.uint8)
                    code = lib.fa_bwd(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                      ctypes.c_void_p(st.cuda_stream))
                    if code != 0:
                        raise RuntimeError(_lib.strerror(code))
                    st.synchronize()
                    if not all(torch.equal(x, y) for x, y in zip((dq, dk, dv, db), refs[i])):
                        raise AssertionError(f"thread {i} call {rep} differs from the single-threaded result")
        except Exception as e:  # reported by the main thread
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(probs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors


def test_dbias_side_stream_not_used_under_capture(monkeypatch):
    """FA_DBIAS_SIDE_STREAM=1: a backward with a causal in-place bias gradient
    captured into a graph writes its zero tails in the dQ pass (the side
    stream would join the capture and pull other calls' work into it); an
    eager backward on another stream while the capture is open still uses the
    side stream, is not pulled into the graph and writes every element; the
    capture ends cleanly, and every replay of the graph (with eager work and
    synchronisations between them) equals the eager result bit for bit."""
    import ctypes
    monkeypatch.setenv("FA_DBIAS_SIDE_STREAM", "1")
    lib = _lib.load()
    B, S, H, D, dt = 1, 384, 2, 64, torch.bfloat16
    say("case: dbias side stream and graph capture, (1, 384, 2, 64) bf16 causal")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dt, seed=29))
    bias = make_bias((B, H, S, S), dt, seed=29).to(DEV)
    o, lse, _ = _lib.fwd(q, k, v, True, D ** -0.5, bias=bias)
    pb = _lib.prepare_bias(bias, B, H, S, S, dt)
    ref = _lib.bwd(q, k, v, o, do, lse, True, D ** -0.5, bias=pb, want_dbias=True)  # creates the side stream

    def buffers():
        dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
        db = torch.full((B, H, S, S), float("nan"), device=DEV, dtype=dt)
        a = _lib.bwd_args(q, k, v, o, do, lse, dq, dk, dv, True, D ** -0.5, 0.0, 0, 0, pb, db)
        ws = torch.empty(max(int(lib.fa_bwd_workspace_size(ctypes.byref(a))), 256), device=DEV, dtype=torch.uint8)
        return a, ws, (dq, dk, dv, db)

    cap_a, cap_ws, cap_out = buffers()
    eag_a, eag_ws, eag_out = buffers()
    torch.cuda.synchronize()
    cap, eag = torch.cuda.Stream(), torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap, capture_error_mode="relaxed"):
        code = lib.fa_bwd(ctypes.byref(cap_a), ctypes.c_void_p(cap_ws.data_ptr()), cap_ws.numel(),
                          ctypes.c_void_p(cap.cuda_stream))
        assert code == 0, _lib.strerror(code)
        code = lib.fa_bwd(ctypes.byref(eag_a), ctypes.c_void_p(eag_ws.data_ptr()), eag_ws.numel(),
                          ctypes.c_void_p(eag.cuda_stream))
        assert code == 0, _lib.strerror(code)
    eag.synchronize()
    torch.cuda.synchronize()
    assert all(torch.equal(x, y) for x, y in zip(eag_out, ref))
    for rep in range(3):
        for t in cap_out:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(x, y) for x, y in zip(cap_out, ref)), f"replay {rep}"
        # eager work between replays
        again = _lib.bwd(q, k, v, o, do, lse, True, D ** -0.5, bias=pb, want_dbias=True)
        assert all(torch.equal(x, y) for x, y in zip(again, ref))


@pytest.mark.parametrize("kind", ["SqSk", "HSqSk"])
@pytest.mark.parametrize("causal", [False, True])
def test_bias_2d_3d_shapes(kind, causal):
    """The reference validator's 2-D (Sq, Sk) position bias and 3-D (H, Sq, Sk)
    per-head bias (utils.py:204-211) through the autograd entry point: read as
    (1, 1, Sq, Sk) and (1, H, Sq, Sk), gradient returned in the caller's shape
    (checked against the oracle's gradient of that 4-D view)."""
    dt, B, S, H, D = torch.bfloat16, 2, 160, 4, 64
    say(f"case: {kind} bias through flash_attention_v100, causal={causal}")
    q, k, v, do = make_inputs(B, S, H, D, dt, seed=12)
    shape = (S, S) if kind == "SqSk" else (H, S, S)
    bias = make_bias(shape, dt)
    view = bias.reshape((1, 1, S, S) if kind == "SqSk" else (1, H, S, S))
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    bd = bias.to(DEV).requires_grad_()
    o, lse = fa.flash_attention_v100(qd, kd, vd, causal=causal, bias=bd, return_softmax_lse=True,
                                     fallback_on_error=False)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    assert bd.grad.shape == shape and bd.grad.dtype == dt
    outs = (o.detach(), lse, qd.grad, kd.grad, vd.grad, bd.grad.reshape(view.shape))
    check(q, k, v, do, causal, D ** -0.5, view, outs, label=f"{kind}-causal{causal}")
