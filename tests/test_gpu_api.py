"""The public API on the GPU: flash_attention_v100, FlashAttentionV100Function
and the kernel-level launchers, including the reference's own property tests
(tests/test_attention.py:229-311, 352-379, 449-486, 602-625, 797-823)
retargeted at the gfx950 kernels instead of the reference's in-file mock."""
import warnings

import pytest
import torch

import flash_attention_v100 as fa
from flash_attention_v100 import _lib
from helpers import assert_parity, c_keep_mask, compare, make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"

REF_SHAPES = [(2, 512, 8, 64), (1, 1024, 12, 64), (2, 2048, 16, 64), (1, 4096, 8, 128)]
REF_DTYPES = [torch.float16, torch.float32, torch.bfloat16]


def say(msg):
    print(msg, flush=True)


def _qkv(shape, dtype, seed=42):
    # reference fixture: randn, q and k scaled by D**-0.5 * 0.5 (tests/test_attention.py:249-283)
    torch.manual_seed(seed)
    B, S, H, D = shape
    s = D ** -0.5 * 0.5
    q = (torch.randn(B, S, H, D, device=DEV) * s).to(dtype)
    k = (torch.randn(B, S, H, D, device=DEV) * s).to(dtype)
    v = torch.randn(B, S, H, D, device=DEV).to(dtype)
    return q, k, v


@pytest.mark.parametrize("shape", REF_SHAPES)
@pytest.mark.parametrize("dtype", REF_DTYPES)
def test_forward_basic(shape, dtype):
    say(f"case: api forward basic {shape} {dtype}")
    q, k, v = _qkv(shape, dtype)
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # no fallback may be taken
        out = fa.flash_attention_v100(q, k, v)
    assert out.shape == q.shape and out.dtype == dtype
    assert torch.isfinite(out).all()
    assert 0.01 < out.float().std().item() < 10


@pytest.mark.parametrize("dtype", REF_DTYPES)
def test_backward_basic(dtype):
    say(f"case: api backward basic {dtype}")
    q, k, v = (t.requires_grad_(True) for t in _qkv((2, 512, 8, 64), dtype))
    out = fa.flash_attention_v100(q, k, v, causal=True)
    out.float().sum().backward()
    for g in (q.grad, k.grad, v.grad):
        assert g is not None and torch.isfinite(g).all()
        assert 1e-8 < g.float().norm().item() < 1e4


def test_causal_differs_from_full():
    q, k, v = _qkv((2, 512, 8, 64), torch.float16)
    a = fa.flash_attention_v100(q, k, v, causal=False)
    b = fa.flash_attention_v100(q, k, v, causal=True)
    assert (a.float() - b.float()).abs().max().item() > 1e-6


def test_strategies_agree():
    q, k, v = _qkv((1, 1024, 12, 64), torch.bfloat16)
    outs = [fa.flash_attention_v100(q, k, v, optimization_strategy=s) for s in
            ("speed", "memory", "balanced", "adaptive")]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_interface_equals_kernel_and_lse():
    say("case: interface vs C ABI")
    q, k, v, do = (t.to(DEV) for t in make_inputs(2, 300, 4, 128, torch.bfloat16))
    o, lse = fa.flash_attention_v100(q, k, v, causal=True, return_softmax_lse=True)
    o2, lse2, _ = _lib.fwd(q, k, v, True, 128 ** -0.5)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert lse.shape == (2, 4, 300) and lse.dtype == torch.float32


def test_autograd_function_matches_abi_and_oracle():
    say("case: FlashAttentionV100Function autograd")
    q, k, v, do = (t.to(DEV) for t in make_inputs(2, 333, 4, 64, torch.float16, Hkv=2))
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = fa.FlashAttentionV100Function.apply(qq, kk, vv, 0.125, True)
    o.backward(do)
    o2, lse2, _ = _lib.fwd(q, k, v, True, 0.125)
    dq, dk, dv = _lib.bwd(q, k, v, o2, do, lse2, True, 0.125)
    assert torch.equal(o, o2)
    assert torch.equal(qq.grad, dq) and torch.equal(kk.grad, dk) and torch.equal(vv.grad, dv)
    res = compare(q, k, v, do, True, 0.125, (o2, lse2, dq, dk, dv), ref_device="cpu")
    assert_parity(res, torch.float16, "autograd GQA")


def test_dropout_through_interface_is_reproducible_and_exact():
    say("case: dropout via interface")
    B, S, H, D, p = 1, 200, 2, 64, 0.1
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.float32, seed=9))
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = fa.flash_attention_v100(qq, kk, vv, causal=True, dropout_p=p, dropout_seed=42, dropout_offset=0)
    o.backward(do)
    o_again = fa.flash_attention_v100(q, k, v, causal=True, dropout_p=p, dropout_seed=42, dropout_offset=0)
    assert torch.equal(o.detach(), o_again)
    keep = torch.from_numpy(c_keep_mask(42, 0, B, H, S, S, p)).bool().to(DEV)
    lse = _lib.fwd(q, k, v, True, D ** -0.5, p, 42, 0)[1]
    res = compare(q, k, v, do, True, D ** -0.5, (o.detach(), lse, qq.grad, kk.grad, vv.grad),
                  keep=keep, p=p, ref_device="cpu")
    assert_parity(res, torch.float32, "dropout interface")


def test_kernel_level_launchers():
    q, k, v, do = (t.to(DEV) for t in make_inputs(1, 256, 2, 64, torch.bfloat16))
    o, lse, mx = fa.flash_attention_forward_triton_enhanced(q, k, v, 0.125, True)
    s = torch.matmul(q.float().transpose(1, 2), k.float().transpose(1, 2).transpose(-2, -1).contiguous()) * 0.125
    s = s.masked_fill(torch.triu(torch.ones(256, 256, dtype=torch.bool, device=DEV), 1), float("-inf"))
    assert torch.allclose(mx, s.amax(-1), atol=1e-4)
    dq, dk, dv = fa.flash_attention_backward_triton_enhanced(q, k, v, o, do, lse, mx, 0.125, True)
    o2, lse2, mx2 = fa.flash_attention_forward_autotuned_enhanced(q, k, v, 0.125, True)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape


def test_invalid_tiles_fall_back_finite():
    # reference tests/test_attention.py:602-625: an unusable tile falls back and stays finite
    q, k, v = _qkv((1, 256, 4, 64), torch.float16)
    with pytest.warns(UserWarning, match="falling back"):
        out = fa.flash_attention_v100(q, k, v, block_size_m=10000, block_size_n=10000)
    assert torch.isfinite(out).all()
    with pytest.raises(ValueError):
        fa.flash_attention_v100(q, k, v, block_size_m=10000, fallback_on_error=False)


def test_bias_runs_on_kernels_and_matches_device_math():
    # the bias is served by the kernels (no fallback warning) and agrees with
    # the PyTorch math the fallback would have used
    q, k, v = _qkv((1, 128, 4, 64), torch.float16)
    bias = torch.randn(1, 4, 128, 128, device=DEV, dtype=torch.float16)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        out = fa.flash_attention_v100(q, k, v, causal=True, bias=bias, fallback_on_error=False)
    ref = fa.interface._fallback_to_pytorch(q, k, v, 64 ** -0.5, True, 0.0, bias, False)
    assert (out.float() - ref.float()).abs().max().item() < 2e-3


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("p", [0.0, 0.1])
def test_causal_dropout_combinations_finite(causal, p):
    q, k, v = _qkv((2, 256, 4, 64), torch.float16)
    out = fa.flash_attention_v100(q, k, v, causal=causal, dropout_p=p)
    assert torch.isfinite(out).all()


def test_kernel_errors_raise_not_fall_back():
    q, k, v = _qkv((1, 64, 2, 320), torch.float16)  # no kernel for head_dim 320 (beyond 256)
    with pytest.warns(UserWarning, match="falling back"):
        fa.flash_attention_v100(q, k, v)
    with pytest.raises(NotImplementedError):
        fa.flash_attention_v100(q, k, v, fallback_on_error=False)


def test_fallback_dropout_uses_the_kernel_mask():
    # the fallback applies the kernels' Philox mask for the same seed / offset
    q, k, v = _qkv((1, 128, 2, 64), torch.float16)
    out_k = fa.flash_attention_v100(q, k, v, dropout_p=0.2, dropout_seed=5, dropout_offset=0)
    out_f = fa.interface._fallback_to_pytorch(q, k, v, 64 ** -0.5, False, 0.2, None, False, 5, 0)
    err = (out_k.float() - out_f.float()).abs().max().item()
    other = fa.interface._fallback_to_pytorch(q, k, v, 64 ** -0.5, False, 0.2, None, False, 6, 0)
    say(f"kernel vs fallback, same seed: {err:.3e}; another seed: {(out_k.float() - other.float()).abs().max().item():.3e}")
    assert err < 5e-3 < (out_k.float() - other.float()).abs().max().item()


def test_standalone_forward_backward_and_compare():
    # reference ops/attention.py:464-718: forward only, backward from saved state, report dict
    from flash_attention_v100 import ops
    q, k, v, do = (t.to(DEV) for t in make_inputs(2, 200, 4, 64, torch.bfloat16, Hkv=2, seed=21))
    bias = torch.randn(1, 4, 200, 200, device=DEV).to(torch.bfloat16)
    o = ops.flash_attention_forward(q, k, v, None, True, 0.0, bias)
    o2, lse, mx = fa.flash_attention_forward_triton_enhanced(q, k, v, 64 ** -0.5, True, bias=bias)
    assert torch.equal(o, o2)
    dq, dk, dv = ops.flash_attention_backward(do, q, k, v, o2, lse, mx, 64 ** -0.5, True, bias=bias)
    dq2, dk2, dv2 = _lib.bwd(q, k, v, o2, do, lse, True, 64 ** -0.5, bias=bias)
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2)
    for p, causal, b in ((0.0, True, bias), (0.1, False, None)):
        r = ops.compare_with_pytorch_attention(q, k, v, causal, b, p, atol=2e-2, rtol=2e-2)
        say(f"compare p={p} causal={causal}: max abs {r['max_absolute_difference']:.3e} "
            f"cos {r['cosine_similarity']:.6f}")
        assert r["allclose"] and r["cosine_similarity"] > 0.9999
        assert r["configuration"]["has_bias"] == (b is not None) and r["input_shape"] == q.shape


@pytest.mark.parametrize("dtype,causal,p,with_bias,Hkv", [
    (torch.bfloat16, True, 0.0, False, 4),
    (torch.float16, True, 0.1, True, 2),     # dropout (bits made by the recomputing pass) + bias grad + GQA
    (torch.float32, False, 0.2, False, 4),
])
def test_gradient_checkpointing_recomputes_output(dtype, causal, p, with_bias, Hkv):
    # enable_gradient_checkpointing keeps q, k, v and the LSE only and recomputes
    # the output in the backward: every gradient equals the stored-output path's
    B, S, H, D = 2, 200, 4, 64
    say(f"case: checkpointing {dtype} causal={causal} p={p} bias={with_bias} Hkv={Hkv}")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dtype, Hkv=Hkv, seed=17))
    bias = torch.randn(1, H, S, S, device=DEV).to(dtype) if with_bias else None
    runs = []
    for ckpt in (False, True):
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        bb = bias.clone().requires_grad_(True) if with_bias else None
        o = fa.FlashAttentionV100Function.apply(qq, kk, vv, D ** -0.5, causal, p, bb, None, None, True, False,
                                                ckpt, True, None, True, "balanced", False, 1, 0, 99, 7)
        saved_ptrs = {t.data_ptr() for t in o.grad_fn.saved_tensors}
        assert (o.data_ptr() in saved_ptrs) == (not ckpt)
        o.backward(do)
        torch.cuda.synchronize()
        runs.append([o.detach(), qq.grad, kk.grad, vv.grad] + ([bb.grad] if with_bias else []))
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    # the context manager switches it on for calls inside the region (a bias
    # that requires grad, as above: dQ is then computed from the stored dS)
    with fa.ops.attention.gradient_checkpointing_mode():
        qq = q.clone().requires_grad_(True)
        bb = bias.clone().requires_grad_(True) if with_bias else None
        o = fa.flash_attention_v100(qq, k, v, causal=causal, dropout_p=p, bias=bb, dropout_seed=99,
                                    dropout_offset=7)
        assert o.data_ptr() not in {t.data_ptr() for t in o.grad_fn.saved_tensors}
        o.backward(do)
    torch.cuda.synchronize()
    assert torch.equal(qq.grad, runs[0][1])


def test_debug_validation_switch(monkeypatch):
    """config.DebugConfig.VALIDATE_OUTPUTS (reference config.py:274,
    ops/attention.py:163-168, 203-206, 271-272, 304-310): off by default, when
    no check runs; on, a NaN in an input or in the incoming gradient raises
    ValueError naming the tensor (with fallback_on_error the interface warns
    and falls back, as the reference's does)."""
    import warnings

    import flash_attention_v100 as fa
    from flash_attention_v100.config import DebugConfig
    from flash_attention_v100.ops import attention as att
    say("case: debug validation switch, (1, 64, 2, 64) bf16")
    q, k, v, do = (t.to(DEV) for t in make_inputs(1, 64, 2, 64, torch.bfloat16, seed=3))
    calls = []
    real = att.check_tensor_nan_inf
    monkeypatch.setattr(att, "check_tensor_nan_inf", lambda t, name, **kw: (calls.append(name), real(t, name, **kw))[1])
    qn = q.clone()
    qn[0, 3, 1, 5] = float("nan")
    o = fa.flash_attention_v100(qn, k, v, fallback_on_error=False)
    torch.cuda.synchronize()
    assert calls == [] and bool(torch.isnan(o).any())
    monkeypatch.setattr(DebugConfig, "VALIDATE_OUTPUTS", True)
    with pytest.raises(ValueError, match=r"^query contains 1 NaN values$"):
        fa.flash_attention_v100(qn, k, v, fallback_on_error=False)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        fa.flash_attention_v100(qn, k, v, fallback_on_error=True)
    assert any("falling back" in str(x.message) for x in w)
    calls.clear()
    qg = q.clone().requires_grad_()
    o = fa.flash_attention_v100(qg, k, v, causal=True, fallback_on_error=False)
    o.backward(do)
    assert calls == ["query", "key", "value", "bias", "output", "lse", "grad_output", "grad_q", "grad_k",
                     "grad_v", "grad_bias"]
    qg.grad = None
    o = fa.flash_attention_v100(qg, k, v, causal=True, fallback_on_error=False)
    dbad = do.clone()
    dbad[0, 0, 0, 0] = float("inf")
    with pytest.raises(ValueError, match=r"^grad_output contains 1 Inf values$"):
        o.backward(dbad)
