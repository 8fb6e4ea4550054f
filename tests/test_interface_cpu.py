"""Host-side logic of the Python interface (no GPU): signatures that mirror the
reference, validation errors and their types, tile-hint checks, the dropout
seed source, layout preparation and the loud failure when the library is
missing."""
import inspect

import pytest
import torch

import flash_attention_v100 as fa
from flash_attention_v100 import _lib
from flash_attention_v100.interface import validate_inputs_enhanced
from flash_attention_v100.ops.attention import check_block_sizes

# interface.py:199-217 of the reference
REF_INTERFACE = [
    ("q", inspect.Parameter.empty), ("k", inspect.Parameter.empty), ("v", inspect.Parameter.empty),
    ("causal", False), ("scale", None), ("dropout_p", 0.0), ("bias", None), ("block_size_m", None),
    ("block_size_n", None), ("enable_autotuning", True), ("return_softmax_lse", False),
    ("optimization_strategy", "balanced"), ("enable_multi_gpu", None), ("enable_profiling", False),
    ("fallback_on_error", True), ("validate_inputs", True),
]
# ops/attention.py:50-72 of the reference
REF_FUNCTION = ["q", "k", "v", "scale", "causal", "dropout_p", "bias", "block_size_m", "block_size_n",
                "enable_autotuning", "return_softmax_lse", "enable_gradient_checkpointing",
                "enable_mixed_precision", "num_checkpoints", "memory_efficient", "performance_mode",
                "enable_multi_gpu", "world_size", "rank"]


def test_interface_signature_mirrors_reference():
    params = list(inspect.signature(fa.flash_attention_v100).parameters.values())
    assert [(p.name, p.default) for p in params[:len(REF_INTERFACE)]] == REF_INTERFACE
    extra = params[len(REF_INTERFACE):]
    assert all(p.kind == inspect.Parameter.KEYWORD_ONLY for p in extra)


def test_function_signature_mirrors_reference():
    params = list(inspect.signature(fa.FlashAttentionV100Function.forward).parameters)[1:]
    assert params[:19] == REF_FUNCTION
    assert params[19:] == ["dropout_seed", "dropout_offset"]
    assert fa.FlashAttentionV100Function is fa.EnhancedFlashAttentionV100Function


def test_kernel_launcher_signatures():
    f = inspect.signature(fa.flash_attention_forward_triton_enhanced).parameters
    assert list(f)[:13] == ["q", "k", "v", "scale", "causal", "dropout_p", "bias", "block_size_m",
                            "block_size_n", "enable_warp_specialization", "enable_double_buffering",
                            "enable_prefetch", "use_fast_math"]
    b = inspect.signature(fa.flash_attention_backward_triton_enhanced).parameters
    assert list(b)[:14] == ["q", "k", "v", "o", "do", "lse", "max_vals", "scale", "causal", "block_size_m",
                            "block_size_n", "enable_fused_delta", "enable_gradient_accumulation", "use_fast_math"]


def test_standalone_function_signatures_and_aliases():
    # reference ops/attention.py:464-475, 539-550, 603-612 and the aliases at :756-759
    from flash_attention_v100 import ops
    f = inspect.signature(ops.flash_attention_forward_enhanced).parameters
    assert list(f)[:9] == ["q", "k", "v", "scale", "causal", "dropout_p", "bias", "enable_multi_gpu",
                           "performance_mode"]
    b = inspect.signature(ops.flash_attention_backward_enhanced).parameters
    assert list(b)[:10] == ["grad_output", "q", "k", "v", "output", "lse", "max_vals", "scale", "causal",
                            "enable_multi_gpu"]
    c = inspect.signature(ops.compare_with_pytorch_attention_enhanced).parameters
    assert [(n, p.default) for n, p in list(c.items())[3:]] == [
        ("causal", False), ("bias", None), ("dropout_p", 0.0), ("atol", 1e-4), ("rtol", 1e-4)]
    assert ops.flash_attention_forward is ops.flash_attention_forward_enhanced is fa.flash_attention_forward
    assert ops.flash_attention_backward is ops.flash_attention_backward_enhanced is fa.flash_attention_backward
    assert ops.compare_with_pytorch_attention is ops.compare_with_pytorch_attention_enhanced
    from flash_attention_v100.ops import attention as att
    assert not att._CHECKPOINTING
    with ops.gradient_checkpointing_mode(), ops.mixed_precision_mode(False):
        assert att._CHECKPOINTING
        with ops.gradient_checkpointing_mode(False):
            assert not att._CHECKPOINTING
        assert att._CHECKPOINTING
    assert not att._CHECKPOINTING


def test_standalone_functions_reject_cpu_tensors():
    from flash_attention_v100 import ops
    q = torch.zeros(1, 8, 2, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        ops.flash_attention_forward(q, q, q)


def _t(*shape, dtype=torch.float16):
    return torch.zeros(*shape, dtype=dtype)


@pytest.mark.parametrize("args,exc,msg", [
    ((_t(2, 8, 4, 64), _t(2, 8, 4, 64), [1]), TypeError, "torch.Tensor"),
    ((_t(8, 4, 64), _t(2, 8, 4, 64), _t(2, 8, 4, 64)), ValueError, "4-dimensional"),
    ((_t(2, 8, 4, 64), _t(3, 8, 4, 64), _t(3, 8, 4, 64)), ValueError, "Batch sizes"),
    ((_t(2, 8, 4, 64), _t(2, 8, 4, 64), _t(2, 9, 4, 64)), ValueError, "Sequence lengths"),
    ((_t(2, 8, 4, 64), _t(2, 8, 4, 32), _t(2, 8, 4, 32)), ValueError, "Head dimensions"),
    ((_t(2, 8, 4, 64), _t(2, 8, 3, 64), _t(2, 8, 3, 64)), ValueError, "divisible"),
    ((_t(2, 8, 4, 64), _t(2, 8, 2, 64), _t(2, 8, 1, 64)), ValueError, "key heads"),
    ((_t(2, 8, 4, 64), _t(2, 8, 4, 64, dtype=torch.float32), _t(2, 8, 4, 64)), ValueError, "same dtype"),
    ((_t(2, 8, 4, 64, dtype=torch.float64),) * 3, ValueError, "Unsupported dtype"),
    ((_t(2, 8, 4, 64),) * 3, ValueError, "GPU tensors"),
])
def test_validation_errors(args, exc, msg):
    with pytest.raises(exc, match=msg):
        validate_inputs_enhanced(*args)


def test_validation_dropout_and_bias(monkeypatch):
    q = _t(2, 8, 4, 64)
    # get past the device check to reach the later checks
    monkeypatch.setattr(torch.Tensor, "device", property(lambda self: torch.device("cuda", 0)))
    with pytest.raises(ValueError, match="dropout_p"):
        validate_inputs_enhanced(q, q, q, None, None, 1.0)
    with pytest.raises(ValueError, match="bias"):
        validate_inputs_enhanced(q, q, q, None, _t(2, 4, 8, 9), 0.0)
    _, _, _, scale = validate_inputs_enhanced(q, q, q, None, _t(1, 4, 8, 8), 0.0)
    assert scale == 64 ** -0.5
    with pytest.raises(ValueError, match="scale"):
        validate_inputs_enhanced(q, q, q, -1.0)


def test_cpu_tensors_never_fall_back():
    q = _t(1, 8, 2, 64)
    with pytest.raises(ValueError, match="GPU"):
        fa.flash_attention_v100(q, q, q, fallback_on_error=True)


def test_strategy_validated():
    q = _t(1, 8, 2, 64)
    with pytest.raises(ValueError, match="optimization_strategy"):
        fa.flash_attention_v100(q, q, q, optimization_strategy="turbo")


@pytest.mark.parametrize("bm,bn,ok", [(None, None, True), (64, 128, True), (16, 256, True),
                                      (10000, None, False), (0, None, False), (None, 48 + 1, False),
                                      (None, 512, False)])
def test_block_size_hints(bm, bn, ok):
    if ok:
        check_block_sizes(bm, bn)
    else:
        with pytest.raises(ValueError):
            check_block_sizes(bm, bn)


def test_seed_offset_source():
    torch.manual_seed(0)
    a = _lib.seed_offset(None, None)
    torch.manual_seed(0)
    b = _lib.seed_offset(None, None)
    assert a == b and a[1] == 0
    assert _lib.seed_offset(42, 7) == (42, 7)
    assert _lib.seed_offset(-1, 2**64 + 3) == (2**64 - 1, 3)


def test_prepare_layout():
    t = torch.zeros(2, 16, 4, 64, dtype=torch.bfloat16)
    assert _lib.prepare(t) is t
    tt = torch.zeros(2, 4, 16, 64, dtype=torch.bfloat16).transpose(1, 2)  # BHSD storage viewed as BSHD
    assert _lib.prepare(tt) is tt  # strides are 16-byte multiples, d stride 1
    td = torch.zeros(2, 16, 4, 64, dtype=torch.bfloat16).transpose(2, 3).transpose(2, 3).transpose(-1, -2)
    assert _lib.prepare(td).stride(-1) == 1
    base = torch.zeros(2 * 16 * 4 * 64 + 1, dtype=torch.bfloat16)
    mis = base[1:].view(2, 16, 4, 64)  # 2-byte misaligned base
    p = _lib.prepare(mis)
    assert p is not mis and p.data_ptr() % 16 == 0 and torch.equal(p, mis)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.FlashAttentionExtensionError, match="build"):
        _lib.load(str(tmp_path / "nope.so"))


# ---- bias shapes of the reference's validator (utils.py:204-211) ----

def test_validation_accepts_reference_bias_shapes(monkeypatch):
    B, S, H, D = 2, 8, 4, 64
    q = _t(B, S, H, D)
    monkeypatch.setattr(torch.Tensor, "device", property(lambda self: torch.device("cuda", 0)))
    for shape in [(B, H, S, S), (1, H, S, S), (B, 1, S, S), (1, 1, S, S), (H, S, S), (S, S)]:
        validate_inputs_enhanced(q, q, q, None, _t(*shape), 0.0)
    for shape in [(B, S, S), (S, S + 1), (H, S, S + 1), (S,), (1, 1, 1, S, S)]:
        with pytest.raises(ValueError, match="bias"):
            validate_inputs_enhanced(q, q, q, None, _t(*shape), 0.0)
    with pytest.raises(TypeError, match="bias"):
        validate_inputs_enhanced(q, q, q, None, [[0.0]], 0.0)


@pytest.mark.parametrize("shape,view", [((3, 5, 7), (1, 3, 5, 7)), ((5, 7), (1, 1, 5, 7)),
                                        ((2, 1, 5, 7), (2, 1, 5, 7))])
def test_prepare_bias_views_and_gradient_shape(shape, view):
    B, H, Sq, Sk = 2, 3, 5, 7
    g = torch.Generator().manual_seed(5)
    bias = torch.randn(*shape, generator=g).to(torch.bfloat16)
    pb = _lib.prepare_bias(bias, B, H, Sq, Sk, torch.bfloat16)
    assert pb.shape == view and pb.caller_shape == shape and pb.dtype == torch.bfloat16
    # the kernels read element (b, h, i, j) at the 4-D strides (zero on broadcast dims)
    st = list(pb.strides)
    seen = torch.as_strided(pb.tensor, (B, H, Sq, Sk), st, pb.tensor.storage_offset())
    assert st[3] == 1 and torch.equal(seen, bias.reshape(view).expand(B, H, Sq, Sk))
    # the score gradient (B, H, Sq, Sk) comes back summed and in the caller's shape
    ds = torch.randn(B, H, Sq, Sk, generator=g)
    want = ds.sum(dim=[d for d in range(4) if view[d] == 1], keepdim=True).reshape(shape).to(torch.bfloat16)
    got = _lib.reduce_dbias(ds, pb)
    assert got.shape == shape and torch.equal(got, want)


# ---- opt-in NaN / Inf validation (reference config.py:274, ops/attention.py:163-168) ----

def test_debug_switches_off_by_default():
    from flash_attention_v100.config import DebugConfig
    assert DebugConfig.VALIDATE_OUTPUTS is False and DebugConfig.CHECK_NUMERICAL_STABILITY is False
    assert fa.DebugConfig is DebugConfig


def test_check_tensor_nan_inf():
    from flash_attention_v100.utils import check_tensor_nan_inf
    x = torch.tensor([1.0, float("nan"), float("inf"), float("-inf"), float("nan")])
    with pytest.raises(ValueError, match=r"^query contains 2 NaN values and 2 Inf values$"):
        check_tensor_nan_inf(x, "query")
    with pytest.raises(ValueError, match=r"^lse contains 2 NaN values and 1 Inf values$"):
        check_tensor_nan_inf(x, "lse", allow_neg_inf=True)
    ok = torch.tensor([0.0, -float("inf")])
    assert check_tensor_nan_inf(ok, "lse", allow_neg_inf=True) is ok
    with pytest.warns(UserWarning, match="Attempting to fix"):
        fixed = check_tensor_nan_inf(x, "x", fix_issues=True)
    assert torch.isfinite(fixed).all() and fixed[1] == 0 and fixed[0] == 1
    assert check_tensor_nan_inf(None, "none") is None


def test_check_numerical_stability():
    from flash_attention_v100.utils import check_numerical_stability
    a = torch.ones(2, 3)
    check_numerical_stability(a, a, a)
    with pytest.raises(ValueError, match="key tensor contains NaN values"):
        check_numerical_stability(a, torch.full((2, 3), float("nan")), a)
    with pytest.raises(ValueError, match="bias tensor contains Inf values"):
        check_numerical_stability(a, a, a, torch.full((2,), float("inf")))
    with pytest.warns(UserWarning, match="very large values"):
        check_numerical_stability(a * 2e4, a, a)
    with pytest.warns(UserWarning, match="very small values"):
        check_numerical_stability(a, a, (a * 1e-8).to(torch.bfloat16))


def test_numerical_scan_only_when_switched_on(monkeypatch):
    from flash_attention_v100 import interface
    from flash_attention_v100.config import DebugConfig
    q = _t(2, 8, 4, 64)
    monkeypatch.setattr(torch.Tensor, "device", property(lambda self: torch.device("cuda", 0)))
    calls = []
    monkeypatch.setattr(interface, "check_numerical_stability", lambda *a: calls.append(a))
    validate_inputs_enhanced(q, q, q)
    assert calls == []
    monkeypatch.setattr(DebugConfig, "CHECK_NUMERICAL_STABILITY", True)
    validate_inputs_enhanced(q, q, q)
    assert len(calls) == 1
