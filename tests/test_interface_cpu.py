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
