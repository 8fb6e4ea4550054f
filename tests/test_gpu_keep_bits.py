"""Dropout keep bits: the forward writes the keep mask it applied, bit-packed,
and the backward reads it (dK/dV transposing 32 x 32 bit blocks across lanes)
instead of regenerating the Philox stream.  The stored bits must equal the
oracle's mask (bit-exact) and every output of the bits path must equal the
regenerating path's bit for bit; the regenerating path itself is held to the
oracle in test_gpu_kernels.py."""
import numpy as np
import pytest
import torch

import flash_attention_v100 as fa
from flash_attention_v100 import _lib
from helpers import assert_parity, c_keep_mask, compare, make_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(msg):
    print(msg, flush=True)


def unpack(words: torch.Tensor, n: int) -> np.ndarray:
    """int32 words (R, W) -> bool (R, n): bit c%32 of word c/32."""
    w = words.cpu().numpy().view(np.uint32)
    bits = (w[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1
    return bits.reshape(w.shape[0], -1)[:, :n].astype(bool)


def defined(B, H, Sq, Sk, causal) -> np.ndarray:
    """Pairs (i, j) whose bits the forward writes: all of them, or under
    top-left causal masking those with j <= i."""
    m = np.ones((Sq, Sk), dtype=bool)
    if causal:
        m = np.tril(m)
    return np.broadcast_to(m, (B, H, Sq, Sk))


CASES = [  # dtype, B, Sq, Sk, H, Hkv, D, causal
    (torch.float16, 2, 150, 150, 3, 3, 64, True),
    (torch.bfloat16, 1, 130, 257, 4, 2, 128, True),   # GQA, Sq < Sk
    (torch.float16, 1, 300, 77, 2, 2, 32, True),      # Sq > Sk (top-left causal)
    (torch.float32, 2, 100, 100, 2, 2, 64, False),
    (torch.float32, 1, 70, 70, 2, 1, 128, True),
    (torch.bfloat16, 1, 1, 50, 2, 1, 64, False),      # one query
    (torch.float16, 1, 64, 1, 2, 2, 128, False),      # one key
    # the benchmark's C5 edge sweep at full size, every head dim and dtype
    (torch.float16, 8, 1000, 1000, 16, 16, 32, True),
    (torch.float16, 8, 1000, 1000, 16, 16, 64, True),
    (torch.float16, 8, 1000, 1000, 16, 16, 128, True),
    (torch.float32, 8, 1000, 1000, 16, 16, 32, True),
    (torch.float32, 8, 1000, 1000, 16, 16, 64, True),
    (torch.float32, 8, 1000, 1000, 16, 16, 128, True),
    (torch.bfloat16, 2, 77, 90, 3, 3, 64, True),      # odd Sq: row pairs of the mask kernel span two heads
    (torch.float16, 1, 33, 600, 2, 1, 128, True),     # odd Sq, keys past the longest causal row
]


def _id(c):
    dt, B, Sq, Sk, H, Hkv, D, causal = c
    return f"{str(dt)[6:]}-B{B}-Sq{Sq}-Sk{Sk}-H{H}-Hkv{Hkv}-D{D}-{'causal' if causal else 'full'}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_keep_bits_path_equals_regeneration(case):
    dt, B, Sq, Sk, H, Hkv, D, causal = case
    say(f"case: keep bits {_id(case)}")
    p, seed, offset = 0.17, 1234, 2**32 - 777
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Sq, H, D, dt, Sk=Sk, Hkv=Hkv, seed=5))
    scale = D ** -0.5
    bits = _lib.alloc_keep_bits(B, H, Sq, Sk, q.device)
    o1, lse1, _ = _lib.fwd(q, k, v, causal, scale, p, seed, offset)
    o2, lse2, _ = _lib.fwd(q, k, v, causal, scale, p, seed, offset, keep_bits=bits)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(lse1, lse2)

    want = c_keep_mask(seed, offset, B, H, Sq, Sk, p).astype(bool)
    sel = defined(B, H, Sq, Sk, causal)
    rows = unpack(bits, Sk).reshape(B, H, Sq, Sk)
    assert np.array_equal(rows[sel], want[sel])

    g1 = _lib.bwd(q, k, v, o1, do, lse1, causal, scale, p, seed, offset)
    g2 = _lib.bwd(q, k, v, o1, do, lse1, causal, scale, p, seed, offset, keep_bits=bits)
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), g1, g2):
        assert torch.equal(a, b), name


def test_keep_bits_parity_with_oracle():
    B, S, H, D, p = 2, 180, 3, 64, 0.2
    say("case: keep bits path vs oracle")
    for dt in (torch.float16, torch.float32):
        q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, dt, seed=13))
        bits = _lib.alloc_keep_bits(B, H, S, S, q.device)
        o, lse, _ = _lib.fwd(q, k, v, True, D ** -0.5, p, 77, 99, keep_bits=bits)
        dq, dk, dv = _lib.bwd(q, k, v, o, do, lse, True, D ** -0.5, p, 77, 99, keep_bits=bits)
        torch.cuda.synchronize()
        keep = torch.from_numpy(c_keep_mask(77, 99, B, H, S, S, p)).bool().to(DEV)
        res = compare(q, k, v, do, True, D ** -0.5, (o, lse, dq, dk, dv), keep=keep, p=p, ref_device="cpu")
        assert_parity(res, dt, f"keep bits {dt}")


def test_keep_bits_with_bias_and_dbias():
    B, S, H, D, p = 1, 200, 2, 64, 0.1
    say("case: keep bits with bias + dbias")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.bfloat16, seed=3))
    bias = torch.randn(B, H, S, S, device=DEV).to(torch.bfloat16)
    bits = _lib.alloc_keep_bits(B, H, S, S, q.device)
    o, lse, _ = _lib.fwd(q, k, v, True, 0.125, p, 5, 6, bias=bias, keep_bits=bits)
    o1, _, _ = _lib.fwd(q, k, v, True, 0.125, p, 5, 6, bias=bias)
    g1 = _lib.bwd(q, k, v, o, do, lse, True, 0.125, p, 5, 6, bias=bias, want_dbias=True)
    g2 = _lib.bwd(q, k, v, o, do, lse, True, 0.125, p, 5, 6, bias=bias, want_dbias=True, keep_bits=bits)
    torch.cuda.synchronize()
    assert torch.equal(o, o1)
    for name, a, b in zip(("dq", "dk", "dv", "dbias"), g1, g2):
        assert torch.equal(a, b), name


def test_autograd_uses_keep_bits(monkeypatch):
    # the autograd function stores the bits when they fit the byte limit;
    # gradients equal those of the regenerating path
    B, S, H, D, p = 2, 256, 4, 128, 0.1
    say("case: autograd keep bits")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, S, H, D, torch.bfloat16, seed=21))
    grads, allocs = [], []
    alloc = _lib.alloc_keep_bits
    monkeypatch.setattr(_lib, "alloc_keep_bits", lambda *a: allocs.append(a) or alloc(*a))
    for limit in (_lib.KEEP_BITS_MAX_BYTES, 0):
        monkeypatch.setattr(_lib, "KEEP_BITS_MAX_BYTES", limit)
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        o = fa.flash_attention_v100(qq, kk, vv, causal=True, dropout_p=p, dropout_seed=8, dropout_offset=0)
        o.backward(do)
        torch.cuda.synchronize()
        grads.append((o.detach(), qq.grad, kk.grad, vv.grad))
    assert len(allocs) == 1  # bits with the default limit, regeneration with 0
    for a, b in zip(*grads):
        assert torch.equal(a, b)
