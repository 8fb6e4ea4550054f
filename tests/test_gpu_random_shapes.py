"""Parity over shapes drawn from a fixed seed: kernels through the C ABI
against the float64 oracle, with the tolerance of the other parity tests
(fp16 / bf16 within 2x the error of the reference math run in the inputs'
dtype, fp32 within 1e-5 of max|oracle|).  The draws mix what the fixed cases
hold apart: dtypes, head dims 32-256, GQA ratios, Sq != Sk, ragged and single
rows, causal or not, and the routing boundaries of the ping-pong and
small-grid kernels; the bias draws add every broadcast form of the bias and
its (summed) gradient."""
import random

import pytest
import torch

import test_gpu_bias as tb
from flash_attention_v100 import _lib
from helpers import assert_parity, compare, make_inputs

pytestmark = pytest.mark.gpu


def _draw_plain(n, seed):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        dt = rng.choice([torch.float16, torch.bfloat16, torch.bfloat16, torch.float32])
        D = rng.choice([32, 64, 128, 128] + ([256] if dt != torch.float32 else []))
        H = rng.choice([1, 2, 4, 6, 8, 12, 16])
        Hkv = rng.choice([d for d in range(1, H + 1) if H % d == 0])
        B = rng.choice([1, 2, 3])
        Sq = rng.choice([1, 7, 63, 64, 65, 127, 128, 129, 255, 256, 300, 511, 777, 1000, 1024, 1500])
        Sk = Sq if rng.random() < 0.6 else rng.choice([1, 33, 128, 200, 513, 1024, 1300])
        out.append((B, Sq, Sk, H, Hkv, D, dt, rng.random() < 0.6))
    return out


PLAIN = _draw_plain(36, 5) + [
    # ping-pong forward / backward (large 16-bit D = 128 grids) and small grids
    (1, 4096, 4096, 64, 64, 128, torch.bfloat16, True),
    (1, 3072, 3072, 48, 16, 128, torch.float16, True),
    (2, 2048, 2048, 64, 8, 128, torch.bfloat16, False),
    (1, 2500, 2600, 40, 40, 128, torch.bfloat16, False),
    (1, 1000, 1000, 8, 2, 64, torch.bfloat16, True),
    (2, 1024, 1024, 12, 12, 64, torch.float16, True),
]


def _id_plain(c):
    B, Sq, Sk, H, Hkv, D, dt, causal = c
    return f"B{B}-Sq{Sq}-Sk{Sk}-H{H}-Hkv{Hkv}-D{D}-{str(dt)[6:]}-{'causal' if causal else 'full'}"


@pytest.mark.parametrize("case", PLAIN, ids=[_id_plain(c) for c in PLAIN])
def test_random_shape(case):
    B, Sq, Sk, H, Hkv, D, dt, causal = case
    print(f"case: random shape {_id_plain(case)}", flush=True)
    q, k, v, do = make_inputs(B, Sq, H, D, dt, Sk=Sk, Hkv=Hkv, seed=Sq * 7 + Sk + H + D, device="cuda")
    scale = D ** -0.5
    o, lse, _ = _lib.fwd(q, k, v, causal, scale)
    dq, dk, dv = _lib.bwd(q, k, v, o, do, lse, causal, scale)
    torch.cuda.synchronize()
    assert_parity(compare(q, k, v, do, causal, scale, (o, lse, dq, dk, dv)), dt, _id_plain(case))


def _draw_bias(n, seed):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        dt = rng.choice([torch.float16, torch.bfloat16, torch.bfloat16, torch.float32])
        D = rng.choice([32, 64, 128])
        H = rng.choice([1, 2, 4, 6])
        Hkv = rng.choice([d for d in range(1, H + 1) if H % d == 0])
        B = rng.choice([1, 2, 3])
        Sq = rng.choice([1, 17, 64, 65, 128, 200, 257, 400])
        Sk = Sq if rng.random() < 0.6 else rng.choice([1, 33, 128, 150, 300])
        causal = rng.random() < 0.6
        kind = rng.choice(["full", "heads", "batch", "both", "q1"])
        shape = {"full": (B, H, Sq, Sk), "heads": (1, H, Sq, Sk), "batch": (B, 1, Sq, Sk),
                 "both": (1, 1, Sq, Sk), "q1": (B, H, 1, Sk)}[kind]
        bdt = torch.float32 if (dt != torch.float32 and rng.random() < 0.25) else None
        out.append((dt, B, Sq, Sk, H, Hkv, D, causal, shape, bdt))
    return out


BIASED = _draw_bias(24, 11)


@pytest.mark.parametrize("case", BIASED, ids=[tb._id(c) for c in BIASED])
def test_random_shape_with_bias(case):
    dt, B, Sq, Sk, H, Hkv, D, causal, shape, bdt = case
    print(f"case: random shape with bias {tb._id(case)}", flush=True)
    q, k, v, do = make_inputs(B, Sq, H, D, dt, Sk=Sk, Hkv=Hkv, seed=Sq + 3 * Sk + H + D)
    bias = tb.make_bias(shape, bdt or dt, seed=Sq + Sk)
    outs = tb.run_kernels(q, k, v, do, causal, D ** -0.5, bias)
    tb.check(q, k, v, do, causal, D ** -0.5, bias, [t.cpu() for t in outs], label=tb._id(case))
