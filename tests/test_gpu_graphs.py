"""fa_fwd + fa_bwd captured into a HIP graph (torch.cuda.graph) and replayed:
every replay, with eager work and a synchronisation between replays, equals
the eager call bit for bit.  Cases cover the launch forms a training or serving
loop would capture: the ping-pong forward and backward kernels of a large
16-bit D = 128 grid, the small-grid backward (delta pre-pass, then one launch
of the dK/dV and dQ workgroups), dropout with the forward's keep bits, and a
(1, H, S, S) bias whose gradient is summed over the batch (parts in the
workspace, then the reduction kernel)."""
import pytest
import torch

from flash_attention_v100 import _lib
from helpers import make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # name, (B, S, H, D), dtype, causal, dropout p, bias shape or None
    ("pingpong", (1, 3072, 48, 128), torch.bfloat16, True, 0.0, None),
    ("small-grid", (2, 1024, 12, 64), torch.float16, True, 0.0, None),
    ("dropout-keep-bits", (2, 500, 4, 64), torch.float16, True, 0.1, None),
    ("summed-bias-grad", (2, 384, 4, 128), torch.bfloat16, True, 0.0, (1, 4, 384, 384)),
]


def _step(q, k, v, do, causal, scale, p, bias):
    kb = _lib.alloc_keep_bits(q.shape[0], q.shape[2], q.shape[1], k.shape[1], q.device) if p > 0 else None
    o, lse, _ = _lib.fwd(q, k, v, causal, scale, p, 1234, 56, bias=bias, keep_bits=kb)
    g = _lib.bwd(q, k, v, o, do, lse, causal, scale, p, 1234, 56, bias=bias, want_dbias=bias is not None,
                 keep_bits=kb)
    return (o, lse) + tuple(g)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_graph_replays_equal_eager(case):
    name, (B, S, H, D), dt, causal, p, bshape = case
    print(f"case: graph capture {name}", flush=True)
    q, k, v, do = make_inputs(B, S, H, D, dt, seed=77, device=DEV)
    bias = None
    if bshape is not None:
        gen = torch.Generator("cpu").manual_seed(5)
        bias = torch.randn(bshape, generator=gen).to(dt).to(DEV)
    scale = D ** -0.5
    eager = _step(q, k, v, do, causal, scale, p, bias)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream's side (allocator pools)
        _step(q, k, v, do, causal, scale, p, bias)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _step(q, k, v, do, causal, scale, p, bias)
    for rep in range(3):
        for t in outs:
            t.fill_(float("nan"))  # a replay must rewrite every output
        torch.cuda.synchronize()
        graph.replay()
        junk = torch.randn(1 << 20, device=DEV).sum()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        for n, a, b in zip(("O", "LSE", "dQ", "dK", "dV", "dBias"), outs, eager):
            assert torch.equal(a, b), (name, rep, n)
