"""Write tests/golden/triton_rand_vectors.json: Triton's own tl.rand /
tl.randint outputs for chosen (seed, 64-bit counter) pairs.

Triton is the third-party library whose ``tl.rand`` the reference's dropout
calls (kernels/forward_kernel.py:201); this script does not import the
reference.  It runs a small kernel written here under Triton's CPU
interpreter (TRITON_INTERPRET=1), so no GPU is needed.  The committed JSON is
the fixture; the GPU box never runs this script.

Usage: TRITON_INTERPRET=1 python tests/golden/make_triton_rand_vectors.py
"""
import json
import os
import sys

os.environ.setdefault("TRITON_INTERPRET", "1")
import numpy as np  # noqa: E402
import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402


@triton.jit
def _rand_kernel(seed, ctr_ptr, u_ptr, x_ptr, N: tl.constexpr):
    offs = tl.arange(0, N)
    c = tl.load(ctr_ptr + offs)  # int64 counters
    tl.store(u_ptr + offs, tl.rand(seed, c))
    tl.store(x_ptr + offs, tl.randint(seed, c))


def main():
    seeds = [0, 42, 0x0123456789ABCDEF, 2**32 - 1, 2**63 + 12345]
    rng = np.random.default_rng(7)
    base = [0, 1, 2, 3, 41, 2**31 - 1, 2**31, 2**32 - 5, 2**32 - 1, 2**32, 2**32 + 7,
            2**40 + 3, 2**62 + 11]
    ctrs = np.array(base + [int(x) for x in rng.integers(0, 2**62, size=64 - len(base))], dtype=np.int64)
    out = {"generator": "triton " + triton.__version__ + " interpreter, tl.rand / tl.randint",
           "cases": []}
    for s in seeds:
        c = torch.from_numpy(ctrs.copy())
        u = torch.empty(64, dtype=torch.float32)
        x = torch.empty(64, dtype=torch.int32)
        # tl.rand's seed argument is an integer scalar; Triton treats it as uint64
        s_arg = s if s < 2**63 else s - 2**64
        _rand_kernel[(1,)](s_arg, c, u, x, N=64)
        out["cases"].append({
            "seed": s,
            "counters": [int(v) for v in ctrs.tolist()],
            "uniform_f32_bits": [int(b) for b in u.numpy().view(np.uint32).tolist()],
            "randint_u32": [int(b) for b in x.numpy().view(np.uint32).tolist()],
        })
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "triton_rand_vectors.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=0)
    print("wrote", path)


if __name__ == "__main__":
    sys.exit(main())
