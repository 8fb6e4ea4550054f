"""numpy restatement of the dropout RNG (TEST INFRASTRUCTURE ONLY).

The reference draws its dropout mask with Triton's ``tl.rand(seed, offset)``
(``kernels/forward_kernel.py:198-203``), i.e. Philox4x32-10 (Salmon, Moraes,
Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11) followed by
Triton's uint32 -> fp32 mapping (triton/language/random.py, ``randint4x`` /
``uint_to_uniform_float``):

* key   = (lo32(seed), hi32(seed));
* ctr   = (lo32(c), hi32(c), 0, 0) for a 64-bit counter ``c``;
* round = ``c0' = mulhi(B, c2) ^ c1 ^ k0``, ``c2' = mulhi(A, c0) ^ c3 ^ k1``,
  ``c1' = lo(B * c2)``, ``c3' = lo(A * c0)``, then ``k0 += 0x9E3779B9``,
  ``k1 += 0xBB67AE85``; A = 0xD2511F53, B = 0xCD9E8D57; ten rounds;
* ``u = fp32(x) * fp32(4.6566127342e-10)`` with ``x`` = word 0 bit-cast to
  int32 and folded ``x < 0 ? -x - 1 : x``.

The dropout counter restores the row index the reference drops
(``forward_kernel.py:110-111, 200``):
``c = offset + ((b * H + h) * Sq + i) * Sk + j`` (mod 2**64); keep = ``u > p``
with ``p`` rounded to fp32 (it is a fp32 kernel argument).
"""
from __future__ import annotations

import numpy as np

M_A = np.uint64(0xD2511F53)
M_B = np.uint64(0xCD9E8D57)
W_A = np.uint32(0x9E3779B9)
W_B = np.uint32(0xBB67AE85)
U_SCALE = np.float32(4.6566127342e-10)
_LO = np.uint64(0xFFFFFFFF)
_S32 = np.uint64(32)


def philox4x32_10(c0, c1, c2, c3, k0, k1, rounds: int = 10):
    """Philox4x32 on uint32 arrays (broadcast); returns four uint32 arrays."""
    c0 = np.asarray(c0, dtype=np.uint32)
    c1 = np.asarray(c1, dtype=np.uint32)
    c2 = np.asarray(c2, dtype=np.uint32)
    c3 = np.asarray(c3, dtype=np.uint32)
    k0 = np.asarray(k0, dtype=np.uint32)
    k1 = np.asarray(k1, dtype=np.uint32)
    with np.errstate(over="ignore"):
        for _ in range(rounds):
            pa = M_A * c0.astype(np.uint64)
            pb = M_B * c2.astype(np.uint64)
            n0 = (pb >> _S32).astype(np.uint32) ^ c1 ^ k0
            n2 = (pa >> _S32).astype(np.uint32) ^ c3 ^ k1
            n1 = (pb & _LO).astype(np.uint32)
            n3 = (pa & _LO).astype(np.uint32)
            c0, c1, c2, c3 = n0, n1, n2, n3
            k0 = k0 + W_A
            k1 = k1 + W_B
    return c0, c1, c2, c3


def uint_to_uniform(x) -> np.ndarray:
    """Triton's uint32 -> [0, 1) fp32 mapping."""
    xi = np.asarray(x, dtype=np.uint32).view(np.int32).astype(np.int64)
    xi = np.where(xi < 0, -xi - 1, xi)
    return xi.astype(np.float32) * U_SCALE


def rand(seed: int, counters) -> np.ndarray:
    """``tl.rand(seed, counters)`` for 64-bit counters."""
    c = np.asarray(counters, dtype=np.uint64)
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    k0 = np.uint32(seed & 0xFFFFFFFF)
    k1 = np.uint32(seed >> 32)
    lo = (c & _LO).astype(np.uint32)
    hi = (c >> _S32).astype(np.uint32)
    z = np.zeros_like(lo)
    x, _, _, _ = philox4x32_10(lo, hi, z, z, k0, k1)
    return uint_to_uniform(x)


def dropout_counters(offset: int, B: int, H: int, Sq: int, Sk: int) -> np.ndarray:
    """(B, H, Sq, Sk) uint64 counters ``offset + ((b*H + h)*Sq + i)*Sk + j``."""
    n = B * H * Sq * Sk
    with np.errstate(over="ignore"):
        c = np.arange(n, dtype=np.uint64) + np.uint64(int(offset) & 0xFFFFFFFFFFFFFFFF)
    return c.reshape(B, H, Sq, Sk)


def dropout_keep_mask(seed: int, offset: int, B: int, H: int, Sq: int, Sk: int, p: float) -> np.ndarray:
    """Bool keep mask (B, H, Sq, Sk): ``rand(seed, counter) > fp32(p)``."""
    u = rand(seed, dropout_counters(offset, B, H, Sq, Sk))
    return u > np.float32(p)
