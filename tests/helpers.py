"""Shared test helpers: the benchmark input recipe, the C oracle library, the
low-precision error envelope and chunked float64 references."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

from oracle import attention as oa  # noqa: E402

_olib = None


def oracle_clib():
    """ctypes handle on oracle/_build/liboracle.so (the C Philox restatement)."""
    global _olib
    if _olib is None:
        lib = ctypes.CDLL(os.path.join(REPO, "oracle", "_build", "liboracle.so"))
        lib.oracle_philox4x32_10.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.oracle_rand.argtypes = [ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        lib.oracle_dropout_keep_mask.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int32, ctypes.c_int32,
                                                 ctypes.c_int32, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p]
        _olib = lib
    return _olib


def c_keep_mask(seed, offset, B, H, Sq, Sk, p) -> np.ndarray:
    keep = np.empty((B, H, Sq, Sk), dtype=np.uint8)
    oracle_clib().oracle_dropout_keep_mask(seed & (2**64 - 1), offset & (2**64 - 1), B, H, Sq, Sk,
                                           float(p), keep.ctypes.data)
    return keep


def c_rand(seed, counters) -> np.ndarray:
    c = np.ascontiguousarray(np.asarray(counters, dtype=np.uint64))
    u = np.empty(c.shape, dtype=np.float32)
    oracle_clib().oracle_rand(seed & (2**64 - 1), c.ctypes.data, c.size, u.ctypes.data)
    return u


def make_inputs(B, Sq, H, D, dtype, Sk=None, Hkv=None, seed=42, qk_scale=1.0, device="cpu"):
    """Benchmark input recipe: torch.Generator('cpu').manual_seed(seed), randn fp32 in
    the order q, k, v, dO, q/k optionally scaled, cast to ``dtype``."""
    Sk = Sq if Sk is None else Sk
    Hkv = H if Hkv is None else Hkv
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, Sq, H, D, generator=g, dtype=torch.float32) * qk_scale
    k = torch.randn(B, Sk, Hkv, D, generator=g, dtype=torch.float32) * qk_scale
    v = torch.randn(B, Sk, Hkv, D, generator=g, dtype=torch.float32)
    do = torch.randn(B, Sq, H, D, generator=g, dtype=torch.float32)
    return tuple(t.to(dtype).to(device) for t in (q, k, v, do))


def lowp_math(q, k, v, do, causal, scale, keep=None, p=0.0, with_bwd=True, bias=None):
    """The reference's math path (tests/test_attention.py:39-79) evaluated in
    the inputs' dtype (the error envelope), with explicit backward formulas.
    dK/dV come back per query head (see reduce_kv).  With an additive ``bias``
    (added in the inputs' dtype after the scale) dBias = dS, summed in float32
    over the broadcast dimensions and rounded to the bias's dtype, is appended.
    Every matmul operand is made contiguous (bf16 batched products with
    transposed views are avoided)."""
    dt = q.dtype
    H = q.shape[2]
    k = oa.expand_kv(k, H)
    v = oa.expand_kv(v, H)
    qh = q.transpose(1, 2).contiguous()
    kh = k.transpose(1, 2).contiguous()
    vh = v.transpose(1, 2).contiguous()
    s = torch.matmul(qh, kh.transpose(-2, -1).contiguous()) * scale
    if bias is not None:
        s = s + bias.to(dt)
    if causal:
        m = torch.triu(torch.ones(s.shape[-2], s.shape[-1], dtype=torch.bool, device=s.device), diagonal=1)
        s = s.masked_fill(m, float("-inf"))
    lse = torch.logsumexp(s.float(), dim=-1)
    pr = torch.softmax(s, dim=-1)
    pz = pr
    if p > 0:
        z = (keep.to(dt) / (1.0 - p)).to(dt)
        pz = pr * z
    o = torch.matmul(pz, vh)
    if not with_bwd:
        return o.transpose(1, 2), lse
    doh = do.transpose(1, 2).contiguous()
    dpz = torch.matmul(doh, vh.transpose(-2, -1).contiguous())
    dp = dpz * z if p > 0 else dpz
    delta = (pr * dp).sum(-1, keepdim=True)
    ds = pr * (dp - delta)
    dv = torch.matmul(pz.transpose(-2, -1).contiguous(), doh)
    dk = torch.matmul(ds.transpose(-2, -1).contiguous(), qh) * scale
    dq = torch.matmul(ds, kh) * scale
    dk = dk.transpose(1, 2)
    dv = dv.transpose(1, 2)
    if bias is not None:
        db = oa.reduce_to_bias_shape(ds.float(), bias.shape).to(bias.dtype)
        return o.transpose(1, 2), lse, dq.transpose(1, 2), dk, dv, db
    return o.transpose(1, 2), lse, dq.transpose(1, 2), dk, dv


def reduce_kv(g, Hkv):
    """Sum per-query-head K/V grads (B, S, H, D) down to (B, S, Hkv, D)."""
    B, S, H, D = g.shape
    if H == Hkv:
        return g
    return g.float().reshape(B, S, Hkv, H // Hkv, D).sum(3).to(g.dtype)


def maxabs(a, b) -> float:
    return (a.double() - b.double()).abs().max().item()


def chunked_reference(q, k, v, do, causal, scale, keep=None, p=0.0, dtype=torch.float64, heads_per_chunk=4,
                      with_bwd=True):
    """oracle.attention_forward/backward evaluated head-chunk by head-chunk
    (on whatever device the tensors live) in ``dtype``; GQA handled by giving
    each chunk its KV head slice.  Returns O, LSE[, dQ, dK, dV] in ``dtype``."""
    B, Sq, H, D = q.shape
    Hkv = k.shape[2]
    g = H // Hkv
    hc = max(g, heads_per_chunk - heads_per_chunk % g)  # whole KV groups per chunk
    O = torch.empty(B, Sq, H, D, dtype=dtype, device=q.device)
    L = torch.empty(B, H, Sq, dtype=dtype, device=q.device)
    if with_bwd:
        dQ = torch.empty_like(O)
        dK = torch.zeros(B, k.shape[1], Hkv, D, dtype=dtype, device=q.device)
        dV = torch.zeros_like(dK)
    for b in range(B):
        for h0 in range(0, H, hc):
            h1 = min(H, h0 + hc)
            k0, k1 = h0 // g, (h1 - 1) // g + 1
            sl = (slice(b, b + 1), slice(None), slice(h0, h1))
            kk = k[b:b + 1, :, k0:k1]
            vv = v[b:b + 1, :, k0:k1]
            mk = keep[b:b + 1, h0:h1] if keep is not None else None
            o, lse = oa.attention_forward(q[sl], kk, vv, causal, scale, mk, p, dtype)
            O[sl] = o
            L[b:b + 1, h0:h1] = lse
            if with_bwd:
                dq, dk, dv = oa.attention_backward(q[sl], kk, vv, o, do[sl], lse, causal, scale, mk, p, dtype)
                dQ[sl] = dq
                dK[b:b + 1, :, k0:k1] += dk
                dV[b:b + 1, :, k0:k1] += dv
    return (O, L, dQ, dK, dV) if with_bwd else (O, L)


NAMES_FWD = ("O", "LSE")
NAMES_BWD = ("O", "LSE", "dQ", "dK", "dV")


def compare(q, k, v, do, causal, scale, outs, keep=None, p=0.0, hpc=4, ref_device=None, with_bwd=True):
    """Chunk by chunk over (batch, whole KV-head groups): the float64 oracle on
    ``ref_device`` (default: the inputs' device) against the kernel outputs
    ``outs`` = (O, LSE[, dQ, dK, dV]) and against the reference math run in the
    inputs' dtype (the error envelope; skipped for float32 inputs).
    Returns {name: [max|kernel - ref|, max|lowp - ref| or None, max|ref|]}."""
    names = NAMES_BWD if with_bwd else NAMES_FWD
    ref_device = ref_device or q.device
    B, Sq, H, D = q.shape
    Hkv = k.shape[2]
    g = H // Hkv
    hc = max(g, hpc - hpc % g)
    env_on = q.dtype != torch.float32
    res = {n: [0.0, 0.0 if env_on else None, 0.0] for n in names}
    for b in range(B):
        for h0 in range(0, H, hc):
            h1 = min(H, h0 + hc)
            k0, k1 = h0 // g, (h1 - 1) // g + 1
            qs, dos = q[b:b + 1, :, h0:h1], do[b:b + 1, :, h0:h1]
            ks, vs = k[b:b + 1, :, k0:k1], v[b:b + 1, :, k0:k1]
            ms = keep[b:b + 1, h0:h1] if keep is not None else None
            r = [t.to(ref_device) for t in (qs, ks, vs, dos)]
            mr = ms.to(ref_device) if ms is not None else None
            o, lse = oa.attention_forward(r[0], r[1], r[2], causal, scale, mr, p, torch.float64)
            refs = [o, lse]
            if with_bwd:
                refs += list(oa.attention_backward(r[0], r[1], r[2], o, r[3], lse, causal, scale, mr, p))
            kern = [outs[0][b:b + 1, :, h0:h1], outs[1][b:b + 1, h0:h1]]
            if with_bwd:
                kern += [outs[2][b:b + 1, :, h0:h1], outs[3][b:b + 1, :, k0:k1], outs[4][b:b + 1, :, k0:k1]]
            env = None
            if env_on:
                env = list(lowp_math(qs, ks, vs, dos, causal, scale,
                                     ms.to(q.device) if ms is not None else None, p, with_bwd))
                if with_bwd:
                    env[3] = reduce_kv(env[3], k1 - k0)
                    env[4] = reduce_kv(env[4], k1 - k0)
            for i, n in enumerate(names):
                rf = refs[i].to(q.device)
                res[n][0] = max(res[n][0], maxabs(kern[i], rf))
                if env_on:
                    res[n][1] = max(res[n][1], maxabs(env[i], rf))
                res[n][2] = max(res[n][2], rf.abs().max().item())
            del refs, env, kern
    return res


def assert_parity(res, dtype, label=""):
    """fp16/bf16: max|kernel - oracle| <= 2 * max|reference lowp math - oracle|;
    fp32: <= 1e-5 * max|oracle|.  Both get an absolute floor of 1e-6 times the
    largest oracle magnitude of the case, for outputs whose exact value is 0
    (e.g. dQ and dK with a single key, where the envelope is exactly 0 too)."""
    lines = []
    ok = True
    floor = 1e-6 * max(mr for _, _, mr in res.values())
    for n, (ek, ee, mr) in res.items():
        if dtype == torch.float32:
            tol = max(1e-5 * mr, floor)
        else:
            tol = 2.0 * ee + floor
        good = ek <= tol
        ok &= good
        lines.append(f"{label} {n}: kernel_err={ek:.3e} env_err={ee if ee is None else f'{ee:.3e}'} "
                     f"max|ref|={mr:.3e} tol={tol:.3e} {'ok' if good else 'FAIL'}")
    print("\n".join(lines), flush=True)
    assert ok, "\n".join(lines)
