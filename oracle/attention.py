"""Restatement of the reference's attention math (TEST INFRASTRUCTURE ONLY).

Device-agnostic torch code: run on the CPU it is the oracle; the GPU tests may
also evaluate it in float64 on the device for shapes too large for the host.

The reference computes attention in its test mock and its import fallback as
plain PyTorch math on (B, S, H, D) tensors:

* ``tests/test_attention.py:39-79``: transpose to (B, H, S, D), ``matmul(q, k^T)
  * scale``, causal ``masked_fill(triu(ones, diagonal=1), -inf)``, ``softmax``,
  optional dropout, ``matmul(p, v)``, transpose back.
* ``__init__.py:34-55``: the same with ``q * scale`` folded before the matmul.
* default ``scale = D ** -0.5`` (``utils.py:148-153``).

The build fixes what the reference's Triton kernels get wrong
(``kernels/forward_kernel.py:206-217`` normalisation, ``:242-243`` where ``L``
holds the row sum, ``kernels/backward_kernel.py:176-194`` racy dQ): this oracle
is the textbook math, with

* LSE = natural-log logsumexp of the scaled, masked scores, shape (B, H, Sq);
* dropout applied after the softmax normalisation, as ``Z / (1 - p)``, with
  ``Z`` the keep mask of :func:`oracle.philox.dropout_keep_mask`
  (reference: ``forward_kernel.py:198-203``, keep = ``u > p``);
* causal masks key ``j > i`` (top-left aligned, ``forward_kernel.py:181``,
  ``tests/test_attention.py:63``), also when Sq != Sk;
* grouped KV heads: query head ``h`` reads KV head ``h // (H // Hkv)``
  (``utils.py:88-97`` allows ``H % Hkv == 0``);
* an optional additive bias of shape (B|1, H|1, Sq|1, Sk) is added to the scaled
  scores before the causal mask (``forward_kernel.py:166-182``: ``qk * scale``,
  ``+ bias_block``, then ``tl.where(causal_mask, qk, -inf)``).

Gradients follow ``kernels/backward_kernel.py:118-176`` with the row index of
the dropout counter and the saved dropout mask restored:
``delta_i = sum_d dO_id O_id``, ``dP = (dO V^T) * Z/(1-p)``,
``dS = P * (dP - delta)``, ``dV = (P * Z/(1-p))^T dO``, ``dK = scale dS^T Q``,
``dQ = scale dS K``.  The bias gradient is ``dS`` itself (the gradient of the
biased scores), summed over the dimensions the bias broadcasts; the reference
returned zeros for it (``ops/attention.py:297-301``).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

__all__ = [
    "expand_kv",
    "attention_forward",
    "attention_backward",
    "attention_autograd",
    "brute_force_forward",
    "reduce_to_bias_shape",
]


def expand_kv(x: torch.Tensor, num_heads: int) -> torch.Tensor:
    """(B, S, Hkv, D) -> (B, S, H, D): query head h uses KV head h // (H // Hkv)."""
    hkv = x.shape[2]
    if hkv == num_heads:
        return x
    if num_heads % hkv != 0:
        raise ValueError(f"num_heads {num_heads} not divisible by kv heads {hkv}")
    return x.repeat_interleave(num_heads // hkv, dim=2)


def _causal_mask(sq: int, sk: int, device=None) -> torch.Tensor:
    # True where masked: key j > query i (triu(ones, diagonal=1)).
    return torch.triu(torch.ones(sq, sk, dtype=torch.bool, device=device), diagonal=1)


def _scores(q, k, causal, scale, dtype, bias=None):
    qh = q.to(dtype).transpose(1, 2)  # (B, H, Sq, D)
    kh = k.to(dtype).transpose(1, 2)
    s = torch.matmul(qh, kh.transpose(-2, -1)) * scale
    if bias is not None:
        s = s + bias.to(dtype)  # broadcasts over B and H
    if causal:
        s = s.masked_fill(_causal_mask(s.shape[-2], s.shape[-1], s.device), float("-inf"))
    return s


def attention_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: Optional[float] = None,
    dropout_mask: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
    dtype: torch.dtype = torch.float64,
    bias: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Forward O (B, Sq, H, D) in ``dtype`` and LSE (B, H, Sq) in ``dtype``.

    ``dropout_mask`` is a bool keep-mask (B, H, Sq, Sk) or None; ``bias`` an
    additive (B|1, H|1, Sq|1, Sk) tensor or None.
    Rows with no visible key (Sk == 0, or a bias that is -inf on every key
    the causal mask leaves) give O = 0, LSE = -inf and zero gradients, as
    FlashAttention-2 does; the reference's ``softmax`` would give NaN there.
    """
    B, Sq, H, D = q.shape
    if scale is None:
        scale = D ** -0.5
    k = expand_kv(k, H)
    v = expand_kv(v, H)
    Sk = k.shape[1]
    if Sk == 0:
        return (torch.zeros(B, Sq, H, D, dtype=dtype, device=q.device),
                torch.full((B, H, Sq), float("-inf"), dtype=dtype, device=q.device))
    s = _scores(q, k, causal, scale, dtype, bias)
    # softmax through the row max, with rows that see no key (max = -inf)
    # shifted by 0 instead: their probabilities are then exp(-inf) = 0 and no
    # -inf - (-inf) = NaN reaches the values or the autograd graph
    m = s.amax(dim=-1, keepdim=True)
    dead = torch.isneginf(m)
    m = torch.where(dead, torch.zeros_like(m), m).detach()
    e = torch.exp(s - m)
    tot = e.sum(dim=-1, keepdim=True)
    lse = (m + torch.log(tot)).squeeze(-1)
    p = e / torch.where(dead, torch.ones_like(tot), tot)
    if dropout_p > 0.0:
        if dropout_mask is None:
            raise ValueError("dropout_p > 0 needs an explicit keep mask")
        p = p * dropout_mask.to(dtype) / (1.0 - dropout_p)
    o = torch.matmul(p, v.to(dtype).transpose(1, 2))  # (B, H, Sq, D)
    return o.transpose(1, 2).contiguous(), lse


def attention_backward(
    q, k, v, o, do, lse,
    causal: bool = False,
    scale: Optional[float] = None,
    dropout_mask: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
    dtype: torch.dtype = torch.float64,
    bias: Optional[torch.Tensor] = None,
):
    """Explicit-formula backward (dQ, dK, dV) in ``dtype``; dK/dV summed over
    the query heads that share a KV head.  With ``bias`` also returns dBias
    (the bias's shape) as a fourth element."""
    B, Sq, H, D = q.shape
    Hkv = k.shape[2]
    if scale is None:
        scale = D ** -0.5
    ke = expand_kv(k, H)
    ve = expand_kv(v, H)
    s = _scores(q, ke, causal, scale, dtype, bias)
    # rows with LSE = -inf saw no key: P = 0 there (exp(s - inf))
    lse_d = lse.to(dtype)
    lse_d = torch.where(torch.isneginf(lse_d), torch.full_like(lse_d, float("inf")), lse_d)
    p = torch.exp(s - lse_d.unsqueeze(-1))  # (B, H, Sq, Sk)
    if causal:
        p = p.masked_fill(_causal_mask(Sq, ke.shape[1], p.device), 0.0)
    qh = q.to(dtype).transpose(1, 2)
    kh = ke.to(dtype).transpose(1, 2)
    vh = ve.to(dtype).transpose(1, 2)
    doh = do.to(dtype).transpose(1, 2)
    oh = o.to(dtype).transpose(1, 2)
    delta = (doh * oh).sum(-1, keepdim=True)  # (B, H, Sq, 1)
    dp = torch.matmul(doh, vh.transpose(-2, -1))
    pz = p
    if dropout_p > 0.0:
        z = dropout_mask.to(dtype) / (1.0 - dropout_p)
        dp = dp * z
        pz = p * z
    ds = p * (dp - delta)
    dv = torch.matmul(pz.transpose(-2, -1), doh)
    dk = torch.matmul(ds.transpose(-2, -1), qh) * scale
    dq = torch.matmul(ds, kh) * scale
    dq = dq.transpose(1, 2).contiguous()
    dk = dk.transpose(1, 2)
    dv = dv.transpose(1, 2)
    if Hkv != H:
        g = H // Hkv
        dk = dk.reshape(B, dk.shape[1], Hkv, g, D).sum(3)
        dv = dv.reshape(B, dv.shape[1], Hkv, g, D).sum(3)
    if bias is None:
        return dq, dk.contiguous(), dv.contiguous()
    return dq, dk.contiguous(), dv.contiguous(), reduce_to_bias_shape(ds, bias.shape)


def reduce_to_bias_shape(ds: torch.Tensor, shape) -> torch.Tensor:
    """Sum a (B, H, Sq, Sk) score gradient over the dimensions a bias of
    ``shape`` (B|1, H|1, Sq|1, Sk) broadcasts."""
    for dim in (0, 1, 2):
        if shape[dim] == 1 and ds.shape[dim] != 1:
            ds = ds.sum(dim, keepdim=True)
    return ds.contiguous()


def attention_autograd(
    q, k, v, do,
    causal: bool = False,
    scale: Optional[float] = None,
    dropout_mask: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
    dtype: torch.dtype = torch.float64,
    bias: Optional[torch.Tensor] = None,
):
    """(O, LSE, dQ, dK, dV) with the gradients taken by torch.autograd through
    :func:`attention_forward` (a second, independent route to the backward);
    with ``bias`` also dBias as a sixth element."""
    qq = q.detach().to(dtype).requires_grad_(True)
    kk = k.detach().to(dtype).requires_grad_(True)
    vv = v.detach().to(dtype).requires_grad_(True)
    bb = None if bias is None else bias.detach().to(dtype).requires_grad_(True)
    o, lse = attention_forward(qq, kk, vv, causal, scale, dropout_mask, dropout_p, dtype, bb)
    o.backward(do.to(dtype))
    if bb is None:
        return o.detach(), lse.detach(), qq.grad, kk.grad, vv.grad
    return o.detach(), lse.detach(), qq.grad, kk.grad, vv.grad, bb.grad


def brute_force_forward(q, k, v, causal=False, scale=None, keep=None, dropout_p=0.0, bias=None):
    """Scalar-loop forward in Python floats for tiny shapes: an implementation
    that shares no code with :func:`attention_forward` (used to pin it)."""
    B, Sq, H, D = q.shape
    Hkv = k.shape[2]
    Sk = k.shape[1]
    if scale is None:
        scale = D ** -0.5
    qf, kf, vf = q.double().tolist(), k.double().tolist(), v.double().tolist()
    bf = None if bias is None else bias.double().tolist()
    o = [[[[0.0] * D for _ in range(H)] for _ in range(Sq)] for _ in range(B)]
    lse = [[[float("-inf")] * Sq for _ in range(H)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            hk = h // (H // Hkv)
            for i in range(Sq):
                js = [j for j in range(Sk) if not (causal and j > i)]
                if not js:
                    continue
                sc = {j: scale * sum(qf[b][i][h][d] * kf[b][j][hk][d] for d in range(D)) for j in js}
                if bf is not None:
                    bb, bh = (b if len(bf) > 1 else 0), (h if len(bf[0]) > 1 else 0)
                    bi = i if len(bf[bb][bh]) > 1 else 0
                    sc = {j: x + bf[bb][bh][bi][j] for j, x in sc.items()}
                m = max(sc.values())
                if m == float("-inf"):  # no visible key: O = 0, LSE = -inf
                    continue
                tot = sum(math.exp(x - m) for x in sc.values())
                lse[b][h][i] = m + math.log(tot)
                for j in js:
                    w = math.exp(sc[j] - m) / tot
                    if dropout_p > 0.0:
                        w = w * (1.0 / (1.0 - dropout_p) if keep[b][h][i][j] else 0.0)
                    for d in range(D):
                        o[b][i][h][d] += w * vf[b][j][hk][d]
    return torch.tensor(o, dtype=torch.float64), torch.tensor(lse, dtype=torch.float64)
