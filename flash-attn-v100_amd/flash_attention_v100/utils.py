"""NaN / Inf scans behind the debug switches of :mod:`.config` (reference
``utils.py:219-254, 686-720``).  Each scan counts on the GPU and brings the
counts to the host in one transfer (one synchronisation per tensor)."""
from __future__ import annotations

import warnings

import torch


def _counts(tensor: torch.Tensor, allow_neg_inf: bool = False):
    t = tensor.detach()
    bad_inf = torch.isposinf(t) if allow_neg_inf else torch.isinf(t)
    nan, inf = torch.stack([torch.isnan(t).sum(), bad_inf.sum()]).tolist()
    return int(nan), int(inf)


def check_tensor_nan_inf(tensor: torch.Tensor, name: str = "tensor", fix_issues: bool = False,
                         allow_neg_inf: bool = False) -> torch.Tensor:
    """Raise ``ValueError("<name> contains <n> NaN values and <m> Inf values")``
    when the tensor holds NaN or Inf (reference ``utils.py:686-720``); with
    ``fix_issues`` warn instead and return a copy with NaN replaced by 0 and
    Inf clamped to half the dtype's largest finite value.  ``allow_neg_inf``
    accepts ``-inf`` (a log-sum-exp of a row without visible keys)."""
    if tensor is None or not tensor.is_floating_point() or tensor.numel() == 0:
        return tensor
    nan, inf = _counts(tensor, allow_neg_inf)
    if nan == 0 and inf == 0:
        return tensor
    issues = []
    if nan:
        issues.append(f"{nan} NaN values")
    if inf:
        issues.append(f"{inf} Inf values")
    msg = f"{name} contains {' and '.join(issues)}"
    if not fix_issues:
        raise ValueError(msg)
    warnings.warn(f"{msg}. Attempting to fix...", UserWarning)
    out = torch.nan_to_num(tensor, nan=0.0, posinf=torch.finfo(tensor.dtype).max / 2,
                           neginf=None if allow_neg_inf else -torch.finfo(tensor.dtype).max / 2)
    return out


def check_numerical_stability(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bias=None) -> None:
    """The reference's input scan (``utils.py:219-254``): ``ValueError`` for
    NaN / Inf in q, k, v or the bias, a warning for magnitudes above 1e4 and,
    for 16-bit inputs, for non-zero magnitudes below 1e-7."""
    named = [("query", q), ("key", k), ("value", v)] + ([("bias", bias)] if bias is not None else [])
    for name, t in named:
        if t.numel() == 0:
            continue
        x = t.detach()
        a = torch.nan_to_num(x.abs().float(), nan=0.0, posinf=0.0)
        # smallest non-zero magnitude without a boolean gather (one sync in all)
        nzmin = torch.where(a != 0, a, torch.full_like(a, float("inf"))).min()
        stats = torch.stack([torch.isnan(x).sum().float(), torch.isinf(x).sum().float(), a.max(),
                             torch.where(torch.isinf(nzmin), torch.ones_like(nzmin), nzmin)]).tolist()
        if stats[0]:
            raise ValueError(f"{name} tensor contains NaN values")
        if stats[1]:
            raise ValueError(f"{name} tensor contains Inf values")
        if stats[2] > 1e4:
            warnings.warn(f"{name} tensor has very large values (max: {stats[2]:.2e}). "
                          "This may cause numerical instability.", UserWarning)
        if t.dtype in (torch.float16, torch.bfloat16) and stats[3] < 1e-7:
            warnings.warn(f"{name} tensor has very small values (min: {stats[3]:.2e}) with dtype {t.dtype}. "
                          "Consider using float32 for better numerical stability.", UserWarning)
