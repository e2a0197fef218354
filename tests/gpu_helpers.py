"""Shared helpers for the GPU parity tests (inputs, oracle glue, tolerances)."""

import math
import sys

import torch

from oracle import ring_oracle as O

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None

# tolerances (max-abs), from the parity bar of the path
TOL_BF16_OUT = 2e-2
TOL_LSE = 1e-3
TOL_FP8_OUT = 5e-2
TOL_MERGE_FP32 = 1e-5


def say(msg: str) -> None:
    """Names the case before GPU work so a crash log still shows it."""
    print(msg, flush=True)
    sys.stdout.flush()


def rounded(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """x rounded to dtype and widened back to fp32 (the oracle's view of device inputs)."""
    return x.to(dtype).float()


def seq_bounds(cu, total, sel):
    """Row ranges of every sequence after a half selection (0 all, 1 front, 2 back)."""
    if cu is None:
        cu = [0, total]
    out = []
    for j in range(len(cu) - 1):
        s, e = int(cu[j]), int(cu[j + 1])
        mid = (s + e) // 2
        if sel == 1:
            e = mid
        elif sel == 2:
            s = mid
        out.append((s, e))
    return out


def oracle_attn(q, k, v, causal, scale, cu_q=None, cu_k=None, q_sel=0, k_sel=0):
    """Oracle attention (O.cpu_attn per sequence) over the same packed layout and selections
    as the kernel: rows not selected are NaN (out) / NaN (lse).  Causal is bottom-right
    aligned per sequence."""
    tq, h, d = q.shape
    out = torch.full((tq, h, v.shape[2]), float("nan"))
    lse = torch.full((tq, h), float("nan"))
    qb = seq_bounds(cu_q, tq, q_sel)
    kb = seq_bounds(cu_k, k.shape[0], k_sel)
    for (qs, qe), (ks, ke) in zip(qb, kb):
        lq, lk = qe - qs, ke - ks
        if lq == 0:
            continue
        if lk == 0:
            out[qs:qe] = 0
            lse[qs:qe] = float("-inf")
            continue
        o, l = O.cpu_attn(q[qs:qe], k[ks:ke], v[ks:ke], causal=causal, scale=scale)
        out[qs:qe] = o
        lse[qs:qe] = l
    return out, lse


def max_err(a: torch.Tensor, b: torch.Tensor, mask=None) -> float:
    d = (a.float().cpu() - b.float().cpu()).abs()
    if mask is not None:
        d = d[mask]
    d = torch.nan_to_num(d, nan=float("inf"))
    return float(d.max()) if d.numel() else 0.0


def lse_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a - b| over rows, treating matching -inf as equal."""
    a = a.float().cpu()
    b = b.float().cpu()
    both_inf = torch.isinf(a) & torch.isinf(b) & (a.sign() == b.sign())
    d = (a - b).abs()
    d[both_inf] = 0
    d = torch.nan_to_num(d, nan=float("inf"))
    return float(d.max()) if d.numel() else 0.0


def scale_for(d: int) -> float:
    return 1.0 / math.sqrt(d)
