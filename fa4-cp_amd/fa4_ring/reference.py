"""Dense causal attention over a whole (unsharded) sequence, for checking ring outputs
(role of fa4_ring/reference.py:30-54).

``full_causal_reference(q, k, v, softmax_scale=None, backend="torch")`` returns
``[N, H_q, D]`` in q's dtype:
  * ``"torch"``: float32 math on q's device.  Queries go in blocks, each block against
    only its causal key prefix, and the query heads that share a kv head are stacked
    into one matrix product with that head's K / V (grouped-query attention without
    replicating K or V).  Memory stays bounded for long sequences.
  * ``"fa4"`` / ``"hip"``: this library's causal attention kernel over the whole
    sequence (one fa4_attn call), for a kernel-against-kernel comparison.
"""

import math
from typing import Optional

import torch

# scores of one block (query rows x heads x keys, float32) are kept under this many bytes
_BLOCK_BYTES = 256 << 20


def _dense_causal_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    group = h_q // h_kv
    out = torch.empty(n, h_q, v.shape[2], dtype=torch.float32, device=q.device)
    if n == 0:
        return out
    # kv-major operands: [H_kv, N, D] for K and V, [H_kv, G * rows, D] for a query block
    kt = k.float().permute(1, 2, 0).contiguous()  # [H_kv, D, N]
    vh = v.float().permute(1, 0, 2).contiguous()  # [H_kv, N, Dv]
    qg = q.float().view(n, h_kv, group, d)
    rows = max(1, min(n, _BLOCK_BYTES // max(1, 4 * h_q * n)))
    for r0 in range(0, n, rows):
        r1 = min(n, r0 + rows)
        b = r1 - r0
        qb = qg[r0:r1].permute(1, 2, 0, 3).reshape(h_kv, group * b, d)
        sc = torch.matmul(qb, kt[:, :, :r1]) * scale  # [H_kv, G * b, r1]
        qpos = (r0 + torch.arange(b, device=q.device)).repeat(group)  # row of each stacked query
        hidden = torch.arange(r1, device=q.device).unsqueeze(0) > qpos.unsqueeze(1)
        sc.masked_fill_(hidden.unsqueeze(0), float("-inf"))
        o = torch.matmul(torch.softmax(sc, dim=-1), vh[:, :r1])  # [H_kv, G * b, Dv]
        out[r0:r1] = o.view(h_kv, group, b, -1).permute(2, 0, 1, 3).reshape(b, h_q, -1)
    return out


def full_causal_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          softmax_scale: Optional[float] = None, backend: str = "torch") -> torch.Tensor:
    """Causal attention of q [N, H_q, D] over k / v [N, H_kv, D]; query head j reads kv head
    j // (H_q / H_kv)."""
    n, h_q, d = q.shape
    if k.shape[0] != n or v.shape[0] != n or k.shape[1] != v.shape[1]:
        raise AssertionError(f"q, k, v must cover one sequence: q {tuple(q.shape)}, k {tuple(k.shape)}, "
                             f"v {tuple(v.shape)}")
    if h_q % k.shape[1]:
        raise AssertionError(f"{h_q} query heads cannot share {k.shape[1]} kv heads evenly")
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else float(softmax_scale)
    if backend in ("fa4", "hip"):
        from .fa4_backend import fa4_attn

        return fa4_attn(q, k, v, causal=True, softmax_scale=scale)[0]
    if backend != "torch":
        raise ValueError(f"unknown backend {backend!r}: use 'torch' or 'hip'")
    return _dense_causal_fp32(q, k, v, scale).to(q.dtype)
