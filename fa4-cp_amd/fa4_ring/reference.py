"""Dense single-GPU references for validating ring outputs (interface of
fa4_ring/reference.py:20-54).

``full_causal_reference`` is ordinary causal attention over the whole sequence:
  * backend "torch": scaled_dot_product_attention in float32 (GQA expanded), runs anywhere;
  * backend "fa4" (alias "hip"): the same gfx950 HIP kernel the ring uses, causal over the
    whole sequence, for an apples-to-apples comparison.
"""

import math
from typing import Optional

import torch
import torch.nn.functional as F


def _expand_kv(k: torch.Tensor, v: torch.Tensor, n_q_heads: int):
    """[T, H_kv, D] -> [T, H_q, D]: query head j reads kv head j // (H_q / H_kv)."""
    h_kv = k.shape[1]
    if h_kv == n_q_heads:
        return k, v
    assert n_q_heads % h_kv == 0, f"H_q={n_q_heads} not a multiple of H_kv={h_kv}"
    rep = n_q_heads // h_kv
    return k.repeat_interleave(rep, dim=1), v.repeat_interleave(rep, dim=1)


def full_causal_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          softmax_scale: Optional[float] = None, backend: str = "torch") -> torch.Tensor:
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    if backend in ("fa4", "hip"):
        from .fa4_backend import fa4_attn

        out, _ = fa4_attn(q, k, v, causal=True, softmax_scale=softmax_scale)
        return out
    if backend != "torch":
        raise ValueError(f"unknown backend {backend!r}")
    kq, vq = _expand_kv(k, v, q.shape[1])
    qt = q.transpose(0, 1).unsqueeze(0).float()
    kt = kq.transpose(0, 1).unsqueeze(0).float().contiguous()
    vt = vq.transpose(0, 1).unsqueeze(0).float().contiguous()
    out = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=softmax_scale)
    return out.squeeze(0).transpose(0, 1).contiguous().to(q.dtype)
