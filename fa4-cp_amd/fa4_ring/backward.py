"""Backward of one rank's causal zig-zag ring sweep (the training side of ring_flash_attn).

The reference is forward-only (README.md: "forward only").  This is the gradient of the same
computation on one GPU, every source rank's K / V resident in HBM (LocalKVRing):

  * ``ring_flash_attn_backward(dout, local_q, local_k, local_v, out, lse, cfg, group=...)``
    returns (dq, dk, dv): dq [T, H, D] float32 for the local q, and per source rank i the
    float32 [T, H_kv, D] contributions dk[i] / dv[i] of this rank's queries to source i's K /
    V gradient (zero for keys this rank does not attend).  A ring's backward sends each to
    its owner and sums them there; ``accumulate=True`` adds into caller buffers for that.
  * ``ring_flash_attn_func(local_q, ring, cfg, ...)``: ring_flash_attn as a differentiable
    function of local_q and of every shard in ``ring`` (torch.autograd), gradients in the
    input dtype.

Both run fa4cp_ring_sweep_bwd: the probabilities come from the forward's final natural-log
LSE, so every step's pairs contribute independently (no merge in reverse).  bf16 / fp16
with head dim 64, 128 or 256.
"""

from __future__ import annotations

import ctypes
import math
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from .config import RingConfig
from .ring_attention import LocalKVRing, _check_even_lengths, ring_flash_attn


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def ring_flash_attn_backward(dout: torch.Tensor, local_q: torch.Tensor, local_k: torch.Tensor,
                             local_v: torch.Tensor, out: torch.Tensor, lse: torch.Tensor, cfg: RingConfig, *,
                             group: Optional[LocalKVRing] = None, cu_seqlens: Optional[torch.Tensor] = None,
                             max_seqlen: Optional[int] = None, dq: Optional[torch.Tensor] = None,
                             dk: Optional[Sequence[torch.Tensor]] = None, dv: Optional[Sequence[torch.Tensor]] = None,
                             accumulate: bool = False
                             ) -> Tuple[torch.Tensor, List[torch.Tensor], List[torch.Tensor]]:
    """Gradients of ring_flash_attn's out (given its ``out`` and ``lse``, from
    ``return_lse=True``) for one rank: (dq, dk per source rank, dv per source rank), float32.
    ``dq`` / ``dk`` / ``dv`` may be given (float32, contiguous); with ``accumulate`` the
    gradients are added to them."""
    lib = _lib.load()
    S, rank = cfg.cp_size, cfg.cp_rank
    total, h_q, d = local_q.shape
    dev = local_q.device
    _require(local_q.is_cuda, "ring_flash_attn_backward runs on the GPU: local_q must be a device tensor")
    _require(local_q.dtype in (torch.bfloat16, torch.float16), "backward takes bf16 / fp16 inputs")
    _require(d in (64, 128, 256), f"backward head dim must be 64, 128 or 256, got {d}")
    if S > 1:
        _require(isinstance(group, LocalKVRing) and group.cp_size == S,
                 "cp_size > 1 needs group=LocalKVRing holding every source rank's K / V")
        ks = [local_k if i == rank else group.k[i] for i in range(S)]
        vs = [local_v if i == rank else group.v[i] for i in range(S)]
    else:
        ks, vs = [local_k], [local_v]
    _require(S <= _lib.MAX_CP, f"cp_size {S} above {_lib.MAX_CP}")
    if cu_seqlens is not None:
        _require(max_seqlen is not None, "max_seqlen required when cu_seqlens is given")
        _require(cu_seqlens.dtype == torch.int32 and cu_seqlens.device == dev and cu_seqlens.is_contiguous(),
                 "cu_seqlens must be contiguous int32 on the device")
    _check_even_lengths(cu_seqlens, total, max_seqlen)
    h_kv = ks[0].shape[1]
    _require(h_q % h_kv == 0, f"{h_q} query heads cannot share {h_kv} kv heads evenly")
    for name, x in (("dout", dout), ("out", out)):
        _require(x.shape == local_q.shape and x.dtype == local_q.dtype and x.device == dev and x.stride(2) == 1,
                 f"{name} must be like local_q: [{total}, {h_q}, {d}] {local_q.dtype}, contiguous in D")
    _require(lse.shape == (total, h_q) and lse.dtype == torch.float32 and lse.device == dev and lse.stride(1) == 1,
             f"lse must be [{total}, {h_q}] float32 with unit head stride")
    _require(local_q.stride(2) == 1, "local_q must be contiguous in D")
    for i, (k, v) in enumerate(zip(ks, vs)):
        _require(k.shape == (total, h_kv, d) and v.shape == k.shape and k.dtype == local_q.dtype
                 and k.device == dev and v.device == dev, f"source {i}'s K / V must be [{total}, {h_kv}, {d}]")
        _require(k.stride() == ks[0].stride() and v.stride() == vs[0].stride() and k.stride(2) == 1
                 and v.stride(2) == 1, "K / V shards must share strides and be contiguous in D")

    def buf(x, shape, what):
        if x is None:
            return (torch.zeros if accumulate else torch.empty)(shape, dtype=torch.float32, device=dev)
        _require(x.shape == shape and x.dtype == torch.float32 and x.is_contiguous() and x.device == dev,
                 f"{what} must be a contiguous float32 tensor of shape {tuple(shape)} on {dev}")
        return x

    dq = buf(dq, (total, h_q, d), "dq")
    dk = [buf(None if dk is None else dk[i], (total, h_kv, d), f"dk[{i}]") for i in range(S)]
    dv = [buf(None if dv is None else dv[i], (total, h_kv, d), f"dv[{i}]") for i in range(S)]
    a = _lib.SweepBwdArgs()
    a.q, a.dout, a.out, a.lse, a.dq = (local_q.data_ptr(), dout.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                       dq.data_ptr())
    a.q_row_stride, a.q_head_stride = local_q.stride(0), local_q.stride(1)
    a.do_row_stride, a.do_head_stride = dout.stride(0), dout.stride(1)
    a.o_row_stride, a.o_head_stride = out.stride(0), out.stride(1)
    a.lse_row_stride = lse.stride(0)
    for i in range(S):
        a.k[i], a.v[i], a.dk[i], a.dv[i] = ks[i].data_ptr(), vs[i].data_ptr(), dk[i].data_ptr(), dv[i].data_ptr()
    a.k_row_stride, a.k_head_stride = ks[0].stride(0), ks[0].stride(1)
    a.v_row_stride, a.v_head_stride = vs[0].stride(0), vs[0].stride(1)
    a.cu = _lib.ptr(cu_seqlens)
    a.nseq = 1 if cu_seqlens is None else cu_seqlens.shape[0] - 1
    a.max_seqlen = int(max_seqlen) if cu_seqlens is not None else total
    a.total = total
    a.h_q, a.h_kv, a.d = h_q, h_kv, d
    a.dtype = _lib.dtype_code(local_q.dtype)
    a.cp_rank, a.cp_size = rank, S
    a.softmax_scale = float(cfg.softmax_scale if cfg.softmax_scale is not None else 1.0 / math.sqrt(d))
    a.accumulate = 1 if accumulate else 0
    ws_bytes = lib.fa4cp_ring_sweep_bwd_workspace_bytes(ctypes.byref(a))
    _lib.check(int(min(ws_bytes, 0)), "fa4cp_ring_sweep_bwd_workspace_bytes")
    # delta and the packed q / dout blocks (caching allocator blocks are 512-byte aligned)
    ws = torch.empty((max(int(ws_bytes), 1),), dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
    _lib.check(lib.fa4cp_ring_sweep_bwd(ctypes.byref(a), _lib.stream_handle(dev)), "fa4cp_ring_sweep_bwd")
    return dq, dk, dv


class _RingAttention(torch.autograd.Function):
    """out = ring_flash_attn(q, ...) with the K / V shards of every source rank as inputs."""

    @staticmethod
    def forward(ctx, q, cfg, cu_seqlens, max_seqlen, *kv):
        S = cfg.cp_size
        ring = LocalKVRing(list(kv[:S]), list(kv[S:]))
        out, lse = ring_flash_attn(q, ring.k[cfg.cp_rank], ring.v[cfg.cp_rank], cfg, group=ring,
                                   cu_seqlens=cu_seqlens, max_seqlen=max_seqlen, return_lse=True)
        ctx.cfg, ctx.cu, ctx.max_seqlen = cfg, cu_seqlens, max_seqlen
        ctx.save_for_backward(q, out, lse, *kv)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, out, lse, *kv = ctx.saved_tensors
        cfg = ctx.cfg
        S = cfg.cp_size
        ring = LocalKVRing(kv[:S], kv[S:])
        dq, dk, dv = ring_flash_attn_backward(dout.contiguous(), q, ring.k[cfg.cp_rank], ring.v[cfg.cp_rank], out, lse,
                                              cfg, group=ring, cu_seqlens=ctx.cu, max_seqlen=ctx.max_seqlen)
        return (dq.to(q.dtype), None, None, None, *[g.to(q.dtype) for g in dk], *[g.to(q.dtype) for g in dv])


def ring_flash_attn_func(local_q: torch.Tensor, ring: LocalKVRing, cfg: RingConfig, *,
                         cu_seqlens: Optional[torch.Tensor] = None, max_seqlen: Optional[int] = None) -> torch.Tensor:
    """ring_flash_attn (fused sweep) that torch.autograd differentiates: gradients flow to
    ``local_q`` and to every K / V shard held by ``ring`` (this rank's contributions)."""
    return _RingAttention.apply(local_q, cfg, cu_seqlens, max_seqlen, *ring.k, *ring.v)
