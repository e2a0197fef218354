"""Online-softmax mergers of ring partial results (interface of fa4_ring/merge.py).

``merge_state_in_place`` and ``merge_states`` keep the names and argument meaning of the
flashinfer.cascade functions the reference calls (fa4_ring/merge.py:31-42) and run the
HBM-bound HIP kernels of libfa4cp.so.  LSEs are float32 natural log on both sides.

``IncrementalMerger`` / ``BatchedMerger`` / ``make_merger`` keep the reference classes'
behaviour (fa4_ring/merge.py:45-94): the first partial added must cover every row with a
finite LSE (step 0 of the ring); a -inf row of a later partial is the identity.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import _lib
from ._lib import SEL_ALL


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def merge_state_in_place(v: torch.Tensor, s: torch.Tensor, v_other: torch.Tensor,
                         s_other: torch.Tensor, *, cu_seqlens: Optional[torch.Tensor] = None,
                         row_sel: int = SEL_ALL) -> None:
    """(v, s) <- merge((v, s), (v_other, s_other)), in place.

    v, v_other: [T, H, D] contiguous bf16 / fp16 / fp32 (same type); s, s_other: [T, H]
    contiguous float32.  ``row_sel`` (SEL_BACK_HALF / SEL_FRONT_HALF) restricts the merge
    to that half of every sequence of ``cu_seqlens`` (one sequence of T rows if None)."""
    lib = _lib.load()
    _require(v.is_cuda, "merge_state_in_place runs on the GPU: v must be a device tensor")
    _require(v.dim() == 3 and v_other.shape == v.shape, "v and v_other must be [T, H, D] alike")
    _require(v.dtype == v_other.dtype, "v and v_other must share a dtype")
    t, h, d = v.shape
    _require(s.shape == (t, h) and s_other.shape == (t, h), "s and s_other must be [T, H]")
    _require(s.dtype == torch.float32 and s_other.dtype == torch.float32, "LSEs must be float32")
    for name, x in (("v", v), ("s", s), ("v_other", v_other), ("s_other", s_other)):
        _require(x.is_contiguous(), f"{name} must be contiguous")
        _require(x.device == v.device, f"{name} must be on {v.device}")
        _require(x.data_ptr() % 16 == 0 or name in ("s", "s_other"), f"{name} must be 16-byte aligned")
    nseq = 0
    if cu_seqlens is not None:
        _require(cu_seqlens.dtype == torch.int32 and cu_seqlens.device == v.device,
                 "cu_seqlens must be int32 on the device")
        nseq = cu_seqlens.shape[0] - 1
    rc = lib.fa4cp_merge_state_inplace(
        v.data_ptr(), s.data_ptr(), v_other.data_ptr(), s_other.data_ptr(), t, h, d,
        _lib.dtype_code(v.dtype), _lib.ptr(cu_seqlens), nseq, int(row_sel),
        _lib.stream_handle(v.device))
    _lib.check(rc, "fa4cp_merge_state_inplace")


def merge_states(v: torch.Tensor, s: torch.Tensor,
                 out: Optional[torch.Tensor] = None,
                 s_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Merges v [T, S, H, D] / s [T, S, H] over S -> (v [T, H, D], s [T, H] float32)."""
    lib = _lib.load()
    _require(v.is_cuda, "merge_states runs on the GPU: v must be a device tensor")
    _require(v.dim() == 4, "v must be [T, num_states, H, D]")
    t, ns, h, d = v.shape
    _require(s.shape == (t, ns, h) and s.dtype == torch.float32, "s must be [T, num_states, H] float32")
    _require(v.is_contiguous() and s.is_contiguous(), "v and s must be contiguous")
    _require(s.device == v.device, "v and s must share a device")
    if out is None:
        out = torch.empty((t, h, d), dtype=v.dtype, device=v.device)
    if s_out is None:
        s_out = torch.empty((t, h), dtype=torch.float32, device=v.device)
    _require(out.shape == (t, h, d) and out.dtype == v.dtype and out.is_contiguous() and out.device == v.device,
             f"out must be a contiguous [{t}, {h}, {d}] {v.dtype} tensor on {v.device}")
    _require(s_out.shape == (t, h) and s_out.dtype == torch.float32 and s_out.is_contiguous()
             and s_out.device == v.device, f"s_out must be a contiguous [{t}, {h}] float32 tensor on {v.device}")
    rc = lib.fa4cp_merge_states(v.data_ptr(), s.data_ptr(), out.data_ptr(), s_out.data_ptr(), t, ns,
                                h, d, _lib.dtype_code(v.dtype), _lib.stream_handle(v.device))
    _lib.check(rc, "fa4cp_merge_states")
    return out, s_out


class IncrementalMerger:
    """Accumulates (out, lse) in place, one ring step at a time."""

    def __init__(self):
        self.out: Optional[torch.Tensor] = None  # [T, H, D]
        self.lse: Optional[torch.Tensor] = None  # [T, H]

    def add(self, out: torch.Tensor, lse: torch.Tensor) -> None:
        if self.out is None:
            # the first partial seeds the accumulator; copies keep the caller's tensors intact
            self.out = out.clone()
            self.lse = lse.clone()
        else:
            merge_state_in_place(self.out, self.lse, out, lse)

    def result(self) -> torch.Tensor:
        assert self.out is not None, "no partials were added"
        return self.out


class BatchedMerger:
    """Keeps every step's (out, lse) and merges them all at the end."""

    def __init__(self):
        self.outs: List[torch.Tensor] = []
        self.lses: List[torch.Tensor] = []

    def add(self, out: torch.Tensor, lse: torch.Tensor) -> None:
        self.outs.append(out)
        self.lses.append(lse)

    def result(self) -> torch.Tensor:
        assert self.outs, "no partials were added"
        if len(self.outs) == 1:
            return self.outs[0]
        v = torch.stack(self.outs, dim=1).contiguous()
        s = torch.stack(self.lses, dim=1).contiguous()
        out, _ = merge_states(v, s)
        return out


def make_merger(merge_mode: str):
    if merge_mode == "incremental":
        return IncrementalMerger()
    if merge_mode == "batched":
        return BatchedMerger()
    raise ValueError(f"unknown merge_mode {merge_mode!r}")
