"""Online-softmax mergers of ring partial results (interface of fa4_ring/merge.py).

``merge_state_in_place`` and ``merge_states`` keep the names and argument meaning of the
flashinfer.cascade functions the reference calls (fa4_ring/merge.py:31-42) and run the
HBM-bound HIP kernels of libfa4cp.so.  LSEs are float32 natural log on both sides.

``IncrementalMerger`` / ``BatchedMerger`` / ``make_merger`` keep the reference classes'
interface (fa4_ring/merge.py:45-94): ``add(out, lse)`` per ring step, ``result()`` at the
end.  The incremental merger copies its first partial and merges every later one into that
copy in place; the batched one merges its partials through a pointer list
(``merge_states_list``) instead of stacking them.  The first partial added must cover
every row with a finite LSE (step 0 of the ring); a -inf row of a later partial is the
identity, and a row that is -inf in both gets NaN, as the reference's formula does.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import SEL_ALL


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def _check_pair(v: torch.Tensor, s: torch.Tensor, v_other: torch.Tensor, s_other: torch.Tensor,
                what: str) -> None:
    """Two states of one shape: v [T, H, D] bf16 / fp16 / fp32, s [T, H] float32, contiguous,
    on one device, v 16-byte aligned."""
    _require(v.is_cuda, f"{what} runs on the GPU: v must be a device tensor")
    _require(v.dim() == 3 and v_other.shape == v.shape, "v and v_other must be [T, H, D] alike")
    _require(v.dtype == v_other.dtype, "v and v_other must share a dtype")
    t, h, _ = v.shape
    _require(s.shape == (t, h) and s_other.shape == (t, h), "s and s_other must be [T, H]")
    _require(s.dtype == torch.float32 and s_other.dtype == torch.float32, "LSEs must be float32")
    for name, x in (("v", v), ("s", s), ("v_other", v_other), ("s_other", s_other)):
        _require(x.is_contiguous(), f"{name} must be contiguous")
        _require(x.device == v.device, f"{name} must be on {v.device}")
        _require(x.data_ptr() % 16 == 0 or name in ("s", "s_other"), f"{name} must be 16-byte aligned")


def merge_state_in_place(v: torch.Tensor, s: torch.Tensor, v_other: torch.Tensor,
                         s_other: torch.Tensor, *, cu_seqlens: Optional[torch.Tensor] = None,
                         row_sel: int = SEL_ALL) -> None:
    """(v, s) <- merge((v, s), (v_other, s_other)), in place.

    v, v_other: [T, H, D] contiguous bf16 / fp16 / fp32 (same type); s, s_other: [T, H]
    contiguous float32.  ``row_sel`` (SEL_BACK_HALF / SEL_FRONT_HALF) restricts the merge
    to that half of every sequence of ``cu_seqlens`` (one sequence of T rows if None)."""
    lib = _lib.load()
    _check_pair(v, s, v_other, s_other, "merge_state_in_place")
    t, h, d = v.shape
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


def merge_state(v: torch.Tensor, s: torch.Tensor, v_other: torch.Tensor, s_other: torch.Tensor,
                out: Optional[torch.Tensor] = None,
                s_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """merge((v, s), (v_other, s_other)) into new tensors (or ``out`` / ``s_out``); the
    inputs are not modified.  Same shapes and types as merge_state_in_place."""
    lib = _lib.load()
    _check_pair(v, s, v_other, s_other, "merge_state")
    t, h, d = v.shape
    if out is None:
        out = torch.empty_like(v)
    if s_out is None:
        s_out = torch.empty_like(s)
    _require(out.shape == v.shape and out.dtype == v.dtype and out.is_contiguous() and out.device == v.device,
             f"out must be a contiguous [{t}, {h}, {d}] {v.dtype} tensor on {v.device}")
    _require(s_out.shape == s.shape and s_out.dtype == torch.float32 and s_out.is_contiguous()
             and s_out.device == v.device, f"s_out must be a contiguous [{t}, {h}] float32 tensor on {v.device}")
    rc = lib.fa4cp_merge_state(v.data_ptr(), s.data_ptr(), v_other.data_ptr(), s_other.data_ptr(),
                               out.data_ptr(), s_out.data_ptr(), t, h, d, _lib.dtype_code(v.dtype), None, 0,
                               SEL_ALL, _lib.stream_handle(v.device))
    _lib.check(rc, "fa4cp_merge_state")
    return out, s_out


def merge_states_list(vs: Sequence[torch.Tensor], ss: Sequence[torch.Tensor],
                      out: Optional[torch.Tensor] = None,
                      s_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """merge_states over states kept in separate tensors: vs[i] [T, H, D], ss[i] [T, H]
    float32 -> (v [T, H, D], s [T, H]).  Equal to merge_states(torch.stack(vs, 1),
    torch.stack(ss, 1)) without building the stack; more than FA4CP_MAX_CP states are
    merged in groups."""
    lib = _lib.load()
    _require(len(vs) == len(ss) and len(vs) >= 1, "merge_states_list needs as many LSEs as states, at least one")
    for v, s in zip(vs, ss):
        _check_pair(vs[0], ss[0], v, s, "merge_states_list")
    t, h, d = vs[0].shape
    dev = vs[0].device
    if out is None:
        out = torch.empty_like(vs[0])
    if s_out is None:
        s_out = torch.empty_like(ss[0])
    _require(out.shape == vs[0].shape and out.dtype == vs[0].dtype and out.is_contiguous() and out.device == dev,
             f"out must be a contiguous [{t}, {h}, {d}] {vs[0].dtype} tensor on {dev}")
    _require(s_out.shape == (t, h) and s_out.dtype == torch.float32 and s_out.is_contiguous() and s_out.device == dev,
             f"s_out must be a contiguous [{t}, {h}] float32 tensor on {dev}")
    vs, ss = list(vs), list(ss)
    while len(vs) > _lib.MAX_CP:
        # fold the first group into one state; the LSE merge is associative
        v1, s1 = merge_states_list(vs[:_lib.MAX_CP], ss[:_lib.MAX_CP])
        vs = [v1] + vs[_lib.MAX_CP:]
        ss = [s1] + ss[_lib.MAX_CP:]
    n = len(vs)
    vp = (ctypes.c_void_p * n)(*[v.data_ptr() for v in vs])
    sp = (ctypes.c_void_p * n)(*[s.data_ptr() for s in ss])
    rc = lib.fa4cp_merge_states_list(vp, sp, n, out.data_ptr(), s_out.data_ptr(), t, h, d,
                                     _lib.dtype_code(vs[0].dtype), _lib.stream_handle(dev))
    _lib.check(rc, "fa4cp_merge_states_list")
    return out, s_out


class IncrementalMerger:
    """Folds ring partials into one (out, lse) state as they arrive (fa4_ring/merge.py:45-64).

    The first partial is copied into buffers the merger owns (as the reference's clone at the
    first add, fa4_ring/merge.py:53-57), so a caller may write the next step into the same
    buffer before the next add.  Every later partial is merged into those buffers in place
    (merge_state_in_place); the caller's tensors are never written.  The first partial must
    give every row a finite LSE (ring step 0); a -inf row of a later partial leaves the row
    unchanged."""

    def __init__(self):
        self.out: Optional[torch.Tensor] = None  # [T, H, D]
        self.lse: Optional[torch.Tensor] = None  # [T, H] float32
        self.count = 0

    def add(self, out: torch.Tensor, lse: torch.Tensor) -> None:
        if self.out is None:
            self.out, self.lse = out.clone(), lse.clone()
        else:
            merge_state_in_place(self.out, self.lse, out, lse)
        self.count += 1

    def result(self) -> torch.Tensor:
        assert self.count > 0, "result() called before any partial was added"
        return self.out


class BatchedMerger:
    """Collects every ring partial and merges them in one launch at the end
    (fa4_ring/merge.py:67-86).  The partials stay where the caller produced them: the merge
    reads them through a list of pointers (merge_states_list), so nothing is stacked."""

    def __init__(self):
        self.outs: List[torch.Tensor] = []
        self.lses: List[torch.Tensor] = []

    def add(self, out: torch.Tensor, lse: torch.Tensor) -> None:
        self.outs.append(out)
        self.lses.append(lse)

    def result_with_lse(self) -> Tuple[torch.Tensor, torch.Tensor]:
        assert self.outs, "result() called before any partial was added"
        if len(self.outs) == 1:
            return self.outs[0], self.lses[0]
        return merge_states_list(self.outs, self.lses)

    def result(self) -> torch.Tensor:
        return self.result_with_lse()[0]


_MERGERS = {"incremental": IncrementalMerger, "batched": BatchedMerger}


def make_merger(merge_mode: str):
    """The merger a RingConfig.merge_mode names (fa4_ring/merge.py:89-94)."""
    try:
        return _MERGERS[merge_mode]()
    except KeyError:
        raise ValueError(f"unknown merge_mode {merge_mode!r}; expected one of {sorted(_MERGERS)}") from None
