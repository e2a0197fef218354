"""Causal zig-zag ring attention for one rank (interface of fa4_ring/ring_attention.py:43-174).

A rank holds its local zig-zag shard ``[first_half (early) | second_half (late)]`` of Q, K
and V and walks ``cp_size`` steps; at step ``s`` it attends to the KV of source rank
``src = (rank - s) % cp_size``:

  * step 0 (src == rank):  causal attention over the local 2h tokens;
  * step s <= rank:        the source's KV is earlier, so all local Q attend only the
                           source's front (early) half;
  * step s > rank:         the source's KV is later, so only the local back (late) half of
                           Q attends, to all of it.

Each step's (out, LSE) partial is merged with the online-softmax merge, incrementally or
all at once at the end.

On MI355X the multi-GPU KV rotation (NCCL point-to-point in the reference) is replaced by
``LocalKVRing``: one GPU holds every source rank's KV shard in HBM and the sweep indexes
them by source rank.  Step ``s`` uses source ``(rank - s) % cp_size`` with that source's
descales, as the reference's CPU algorithm does (tests/test_algorithm_cpu.py:75-88).

No host synchronisation happens inside the sweep: the half selections are done inside the
attention kernel (no index_select gathers, no zero / -inf padding of the late-Q partial),
and every launch goes to torch's current stream.
"""

from __future__ import annotations

import ctypes
import dataclasses
import math
import weakref
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from .config import RingConfig
from .fa4_backend import (SEL_ALL, SEL_BACK_HALF, SEL_FRONT_HALF, SUPPORTED_HEAD_DIMS, fa4_attn, kernel_head_dim,
                          out_dtype_for, pad_head_dim, sweep_descales, transpose_v, transpose_v_many, uses_vt)
from .merge import merge_state_in_place, merge_states
from .paged import PagedKVRing, gather_kv_pages, transpose_v_paged_many
from .zigzag import zigzag_shard, zigzag_shard_varlen


@dataclass
class Descales:
    """FP8 descales.  ``k`` / ``v`` are indexed by the SOURCE rank whose KV is attended;
    each entry is a float32 scalar, [H_kv] or (1, H_kv) tensor."""

    q: Optional[torch.Tensor] = None
    k: Optional[List[torch.Tensor]] = None
    v: Optional[List[torch.Tensor]] = None


class LocalKVRing:
    """The ring's KV source on one GPU: the (k, v) zig-zag shard of every source rank,
    resident in HBM and indexed by rank.  Pass it as ``group=`` to ring_flash_attn."""

    def __init__(self, k_shards: Sequence[torch.Tensor], v_shards: Sequence[torch.Tensor]):
        assert len(k_shards) == len(v_shards) and len(k_shards) >= 1
        for k, v in zip(k_shards, v_shards):
            assert k.shape == v.shape == k_shards[0].shape, "every shard must have one shape"
            assert k.dtype == v.dtype == k_shards[0].dtype
            assert k.dim() == 3, "K and V shards must be [T, H_kv, D]"
        # the kernels read rows contiguous in D: shards laid out otherwise are copied once
        self.k = [k if k.stride(2) == 1 else k.contiguous() for k in k_shards]
        self.v = [v if v.stride(2) == 1 else v.contiguous() for v in v_shards]
        if len({x.stride() for x in self.k}) > 1 or len({x.stride() for x in self.v}) > 1:
            self.k = [x.contiguous() for x in self.k]
            self.v = [x.contiguous() for x in self.v]

    @property
    def cp_size(self) -> int:
        return len(self.k)

    def kv(self, src: int) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.k[src], self.v[src]

    @classmethod
    def from_full(cls, k: torch.Tensor, v: torch.Tensor, cp_size: int, full_cu_seqlens=None):
        """Shards full-sequence K and V for every rank with the zig-zag gather kernel."""
        if full_cu_seqlens is None:
            ks = [zigzag_shard(k, r, cp_size) for r in range(cp_size)]
            vs = [zigzag_shard(v, r, cp_size) for r in range(cp_size)]
        else:
            ks = [zigzag_shard_varlen(k, full_cu_seqlens, r, cp_size)[0] for r in range(cp_size)]
            vs = [zigzag_shard_varlen(v, full_cu_seqlens, r, cp_size)[0] for r in range(cp_size)]
        return cls(ks, vs)


_checked_cu = {}  # id(cu tensor) -> (weak reference, tensor version, longest sequence) of cu tables found even


def _check_even_lengths(cu_seqlens: Optional[torch.Tensor], total: int,
                        max_seqlen: Optional[int] = None) -> None:
    """Every local sequence is two zig-zag chunks of equal size, so its length must be even
    (the reference asserts it through get_half_index, fa4_ring/zigzag.py:75, on every call).
    The kernels split a sequence at (start + end) / 2 and the half-row merges at cu / 2,
    which agree only for even lengths.  ``max_seqlen``, when given, must cover the longest
    sequence: the kernels size their grids by it, and rows past it would be left unwritten.

    A device cu table is read once (one host synchronisation, which must therefore happen
    outside any graph capture: make one call with the table before capturing) and
    remembered until it is modified through torch or freed.  A table refilled by writes
    torch does not see (a raw pointer, a foreign kernel) is not checked again."""
    if cu_seqlens is None:
        if total % 2:
            raise AssertionError(f"the local sequence has odd length {total}: a zig-zag shard is two "
                                 "chunks of equal size")
        return
    key = id(cu_seqlens)
    seen = _checked_cu.get(key)
    if seen is not None and seen[0]() is cu_seqlens and seen[1] == cu_seqlens._version:
        longest = seen[2]
    else:
        cu = cu_seqlens.to("cpu", torch.int64)
        lens = cu[1:] - cu[:-1]
        odd = (lens % 2 != 0).nonzero().flatten().tolist()
        if odd:
            raise AssertionError(f"local sequences {odd[:8]} have odd length: a zig-zag shard is two chunks of "
                                 "equal size")
        longest = int(lens.max()) if lens.numel() else 0
        if len(_checked_cu) > 256:
            _checked_cu.clear()
        _checked_cu[key] = (weakref.ref(cu_seqlens), cu_seqlens._version, longest)
    if max_seqlen is not None and max_seqlen < longest:
        raise AssertionError(f"max_seqlen {max_seqlen} is below the longest local sequence ({longest})")


def ring_flash_attn(
    local_q: torch.Tensor,  # [T, H, D] zig-zag local shard (T = sum of 2*h_j)
    local_k: Optional[torch.Tensor],  # [T, H_kv, D] (None with a PagedKVRing)
    local_v: Optional[torch.Tensor],  # [T, H_kv, D] (None with a PagedKVRing)
    cfg: RingConfig,
    *,
    group=None,  # LocalKVRing or PagedKVRing holding every source rank's K/V
    descales: Optional[Descales] = None,
    cu_seqlens: Optional[torch.Tensor] = None,  # local int32 [num_seq+1]; None -> one sequence
    max_seqlen: Optional[int] = None,
    fused: Optional[bool] = None,
    return_lse: bool = False,
):
    """This rank's local causal ring-attention output ``[T, H, D]`` (with ``return_lse``:
    ``(out, lse)``, lse ``[T, H]`` float32, the natural-log LSE of every row over all the
    keys it attends).

    ``fused`` (default: whenever supported) runs the whole sweep as one kernel over every
    source's K / V^T (``ring_sweep``): no per-step partials, no merges.  It needs
    cp_size in [2, 16] with a LocalKVRing and either bf16 / fp16 with head dim 64, 128 or 256 and
    no descales, or e4m3 with head dim 128 or 256 (any descales); ``fused=False`` runs the
    per-step path of the reference (attention + LSE merge per step), which covers every
    case.  ``cfg.merge_mode`` chooses how the per-step path merges its partials
    (incremental: in place after every step; batched: one merge_states at the end).  The
    fused sweep has no partials to merge, so it runs for either mode; pass
    ``fused=False`` to get the merge the mode names.  Other head dims up to 256 run at the
    next supported one, on copies of Q and every K / V shard zero-padded in D.

    One sequence per rank: leave ``cu_seqlens=None``.  Packed sequences: pass the LOCAL
    ``cu_seqlens`` (each entry a zig-zag ``2*h_j`` shard length) on the device and
    ``max_seqlen``.  Every local sequence length must be even.  For cp_size > 1 ``group``
    must be a LocalKVRing holding every source rank's KV shard (KV is not moved between
    GPUs here), or a PagedKVRing holding every source's paged K/V cache (the rank's own K/V
    come from it, so ``local_k`` / ``local_v`` are ignored; the per-step form gathers the
    pages into contiguous shards first)."""
    S = cfg.cp_size
    rank = cfg.cp_rank
    d = local_q.shape[2]
    dp = kernel_head_dim(local_q.dtype, d) if local_q.dtype in SUPPORTED_HEAD_DIMS else d
    if dp != d:
        # no kernel at this head dim: pad Q and every source's K / V with zero columns once
        # and run the sweep at the next supported head dim (scores are unchanged; the output's
        # padded columns are dropped)
        cfg_p = dataclasses.replace(cfg, softmax_scale=cfg.softmax_scale if cfg.softmax_scale is not None
                                    else 1.0 / math.sqrt(d))
        if isinstance(group, PagedKVRing):
            group_p = PagedKVRing([pad_head_dim(x, dp) for x in group.k], [pad_head_dim(x, dp) for x in group.v],
                                  group.page_tables)
            lk = lv = None
        else:
            group_p = None if group is None else LocalKVRing([pad_head_dim(x, dp) for x in group.k],
                                                             [pad_head_dim(x, dp) for x in group.v])
            same = group is not None and S > 1 and local_k is group.k[rank] and local_v is group.v[rank]
            lk, lv = group_p.kv(rank) if same else (pad_head_dim(local_k, dp), pad_head_dim(local_v, dp))
        res = ring_flash_attn(pad_head_dim(local_q, dp), lk, lv, cfg_p, group=group_p, descales=descales,
                              cu_seqlens=cu_seqlens, max_seqlen=max_seqlen, fused=fused, return_lse=return_lse)
        if return_lse:
            return res[0][..., :d].contiguous(), res[1]
        return res[..., :d].contiguous()
    # the kernels read rows contiguous in D (the reference copies with .contiguous() too)
    local_q = local_q if local_q.stride(2) == 1 else local_q.contiguous()
    if local_k is not None and local_k.stride(2) != 1:
        local_k = local_k.contiguous()
    if local_v is not None and local_v.stride(2) != 1:
        local_v = local_v.contiguous()
    scale = cfg.softmax_scale
    total = local_q.shape[0]
    if cu_seqlens is not None:
        assert max_seqlen is not None, "max_seqlen required when cu_seqlens is given"
    else:
        max_seqlen = total
    _check_even_lengths(cu_seqlens, total, max_seqlen)
    paged = isinstance(group, PagedKVRing)
    if paged:
        assert group.cp_size == S, f"PagedKVRing holds {group.cp_size} caches, cp_size is {S}"
    elif S > 1:
        if not isinstance(group, LocalKVRing):
            raise RuntimeError(
                "ring_flash_attn: cp_size > 1 needs group=LocalKVRing(k_shards, v_shards) or a "
                "PagedKVRing: every source rank's K/V on this GPU (no KV rotation between GPUs)")
        assert group.cp_size == S, f"LocalKVRing holds {group.cp_size} shards, cp_size is {S}"

    d = local_q.shape[2]
    e4m3 = local_q.dtype == torch.float8_e4m3fn
    can_fuse = 1 < S <= _lib.MAX_CP and (
        (descales is None and local_q.dtype in (torch.bfloat16, torch.float16) and d in (64, 128, 256))
        or (e4m3 and d in (128, 256)))
    def finish(out, lse):
        return (out, lse) if return_lse else out

    if paged:
        if fused is not False and can_fuse:
            lse = _new_lse(local_q) if return_lse else None
            return finish(ring_sweep_paged(local_q, cfg, group, cu_seqlens, max_seqlen, lse=lse,
                                           descales=descales), lse)
        if fused:
            raise AssertionError("fused ring sweep needs cp_size in [2, 16] and bf16/fp16 with head dim "
                                 "64/128/256 and no descales, or e4m3 with head dim 128/256")
        # the per-step form reads contiguous shards: gather every source's K and V pages first
        group = LocalKVRing(gather_kv_pages(group, "k", total, cu_seqlens, max_seqlen),
                            gather_kv_pages(group, "v", total, cu_seqlens, max_seqlen))
        local_k, local_v = group.kv(rank)
        fused = False
    if fused and not can_fuse:
        raise AssertionError("fused ring sweep needs cp_size in [2, 16] and bf16/fp16 with head dim "
                             "64/128/256 and no descales, or e4m3 with head dim 128/256")
    if fused is None:
        fused = can_fuse
    if fused:
        lse = _new_lse(local_q) if return_lse else None
        return finish(ring_sweep(local_q, local_k, local_v, cfg, group, cu_seqlens, max_seqlen, lse=lse,
                                 descales=descales), lse)

    qd = descales.q if descales else None

    def kd(src):
        return descales.k[src] if (descales and descales.k) else None

    def vd(src):
        return descales.v[src] if (descales and descales.v) else None

    h_q, d = local_q.shape[1], local_q.shape[2]
    odt = out_dtype_for(local_q.dtype)
    dev = local_q.device
    common = dict(softmax_scale=scale, cu_seqlens_q=cu_seqlens, cu_seqlens_k=cu_seqlens,
                  max_seqlen_q=max_seqlen, max_seqlen_k=max_seqlen, q_descale=qd)
    vt_kernels = uses_vt(local_q.dtype, d)

    def attn(k, v, src, causal, k_sel=SEL_ALL, **kw):
        """One ring step's attention; V is transposed first (only the selected keys) when the
        kernel for this type reads V^T."""
        v_t = None
        if vt_kernels:
            v_t = transpose_v(v, cu_seqlens_k=cu_seqlens, max_seqlen_k=max_seqlen, k_sel=k_sel)
        return fa4_attn(local_q, k, v, causal=causal, k_sel=k_sel, k_descale=kd(src), v_descale=vd(src),
                        v_t=v_t, **kw, **common)

    if cfg.merge_mode == "batched" and S > 1:
        # every step writes its partial straight into slot `step` of the merge buffer
        vbuf = torch.empty((total, S, h_q, d), dtype=odt, device=dev)
        sbuf = torch.empty((total, S, h_q), dtype=torch.float32, device=dev)
        attn(local_k, local_v, rank, True, out=vbuf[:, 0], lse=sbuf[:, 0])
        for step in range(1, S):
            src = (rank - step) % S
            k, v = group.kv(src)
            if step <= rank:
                attn(k, v, src, False, k_sel=SEL_FRONT_HALF, out=vbuf[:, step], lse=sbuf[:, step])
            else:
                # front rows of this slot stay empty: -inf LSE makes them the identity
                sbuf[:, step].fill_(float("-inf"))
                attn(k, v, src, False, q_sel=SEL_BACK_HALF, out=vbuf[:, step], lse=sbuf[:, step])
        return finish(*merge_states(vbuf, sbuf))

    # incremental (and cp_size == 1): step 0 seeds the accumulator with every row finite
    acc, acc_lse = attn(local_k, local_v, rank, True)
    if S == 1:
        return finish(acc, acc_lse)
    part = torch.empty_like(acc)
    part_lse = torch.empty_like(acc_lse)
    for step in range(1, S):
        src = (rank - step) % S
        k, v = group.kv(src)
        if step <= rank:
            attn(k, v, src, False, k_sel=SEL_FRONT_HALF, out=part, lse=part_lse)
            merge_state_in_place(acc, acc_lse, part, part_lse)
        else:
            attn(k, v, src, False, q_sel=SEL_BACK_HALF, out=part, lse=part_lse)
            merge_state_in_place(acc, acc_lse, part, part_lse, cu_seqlens=cu_seqlens,
                                 row_sel=SEL_BACK_HALF)
    return finish(acc, acc_lse)


def _new_lse(local_q: torch.Tensor) -> torch.Tensor:
    return torch.empty(local_q.shape[:2], dtype=torch.float32, device=local_q.device)


def ring_sweep(local_q: torch.Tensor, local_k: torch.Tensor, local_v: torch.Tensor, cfg: RingConfig,
               group: "LocalKVRing", cu_seqlens: Optional[torch.Tensor] = None,
               max_seqlen: Optional[int] = None, out: Optional[torch.Tensor] = None,
               lse: Optional[torch.Tensor] = None, descales: Optional[Descales] = None) -> torch.Tensor:
    """The whole sweep of ring_flash_attn (fa4_ring/ring_attention.py:61-174) in one
    fa4cp_ring_sweep_fwd launch: every source's V is transposed (one fa4cp_transpose_v_many
    launch), then one kernel carries each row tile's online softmax through the causal local keys, the front
    halves of the earlier sources and, for the back-half rows, all keys of the later ones.
    e4m3 inputs take ``descales`` (the k / v descales per source rank, as ring_flash_attn)
    and give a bf16 out.  Returns out [T, H, D] (``lse`` [T, H], if given, receives the
    natural-log LSE)."""
    _lib.load()  # fails here, before any allocation, without the library
    S, rank = cfg.cp_size, cfg.cp_rank
    total, h_q, d = local_q.shape
    dev = local_q.device
    assert local_q.is_cuda and local_q.stride(2) == 1, "local_q must be a device tensor, contiguous in D"
    nseq = 1 if cu_seqlens is None else cu_seqlens.shape[0] - 1
    ks = [local_k if i == rank else group.k[i] for i in range(S)]
    vs = [local_v if i == rank else group.v[i] for i in range(S)]
    h_kv = ks[0].shape[1]
    for k, v in zip(ks, vs):
        assert k.shape == (total, h_kv, d) and v.shape == k.shape and k.dtype == local_q.dtype
        assert k.stride() == ks[0].stride(), "all K shards must share strides"
        # the sweep's arguments carry K's row and head strides only: D must be contiguous
        assert k.stride(2) == 1 and v.stride(2) == 1, "K and V shards must be contiguous in D"
    assert all(v.stride() == vs[0].stride() for v in vs), "all V shards must share strides"
    vts, stride = transpose_v_many(vs, cu_seqlens_k=cu_seqlens, max_seqlen_k=max_seqlen)
    return _sweep_launch(local_q, [k.data_ptr() for k in ks], (ks[0].stride(0), ks[0].stride(1)), h_kv, vts,
                         stride, cfg, cu_seqlens, max_seqlen, out, lse, descales)


def ring_sweep_paged(local_q: torch.Tensor, cfg: RingConfig, ring: "PagedKVRing",
                     cu_seqlens: Optional[torch.Tensor] = None, max_seqlen: Optional[int] = None,
                     out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
                     descales: Optional[Descales] = None) -> torch.Tensor:
    """ring_sweep over paged K/V caches: one launch writes every source's V^T from its V
    pages, then the sweep kernel reads K straight from the caches through the page tables
    (fa4cp_ring_sweep_fwd_paged: one table entry per page, no contiguous K copy).  The result
    is bit-identical to ring_sweep on the contiguous shards."""
    _lib.load()  # fails here, before any allocation, without the library
    total, _, d = local_q.shape
    assert local_q.is_cuda and local_q.stride(2) == 1, "local_q must be a device tensor, contiguous in D"
    kc = ring.k[0]
    assert kc.dtype == local_q.dtype and kc.shape[3] == d and kc.device == local_q.device, \
        "caches must match local_q's dtype, head dim and device"
    nseq = 1 if cu_seqlens is None else cu_seqlens.shape[0] - 1
    assert ring.page_tables[0].shape[0] == nseq, "page tables need one row per local sequence"
    vts, stride = transpose_v_paged_many(ring, total, cu_seqlens, max_seqlen)
    kp = _lib.SweepKPages()
    for i, pt in enumerate(ring.page_tables):
        kp.page_table[i] = pt.data_ptr()
    kp.pt_stride = ring.page_tables[0].shape[1]
    kp.page_size = ring.page_size
    kp.num_pages = kc.shape[0]
    # a cache is [num_pages, page_size, H_kv, D]: rows at stride(1), heads at stride(2)
    return _sweep_launch(local_q, [k.data_ptr() for k in ring.k], (kc.stride(1), kc.stride(2)), kc.shape[2],
                         vts, stride, cfg, cu_seqlens, max_seqlen, out, lse, descales, kpages=kp)


def _sweep_launch(local_q: torch.Tensor, k_ptrs: List[int], k_strides: Tuple[int, int], h_kv: int,
                  vts: List[torch.Tensor], stride: int, cfg: RingConfig, cu_seqlens: Optional[torch.Tensor],
                  max_seqlen: Optional[int], out: Optional[torch.Tensor], lse: Optional[torch.Tensor],
                  descales: Optional[Descales], kpages: Optional["_lib.SweepKPages"] = None) -> torch.Tensor:
    """Queues fa4cp_ring_sweep_fwd over every source rank's K (device addresses `k_ptrs`, row
    and head strides `k_strides`) and V^T buffers `vts` (row stride `stride`); with `kpages`,
    fa4cp_ring_sweep_fwd_paged, the K addresses being the sources' paged caches."""
    S, rank = cfg.cp_size, cfg.cp_rank
    total, h_q, d = local_q.shape
    dev = local_q.device
    nseq = 1 if cu_seqlens is None else cu_seqlens.shape[0] - 1
    e4m3 = local_q.dtype == torch.float8_e4m3fn
    if out is None:
        out = torch.empty(local_q.shape, dtype=torch.bfloat16 if e4m3 else local_q.dtype, device=dev)
    qd = kd = vd = None
    if e4m3 and descales is not None:
        qd, kd, vd = sweep_descales(descales.q, None if descales.k is None else descales.k[:S],
                                    None if descales.v is None else descales.v[:S], h_kv, dev)
    if lse is None:
        lse = torch.empty((total, h_q), dtype=torch.float32, device=dev)
    odt = torch.bfloat16 if e4m3 else local_q.dtype
    assert out.shape == local_q.shape and out.dtype == odt and out.device == dev and out.stride(2) == 1, \
        f"out must be [{total}, {h_q}, {d}] {odt} on {dev}, contiguous in D"
    assert lse.shape == (total, h_q) and lse.dtype == torch.float32 and lse.device == dev and lse.stride(1) == 1, \
        f"lse must be [{total}, {h_q}] float32 on {dev} with unit head stride"
    for i, vt in enumerate(vts):
        assert vt.device == dev, f"source {i}'s V^T must be on {dev}"
    if cu_seqlens is not None:
        assert cu_seqlens.dtype == torch.int32 and cu_seqlens.device == dev and cu_seqlens.is_contiguous(), \
            "cu_seqlens must be contiguous int32 on the device"
        assert max_seqlen is not None, "max_seqlen required when cu_seqlens is given"
    a = _lib.SweepArgs()
    a.q, a.out, a.lse = local_q.data_ptr(), out.data_ptr(), lse.data_ptr()
    a.q_row_stride, a.q_head_stride = local_q.stride(0), local_q.stride(1)
    a.o_row_stride, a.o_head_stride = out.stride(0), out.stride(1)
    a.lse_row_stride = lse.stride(0)
    for i in range(S):
        a.k[i] = k_ptrs[i]
        a.v_t[i] = vts[i].data_ptr()
    a.k_row_stride, a.k_head_stride = k_strides
    a.vt_d_stride = stride
    a.cu = _lib.ptr(cu_seqlens)
    a.nseq = nseq
    a.max_seqlen = int(max_seqlen) if cu_seqlens is not None else total
    a.total = total
    a.h_q, a.h_kv, a.d = h_q, h_kv, d
    a.dtype = _lib.dtype_code(local_q.dtype)
    a.cp_rank, a.cp_size = rank, S
    a.softmax_scale = float(cfg.softmax_scale if cfg.softmax_scale is not None else 1.0 / math.sqrt(d))
    a.q_descale, a.k_descale, a.v_descale = _lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd)
    launch_sweep(a, dev, kpages)
    return out


def launch_sweep(args: "_lib.SweepArgs", device: torch.device,
                 kpages: Optional["_lib.SweepKPages"] = None) -> None:
    """Queues the fused sweep kernel on the current stream of `device` (with `kpages`: the
    paged-K sweep)."""
    lib = _lib.load()
    if kpages is None:
        _lib.check(lib.fa4cp_ring_sweep_fwd(ctypes.byref(args), _lib.stream_handle(device)),
                   "fa4cp_ring_sweep_fwd")
    else:
        _lib.check(lib.fa4cp_ring_sweep_fwd_paged(ctypes.byref(args), ctypes.byref(kpages),
                                                  _lib.stream_handle(device)), "fa4cp_ring_sweep_fwd_paged")
