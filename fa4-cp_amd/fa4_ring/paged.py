"""Paged K/V caches in front of the fused ring sweep.

The reference keeps every rotated K/V shard contiguous and lists paged KV as not supported
(README.md:139-140).  Here a source rank's K and V may live in a paged cache
``[num_pages, page_size, H_kv, D]`` with an int32 page table ``[nseq, max_pages]`` per source:
entry ``[j, k]`` names the page holding rows ``[k * page_size, (k + 1) * page_size)`` of local
sequence ``j`` (the zig-zag local layout of ``cu_seqlens``).  ``page_size`` is a multiple of 128.

The fused sweep reads K in place: its K loads walk the page tables (one table entry per
page, fa4cp_ring_sweep_fwd_paged), so no contiguous K copy is made.  V is read once anyway
to write the V^T layout the sweep loads, and that launch reads it from the V pages.  Table
entries that name no page of the cache read as zero rows, and rows past a sequence's end
are never read, so unused cache rows (stale or NaN) never reach the attention.  The per-step
form (``fused=False``, and the shapes the fused sweep does not take) gathers the K and V
pages into contiguous shards first (``gather_kv_pages``).
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from .fa4_backend import _require


class PagedKVRing:
    """Every source rank's paged K/V cache on this GPU (the paged form of LocalKVRing).

    k_caches[i], v_caches[i]: ``[num_pages, page_size, H_kv, D]`` (one shape and dtype for all);
    page_tables[i]: int32 ``[nseq, max_pages]`` on the device, contiguous."""

    def __init__(self, k_caches: Sequence[torch.Tensor], v_caches: Sequence[torch.Tensor],
                 page_tables: Sequence[torch.Tensor]):
        _require(len(k_caches) == len(v_caches) == len(page_tables) >= 1,
                 "one K cache, V cache and page table per source rank")
        shape = k_caches[0].shape
        _require(len(shape) == 4, "caches are [num_pages, page_size, H_kv, D]")
        for k, v, pt in zip(k_caches, v_caches, page_tables):
            _require(k.shape == v.shape == shape and k.dtype == v.dtype == k_caches[0].dtype,
                     "every cache must have one shape and dtype")
            _require(k.is_cuda and v.is_cuda and k.stride() == k_caches[0].stride() and v.stride() == k.stride(),
                     "caches must be device tensors with one set of strides")
            _require(k.stride(3) == 1 and k.stride(0) == shape[1] * k.stride(1),
                     "each page must be page_size rows at one row stride, contiguous in D")
            _require(pt.dtype == torch.int32 and pt.dim() == 2 and pt.is_contiguous() and pt.device == k.device,
                     "page tables are contiguous int32 [nseq, max_pages] on the caches' device")
            _require(pt.shape == page_tables[0].shape, "every page table must have one shape")
        self.k = list(k_caches)
        self.v = list(v_caches)
        self.page_tables = list(page_tables)
        self.page_size = int(shape[1])
        _require(self.page_size % 128 == 0, f"page_size {self.page_size} must be a multiple of 128")

    @property
    def cp_size(self) -> int:
        return len(self.k)

    @classmethod
    def from_shards(cls, k_shards: Sequence[torch.Tensor], v_shards: Sequence[torch.Tensor], page_size: int,
                    cu_seqlens: Optional[Sequence[int]] = None, spare_pages: int = 0,
                    generator: Optional[torch.Generator] = None, fill: float = float("nan")) -> "PagedKVRing":
        """Scatters contiguous local shards ``[T, H_kv, D]`` into caches whose pages are handed
        out in a random order (``generator``), with ``spare_pages`` extra pages and every row
        no sequence uses set to ``fill``.  ``cu_seqlens``: the local layout (host list or
        tensor), None for one sequence of T rows."""
        t = k_shards[0].shape[0]
        cu = [0, t] if cu_seqlens is None else [int(c) for c in (
            cu_seqlens.tolist() if torch.is_tensor(cu_seqlens) else cu_seqlens)]
        lens = [cu[j + 1] - cu[j] for j in range(len(cu) - 1)]
        npg = [(n + page_size - 1) // page_size for n in lens]
        max_pages = max(1, max(npg))
        num_pages = sum(npg) + spare_pages
        dev = k_shards[0].device
        kcs, vcs, pts = [], [], []
        for ks, vs in zip(k_shards, v_shards):
            perm = torch.randperm(num_pages, generator=generator).tolist()
            table = torch.full((len(lens), max_pages), -1, dtype=torch.int32)
            rows = []
            nxt = 0
            for j, n in enumerate(lens):
                for k in range(npg[j]):
                    table[j, k] = perm[nxt]
                    nxt += 1
                    rows.append((j, k))
            kc = torch.full((num_pages, page_size) + tuple(ks.shape[1:]), fill, device=dev).to(ks.dtype)
            vc = torch.full_like(kc, fill)
            for j, k in rows:
                r0 = cu[j] + k * page_size
                n = min(page_size, cu[j + 1] - r0)
                p = int(table[j, k])
                kc[p, :n] = ks[r0:r0 + n]
                vc[p, :n] = vs[r0:r0 + n]
            kcs.append(kc)
            vcs.append(vc)
            pts.append(table.to(dev))
        return cls(kcs, vcs, pts)


def _paged_args(ring: PagedKVRing, total: int, cu_seqlens: Optional[torch.Tensor],
                max_seqlen: Optional[int]) -> "_lib.PagedArgs":
    k0 = ring.k[0]
    a = _lib.PagedArgs()
    a.cu = _lib.ptr(cu_seqlens)
    a.nseq = 1 if cu_seqlens is None else cu_seqlens.shape[0] - 1
    a.max_seqlen = int(max_seqlen) if cu_seqlens is not None else total
    a.total = total
    a.h_kv, a.d = k0.shape[2], k0.shape[3]
    a.dtype = _lib.dtype_code(k0.dtype)
    a.page_size = ring.page_size
    a.num_pages = k0.shape[0]
    a.cache_row_stride, a.cache_head_stride = k0.stride(1), k0.stride(2)
    a.pt_stride = ring.page_tables[0].shape[1]
    return a


def gather_kv_pages(ring: PagedKVRing, which: str, total: int, cu_seqlens: Optional[torch.Tensor] = None,
                    max_seqlen: Optional[int] = None) -> List[torch.Tensor]:
    """Every source's K (``which="k"``) or V rows as contiguous ``[total, H_kv, D]`` tensors in
    the local layout of ``cu_seqlens`` (one fa4cp_gather_kv_pages launch, current stream)."""
    lib = _lib.load()
    _require(which in ("k", "v"), f"which must be 'k' or 'v', got {which!r}")
    caches = ring.k if which == "k" else ring.v
    n, (_, _, h_kv, d) = ring.cp_size, caches[0].shape
    outs = [torch.empty((total, h_kv, d), dtype=caches[0].dtype, device=caches[0].device) for _ in range(n)]
    a = _paged_args(ring, total, cu_seqlens, max_seqlen)
    arr = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])  # noqa: E731
    _lib.check(lib.fa4cp_gather_kv_pages(ctypes.byref(a), arr(caches), arr(ring.page_tables), arr(outs),
                                         h_kv * d, d, n, _lib.stream_handle(caches[0].device)),
               "fa4cp_gather_kv_pages")
    return outs


def transpose_v_paged_many(ring: PagedKVRing, total: int, cu_seqlens: Optional[torch.Tensor] = None,
                           max_seqlen: Optional[int] = None) -> Tuple[List[torch.Tensor], int]:
    """Every source's V^T (the fa4cp_transpose_v layout of the contiguous V with the same
    ``cu_seqlens``) written from its V pages in one launch; returns (V^T list, row stride)."""
    lib = _lib.load()
    n, (_, _, h_kv, d) = ring.cp_size, ring.v[0].shape
    nseq = 1 if cu_seqlens is None else cu_seqlens.shape[0] - 1
    stride = int(lib.fa4cp_vt_min_d_stride(total, nseq))
    vts = [torch.empty(h_kv * d * stride, dtype=ring.v[0].dtype, device=ring.v[0].device) for _ in range(n)]
    a = _paged_args(ring, total, cu_seqlens, max_seqlen)
    arr = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])  # noqa: E731
    _lib.check(lib.fa4cp_transpose_v_paged_many(ctypes.byref(a), arr(ring.v), arr(ring.page_tables), arr(vts),
                                                stride, n, _lib.stream_handle(ring.v[0].device)),
               "fa4cp_transpose_v_paged_many")
    return vts, stride
