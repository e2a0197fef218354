"""Zig-zag context-parallel sharding (interface of fa4_ring/zigzag.py).

A sequence of N tokens is cut into 2*cp_size chunks of h = N / (2*cp_size) tokens; rank i
holds chunk i (early) followed by chunk 2*cp_size-1-i (late) as its local [2h] sequence,
which balances the causal work across ranks.  Packed varlen input is sharded sequence by
sequence and the local shards are concatenated.

The row copies run on the gfx950 gather / scatter kernels of libfa4cp.so (bit-exact, one
launch per call).  The index helpers (``half_indices``, ``get_half_index``,
``local_seqlen``) are host-side index math, as in the reference.
"""

from __future__ import annotations

from typing import List, Sequence, Tuple, Union

import ctypes

import torch

from . import _lib


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def local_seqlen(n: int, cp_size: int) -> int:
    assert n % (2 * cp_size) == 0, f"seqlen {n} must be divisible by 2*cp_size={2 * cp_size}"
    return n // cp_size


def _row_bytes(x: torch.Tensor) -> int:
    return (x[0].numel() if x.shape[0] else int(torch.Size(x.shape[1:]).numel())) * x.element_size()


def _as_cu_list(cu) -> List[int]:
    return [int(c) for c in (cu.tolist() if torch.is_tensor(cu) else list(cu))]


def _device_cu(cu, device) -> torch.Tensor:
    if torch.is_tensor(cu) and cu.device == device and cu.dtype == torch.int32 and cu.is_contiguous():
        return cu
    return torch.tensor(_as_cu_list(cu), dtype=torch.int32, device=device)


def _shard(x: torch.Tensor, cp_rank: int, cp_size: int, full_cu_dev, nseq: int) -> torch.Tensor:
    lib = _lib.load()
    _require(x.is_cuda, "zig-zag sharding runs on the GPU: x must be a device tensor")
    _require(x.is_contiguous(), "x must be contiguous")
    n = x.shape[0]
    out = x.new_empty((n // cp_size,) + tuple(x.shape[1:]))
    rc = lib.fa4cp_zigzag_shard(x.data_ptr(), out.data_ptr(), _row_bytes(x), _lib.ptr(full_cu_dev),
                                nseq, n, cp_rank, cp_size, _lib.stream_handle(x.device))
    _lib.check(rc, "fa4cp_zigzag_shard")
    return out


def zigzag_shard(x: torch.Tensor, cp_rank: int, cp_size: int) -> torch.Tensor:
    """Full [N, ...] sequence -> this rank's local [2h, ...] shard."""
    n = x.shape[0]
    assert n % (2 * cp_size) == 0, f"seqlen {n} must be divisible by 2*cp_size={2 * cp_size}"
    assert 0 <= cp_rank < cp_size
    return _shard(x, cp_rank, cp_size, None, 1)


def _unshard(local_shards: Sequence[torch.Tensor], cp_size: int, full_cu_dev, nseq: int,
             n: int) -> torch.Tensor:
    lib = _lib.load()
    first = local_shards[0]
    _require(first.is_cuda, "zig-zag unsharding runs on the GPU: shards must be device tensors")
    for s in local_shards:
        _require(s.shape == first.shape and s.dtype == first.dtype and s.device == first.device,
                 "all shards must have the same shape, dtype and device")
        _require(s.is_contiguous(), "shards must be contiguous")
    out = first.new_empty((n,) + tuple(first.shape[1:]))
    ptrs = (ctypes.c_void_p * cp_size)(*[s.data_ptr() for s in local_shards])
    rc = lib.fa4cp_zigzag_unshard(ptrs, out.data_ptr(), _row_bytes(first), _lib.ptr(full_cu_dev), nseq,
                                  n, cp_size, _lib.stream_handle(first.device))
    _lib.check(rc, "fa4cp_zigzag_unshard")
    return out


def zigzag_unshard(local_shards: List[torch.Tensor], cp_size: int) -> torch.Tensor:
    """Inverse of zigzag_shard: stitch the cp_size per-rank [2h, ...] shards into [N, ...]."""
    assert len(local_shards) == cp_size
    return _unshard(local_shards, cp_size, None, 1, local_shards[0].shape[0] * cp_size)


def half_indices(local_len: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """(first_half, second_half) row indices of a local [2h] sequence."""
    h = local_len // 2
    return (torch.arange(0, h, device=device), torch.arange(h, local_len, device=device))


def get_half_index(cu_seqlens: torch.Tensor, *, front: bool) -> torch.Tensor:
    """Long indices of the front (early) or back (late) half of each packed sequence of
    ``cu_seqlens`` (int32 [num_seq+1]); each local sequence has even length and its
    midpoint is (start + end) // 2."""
    device = cu_seqlens.device
    cu = _as_cu_list(cu_seqlens)
    parts = []
    for i in range(len(cu) - 1):
        start, end = cu[i], cu[i + 1]
        assert (end - start) % 2 == 0, "each local sequence length must be even (zig-zag)"
        mid = (start + end) // 2
        parts.append(torch.arange(start, mid, device=device) if front
                     else torch.arange(mid, end, device=device))
    return torch.cat(parts) if parts else torch.empty(0, dtype=torch.long, device=device)


def zigzag_shard_varlen(x: torch.Tensor, full_cu_seqlens: Union[torch.Tensor, Sequence[int]],
                        cp_rank: int, cp_size: int):
    """Shard packed sequences zig-zag for this rank.

    ``full_cu_seqlens`` holds the FULL sequence boundaries (int list or tensor).  Returns
    (local_packed, local_cu_seqlens) with local_cu_seqlens int32 on x's device."""
    cu = _as_cu_list(full_cu_seqlens)
    assert 0 <= cp_rank < cp_size
    local_cu = [0]
    for j in range(len(cu) - 1):
        n = cu[j + 1] - cu[j]
        assert n % (2 * cp_size) == 0, f"seqlen {n} must be divisible by 2*cp_size={2 * cp_size}"
        local_cu.append(local_cu[-1] + n // cp_size)
    _require(cu[0] == 0 and cu[-1] == x.shape[0], "full_cu_seqlens must span x from row 0")
    local_cu_t = torch.tensor(local_cu, dtype=torch.int32, device=x.device)
    if len(cu) < 2:
        return x.new_empty((0,) + tuple(x.shape[1:])), local_cu_t
    local = _shard(x, cp_rank, cp_size, _device_cu(full_cu_seqlens, x.device), len(cu) - 1)
    return local, local_cu_t


def zigzag_unshard_varlen(local_shards: List[torch.Tensor],
                          full_cu_seqlens: Union[torch.Tensor, Sequence[int]], cp_size: int):
    """Inverse of zigzag_shard_varlen over all ranks -> the packed full tensor."""
    assert len(local_shards) == cp_size
    cu = _as_cu_list(full_cu_seqlens)
    for j in range(len(cu) - 1):
        assert (cu[j + 1] - cu[j]) % (2 * cp_size) == 0
    return _unshard(local_shards, cp_size, _device_cu(full_cu_seqlens, local_shards[0].device),
                    len(cu) - 1, cu[-1])
