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
    """Rows one rank holds of a length-n sequence: two zig-zag chunks of n / (2 cp_size)
    (fa4_ring/zigzag.py:26-28)."""
    chunks = 2 * cp_size
    _require(n % chunks == 0, f"sequence length {n} is not a multiple of 2*cp_size = {chunks}")
    return 2 * (n // chunks)


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
    local_seqlen(n, cp_size)
    _require(0 <= cp_rank < cp_size, f"cp_rank {cp_rank} outside [0, {cp_size})")
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
    _require(len(local_shards) == cp_size, f"{len(local_shards)} shards given for cp_size {cp_size}")
    return _unshard(local_shards, cp_size, None, 1, local_shards[0].shape[0] * cp_size)


def half_indices(local_len: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Row indices of the early and the late zig-zag chunk of one local sequence of
    ``local_len`` rows (fa4_ring/zigzag.py:53-62)."""
    rows = torch.arange(local_len, device=device)
    return rows[:local_len // 2], rows[local_len // 2:]


def get_half_index(cu_seqlens: torch.Tensor, *, front: bool) -> torch.Tensor:
    """int64 row indices of the early (``front``) or late chunk of every packed local
    sequence of ``cu_seqlens`` (int32 [num_seq+1]), in order (fa4_ring/zigzag.py:65-79).
    Every local sequence is two chunks of equal size, so its length must be even.

    Built in one pass without a per-sequence loop: sequence j contributes
    ``first_j + [0, half_j)`` with ``half_j = len_j / 2`` and ``first_j = cu[j]`` (front) or
    ``cu[j] + half_j`` (late).  Reads cu on the host (one synchronisation), as the reference
    does."""
    cu = torch.as_tensor(cu_seqlens).to("cpu", torch.int64)
    lens = cu[1:] - cu[:-1]
    _require(bool((lens % 2 == 0).all()), "every local sequence must have an even length "
             "(two zig-zag chunks of equal size)")
    half = lens // 2
    first = cu[:-1] if front else cu[:-1] + half
    offset_in_seq = torch.arange(int(half.sum())) - torch.repeat_interleave(torch.cumsum(half, 0) - half, half)
    rows = torch.repeat_interleave(first, half) + offset_in_seq
    return rows.to(torch.as_tensor(cu_seqlens).device)


def zigzag_shard_varlen(x: torch.Tensor, full_cu_seqlens: Union[torch.Tensor, Sequence[int]],
                        cp_rank: int, cp_size: int):
    """Shard packed sequences zig-zag for this rank.

    ``full_cu_seqlens`` holds the FULL sequence boundaries (int list or tensor).  Returns
    (local_packed, local_cu_seqlens) with local_cu_seqlens int32 on x's device."""
    cu = _as_cu_list(full_cu_seqlens)
    _require(0 <= cp_rank < cp_size, f"cp_rank {cp_rank} outside [0, {cp_size})")
    local_cu = [0]
    for j in range(len(cu) - 1):
        n = cu[j + 1] - cu[j]
        local_cu.append(local_cu[-1] + local_seqlen(n, cp_size))
    _require(cu[0] == 0 and cu[-1] == x.shape[0], "full_cu_seqlens must span x from row 0")
    local_cu_t = torch.tensor(local_cu, dtype=torch.int32, device=x.device)
    if len(cu) < 2:
        return x.new_empty((0,) + tuple(x.shape[1:])), local_cu_t
    local = _shard(x, cp_rank, cp_size, _device_cu(full_cu_seqlens, x.device), len(cu) - 1)
    return local, local_cu_t


def zigzag_unshard_varlen(local_shards: List[torch.Tensor],
                          full_cu_seqlens: Union[torch.Tensor, Sequence[int]], cp_size: int):
    """Inverse of zigzag_shard_varlen over all ranks -> the packed full tensor."""
    _require(len(local_shards) == cp_size, f"{len(local_shards)} shards given for cp_size {cp_size}")
    cu = _as_cu_list(full_cu_seqlens)
    for j in range(len(cu) - 1):
        local_seqlen(cu[j + 1] - cu[j], cp_size)
    return _unshard(local_shards, cp_size, _device_cu(full_cu_seqlens, local_shards[0].device),
                    len(cu) - 1, cu[-1])
