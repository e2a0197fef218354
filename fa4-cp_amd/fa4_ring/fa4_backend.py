"""Per-chunk attention forward on the gfx950 HIP kernel (operator level of the ring).

Keeps the interface of fa4_ring/fa4_backend.py:58-123 (``fa4_attn`` returning out and a
natural-log LSE laid out [T_q, H]) so the module drops in where the reference called
FlashAttention-4's ``_flash_attn_fwd``; the computation is ``fa4cp_attn_fwd`` of
libfa4cp.so, launched on torch's current stream without any host synchronisation.

Beyond the reference signature, ``q_sel`` / ``k_sel`` select the back half of every
query sequence or the front half of every key sequence inside the kernel (the two
non-local zig-zag step patterns, fa4_ring/ring_attention.py:139-165, without the
index_select gathers), and ``out`` / ``lse`` accept preallocated (possibly strided)
destinations, such as one slot of a batched-merge buffer.
"""

from __future__ import annotations

import ctypes
import math
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import SEL_ALL, SEL_BACK_HALF, SEL_FRONT_HALF

SUPPORTED_HEAD_DIMS = {torch.bfloat16: (64, 128, 256), torch.float16: (64, 128, 256),
                       torch.float8_e4m3fn: (128, 256)}
# (dtype, head dim) pairs whose kernels read a pre-transposed V^T (fa4cp_transpose_v)
VT_HEAD_DIMS = {torch.bfloat16: (64, 128, 256), torch.float16: (64, 128, 256), torch.float8_e4m3fn: (128, 256)}


def has_fa4() -> bool:
    """True when the HIP attention library is built and loadable (the reference's
    ``has_fa4`` probes the FlashAttention-4 import, fa4_backend.py:41-42)."""
    return _lib.available()


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def kernel_head_dim(dtype: torch.dtype, d: int) -> int:
    """The head dim the kernels run a head dim ``d`` at: ``d`` itself where a kernel exists,
    else the smallest supported one above it (q, k and v are then zero-padded in D: the
    padded columns add nothing to any score, and the output's padded columns are dropped).
    Raises for ``d`` above the largest supported head dim."""
    dims = SUPPORTED_HEAD_DIMS.get(dtype)
    _require(dims is not None, f"unsupported dtype {dtype}")
    _require(1 <= d <= max(dims), f"head dim {d} above {max(dims)} is not supported for {dtype}")
    return min(x for x in dims if x >= d)


def pad_head_dim(x: torch.Tensor, dp: int) -> torch.Tensor:
    """x [..., d] -> a new contiguous [..., dp] tensor, zeros in columns d..dp-1 (x itself
    when d == dp and x is contiguous in D)."""
    d = x.shape[-1]
    if d == dp:
        return x if x.stride(-1) == 1 else x.contiguous()
    y = torch.zeros((*x.shape[:-1], dp), dtype=x.dtype, device=x.device)
    y[..., :d] = x
    return y


def _descale_view(d, h_kv: int, device) -> torch.Tensor:
    """Descale -> a float32 [h_kv] view on `device` (a scalar broadcasts to every kv head,
    [h_kv] and (1, h_kv) are taken as is; fa4_backend.py:45-55), copied only if its dtype or
    device differ."""
    if not torch.is_tensor(d):
        d = torch.tensor(float(d))
    d = d.to(device=device, dtype=torch.float32)
    if d.dim() == 0:
        d = d.reshape(1).expand(h_kv)
    elif d.dim() == 2:
        _require(d.shape[0] == 1, f"descale batch dimension must be 1, got {tuple(d.shape)}")
        d = d[0]
    _require(d.dim() == 1 and d.shape[0] == h_kv,
             f"descale must be a scalar, [H_kv] or (1, H_kv) with H_kv={h_kv}, got {tuple(d.shape)}")
    return d


def _norm_descale(d: Optional[torch.Tensor], h_kv: int, device) -> Optional[torch.Tensor]:
    """Descale -> float32 contiguous [h_kv] on `device` (see _descale_view)."""
    if d is None:
        return None
    return _descale_view(d, h_kv, device).contiguous()


def descale_table(ds, h_kv: int, device) -> torch.Tensor:
    """Per-source descales -> one float32 contiguous [len(ds), h_kv] table, built by a single
    stack over views (one small device copy, where normalising each entry on its own and
    stacking takes one launch per source)."""
    return torch.stack([_descale_view(d, h_kv, device) for d in ds])


def sweep_descales(q, ks, vs, h_kv: int, device):
    """The fused sweep's descales -> (q [h_kv], k [len(ks), h_kv], v [len(vs), h_kv]), float32
    rows of one contiguous table built by a single stack (one device copy per call instead of
    three); a part given as None comes back None."""
    parts = [[] if q is None else [q], list(ks or []), list(vs or [])]
    views = [_descale_view(d, h_kv, device) for part in parts for d in part]
    if not views:
        return None, None, None
    table = torch.stack(views)
    out, row = [], 0
    for part, given in zip(parts, (q is not None, ks is not None, vs is not None)):
        out.append(table[row:row + len(part)] if given else None)
        row += len(part)
    return out[0][0] if q is not None else None, out[1], out[2]


def _cu_ok(cu: torch.Tensor, device, name: str) -> None:
    _require(cu.dtype == torch.int32, f"{name} must be int32, got {cu.dtype}")
    _require(cu.device == device, f"{name} must live on {device}, got {cu.device}")
    _require(cu.dim() == 1 and cu.shape[0] >= 2, f"{name} must be [num_seq + 1]")
    _require(cu.is_contiguous(), f"{name} must be contiguous")


def out_dtype_for(dt: torch.dtype) -> torch.dtype:
    """FP8 inputs produce a bf16 output, other inputs their own type."""
    return torch.bfloat16 if dt == torch.float8_e4m3fn else dt


def uses_vt(dtype: torch.dtype, d: int) -> bool:
    """True when fa4_attn runs a kernel that reads V^T for this input type and head dim."""
    return d in VT_HEAD_DIMS.get(dtype, ())


def transpose_v(v: torch.Tensor, *, cu_seqlens_k: Optional[torch.Tensor] = None,
                max_seqlen_k: Optional[int] = None, k_sel: int = SEL_ALL) -> Tuple[torch.Tensor, int]:
    """V [T_k, H_kv, D] -> (V^T, row stride): the keys selected by ``k_sel`` of every packed
    sequence, transposed to [H_kv, D, positions] (fa4cp_transpose_v layout: each sequence
    starts at a multiple of 128 positions, zero padded).  Runs on the current stream."""
    lib = _lib.load()
    _require(v.dim() == 3 and v.is_cuda, "v must be a [T, H_kv, D] device tensor")
    _require(v.stride(2) == 1, "v must be contiguous in the head dim")
    t_k, h_kv, d = v.shape
    nseq = 1
    if cu_seqlens_k is not None:
        _cu_ok(cu_seqlens_k, v.device, "cu_seqlens_k")
        _require(max_seqlen_k is not None, "max_seqlen_k required with cu_seqlens_k")
        nseq = cu_seqlens_k.shape[0] - 1
    stride = int(lib.fa4cp_vt_min_d_stride(t_k, nseq))
    vt = torch.empty(h_kv * d * stride, dtype=v.dtype, device=v.device)
    a = _lib.TransposeArgs()
    a.v = v.data_ptr()
    a.v_row_stride, a.v_head_stride = v.stride(0), v.stride(1)
    a.cu_k = _lib.ptr(cu_seqlens_k)
    a.nseq = nseq
    a.total_k = t_k
    a.max_seqlen_k = int(max_seqlen_k) if cu_seqlens_k is not None else t_k
    a.k_sel = int(k_sel)
    a.h_kv, a.d = h_kv, d
    a.dtype = _lib.dtype_code(v.dtype)
    a.v_t = vt.data_ptr()
    a.vt_d_stride = stride
    _lib.check(lib.fa4cp_transpose_v(ctypes.byref(a), _lib.stream_handle(v.device)), "fa4cp_transpose_v")
    return vt, stride


def transpose_v_many(vs: Sequence[torch.Tensor], *, cu_seqlens_k: Optional[torch.Tensor] = None,
                     max_seqlen_k: Optional[int] = None) -> Tuple[List[torch.Tensor], int]:
    """transpose_v (k_sel = all) of up to 16 tensors of one shape and stride in one launch
    (fa4cp_transpose_v_many), e.g. every source rank's V before a fused sweep."""
    lib = _lib.load()
    _require(1 <= len(vs) <= _lib.MAX_CP, f"1..{_lib.MAX_CP} tensors")
    v = vs[0]
    _require(v.dim() == 3 and v.is_cuda and v.stride(2) == 1, "v must be a [T, H_kv, D] device tensor, unit stride in D")
    for x in vs:
        _require(x.shape == v.shape and x.stride() == v.stride() and x.dtype == v.dtype, "tensors must share shape, strides and dtype")
    t_k, h_kv, d = v.shape
    nseq = 1
    if cu_seqlens_k is not None:
        _cu_ok(cu_seqlens_k, v.device, "cu_seqlens_k")
        _require(max_seqlen_k is not None, "max_seqlen_k required with cu_seqlens_k")
        nseq = cu_seqlens_k.shape[0] - 1
    stride = int(lib.fa4cp_vt_min_d_stride(t_k, nseq))
    vts = [torch.empty(h_kv * d * stride, dtype=v.dtype, device=v.device) for _ in vs]
    a = _lib.TransposeArgs()
    a.v_row_stride, a.v_head_stride = v.stride(0), v.stride(1)
    a.cu_k = _lib.ptr(cu_seqlens_k)
    a.nseq = nseq
    a.total_k = t_k
    a.max_seqlen_k = int(max_seqlen_k) if cu_seqlens_k is not None else t_k
    a.k_sel = SEL_ALL
    a.h_kv, a.d = h_kv, d
    a.dtype = _lib.dtype_code(v.dtype)
    a.vt_d_stride = stride
    src = (ctypes.c_void_p * len(vs))(*[x.data_ptr() for x in vs])
    dst = (ctypes.c_void_p * len(vs))(*[x.data_ptr() for x in vts])
    _lib.check(lib.fa4cp_transpose_v_many(ctypes.byref(a), src, dst, len(vs), _lib.stream_handle(v.device)),
               "fa4cp_transpose_v_many")
    return vts, stride


def fa4_attn(
    q: torch.Tensor,  # [T_q, H, D]
    k: torch.Tensor,  # [T_k, H_kv, D]
    v: torch.Tensor,  # [T_k, H_kv, D]
    *,
    causal: bool,
    softmax_scale: Optional[float] = None,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    cu_seqlens_k: Optional[torch.Tensor] = None,
    max_seqlen_q: Optional[int] = None,
    max_seqlen_k: Optional[int] = None,
    q_descale: Optional[torch.Tensor] = None,
    k_descale: Optional[torch.Tensor] = None,
    v_descale: Optional[torch.Tensor] = None,
    q_sel: int = SEL_ALL,
    k_sel: int = SEL_ALL,
    out: Optional[torch.Tensor] = None,
    lse: Optional[torch.Tensor] = None,
    v_t: Optional[Tuple[torch.Tensor, int]] = None,
    use_vt: bool = True,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Varlen flash-attention forward.

    Returns ``out [T_q, H, D]`` (bf16 for e4m3 inputs, else the input type) and
    ``lse [T_q, H]`` float32 natural log.  ``cu_seqlens_q/k`` (int32 [num_seq+1], on the
    device) with ``max_seqlen_q/k`` describe packed sequences; omitted, each side is one
    sequence.  Causal masking is bottom-right aligned per sequence.  With
    ``q_sel=SEL_BACK_HALF`` only the back half of each query sequence is computed and
    written (at its own rows of ``out`` / ``lse``); with ``k_sel=SEL_FRONT_HALF`` only
    the front half of each key sequence is attended.

    Where a kernel reading V^T exists (``VT_HEAD_DIMS``) and ``use_vt`` is set, V is first
    transposed with ``transpose_v`` (or ``v_t`` from an earlier ``transpose_v`` call with
    the same keys and selection is used)."""
    lib = _lib.load()
    _require(q.dim() == 3 and k.dim() == 3 and v.dim() == 3, "q, k, v must be [T, H, D]")
    _require(q.is_cuda, "fa4_attn runs on the GPU: q must be a device tensor")
    dev = q.device
    _require(k.device == dev and v.device == dev, "q, k, v must share a device")
    _require(q.dtype == k.dtype == v.dtype, f"q/k/v dtypes differ: {q.dtype} {k.dtype} {v.dtype}")
    dt = q.dtype
    _require(dt in SUPPORTED_HEAD_DIMS, f"unsupported dtype {dt}")
    t_q, h_q, d = q.shape
    t_k, h_kv, dk = k.shape
    _require(v.shape == k.shape, f"k {tuple(k.shape)} and v {tuple(v.shape)} must match")
    _require(dk == d, f"q head dim {d} != k head dim {dk}")
    _require(h_q % h_kv == 0, f"H_q={h_q} not a multiple of H_kv={h_kv}")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(d)
    # the kernels read rows contiguous in D; other layouts are copied (as the reference's
    # .contiguous() before FA4, fa4_backend.py:106-109)
    q, k, v = (t if t.stride(2) == 1 else t.contiguous() for t in (q, k, v))
    dp = kernel_head_dim(dt, d)
    if dp != d:
        # no kernel at this head dim: run the next one up on zero-padded copies
        _require(v_t is None, f"v_t cannot be given at head dim {d} (the kernels run at {dp})")
        odt = out_dtype_for(dt)
        if out is not None:
            _require(out.shape == (t_q, h_q, d) and out.dtype == odt and out.device == dev,
                     f"out must be [{t_q}, {h_q}, {d}] {odt}")
        # (a given out is padded too, so the rows outside a q selection keep what it held)
        o_p, lse = fa4_attn(pad_head_dim(q, dp), pad_head_dim(k, dp), pad_head_dim(v, dp), causal=causal,
                            softmax_scale=softmax_scale, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
                            max_seqlen_q=max_seqlen_q, max_seqlen_k=max_seqlen_k, q_descale=q_descale,
                            k_descale=k_descale, v_descale=v_descale, q_sel=q_sel, k_sel=k_sel,
                            out=None if out is None else pad_head_dim(out, dp), lse=lse, use_vt=use_vt)
        if out is None:
            return o_p[..., :d].contiguous(), lse
        out.copy_(o_p[..., :d])
        return out, lse

    if (cu_seqlens_q is None) != (cu_seqlens_k is None):
        # one side packed, the other a single sequence: describe the latter explicitly
        if cu_seqlens_q is None:
            cu_seqlens_q = torch.tensor([0, t_q], dtype=torch.int32, device=dev)
            max_seqlen_q = t_q
        else:
            cu_seqlens_k = torch.tensor([0, t_k], dtype=torch.int32, device=dev)
            max_seqlen_k = t_k
    nseq = 1
    if cu_seqlens_q is not None:
        _cu_ok(cu_seqlens_q, dev, "cu_seqlens_q")
        _cu_ok(cu_seqlens_k, dev, "cu_seqlens_k")
        _require(cu_seqlens_q.shape == cu_seqlens_k.shape,
                 "cu_seqlens_q and cu_seqlens_k must describe the same number of sequences")
        _require(max_seqlen_q is not None and max_seqlen_k is not None,
                 "max_seqlen_q/k required when cu_seqlens are given")
        nseq = cu_seqlens_q.shape[0] - 1
    else:
        max_seqlen_q, max_seqlen_k = t_q, t_k

    odt = out_dtype_for(dt)
    if out is None:
        out = torch.empty((t_q, h_q, d), dtype=odt, device=dev)
    if lse is None:
        lse = torch.empty((t_q, h_q), dtype=torch.float32, device=dev)
    _require(out.shape == (t_q, h_q, d) and out.dtype == odt and out.device == dev,
             f"out must be [{t_q}, {h_q}, {d}] {odt}")
    _require(out.stride(2) == 1, "out must be contiguous in the head dim")
    _require(lse.shape == (t_q, h_q) and lse.dtype == torch.float32 and lse.stride(1) == 1
             and lse.device == dev, "lse must be [T_q, H] float32 on q's device with unit head stride")

    vt_ptr, vt_stride = None, 0
    if use_vt and uses_vt(dt, d):
        if v_t is None:
            v_t = transpose_v(v, cu_seqlens_k=cu_seqlens_k, max_seqlen_k=max_seqlen_k, k_sel=k_sel)
        vt_ptr, vt_stride = v_t[0].data_ptr(), int(v_t[1])

    qd = _norm_descale(q_descale, h_kv, dev)
    kd = _norm_descale(k_descale, h_kv, dev)
    vd = _norm_descale(v_descale, h_kv, dev)

    a = _lib.AttnArgs()
    a.q, a.k, a.v, a.out, a.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr()
    a.q_row_stride, a.q_head_stride = q.stride(0), q.stride(1)
    a.k_row_stride, a.k_head_stride = k.stride(0), k.stride(1)
    a.v_row_stride, a.v_head_stride = v.stride(0), v.stride(1)
    a.o_row_stride, a.o_head_stride = out.stride(0), out.stride(1)
    a.lse_row_stride = lse.stride(0)
    a.cu_q = _lib.ptr(cu_seqlens_q)
    a.cu_k = _lib.ptr(cu_seqlens_k)
    a.nseq = nseq
    a.max_seqlen_q, a.max_seqlen_k = int(max_seqlen_q), int(max_seqlen_k)
    a.total_q, a.total_k = t_q, t_k
    a.h_q, a.h_kv, a.d = h_q, h_kv, d
    a.dtype = _lib.dtype_code(dt)
    a.causal = 1 if causal else 0
    a.q_sel, a.k_sel = int(q_sel), int(k_sel)
    a.softmax_scale = float(softmax_scale)
    a.q_descale, a.k_descale, a.v_descale = _lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd)
    a.v_t, a.vt_d_stride = vt_ptr, vt_stride
    rc = lib.fa4cp_attn_fwd(ctypes.byref(a), _lib.stream_handle(dev))
    _lib.check(rc, "fa4cp_attn_fwd")
    return out, lse


__all__ = ["fa4_attn", "kernel_head_dim", "pad_head_dim", "transpose_v", "uses_vt", "has_fa4", "out_dtype_for", "SEL_ALL", "SEL_BACK_HALF",
           "SEL_FRONT_HALF"]
