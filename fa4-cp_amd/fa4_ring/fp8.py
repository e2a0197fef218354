"""FP8 producer: OCP e4m3 shards and their descales for the e4m3 ring sweep.

The reference leaves this step to its caller (README.md:63-70: pass e4m3 q/k/v shards and
per-tensor descales, the k/v ones all-gathered and indexed by source rank; Descales at
ring_attention.py:43-52).  The recipe is the one its FP8 inputs assume:
``scale = amax / 448``, ``x8 = clamp(x / scale, -448, 448).to(float8_e4m3fn)``,
descale = scale.  Here it is one library call per tensor (``fa4cp_quantize_e4m3``: an amax
pass and a quantise pass over HBM) instead of the four torch passes.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from .ring_attention import Descales


def quantize_e4m3(x: torch.Tensor, *, heads_per_scale: int = 0,
                  out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [rows, h, d] (bf16 / fp16 / fp32, on the device, unit stride in d) ->
    (x8 [rows, h, d] float8_e4m3fn contiguous, descale float32).

    ``heads_per_scale`` 0 gives one scale (a 0-dim descale); g > 0 one scale per g
    consecutive heads (a [h / g] descale): 1 for K/V per kv head, ``H_q / H_kv`` for Q in
    the (1, H_kv) layout of the sweep's q descale.  An all-zero group gets scale 1."""
    lib = _lib.load()
    assert x.is_cuda and x.dim() == 3 and x.stride(2) == 1, "x must be a [rows, h, d] device tensor, unit stride in d"
    rows, h, d = x.shape
    g = int(heads_per_scale)
    assert g == 0 or (g > 0 and h % g == 0), f"heads_per_scale {g} must be 0 or divide h = {h}"
    nscale = 1 if g == 0 else h // g
    if out is None:
        out = torch.empty((rows, h, d), dtype=torch.float8_e4m3fn, device=x.device)
    assert out.shape == (rows, h, d) and out.dtype == torch.float8_e4m3fn and out.is_contiguous() \
        and out.device == x.device, f"out must be a contiguous [{rows}, {h}, {d}] float8_e4m3fn tensor on {x.device}"
    amax = torch.empty(nscale, dtype=torch.float32, device=x.device)
    descale = torch.empty(nscale, dtype=torch.float32, device=x.device)
    a = _lib.QuantArgs()
    a.x, a.rows, a.h, a.d = x.data_ptr(), rows, h, d
    a.row_stride, a.head_stride = x.stride(0), x.stride(1)
    a.dtype = _lib.dtype_code(x.dtype)
    a.heads_per_scale = g
    a.amax, a.descale, a.y = amax.data_ptr(), descale.data_ptr(), out.data_ptr()
    _lib.check(lib.fa4cp_quantize_e4m3(ctypes.byref(a), _lib.stream_handle(x.device)), "fa4cp_quantize_e4m3")
    return out, (descale.reshape(()) if g == 0 else descale)


QUANT_MAX_SCALES = 1024  # FA4CP_QUANT_MAX_SCALES


def quantize_e4m3_into(x: torch.Tensor, out: torch.Tensor, descale: torch.Tensor, *,
                       heads_per_scale: int = 0) -> None:
    """quantize_e4m3 into caller-provided ``out`` ([rows, h, d] float8_e4m3fn, contiguous) and
    ``descale`` (float32, one element per scale, contiguous), allocating nothing on the
    device: the amax workspace is the library's static per-GPU array
    (fa4cp_quantize_e4m3_noalloc), so this can run where allocation is not allowed.  At most
    QUANT_MAX_SCALES scales.  Calls that overlap on one GPU (on different streams) share that
    workspace and race."""
    lib = _lib.load()
    assert x.is_cuda and x.dim() == 3 and x.stride(2) == 1, "x must be a [rows, h, d] device tensor, unit stride in d"
    rows, h, d = x.shape
    g = int(heads_per_scale)
    assert g == 0 or (g > 0 and h % g == 0), f"heads_per_scale {g} must be 0 or divide h = {h}"
    nscale = 1 if g == 0 else h // g
    assert nscale <= QUANT_MAX_SCALES, f"{nscale} scales exceed the static workspace ({QUANT_MAX_SCALES})"
    assert out.shape == (rows, h, d) and out.dtype == torch.float8_e4m3fn and out.is_contiguous() \
        and out.device == x.device, f"out must be a contiguous [{rows}, {h}, {d}] float8_e4m3fn tensor on {x.device}"
    assert descale.numel() == nscale and descale.dtype == torch.float32 and descale.is_contiguous() \
        and descale.device == x.device, f"descale must be {nscale} contiguous float32 values on {x.device}"
    a = _lib.QuantArgs()
    a.x, a.rows, a.h, a.d = x.data_ptr(), rows, h, d
    a.row_stride, a.head_stride = x.stride(0), x.stride(1)
    a.dtype = _lib.dtype_code(x.dtype)
    a.heads_per_scale = g
    a.amax, a.descale, a.y = None, descale.data_ptr(), out.data_ptr()
    with torch.cuda.device(x.device):  # the library looks up the current device's workspace
        rc = lib.fa4cp_quantize_e4m3_noalloc(ctypes.byref(a), _lib.stream_handle(x.device))
    _lib.check(rc, "fa4cp_quantize_e4m3_noalloc")


def quantize_ring(local_q: torch.Tensor, k_shards: Sequence[torch.Tensor], v_shards: Sequence[torch.Tensor],
                  *, per_head: bool = False
                  ) -> Tuple[torch.Tensor, List[torch.Tensor], List[torch.Tensor], Descales]:
    """The e4m3 inputs of one rank's sweep: its local q and every source rank's k / v shard
    quantised, with the Descales ring_flash_attn takes (k / v indexed by source rank).
    ``per_head`` scales q per kv-head group and k / v per kv head; otherwise per tensor."""
    h_q, h_kv = local_q.shape[1], k_shards[0].shape[1]
    assert h_q % h_kv == 0
    q8, qd = quantize_e4m3(local_q, heads_per_scale=(h_q // h_kv) if per_head else 0)
    g = 1 if per_head else 0
    k8, kd = zip(*(quantize_e4m3(k, heads_per_scale=g) for k in k_shards))
    v8, vd = zip(*(quantize_e4m3(v, heads_per_scale=g) for v in v_shards))
    return q8, list(k8), list(v8), Descales(q=qd, k=list(kd), v=list(vd))
