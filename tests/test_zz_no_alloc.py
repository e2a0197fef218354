"""fa4cp_quantize_e4m3_noalloc (the FP8 producer with its amax words in the library's static
per-GPU array) against fa4cp_quantize_e4m3 (caller workspace), through the C ABI.

Two calls in a row on one GPU, the second smaller and with fewer scales, its values a
hundred times smaller than the first's: a workspace not cleared between calls would give
the second call the first call's amax.  Bytes and descales must be equal bit for bit, and
equal to the oracle's quantisation."""

import ctypes

import pytest
import torch

from fa4_ring import _lib
from fa4_ring.fp8 import QUANT_MAX_SCALES, quantize_e4m3_into
from gpu_helpers import DEV, say
from oracle import ring_oracle as O

pytestmark = pytest.mark.gpu


def _args(x, y, descale, amax, g):
    a = _lib.QuantArgs()
    a.x, a.rows, a.h, a.d = x.data_ptr(), x.shape[0], x.shape[1], x.shape[2]
    a.row_stride, a.head_stride = x.stride(0), x.stride(1)
    a.dtype = _lib.dtype_code(x.dtype)
    a.heads_per_scale = g
    a.amax = None if amax is None else amax.data_ptr()
    a.descale, a.y = descale.data_ptr(), y.data_ptr()
    return a


def _both(x, g):
    """(bytes, descale) from the allocating entry point and from the one that allocates nothing."""
    lib = _lib.load()
    nscale = 1 if g == 0 else x.shape[1] // g
    stream = _lib.stream_handle(x.device)
    y_ref = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=DEV)
    d_ref = torch.empty(nscale, dtype=torch.float32, device=DEV)
    amax = torch.empty(nscale, dtype=torch.float32, device=DEV)
    _lib.check(lib.fa4cp_quantize_e4m3(ctypes.byref(_args(x, y_ref, d_ref, amax, g)), stream), "quantize_e4m3")
    y = torch.empty_like(y_ref)
    d = torch.empty_like(d_ref)
    _lib.check(lib.fa4cp_quantize_e4m3_noalloc(ctypes.byref(_args(x, y, d, None, g)), stream),
               "quantize_e4m3_noalloc")
    torch.cuda.synchronize()
    return (y_ref, d_ref), (y, d)


def _same_bits(a, b):
    return torch.equal(a.cpu().view(torch.uint8), b.cpu().view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_quantize_equals_workspace_entry_point_twice(dtype):
    gen = torch.Generator().manual_seed(31)
    cases = [  # (rows, h, d, heads_per_scale, magnitude): the second call smaller, fewer scales
        (4096, 32, 128, 1, 100.0),
        (1000, 8, 128, 4, 1.0),
    ]
    for rows, h, d, g, mag in cases:
        say(f"quantize_e4m3_noalloc dtype={dtype} rows={rows} h={h} d={d} heads_per_scale={g}")
        x = (mag * torch.randn(rows, h, d, generator=gen)).to(dtype)
        (y_ref, d_ref), (y, dsc) = _both(x.to(DEV), g)
        assert _same_bits(y, y_ref), "e4m3 bytes differ from the workspace entry point"
        assert _same_bits(dsc, d_ref), "descales differ from the workspace entry point"
        # and both equal the oracle's recipe, one scale per group of g heads
        xf = x.float()
        for s in range(h // g):
            grp = xf[:, s * g:(s + 1) * g]
            scale = O.amax_scale(grp)
            assert float(dsc[s]) == float(torch.tensor(scale, dtype=torch.float32))
            assert _same_bits(y[:, s * g:(s + 1) * g].contiguous(), O.quantize_e4m3(grp, scale).contiguous())


def test_noalloc_quantize_python_wrapper_and_limits():
    say("quantize_e4m3_into: one scale, then the static workspace's limit")
    x = torch.randn(512, 4, 64, device=DEV).to(torch.bfloat16)
    out = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=DEV)
    dsc = torch.empty(1, dtype=torch.float32, device=DEV)
    quantize_e4m3_into(x, out, dsc)
    (y_ref, d_ref), _ = _both(x, 0)
    assert _same_bits(out, y_ref) and _same_bits(dsc, d_ref)
    # more scales than the static array holds: refused before any launch
    lib = _lib.load()
    big = torch.zeros(2, QUANT_MAX_SCALES + 8, 8, dtype=torch.bfloat16, device=DEV)
    y = torch.empty(big.shape, dtype=torch.float8_e4m3fn, device=DEV)
    d = torch.empty(QUANT_MAX_SCALES + 8, dtype=torch.float32, device=DEV)
    rc = lib.fa4cp_quantize_e4m3_noalloc(ctypes.byref(_args(big, y, d, None, 1)), _lib.stream_handle(DEV))
    assert rc == -2 and b"scales, at most 1024" in lib.fa4cp_last_error()
    torch.cuda.synchronize()
