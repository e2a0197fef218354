"""FP8 producer (fa4cp_quantize_e4m3) on the GPU: amax, descales and e4m3 bytes against the
oracle's quantisation (fp32 quotient, clamp, round to nearest even), bit for bit, and the
producer feeding the e4m3 ring sweep."""

import pytest
import torch

from fa4_ring import LocalKVRing, RingConfig, quantize_e4m3, quantize_ring, ring_flash_attn, zigzag_shard
from gpu_helpers import DEV, TOL_FP8_OUT, max_err, say, scale_for
from oracle import ring_oracle as O

pytestmark = pytest.mark.gpu


def _oracle(x: torch.Tensor, g: int):
    """(e4m3 bytes [rows, h, d], descales as float32) of the oracle, scale groups of g heads."""
    xf = x.float()
    h = x.shape[1]
    groups = [(0, h)] if g == 0 else [(i, i + g) for i in range(0, h, g)]
    ys, ds = [], []
    for a, b in groups:
        s = O.amax_scale(xf[:, a:b])
        ys.append(O.quantize_e4m3(xf[:, a:b], s))
        ds.append(s)
    return torch.cat(ys, dim=1).view(torch.uint8), torch.tensor(ds, dtype=torch.float32)


def _heads_scaled(rows, h, d, dtype, seed):
    """N(0, 1) * 3 with each head on its own range (so per-head scales differ)."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, h, d, generator=gen) * 3
    x = x * torch.logspace(-2, 2, h).reshape(1, h, 1)
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,h,d,g", [(1000, 8, 128, 0), (333, 32, 128, 4), (17, 2, 256, 1),
                                        (64, 16, 64, 2), (5, 1, 16, 0), (4096, 8, 128, 1),
                                        (9, 24, 512, 6), (9, 48, 512, 6)])
def test_quantize_matches_oracle(dtype, rows, h, d, g):
    """The last two cases have rows of more than 2048 16-byte chunks (fp32 / 16-bit); fp32
    rows of more than 4096 chunks are refused."""
    say(f"quantize_e4m3 {dtype} rows={rows} h={h} d={d} heads_per_scale={g}")
    x = _heads_scaled(rows, h, d, dtype, seed=rows + h)
    if h * d * x.element_size() > 16 * 4096:
        with pytest.raises(RuntimeError, match="elements per row"):
            quantize_e4m3(x.to(DEV), heads_per_scale=g)
        return
    y, ds = quantize_e4m3(x.to(DEV), heads_per_scale=g)
    y_ref, ds_ref = _oracle(x, g)
    assert y.dtype == torch.float8_e4m3fn and y.shape == (rows, h, d)
    assert ds.shape == (() if g == 0 else (h // g,))
    assert torch.equal(ds.reshape(-1).cpu(), ds_ref), "descales"
    assert torch.equal(y.view(torch.uint8).cpu(), y_ref), "e4m3 bytes"
    # the largest magnitude of every group maps to +-448
    assert int((y.view(torch.uint8).cpu() & 0x7F).max()) == 0x7E


def _e4m3_midpoints() -> torch.Tensor:
    """The 126 points halfway between consecutive non-negative e4m3 values (fp32, exact)."""
    vals = torch.arange(0, 0x7F, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float()
    vals = vals.sort().values
    return (vals[:-1] + vals[1:]) / 2


@pytest.mark.parametrize("amax", [1.0, 3.7, 0.0123, 1000.5, 1.3 * 2.0 ** -20])
def test_quantize_rounds_at_every_e4m3_midpoint(amax):
    """fp32 inputs a few ulps either side of every e4m3 rounding midpoint (times the scale),
    both signs: the quotient x / scale must be the correctly rounded one wherever that decides
    the e4m3 byte, as the oracle's fp32 division and round-to-nearest-even conversion give."""
    say(f"quantize_e4m3 midpoint sweep amax={amax}")
    s = torch.tensor(amax, dtype=torch.float32) / 448  # the producer's scale, in fp32
    x0 = (_e4m3_midpoints() * s).float()
    xs = [x0]
    lo, hi = x0.clone(), x0.clone()
    for _ in range(3):
        lo = torch.nextafter(lo, torch.tensor(-float("inf")))
        hi = torch.nextafter(hi, torch.tensor(float("inf")))
        xs += [lo, hi]
    x = torch.cat(xs)
    x = torch.cat([x, -x, torch.tensor([amax], dtype=torch.float32)])
    x = x[x.abs() <= amax]
    pad = (-x.numel()) % 16
    x = torch.cat([x, torch.zeros(pad)]).reshape(-1, 1, 16)
    y, ds = quantize_e4m3(x.to(DEV))
    y_ref, ds_ref = _oracle(x, 0)
    assert float(ds) == float(ds_ref[0]) == float(s)
    assert torch.equal(y.view(torch.uint8).cpu(), y_ref)


def test_quantize_strided_input():
    say("quantize_e4m3 strided head stride")
    base = _heads_scaled(300, 4, 136, torch.bfloat16, seed=9)
    xd = base.to(DEV)[:, :, :128]
    assert xd.stride() == (4 * 136, 136, 1)
    y, ds = quantize_e4m3(xd, heads_per_scale=1)
    y_ref, ds_ref = _oracle(base[:, :, :128], 1)
    assert torch.equal(ds.cpu(), ds_ref) and torch.equal(y.view(torch.uint8).cpu(), y_ref)


def test_quantize_zero_and_empty():
    say("quantize_e4m3 all-zero and empty")
    y, ds = quantize_e4m3(torch.zeros(64, 2, 128, dtype=torch.bfloat16, device=DEV), heads_per_scale=1)
    assert ds.tolist() == [1.0, 1.0] and int(y.view(torch.uint8).abs().sum()) == 0
    y, ds = quantize_e4m3(torch.zeros(0, 2, 128, dtype=torch.bfloat16, device=DEV))
    assert y.shape == (0, 2, 128) and float(ds) == 1.0


def test_quantize_rejects_bad_arguments():
    say("quantize_e4m3 argument checks")
    with pytest.raises(AssertionError):
        quantize_e4m3(torch.zeros(8, 3, 128, dtype=torch.bfloat16, device=DEV), heads_per_scale=2)
    with pytest.raises(RuntimeError, match="multiple"):
        quantize_e4m3(torch.zeros(8, 2, 12, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(RuntimeError, match="elements per row"):
        quantize_e4m3(torch.zeros(8, 64, 1024, dtype=torch.bfloat16, device=DEV))


@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("fused", [True, False])
def test_producer_feeds_the_e4m3_sweep(per_head, fused):
    n, h, hkv, d, cp = 2048, 8, 2, 128, 4
    say(f"quantize_ring -> e4m3 sweep per_head={per_head} fused={fused}")
    q, k, v = O.random_qkv(n, h, hkv, d, seed=11)
    scale = scale_for(d)
    ks = [zigzag_shard(k.to(DEV), r, cp) for r in range(cp)]
    vs = [zigzag_shard(v.to(DEV), r, cp) for r in range(cp)]
    for rank in range(cp):
        lq = zigzag_shard(q.to(DEV), rank, cp)
        q8, k8, v8, desc = quantize_ring(lq, ks, vs, per_head=per_head)
        ring = LocalKVRing(k8, v8)
        out = ring_flash_attn(q8, ring.k[rank], ring.v[rank], RingConfig(cp_size=cp, cp_rank=rank), group=ring,
                              descales=desc, fused=fused)
        # the oracle on the dequantised tensors (q descale per kv-head group of heads)
        qs = desc.q.reshape(-1).cpu().repeat_interleave(h // desc.q.numel()) if per_head else desc.q.cpu()
        dq = q8.float().cpu() * (qs.reshape(1, -1, 1) if per_head else qs)
        dk = [x.float().cpu() * s.reshape(1, -1, 1).cpu() for x, s in zip(k8, desc.k)]
        dv = [x.float().cpu() * s.reshape(1, -1, 1).cpu() for x, s in zip(v8, desc.v)]
        ref, _ = O.ring_rank(dq, dk, dv, rank, cp, scale)
        assert max_err(out, ref) <= TOL_FP8_OUT, f"rank {rank}"
        # and the dequantised inputs are close to the originals (scale / 16 per element at most)
        assert float((dq - O.zigzag_shard(q, rank, cp)).abs().max()) <= float(qs.max()) * 448 / 16
