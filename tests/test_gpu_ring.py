"""GPU parity of the whole per-rank ring sweep (ring_flash_attn on the HIP kernels).

Small shapes: every rank against the oracle's ring (same rounded inputs) and the stitched
output against dense causal attention.  Benchmark sizes: one rank's sweep checked on
sampled rows against exact dense causal attention (a row's ring output must equal plain
causal attention over every key before it), plus run-to-run bit reproducibility.
"""

import functools
import math

import numpy as np
import pytest
import torch

from fa4_ring import Descales, LocalKVRing, RingConfig, ring_flash_attn, zigzag_shard, zigzag_unshard
from fa4_ring.reference import full_causal_reference
from fa4_ring.zigzag import zigzag_shard_varlen, zigzag_unshard_varlen
from gpu_helpers import DEV, TOL_BF16_OUT, TOL_FP8_OUT, TOL_LSE, lse_err, max_err, rounded, say, scale_for
from oracle import ring_oracle as O

pytestmark = pytest.mark.gpu

SMALL_CASES = [  # (N, H, H_kv, D, cp): the reference's CPU cases' structure at GPU head dims
    (256, 4, 4, 64, 2), (512, 8, 2, 128, 4), (1024, 8, 8, 64, 4), (1024, 4, 1, 128, 8),
    (2048, 8, 2, 128, 8), (768, 6, 3, 64, 2), (1536, 8, 8, 128, 4),
    (2048, 8, 2, 128, 4),  # the CPU benchmark configuration's shape
    (1024, 16, 2, 128, 4), (1024, 16, 1, 64, 2),  # GQA 8 and 16 query heads per kv head
    (2048, 4, 2, 128, 16),  # the largest ring the fused sweep takes
    (1024, 8, 2, 256, 4), (512, 4, 4, 256, 2), (2048, 16, 2, 256, 8),  # head dim 256 (32-key tiles)
    (1024, 4, 2, 256, 4),  # head dim 256, two query heads per kv head
]


def _device_ring(q, k, v, cp, dtype):
    qd, kd, vd = (t.to(dtype).to(DEV) for t in (q, k, v))
    return qd, LocalKVRing.from_full(kd, vd, cp)


PATHS = ["fused", "incremental", "batched"]  # one-kernel sweep; per-step paths with merges


def _cfg_path(path, cp, rank):
    """RingConfig and ring_flash_attn `fused` flag of a test path."""
    mode = "incremental" if path == "fused" else path
    return RingConfig(cp_size=cp, cp_rank=rank, merge_mode=mode), path == "fused"


@pytest.mark.parametrize("mode", PATHS)
@pytest.mark.parametrize("n,h,hkv,d,cp", SMALL_CASES)
def test_ring_all_ranks_small(n, h, hkv, d, cp, mode):
    say(f"ring bf16 n={n} h={h}/{hkv} d={d} cp={cp} path={mode}")
    q, k, v = O.random_qkv(n, h, hkv, d, seed=0)
    q, k, v = (rounded(t, torch.bfloat16) for t in (q, k, v))
    scale = scale_for(d)
    qd, ring = _device_ring(q, k, v, cp, torch.bfloat16)
    ks = [O.zigzag_shard(k, r, cp) for r in range(cp)]
    vs = [O.zigzag_shard(v, r, cp) for r in range(cp)]
    outs = []
    for rank in range(cp):
        cfg, fused = _cfg_path(mode, cp, rank)
        out, lse = ring_flash_attn(zigzag_shard(qd, rank, cp), ring.k[rank], ring.v[rank], cfg, group=ring,
                                   fused=fused, return_lse=True)
        assert out.dtype == torch.bfloat16 and out.shape == (n // cp, h, d)
        assert lse.dtype == torch.float32 and lse.shape == (n // cp, h)
        ref, ref_lse = O.ring_rank(O.zigzag_shard(q, rank, cp), ks, vs, rank, cp, scale,
                                   merge_mode=cfg.merge_mode)
        assert max_err(out, ref) <= TOL_BF16_OUT, f"rank {rank}"
        assert lse_err(lse, ref_lse) <= TOL_LSE, f"rank {rank} lse"
        outs.append(out.float().cpu())
    dense = O.dense_causal(q, k, v, scale)
    assert max_err(O.zigzag_unshard(outs, cp), dense) <= TOL_BF16_OUT


@pytest.mark.parametrize("mode", PATHS)
@pytest.mark.parametrize("d", [128, 256])
def test_ring_fp16_all_ranks(d, mode):
    """fp16 inputs and out on every rank of a cp 4 ring, at both 64-key (D 128) and 32-key
    (D 256) tiles, against the oracle at the fp16 bar (5e-3) and dense causal attention."""
    n, h, hkv, cp = 1024, 8, 2, 4
    say(f"ring fp16 n={n} h={h}/{hkv} d={d} cp={cp} path={mode}")
    q, k, v = O.random_qkv(n, h, hkv, d, seed=6)
    q, k, v = (rounded(t, torch.float16) for t in (q, k, v))
    scale = scale_for(d)
    qd, ring = _device_ring(q, k, v, cp, torch.float16)
    ks = [O.zigzag_shard(k, r, cp) for r in range(cp)]
    vs = [O.zigzag_shard(v, r, cp) for r in range(cp)]
    outs = []
    for rank in range(cp):
        cfg, fused = _cfg_path(mode, cp, rank)
        out, lse = ring_flash_attn(zigzag_shard(qd, rank, cp), ring.k[rank], ring.v[rank], cfg, group=ring,
                                   fused=fused, return_lse=True)
        assert out.dtype == torch.float16
        ref, ref_lse = O.ring_rank(O.zigzag_shard(q, rank, cp), ks, vs, rank, cp, scale, merge_mode=cfg.merge_mode)
        assert max_err(out, ref) <= 5e-3, f"rank {rank}"
        assert lse_err(lse, ref_lse) <= TOL_LSE, f"rank {rank} lse"
        outs.append(out.float().cpu())
    assert max_err(O.zigzag_unshard(outs, cp), O.dense_causal(q, k, v, scale)) <= 5e-3


@functools.lru_cache(maxsize=4)
def _reference_gpu_case(dtype_name: str, num_seqs: int):
    """Inputs and dense fp32 reference of the reference's own GPU test at its defaults
    (tests/test_ring_correctness.py:41-47: N=4096, H=16, H_kv=4, D=128, 4 ranks, seed 1234,
    ~N(0,1) in the test dtype; the generator here is the CPU one, so the draws differ), each
    packed sequence compared on its own (block-diagonal causal, :96-103)."""
    dtype = getattr(torch, dtype_name)
    n, h, hkv, d = 4096, 16, 4, 128
    gen = torch.Generator().manual_seed(1234)
    q = torch.randn(n, h, d, generator=gen).to(dtype)
    k = torch.randn(n, hkv, d, generator=gen).to(dtype)
    v = torch.randn(n, hkv, d, generator=gen).to(dtype)
    per = n // num_seqs
    ref = torch.cat([full_causal_reference(q[i * per:(i + 1) * per], k[i * per:(i + 1) * per],
                                           v[i * per:(i + 1) * per]) for i in range(num_seqs)]).float()
    return q, k, v, ref


@pytest.mark.parametrize("num_seqs", [1, 4])
@pytest.mark.parametrize("mode", PATHS)
@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
def test_reference_gpu_test_configuration(dtype_name, mode, num_seqs):
    """The reference's GPU correctness check (test_ring_correctness.py:55-116) on one GPU: every
    rank's sweep over its zig-zag shard, the outputs stitched back and compared with dense
    causal attention over the whole sequence, max error below 2e-2 (bf16) / 5e-3 (fp16) and
    cosine similarity above 0.999 (:108-109)."""
    world = 4
    say(f"reference GPU test config dtype={dtype_name} path={mode} num_seqs={num_seqs}")
    q, k, v, ref = _reference_gpu_case(dtype_name, num_seqs)
    n = q.shape[0]
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    full_cu = list(range(0, n + 1, n // num_seqs))
    ring = LocalKVRing.from_full(kd, vd, world, full_cu if num_seqs > 1 else None)
    outs = []
    for rank in range(world):
        cfg, fused = _cfg_path(mode, world, rank)
        if num_seqs > 1:
            lq, local_cu = zigzag_shard_varlen(qd, full_cu, rank, world)
            max_local = int((local_cu[1:] - local_cu[:-1]).max())
            out = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, cu_seqlens=local_cu,
                                  max_seqlen=max_local, fused=fused)
        else:
            out = ring_flash_attn(zigzag_shard(qd, rank, world), ring.k[rank], ring.v[rank], cfg, group=ring,
                                  fused=fused)
        assert out.dtype == q.dtype
        outs.append(out)
    full = (zigzag_unshard_varlen(outs, full_cu, world) if num_seqs > 1 else zigzag_unshard(outs, world))
    full = full.float().cpu()
    err = float((full - ref).abs().max())
    # in float64: an fp32 cosine over 8M elements drifts above 1
    cos = float(torch.nn.functional.cosine_similarity(full.double().flatten(), ref.double().flatten(), dim=0))
    tol = 2e-2 if dtype_name == "bfloat16" else 5e-3
    say(f"  max_err={err:.3e} cos={cos:.6f}")
    assert err < tol and cos > 0.999


@pytest.mark.parametrize("dtype_name,d,h,hkv", [("bfloat16", 128, 8, 2), ("float16", 64, 4, 4),
                                                ("bfloat16", 256, 4, 1)])
def test_full_causal_reference_hip_matches_torch(dtype_name, d, h, hkv):
    """full_causal_reference's two backends agree: the library's causal kernel over the whole
    sequence against the fp32 blocked reference (and both against the oracle)."""
    dtype = getattr(torch, dtype_name)
    say(f"full_causal_reference hip vs torch {dtype_name} d={d} h={h}/{hkv}")
    q, k, v = O.random_qkv(1536, h, hkv, d, seed=13)
    q, k, v = (rounded(x, dtype) for x in (q, k, v))
    qd, kd, vd = (x.to(dtype).to(DEV) for x in (q, k, v))
    hip = full_causal_reference(qd, kd, vd, backend="hip")
    ref = full_causal_reference(qd, kd, vd, backend="torch")
    assert hip.dtype == ref.dtype == dtype
    tol = TOL_BF16_OUT if dtype == torch.bfloat16 else 5e-3
    assert max_err(hip, ref) <= tol
    assert max_err(ref, O.dense_causal(q, k, v, scale_for(d))) <= tol


def test_ring_cp1_is_causal_attention():
    say("ring cp=1")
    q, k, v = O.random_qkv(512, 8, 2, 128, seed=2)
    q, k, v = (rounded(t, torch.bfloat16) for t in (q, k, v))
    out = ring_flash_attn(q.to(torch.bfloat16).to(DEV), k.to(torch.bfloat16).to(DEV),
                          v.to(torch.bfloat16).to(DEV), RingConfig(cp_size=1, cp_rank=0))
    assert max_err(out, O.dense_causal(q, k, v, scale_for(128))) <= TOL_BF16_OUT


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("mode", PATHS)
def test_ring_varlen_all_ranks(mode, d):
    lens = [608, 1216, 1072, 608, 232, 1928, 344, 200]  # the packed benchmark lengths / 8
    cp, h, hkv = 4, 8, 2
    say(f"ring varlen lens={lens} cp={cp} d={d} path={mode}")
    full_cu = [0]
    for n in lens:
        full_cu.append(full_cu[-1] + n)
    q, k, v = O.random_qkv(full_cu[-1], h, hkv, d, seed=3)
    q, k, v = (rounded(t, torch.bfloat16) for t in (q, k, v))
    scale = scale_for(d)
    qd, kd, vd = (t.to(torch.bfloat16).to(DEV) for t in (q, k, v))
    ring = LocalKVRing.from_full(kd, vd, cp, full_cu)
    ks = [O.zigzag_shard_varlen(k, full_cu, r, cp)[0] for r in range(cp)]
    vs = [O.zigzag_shard_varlen(v, full_cu, r, cp)[0] for r in range(cp)]
    outs = []
    for rank in range(cp):
        lq, local_cu = zigzag_shard_varlen(qd, full_cu, rank, cp)
        max_local = int((local_cu[1:] - local_cu[:-1]).max())
        cfg, fused = _cfg_path(mode, cp, rank)
        out, lse = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring,
                                   cu_seqlens=local_cu, max_seqlen=max_local, fused=fused, return_lse=True)
        oq, ocu = O.zigzag_shard_varlen(q, full_cu, rank, cp)
        ref, ref_lse = O.ring_rank(oq, ks, vs, rank, cp, scale, cu=ocu, merge_mode=cfg.merge_mode)
        assert max_err(out, ref) <= TOL_BF16_OUT, f"rank {rank}"
        assert lse_err(lse, ref_lse) <= TOL_LSE, f"rank {rank} lse"
        outs.append(out.float().cpu())
    lcu = O.local_cu_from_full(full_cu, cp)
    for j in range(len(lens)):
        seq = O.zigzag_unshard([outs[r][lcu[j]:lcu[j + 1]] for r in range(cp)], cp)
        s, e = full_cu[j], full_cu[j + 1]
        assert max_err(seq, O.dense_causal(q[s:e], k[s:e], v[s:e], scale)) <= TOL_BF16_OUT


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("mode", ["fused", "incremental"])
def test_ring_varlen_many_sequences(mode, d):
    """80 packed sequences (some empty, some of 4 rows): every kernel finds a sequence's V^T
    start by summing the padded lengths of up to 79 earlier ones, 64 per wavefront pass; at
    head dim 256 with 32-key tiles, most segments end in a partial tile."""
    cp, h, hkv = 2, 4, 2
    g = torch.Generator().manual_seed(12)
    lens = (torch.randint(0, 33, (80,), generator=g) * 4).tolist()
    lens[5] = 0
    lens[66] = 4
    say(f"ring varlen {len(lens)} sequences cp={cp} d={d} path={mode}")
    full_cu = [0]
    for n in lens:
        full_cu.append(full_cu[-1] + n)
    q, k, v = O.random_qkv(full_cu[-1], h, hkv, d, seed=4)
    q, k, v = (rounded(t, torch.bfloat16) for t in (q, k, v))
    scale = scale_for(d)
    qd, kd, vd = (t.to(torch.bfloat16).to(DEV) for t in (q, k, v))
    ring = LocalKVRing.from_full(kd, vd, cp, full_cu)
    ks = [O.zigzag_shard_varlen(k, full_cu, r, cp)[0] for r in range(cp)]
    vs = [O.zigzag_shard_varlen(v, full_cu, r, cp)[0] for r in range(cp)]
    for rank in range(cp):
        lq, local_cu = zigzag_shard_varlen(qd, full_cu, rank, cp)
        max_local = int((local_cu[1:] - local_cu[:-1]).max())
        cfg, fused = _cfg_path(mode, cp, rank)
        out, lse = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring,
                                   cu_seqlens=local_cu, max_seqlen=max_local, fused=fused, return_lse=True)
        oq, ocu = O.zigzag_shard_varlen(q, full_cu, rank, cp)
        ref, ref_lse = O.ring_rank(oq, ks, vs, rank, cp, scale, cu=ocu, merge_mode=cfg.merge_mode)
        assert max_err(out, ref) <= TOL_BF16_OUT, f"rank {rank}"
        assert lse_err(lse, ref_lse) <= TOL_LSE, f"rank {rank} lse"


def _fp8_ring_inputs(q, k, v, cp, rank, full_cu=None):
    """Per-tensor q scale (local shard amax / 448), per-source-rank k / v scales."""
    if full_cu is None:
        lq = O.zigzag_shard(q, rank, cp)
        ks = [O.zigzag_shard(k, r, cp) for r in range(cp)]
        vs = [O.zigzag_shard(v, r, cp) for r in range(cp)]
    else:
        lq = O.zigzag_shard_varlen(q, full_cu, rank, cp)[0]
        ks = [O.zigzag_shard_varlen(k, full_cu, r, cp)[0] for r in range(cp)]
        vs = [O.zigzag_shard_varlen(v, full_cu, r, cp)[0] for r in range(cp)]
    sq = O.amax_scale(lq)
    sk = [O.amax_scale(x) for x in ks]
    sv = [O.amax_scale(x) for x in vs]
    q8 = O.quantize_e4m3(lq, sq)
    k8 = [O.quantize_e4m3(x, s) for x, s in zip(ks, sk)]
    v8 = [O.quantize_e4m3(x, s) for x, s in zip(vs, sv)]
    deq = (O.dequantize_e4m3(q8, sq), [O.dequantize_e4m3(x, s) for x, s in zip(k8, sk)],
           [O.dequantize_e4m3(x, s) for x, s in zip(v8, sv)])
    return (q8, k8, v8, sq, sk, sv), deq


@pytest.mark.parametrize("mode", PATHS)
@pytest.mark.parametrize("n,h,hkv,d,cp", [(2048, 8, 2, 128, 8), (1024, 16, 2, 256, 4),
                                          (1024, 8, 8, 128, 2), (2048, 16, 1, 128, 16)])
def test_ring_fp8_all_ranks(n, h, hkv, d, cp, mode):
    say(f"ring e4m3 n={n} h={h}/{hkv} d={d} cp={cp} mode={mode}")
    q, k, v = O.random_qkv(n, h, hkv, d, seed=4)
    scale = scale_for(d)
    for rank in range(cp):
        (q8, k8, v8, sq, sk, sv), (dq, dk, dv) = _fp8_ring_inputs(q, k, v, cp, rank)
        ring = LocalKVRing([x.to(DEV) for x in k8], [x.to(DEV) for x in v8])
        desc = Descales(q=torch.tensor(sq, device=DEV),
                        k=[torch.tensor(s, device=DEV) for s in sk],
                        v=[torch.tensor([s] * hkv, device=DEV) for s in sv])
        cfg, fused = _cfg_path(mode, cp, rank)
        out, lse = ring_flash_attn(q8.to(DEV), ring.k[rank], ring.v[rank], cfg, group=ring, descales=desc,
                                   fused=fused, return_lse=True)
        assert out.dtype == torch.bfloat16
        ref, ref_lse = O.ring_rank(dq, dk, dv, rank, cp, scale, merge_mode=cfg.merge_mode)
        assert max_err(out, ref) <= TOL_FP8_OUT, f"rank {rank}"
        assert lse_err(lse, ref_lse) <= TOL_LSE, f"rank {rank} lse"


@pytest.mark.parametrize("mode", PATHS)
@pytest.mark.parametrize("dtype_name,d", [("bf16", 96), ("fp16", 48), ("bf16", 192), ("e4m3", 64)])
def test_ring_padded_head_dim_all_ranks(dtype_name, d, mode):
    """Head dims without a kernel: ring_flash_attn pads Q and every shard once and runs the
    sweep at the next supported head dim; every rank against the oracle's ring."""
    n, h, hkv, cp = 1024, 8, 2, 4
    say(f"ring padded head dim {dtype_name} d={d} n={n} cp={cp} path={mode}")
    q, k, v = O.random_qkv(n, h, hkv, d, seed=6)
    scale = scale_for(d)
    for rank in range(cp):
        cfg, fused = _cfg_path(mode, cp, rank)
        if dtype_name == "e4m3":
            (q8, k8, v8, sq, sk, sv), (lq, ks, vs) = _fp8_ring_inputs(q, k, v, cp, rank)
            ring = LocalKVRing([x.to(DEV) for x in k8], [x.to(DEV) for x in v8])
            desc = Descales(q=torch.tensor(sq, device=DEV), k=[torch.tensor(s, device=DEV) for s in sk],
                            v=[torch.tensor(s, device=DEV) for s in sv])
            out, lse = ring_flash_attn(q8.to(DEV), ring.k[rank], ring.v[rank], cfg, group=ring, descales=desc,
                                       fused=fused, return_lse=True)
            tol = TOL_FP8_OUT
        else:
            dt = torch.bfloat16 if dtype_name == "bf16" else torch.float16
            qr, kr, vr = (rounded(t, dt) for t in (q, k, v))
            qd, ring = _device_ring(qr, kr, vr, cp, dt)
            lq = O.zigzag_shard(qr, rank, cp)
            ks = [O.zigzag_shard(kr, r, cp) for r in range(cp)]
            vs = [O.zigzag_shard(vr, r, cp) for r in range(cp)]
            out, lse = ring_flash_attn(zigzag_shard(qd, rank, cp), ring.k[rank], ring.v[rank], cfg, group=ring,
                                       fused=fused, return_lse=True)
            tol = TOL_BF16_OUT
        assert out.shape == (n // cp, h, d) and out.is_contiguous()
        ref, ref_lse = O.ring_rank(lq, ks, vs, rank, cp, scale, merge_mode=cfg.merge_mode)
        assert max_err(out, ref) <= tol, f"rank {rank}"
        assert lse_err(lse, ref_lse) <= TOL_LSE, f"rank {rank} lse"


def test_ring_inputs_not_contiguous_in_d():
    """local q and every K / V shard with a strided head dim: copied to contiguous rows, the
    sweep's result equals the one on contiguous inputs bit for bit."""
    n, h, hkv, d, cp, rank = 1024, 8, 2, 128, 4, 2
    say(f"ring inputs strided in D n={n} cp={cp} rank={rank}")
    q, k, v = O.random_qkv(n, h, hkv, d, seed=8)
    qd, ring = _device_ring(q, k, v, cp, torch.bfloat16)
    strided = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)  # noqa: E731
    ring_s = LocalKVRing([strided(x) for x in ring.k], [strided(x) for x in ring.v])
    lq = zigzag_shard(qd, rank, cp)
    cfg = RingConfig(cp_size=cp, cp_rank=rank)
    want = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring)
    got = ring_flash_attn(strided(lq), strided(ring.k[rank]), strided(ring.v[rank]), cfg, group=ring_s)
    assert torch.equal(got, want)


@pytest.mark.parametrize("mode", PATHS)
def test_ring_fp8_varlen_all_ranks(mode):
    lens = [608, 1216, 1072, 608, 232, 1928, 344, 200]
    cp, h, hkv, d = 4, 8, 2, 128
    say(f"ring e4m3 varlen lens={lens} cp={cp} path={mode}")
    full_cu = [0]
    for n in lens:
        full_cu.append(full_cu[-1] + n)
    q, k, v = O.random_qkv(full_cu[-1], h, hkv, d, seed=6)
    scale = scale_for(d)
    for rank in range(cp):
        (q8, k8, v8, sq, sk, sv), (dq, dk, dv) = _fp8_ring_inputs(q, k, v, cp, rank, full_cu)
        ring = LocalKVRing([x.to(DEV) for x in k8], [x.to(DEV) for x in v8])
        desc = Descales(q=torch.tensor(sq, device=DEV), k=[torch.tensor(s, device=DEV) for s in sk],
                        v=[torch.tensor([s] * hkv, device=DEV) for s in sv])
        local_cu = torch.tensor(O.local_cu_from_full(full_cu, cp), dtype=torch.int32)
        max_local = int((local_cu[1:] - local_cu[:-1]).max())
        cfg, fused = _cfg_path(mode, cp, rank)
        out, lse = ring_flash_attn(q8.to(DEV), ring.k[rank], ring.v[rank], cfg, group=ring, descales=desc,
                                   cu_seqlens=local_cu.to(DEV), max_seqlen=max_local, fused=fused,
                                   return_lse=True)
        assert out.dtype == torch.bfloat16
        ref, ref_lse = O.ring_rank(dq, dk, dv, rank, cp, scale, cu=local_cu.tolist(), merge_mode=cfg.merge_mode)
        assert max_err(out, ref) <= TOL_FP8_OUT, f"rank {rank}"
        assert lse_err(lse, ref_lse) <= TOL_LSE, f"rank {rank} lse"


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("mode", PATHS)
@pytest.mark.parametrize("growth", [5.0, 8.8, 150.0])
def test_ring_fp8_row_max_grows_inside_a_later_source(growth, mode, d):
    """The row max jumps by `growth` (log2 units) on key 300 of the second source (rank 1 of
    2: local causal keys, then the front half of source 0; the third 128-key tile at head dim
    128, the fifth 64-key tile at 256, where the mask, row max and rescale run in the softmax
    phase), whose v descale is ten times the first source's: 5 stays under the lazy-rescale
    bound, 8.8 moves the reference max mid-segment (O must change units once, at the segment
    start, not again here), 150 overflows the exponentials taken against the old max."""
    n, h, hkv, cp, rank = 2048, 2, 1, 2, 1
    say(f"ring e4m3 late max growth={growth} d={d} path={mode}")
    g = torch.Generator().manual_seed(8)
    u = torch.randn(d, generator=g)
    u = u / u.norm()
    a = 4.0
    scale = scale_for(d)
    q = (a * u).expand(n, h, d).clone()
    k = 1e-3 * torch.randn(n, hkv, d, generator=g)
    k[300, 0] = u * (growth * math.log(2) / (a * scale))  # source 0, local key 300: tile 2
    v = 4 * torch.randn(n, hkv, d, generator=g)
    v[512:1536] = 1 + 0.1 * torch.randn(1024, hkv, d, generator=g)  # source 1's keys, mean 1
    (q8, k8, v8, sq, sk, sv), (dq, dk, dv) = _fp8_ring_inputs(q, k, v, cp, rank)
    assert sv[0] > 5 * sv[1]
    ring = LocalKVRing([x.to(DEV) for x in k8], [x.to(DEV) for x in v8])
    desc = Descales(q=torch.tensor(sq, device=DEV), k=[torch.tensor(s, device=DEV) for s in sk],
                    v=[torch.tensor(s, device=DEV) for s in sv])
    cfg, fused = _cfg_path(mode, cp, rank)
    out = ring_flash_attn(q8.to(DEV), ring.k[rank], ring.v[rank], cfg, group=ring, descales=desc,
                          fused=fused)
    ref, _ = O.ring_rank(dq, dk, dv, rank, cp, scale, merge_mode=cfg.merge_mode)
    assert torch.isfinite(out.float()).all()
    assert max_err(out, ref) <= TOL_FP8_OUT


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("mode", PATHS)
@pytest.mark.parametrize("growth", [5.0, 8.8, 150.0])
def test_ring_bf16_row_max_grows_mid_sweep(growth, mode, d):
    """As the e4m3 case above in bf16: the row max jumps by `growth` (log2 units) on key 300 of
    source 0, inside rank 1's second step (its fifth 64-key tile at head dim 128, its tenth
    32-key tile at 256)."""
    n, h, hkv, cp, rank = 2048, 2, 1, 2, 1
    say(f"ring bf16 late max growth={growth} d={d} path={mode}")
    g = torch.Generator().manual_seed(9)
    u = torch.randn(d, generator=g)
    u = u / u.norm()
    a = 4.0
    scale = scale_for(d)
    q = (a * u).expand(n, h, d).clone()
    k = 1e-3 * torch.randn(n, hkv, d, generator=g)
    k[300, 0] = u * (growth * math.log(2) / (a * scale))
    # outputs of order 1, where the absolute bf16 bound applies (the per-step paths round each
    # step's output and the merged accumulator to bf16)
    v = 0.5 * torch.randn(n, hkv, d, generator=g)
    v[512:1536] = 0.5 + 0.05 * torch.randn(1024, hkv, d, generator=g)
    q, k, v = (rounded(t, torch.bfloat16) for t in (q, k, v))
    qd, ring = _device_ring(q, k, v, cp, torch.bfloat16)
    cfg, fused = _cfg_path(mode, cp, rank)
    out = ring_flash_attn(zigzag_shard(qd, rank, cp), ring.k[rank], ring.v[rank], cfg, group=ring, fused=fused)
    ks = [O.zigzag_shard(k, r, cp) for r in range(cp)]
    vs = [O.zigzag_shard(v, r, cp) for r in range(cp)]
    ref, _ = O.ring_rank(O.zigzag_shard(q, rank, cp), ks, vs, rank, cp, scale, merge_mode=cfg.merge_mode)
    assert torch.isfinite(out.float()).all()
    assert max_err(out, ref) <= TOL_BF16_OUT


# ----------------------------------------------------------------- benchmark sizes
#
# At full size the oracle cannot run the whole sweep, so every rank output is checked two
# ways: one row of every 64-row tile (a seeded random row inside the tile, plus the shard's
# first, middle and last rows), every head, out and LSE, against exact dense causal
# attention; and, on the device over every row, the fused sweep against the per-step form
# (two different kernels: a mis-scheduled row tile or head group of one shows as a
# difference there).


def _tile_rows(t, seed, tile=64):
    rng = np.random.default_rng(seed)
    rows = {int(t0 + rng.integers(0, min(tile, t - t0))) for t0 in range(0, t, tile)}
    rows.update([0, t // 2 - 1, t // 2, t - 1])
    return sorted(r for r in rows if 0 <= r < t)


def _check_tiles(name, outs, lq_f, rows, positions, starts, k_full, v_full, scale, tol):
    """Every form's out / lse (device, local rows) against dense causal attention at the
    given rows, every head.  lq_f: the local q in fp32 on the host (the device inputs,
    dequantised)."""
    exp, exp_lse = O.dense_causal_rows_all_heads(lq_f[rows], positions, starts, k_full, v_full, scale)
    idx = torch.tensor(rows, device=DEV)
    for form, (out, lse) in outs.items():
        got = out.index_select(0, idx).float().cpu()
        got_lse = lse.index_select(0, idx).cpu()
        err = float((got - exp).abs().max())
        lerr = float((got_lse - exp_lse).abs().max())
        say(f"  {name} {form}: {len(rows)} rows x {out.shape[1]} heads: max |out err| {err:.3e} (bar {tol}), "
            f"max |lse err| {lerr:.3e} (bar {TOL_LSE})")
        assert err <= tol, f"{name} {form}: out {err}"
        assert lerr <= TOL_LSE, f"{name} {form}: lse {lerr}"


def _check_forms_agree(name, ref_form, outs, tol):
    """Every row of every form against the reference form, on the device."""
    o0, l0 = outs[ref_form]
    for form, (o, l) in outs.items():
        if form == ref_form:
            continue
        e = float((o.float() - o0.float()).abs().max())
        le = float((l - l0).abs().max())
        say(f"  {name}: {form} vs {ref_form} over all rows: max |out diff| {e:.3e}, max |lse diff| {le:.3e}")
        assert e <= tol and le <= TOL_LSE, f"{name}: {form} differs from {ref_form}: {e}, {le}"


def _run_forms(lq, ring, cp, rank, forms, **kw):
    outs = {}
    for form in forms:
        cfg, fused = _cfg_path(form, cp, rank)
        outs[form] = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, fused=fused,
                                     return_lse=True, **kw)
    return outs


@pytest.mark.parametrize("rank", [3, 7])
def test_ring_c2_bf16_full_size(rank):
    n, cp, hq, hkv, d = 131072, 8, 32, 8, 128
    say(f"ring C2 bf16 n={n} rank={rank}")
    gen = torch.Generator(device=DEV).manual_seed(0)
    q = torch.randn(n, hq, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    k = torch.randn(n, hkv, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    v = torch.randn(n, hkv, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    ring = LocalKVRing.from_full(k, v, cp)
    lq = zigzag_shard(q, rank, cp)
    del q
    outs = _run_forms(lq, ring, cp, rank, PATHS)
    for form, fused in (("fused", True), ("incremental", False)):
        again = ring_flash_attn(lq, ring.k[rank], ring.v[rank], RingConfig(cp_size=cp, cp_rank=rank),
                                group=ring, fused=fused)
        assert torch.equal(again, outs[form][0]), f"{form} sweep is not bit-reproducible"
    _check_forms_agree(f"C2 rank {rank}", "fused", outs, TOL_BF16_OUT)
    t = lq.shape[0]
    rows = _tile_rows(t, seed=rank)
    grow = O.zigzag_rows(n, rank, cp)
    kc, vc = k.float().cpu(), v.float().cpu()
    lq_f = lq.float().cpu()
    _check_tiles(f"C2 rank {rank}", outs, lq_f, rows, [int(grow[i]) for i in rows], [0] * len(rows), kc, vc,
                 scale_for(d), TOL_BF16_OUT)


def _fp8_full_size(n, cp, hq, hkv, d, rank, forms, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(n, hq, d, device=DEV, generator=gen)
    k = torch.randn(n, hkv, d, device=DEV, generator=gen)
    v = torch.randn(n, hkv, d, device=DEV, generator=gen)
    lq = zigzag_shard(q, rank, cp)
    sq = float(lq.abs().max()) / 448.0
    q8 = (lq / sq).clamp(-448, 448).to(torch.float8_e4m3fn)
    ks = [zigzag_shard(k, r, cp) for r in range(cp)]
    vs = [zigzag_shard(v, r, cp) for r in range(cp)]
    sk = [float(x.abs().max()) / 448.0 for x in ks]
    sv = [float(x.abs().max()) / 448.0 for x in vs]
    k8 = [(x / s).clamp(-448, 448).to(torch.float8_e4m3fn) for x, s in zip(ks, sk)]
    v8 = [(x / s).clamp(-448, 448).to(torch.float8_e4m3fn) for x, s in zip(vs, sv)]
    del q, k, v, ks, vs, lq
    ring = LocalKVRing(k8, v8)
    desc = Descales(q=torch.tensor(sq, device=DEV), k=[torch.tensor(s, device=DEV) for s in sk],
                    v=[torch.tensor(s, device=DEV) for s in sv])
    outs = _run_forms(q8, ring, cp, rank, forms, descales=desc)
    name = f"e4m3 n={n} d={d} rank {rank}"
    _check_forms_agree(name, "fused", outs, TOL_FP8_OUT)
    # dense reference on the dequantised tensors
    kf = O.zigzag_unshard([x.float().cpu() * s for x, s in zip(k8, sk)], cp)
    vf = O.zigzag_unshard([x.float().cpu() * s for x, s in zip(v8, sv)], cp)
    lq_f = q8.float().cpu() * sq
    rows = _tile_rows(q8.shape[0], seed=rank + 10)
    grow = O.zigzag_rows(n, rank, cp)
    _check_tiles(name, outs, lq_f, rows, [int(grow[i]) for i in rows], [0] * len(rows), kf, vf, scale_for(d),
                 TOL_FP8_OUT)


@pytest.mark.parametrize("rank", [0, 3, 7])
def test_ring_c3_fp8_full_size(rank):
    say(f"ring C3 e4m3 n=131072 rank={rank}")
    _fp8_full_size(131072, 8, 32, 8, 128, rank, ("fused", "incremental"), seed=1)


def test_ring_c5_bf16_d256_full_size():
    """The C5 shape (N=262144, cp 8, H 16/2, D 256) in bf16, rank 3: the fused sweep (32-key
    tiles) against the per-step form on every row, and sampled rows of every 64-row tile
    against dense causal attention."""
    n, cp, hq, hkv, d, rank = 262144, 8, 16, 2, 256, 3
    say(f"ring C5-shape bf16 d={d} n={n} rank={rank}")
    gen = torch.Generator(device=DEV).manual_seed(4)
    q = torch.randn(n, hq, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    k = torch.randn(n, hkv, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    v = torch.randn(n, hkv, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    ring = LocalKVRing.from_full(k, v, cp)
    lq = zigzag_shard(q, rank, cp)
    del q
    outs = _run_forms(lq, ring, cp, rank, ("fused", "incremental"))
    _check_forms_agree(f"C5-shape bf16 rank {rank}", "fused", outs, TOL_BF16_OUT)
    rows = _tile_rows(lq.shape[0], seed=rank + 20)
    grow = O.zigzag_rows(n, rank, cp)
    _check_tiles(f"C5-shape bf16 rank {rank}", outs, lq.float().cpu(), rows, [int(grow[i]) for i in rows],
                 [0] * len(rows), k.float().cpu(), v.float().cpu(), scale_for(d), TOL_BF16_OUT)


def test_ring_c5_fp8_d256_full_size():
    say("ring C5 e4m3 d=256 n=262144 rank=3")
    _fp8_full_size(262144, 8, 16, 2, 256, 3, ("fused", "batched", "incremental"), seed=2)


@pytest.mark.parametrize("rank", [0, 3])
def test_ring_c4_varlen_full_size(rank):
    lens = [4856, 9720, 8592, 4864, 1832, 15456, 2784, 1576]
    cp, hq, hkv, d = 4, 32, 8, 128
    say(f"ring C4 varlen rank={rank}")
    full_cu = [0]
    for n in lens:
        full_cu.append(full_cu[-1] + n)
    gen = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn(full_cu[-1], hq, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    k = torch.randn(full_cu[-1], hkv, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    v = torch.randn(full_cu[-1], hkv, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    ring = LocalKVRing.from_full(k, v, cp, full_cu)
    lq, local_cu = zigzag_shard_varlen(q, full_cu, rank, cp)
    max_local = int((local_cu[1:] - local_cu[:-1]).max())
    outs = _run_forms(lq, ring, cp, rank, PATHS, cu_seqlens=local_cu, max_seqlen=max_local)
    _check_forms_agree(f"C4 rank {rank}", "fused", outs, TOL_BF16_OUT)
    kc, vc = k.float().cpu(), v.float().cpu()
    lq_f = lq.float().cpu()
    grow = O.zigzag_rows_varlen(full_cu, rank, cp)
    # one row of every 64-row tile of every local sequence, plus each sequence's halves' ends
    lcu = local_cu.tolist()
    rows = set()
    rng = np.random.default_rng(rank)
    for j in range(len(lens)):
        a, b = lcu[j], lcu[j + 1]
        for t0 in range(a, b, 64):
            rows.add(int(t0 + rng.integers(0, min(64, b - t0))))
        rows.update([a, (a + b) // 2 - 1, (a + b) // 2, b - 1])
    rows = sorted(rows)
    starts = [full_cu[int(np.searchsorted(full_cu, int(grow[i]), side="right")) - 1] for i in rows]
    _check_tiles(f"C4 rank {rank}", outs, lq_f, rows, [int(grow[i]) for i in rows], starts, kc, vc,
                 scale_for(d), TOL_BF16_OUT)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("packed", [False, True])
def test_sweep_handout_counters_reused(packed, dtype):
    """The fused sweep over one sequence hands its row tiles out from counters that each
    launch takes from a set of 64 per GPU and that the launch's last workgroup clears
    (packed sequences keep the fixed order and are checked the same way).  The first launch
    matches the oracle, and 70 more in a row (every counter set reused) and 6 alternating
    between two streams give bit-identical out and LSE."""
    lens = [608, 1216, 1072, 608, 232, 1928, 344, 200] if packed else [2048]
    cp, h, hkv, d, rank = 4, 32, 8, 128, 3
    fp8 = dtype == torch.float8_e4m3fn
    say(f"sweep hand-out reuse packed={packed} {dtype}")
    full_cu = [0]
    for n in lens:
        full_cu.append(full_cu[-1] + n)
    q, k, v = O.random_qkv(full_cu[-1], h, hkv, d, seed=6)
    q, k, v = (rounded(t, torch.bfloat16) for t in (q, k, v))
    qd, kd, vd = (t.to(torch.bfloat16).to(DEV) for t in (q, k, v))
    cfg = RingConfig(cp_size=cp, cp_rank=rank)
    if packed:
        ring = LocalKVRing.from_full(kd, vd, cp, full_cu)
        lq, local_cu = zigzag_shard_varlen(qd, full_cu, rank, cp)
        kw = dict(cu_seqlens=local_cu, max_seqlen=int((local_cu[1:] - local_cu[:-1]).max()))
    else:
        ring = LocalKVRing.from_full(kd, vd, cp)
        lq = zigzag_shard(qd, rank, cp)
        kw = {}
    if fp8:
        from fa4_ring import quantize_ring
        lq, k8, v8, desc = quantize_ring(lq, list(ring.k), list(ring.v))
        ring = LocalKVRing(k8, v8)
        kw["descales"] = desc

    def sweep():
        return ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, return_lse=True, **kw)

    out0, lse0 = sweep()
    if fp8:
        # the oracle on the dequantised e4m3 inputs
        qo = lq.float().cpu() * float(desc.q)
        ks = [ring.k[r].float().cpu() * float(desc.k[r]) for r in range(cp)]
        vs = [ring.v[r].float().cpu() * float(desc.v[r]) for r in range(cp)]
    else:
        qo = lq.float().cpu()
        ks = [ring.k[r].float().cpu() for r in range(cp)]
        vs = [ring.v[r].float().cpu() for r in range(cp)]
    ocu = kw["cu_seqlens"].cpu().tolist() if packed else None
    ref, ref_lse = O.ring_rank(qo, ks, vs, rank, cp, scale_for(d), cu=ocu)
    assert max_err(out0, ref) <= (TOL_FP8_OUT if fp8 else TOL_BF16_OUT)
    assert lse_err(lse0, ref_lse) <= TOL_LSE
    for i in range(70):
        out, lse = sweep()
        assert torch.equal(out, out0) and torch.equal(lse, lse0), f"launch {i + 1}"
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    res = []
    for i in range(6):
        with torch.cuda.stream(streams[i % 2]):
            res.append(sweep())
    torch.cuda.synchronize()
    for i, (out, lse) in enumerate(res):
        assert torch.equal(out, out0) and torch.equal(lse, lse0), f"stream launch {i}"


def test_sweep_graph_replays():
    """A captured fused sweep (one sequence: the V transposes and the sweep launch, which keeps
    the set of hand-out counters it took at capture) replayed five times, with eager sweeps
    and synchronisations between the replays, gives the eager result every time."""
    cp, h, hkv, d, rank, n = 4, 32, 8, 128, 2, 2048
    say("sweep graph replays")
    q, k, v = O.random_qkv(n, h, hkv, d, seed=9)
    qd, ring = _device_ring(q, k, v, cp, torch.bfloat16)
    lq = zigzag_shard(qd, rank, cp)
    cfg = RingConfig(cp_size=cp, cp_rank=rank)

    def sweep():
        return ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, return_lse=True)

    out0, lse0 = sweep()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm the allocator off the default stream, as capture requires
        sweep()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout, glse = sweep()
    for i in range(5):
        gout.zero_()
        glse.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, out0) and torch.equal(glse, lse0), f"replay {i}"
        out, lse = sweep()  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(out, out0) and torch.equal(lse, lse0), f"eager after replay {i}"


EMPTY_CASES = [(torch.bfloat16, p) for p in PATHS] + [(torch.float8_e4m3fn, "fused"),
                                                       (torch.float8_e4m3fn, "incremental")]


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("dtype,path", EMPTY_CASES)
def test_ring_empty_shard(dtype, path, packed):
    """A rank with no rows (N = 0, or packed sequences that are all empty) gets an empty out
    of the output type: every kernel call sees no rows and launches nothing."""
    say(f"ring empty shard {dtype} path={path} packed={packed}")
    cp, rank, h, hkv, d = 4, 1, 8, 2, 128
    q = torch.empty(0, h, d, dtype=dtype, device=DEV)
    k = torch.empty(0, hkv, d, dtype=dtype, device=DEV)
    cfg, fused = _cfg_path(path, cp, rank)
    kw = dict(cu_seqlens=torch.zeros(3, dtype=torch.int32, device=DEV), max_seqlen=0) if packed else {}
    out = ring_flash_attn(q, k, k, cfg, group=LocalKVRing([k] * cp, [k] * cp), fused=fused, **kw)
    torch.cuda.synchronize()
    assert out.shape == (0, h, d)
    assert out.dtype == (torch.bfloat16 if dtype == torch.float8_e4m3fn else dtype)


def test_empty_operators():
    """The operator level on zero rows: zig-zag shard / unshard (one and packed sequences),
    fa4_attn, both merges, all returning empty results."""
    from fa4_ring.fa4_backend import fa4_attn
    from fa4_ring.merge import merge_state_in_place, merge_states

    say("operators on zero rows")
    x = torch.empty(0, 4, 64, dtype=torch.bfloat16, device=DEV)
    shards = [zigzag_shard(x, r, 4) for r in range(4)]
    assert all(s.shape == (0, 4, 64) for s in shards)
    assert zigzag_unshard(shards, 4).shape == (0, 4, 64)
    local, local_cu = zigzag_shard_varlen(x, [0, 0, 0], 1, 4)
    assert local.shape == (0, 4, 64) and local_cu.tolist() == [0, 0, 0]
    kv = torch.empty(0, 2, 64, dtype=torch.bfloat16, device=DEV)
    out, lse = fa4_attn(x, kv, kv, causal=True)
    assert out.shape == (0, 4, 64) and lse.shape == (0, 4)
    acc, acc_lse = out.clone(), lse.clone()
    merge_state_in_place(acc, acc_lse, out, lse)
    v, s = merge_states(torch.empty(0, 3, 4, 64, dtype=torch.bfloat16, device=DEV),
                        torch.empty(0, 3, 4, dtype=torch.float32, device=DEV))
    torch.cuda.synchronize()
    assert v.shape == (0, 4, 64) and s.shape == (0, 4)


def test_ring_sweep_rejects_bad_out_and_lse():
    """Caller-provided out / lse of the wrong shape, type or layout are refused before the
    sweep kernel is queued."""
    from fa4_ring.ring_attention import ring_sweep

    say("ring_sweep argument checks")
    q = torch.randn(256, 4, 128, device=DEV).to(torch.bfloat16)
    k = torch.randn(256, 2, 128, device=DEV).to(torch.bfloat16)
    ring = LocalKVRing([k, k], [k, k])
    cfg = RingConfig(cp_size=2, cp_rank=0)
    bad_outs = [torch.empty(128, 4, 128, dtype=torch.bfloat16, device=DEV),
                torch.empty(256, 4, 128, dtype=torch.float16, device=DEV),
                torch.empty(256, 128, 4, dtype=torch.bfloat16, device=DEV).transpose(1, 2)]
    for out in bad_outs:
        with pytest.raises(AssertionError, match="out must be"):
            ring_sweep(q, k, k, cfg, ring, out=out)
    for lse in (torch.empty(256, 3, device=DEV), torch.empty(256, 4, dtype=torch.float16, device=DEV)):
        with pytest.raises(AssertionError, match="lse must be"):
            ring_sweep(q, k, k, cfg, ring, lse=lse)
    torch.cuda.synchronize()
