"""GPU parity of paged K/V caches in front of the fused sweep.

The caches here are built on the host (pages handed out in a random order, unused rows NaN),
independently of PagedKVRing.from_shards.  The page gather must return the contiguous shards
bit for bit, the paged V^T must equal fa4cp_transpose_v_many's V^T of the contiguous V bit for
bit, table entries naming no page read as zeros, and a sweep over the paged ring must equal
the sweep over the contiguous ring bit for bit (which the oracle pins, checked again here).
"""

import pytest
import torch

from fa4_ring import Descales, LocalKVRing, PagedKVRing, RingConfig, ring_flash_attn, zigzag_shard
from fa4_ring.fa4_backend import transpose_v_many
from fa4_ring.paged import gather_kv_pages, transpose_v_paged_many
from fa4_ring.zigzag import zigzag_shard_varlen
from gpu_helpers import DEV, TOL_BF16_OUT, TOL_LSE, lse_err, max_err, rounded, say, scale_for
from oracle import ring_oracle as O

pytestmark = pytest.mark.gpu

NAN = float("nan")


def bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().cpu().view(torch.uint8)


def host_pages(shards, cu, page_size, spare, seed, extra_cols=0):
    """(caches, tables) on the host: sequence j's rows [k P, (k+1) P) go to a random page;
    `extra_cols` more table columns than the longest sequence needs, holding -1."""
    gen = torch.Generator().manual_seed(seed)
    lens = [cu[j + 1] - cu[j] for j in range(len(cu) - 1)]
    npg = [(n + page_size - 1) // page_size for n in lens]
    num_pages = sum(npg) + spare
    caches, tables = [], []
    for x in shards:
        perm = torch.randperm(num_pages, generator=gen)
        table = torch.full((len(lens), max(1, max(npg)) + extra_cols), -1, dtype=torch.int32)
        cache = torch.full((num_pages, page_size) + tuple(x.shape[1:]), NAN).to(x.dtype)
        i = 0
        for j in range(len(lens)):
            for k in range(npg[j]):
                p = int(perm[i])
                i += 1
                table[j, k] = p
                r0 = cu[j] + k * page_size
                n = min(page_size, cu[j + 1] - r0)
                cache[p, :n] = x[r0:r0 + n]
        caches.append(cache)
        tables.append(table)
    return caches, tables


def _rand(n, h, d, dtype, gen):
    x = torch.randn(n, h, d, generator=gen)
    return x.to(dtype)


PAGE_CASES = [  # (dtype, d, page_size, local sequence lengths)
    (torch.bfloat16, 128, 128, [512]),
    (torch.bfloat16, 64, 256, [130, 0, 388, 2]),
    (torch.float16, 128, 128, [256, 1000]),
    (torch.float8_e4m3fn, 128, 128, [300, 86]),
    (torch.float8_e4m3fn, 256, 256, [700]),
]


@pytest.mark.parametrize("dtype,d,page_size,lens", PAGE_CASES)
def test_gather_and_paged_vt_bit_exact(dtype, d, page_size, lens):
    say(f"paged gather / V^T {dtype} d={d} page={page_size} lens={lens}")
    gen = torch.Generator().manual_seed(7)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    total, h_kv, S = cu[-1], 2, 3
    ks = [_rand(total, h_kv, d, dtype, gen) for _ in range(S)]
    vs = [_rand(total, h_kv, d, dtype, gen) for _ in range(S)]
    kc, pt = host_pages(ks, cu, page_size, spare=3, seed=1)
    vc, _ = host_pages(vs, cu, page_size, spare=3, seed=1)  # same seed: the same tables
    ring = PagedKVRing([c.to(DEV) for c in kc], [c.to(DEV) for c in vc], [t.to(DEV) for t in pt])
    packed = len(lens) > 1
    cu_dev = torch.tensor(cu, dtype=torch.int32, device=DEV) if packed else None
    mx = max(lens)
    got = gather_kv_pages(ring, "k", total, cu_dev, mx)
    for i in range(S):
        assert torch.equal(bits(got[i]), bits(ks[i])), f"K source {i}"
    vt, stride = transpose_v_paged_many(ring, total, cu_dev, mx)
    ref, ref_stride = transpose_v_many([v.to(DEV) for v in vs], cu_seqlens_k=cu_dev, max_seqlen_k=mx)
    used = sum((n + 127) // 128 * 128 for n in lens)  # positions the layout defines
    assert stride == ref_stride
    for i in range(S):
        a = bits(vt[i].view(h_kv * d, stride)[:, :used])
        b = bits(ref[i].view(h_kv * d, stride)[:, :used])
        assert torch.equal(a, b), f"V^T source {i}"


def test_page_entries_outside_the_cache_read_as_zeros():
    say("paged gather with table entries outside the cache")
    gen = torch.Generator().manual_seed(3)
    cu, h_kv, d, P = [0, 384], 2, 128, 128
    ks = [_rand(384, h_kv, d, torch.bfloat16, gen) for _ in range(2)]
    kc, pt = host_pages(ks, cu, P, spare=1, seed=2)
    num_pages = kc[0].shape[0]
    pt[0][0, 1] = -5
    pt[1][0, 2] = num_pages + 7
    ring = PagedKVRing([c.to(DEV) for c in kc], [c.to(DEV) for c in kc], [t.to(DEV) for t in pt])
    got = gather_kv_pages(ring, "k", 384)
    want0, want1 = ks[0].clone(), ks[1].clone()
    want0[128:256] = 0
    want1[256:384] = 0
    assert torch.equal(bits(got[0]), bits(want0)) and torch.equal(bits(got[1]), bits(want1))
    vt, stride = transpose_v_paged_many(ring, 384)
    v0 = vt[0].view(h_kv, d, stride).float().cpu()
    assert torch.all(v0[:, :, 128:256] == 0) and torch.equal(v0[:, :, :128], ks[0][:128].float().permute(1, 2, 0))


RING_CASES = [  # (dtype, d, cp, full lengths (None: one sequence of n), n, page_size, descaled)
    (torch.bfloat16, 128, 4, None, 2048, 128, False),
    (torch.bfloat16, 64, 2, [512, 1024, 256], 0, 256, False),
    (torch.float16, 128, 8, None, 4096, 128, False),
    (torch.float8_e4m3fn, 128, 4, [1024, 520, 2048], 0, 128, True),
    (torch.float8_e4m3fn, 256, 2, None, 1024, 256, True),
    (torch.bfloat16, 256, 4, [768, 1280], 0, 128, False),
]


@pytest.mark.parametrize("dtype,d,cp,full_lens,n,page_size,descaled", RING_CASES)
def test_paged_sweep_equals_contiguous(dtype, d, cp, full_lens, n, page_size, descaled):
    say(f"paged sweep {dtype} d={d} cp={cp} lens={full_lens or n} page={page_size}")
    h, h_kv = 8, 2
    gen = torch.Generator().manual_seed(11)
    full_cu = None
    if full_lens:
        full_cu = [0]
        for x in full_lens:
            full_cu.append(full_cu[-1] + x)
        n = full_cu[-1]
    q, k, v = (torch.randn(n, hh, d, generator=gen) for hh in (h, h_kv, h_kv))
    qd, kd, vd = (t.to(dtype).to(DEV) for t in (q, k, v))
    ring = LocalKVRing.from_full(kd, vd, cp, full_cu)
    desc = None
    if descaled:
        desc = Descales(q=torch.tensor(0.75, device=DEV),
                        k=[torch.full((h_kv,), 0.5 + 0.1 * r, device=DEV) for r in range(cp)],
                        v=[torch.full((h_kv,), 1.25 - 0.05 * r, device=DEV) for r in range(cp)])
    for rank in range(cp):
        if full_cu is None:
            lq, lcu, mx = zigzag_shard(qd, rank, cp), None, None
            local_cu = None
        else:
            lq, lcu = zigzag_shard_varlen(qd, full_cu, rank, cp)
            local_cu = lcu.tolist()
            mx = max(local_cu[j + 1] - local_cu[j] for j in range(len(local_cu) - 1))
        paged = PagedKVRing.from_shards(ring.k, ring.v, page_size, local_cu, spare_pages=2,
                                        generator=torch.Generator().manual_seed(rank))
        cfg = RingConfig(cp_size=cp, cp_rank=rank)
        want, want_lse = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, descales=desc,
                                         cu_seqlens=lcu, max_seqlen=mx, fused=True, return_lse=True)
        got, got_lse = ring_flash_attn(lq, None, None, cfg, group=paged, descales=desc, cu_seqlens=lcu,
                                       max_seqlen=mx, return_lse=True)
        assert torch.equal(bits(got), bits(want)), f"rank {rank}"
        assert torch.equal(bits(got_lse), bits(want_lse)), f"rank {rank} lse"
    if dtype == torch.bfloat16 and full_cu is None:  # the oracle, on the last rank
        qr, kr, vr = (rounded(t, dtype) for t in (q, k, v))
        ks = [O.zigzag_shard(kr, r, cp) for r in range(cp)]
        vs = [O.zigzag_shard(vr, r, cp) for r in range(cp)]
        ref, ref_lse = O.ring_rank(O.zigzag_shard(qr, rank, cp), ks, vs, rank, cp, scale_for(d))
        assert max_err(got, ref) <= TOL_BF16_OUT
        assert lse_err(got_lse, ref_lse) <= TOL_LSE


def test_paged_sweep_full_size_bf16_rank3():
    """N=131072, cp=8, H 32/8, D=128, rank 3, pages of 256 rows: bit-identical to the
    contiguous sweep."""
    say("paged sweep bf16 N=131072 cp=8 rank 3 page 256")
    n, cp, rank, d = 131072, 8, 3, 128
    gen = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn(n // cp, 32, d, generator=gen, device=DEV).to(torch.bfloat16)
    ks = [torch.randn(n // cp, 8, d, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(cp)]
    vs = [torch.randn(n // cp, 8, d, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(cp)]
    ring = LocalKVRing(ks, vs)
    paged = PagedKVRing.from_shards(ks, vs, 256, spare_pages=5, generator=torch.Generator().manual_seed(9))
    cfg = RingConfig(cp_size=cp, cp_rank=rank)
    want, want_lse = ring_flash_attn(q, ks[rank], vs[rank], cfg, group=ring, return_lse=True)
    got, got_lse = ring_flash_attn(q, None, None, cfg, group=paged, return_lse=True)
    assert torch.equal(bits(got), bits(want))
    assert torch.equal(bits(got_lse), bits(want_lse))


PER_STEP_CASES = [  # (dtype, d, cp, merge mode): shapes the fused sweep does not take, and fused=False
    (torch.bfloat16, 256, 2, "incremental"),
    (torch.float16, 256, 4, "batched"),
    (torch.bfloat16, 128, 4, "batched"),
    (torch.bfloat16, 128, 1, "incremental"),
]


@pytest.mark.parametrize("dtype,d,cp,mode", PER_STEP_CASES)
def test_paged_per_step_equals_contiguous(dtype, d, cp, mode):
    say(f"paged per-step {dtype} d={d} cp={cp} {mode}")
    n, h, h_kv = 1024, 4, 2
    gen = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(n, hh, d, generator=gen).to(dtype).to(DEV) for hh in (h, h_kv, h_kv))
    ring = LocalKVRing.from_full(k, v, cp)
    for rank in range(cp):
        lq = zigzag_shard(q, rank, cp)
        paged = PagedKVRing.from_shards(ring.k, ring.v, 128, spare_pages=1,
                                        generator=torch.Generator().manual_seed(rank))
        cfg = RingConfig(cp_size=cp, cp_rank=rank, merge_mode=mode)
        want, want_lse = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, fused=False,
                                         return_lse=True)
        got, got_lse = ring_flash_attn(lq, None, None, cfg, group=paged, fused=False, return_lse=True)
        assert torch.equal(bits(got), bits(want)), f"rank {rank}"
        assert torch.equal(bits(got_lse), bits(want_lse)), f"rank {rank} lse"


WALK_CASES = [  # (dtype, d, cp, rank, page_size, local sequence lengths, extra table columns)
    (torch.bfloat16, 128, 4, 2, 384, [1536], 0),             # six 64-key tiles per page
    (torch.bfloat16, 64, 3, 1, 384, [770, 2, 1150], 3),      # ragged packed sequences, wider table
    (torch.float16, 128, 2, 1, 128, [640, 0, 256], 1),       # two tiles per page, an empty sequence
    (torch.float8_e4m3fn, 128, 4, 3, 384, [1152, 514], 2),   # three 128-key tiles per page
    (torch.float8_e4m3fn, 128, 2, 0, 128, [1024], 0),        # one tile per page: every step a new page
    (torch.float8_e4m3fn, 256, 3, 2, 128, [896], 0),         # two 64-key tiles per page
    (torch.bfloat16, 256, 4, 1, 128, [640, 386], 1),         # four 32-key tiles per page
]


@pytest.mark.parametrize("dtype,d,cp,rank,page_size,lens,extra", WALK_CASES)
@pytest.mark.parametrize("bad_entries", [False, True])
def test_in_kernel_page_walk_equals_contiguous(dtype, d, cp, rank, page_size, lens, extra, bad_entries):
    """The fused sweep reading K through the page tables (fa4cp_ring_sweep_fwd_paged) against
    the contiguous sweep over the same rows, bit for bit: caches built on the host with pages
    in a random order and NaN in every unused row.  bad_entries: a few table entries name no
    page of the cache (negative, or past num_pages); those rows read as zeros, so the
    reference is the contiguous sweep with the same K and V rows zeroed."""
    say(f"paged K walk {dtype} d={d} cp={cp} rank={rank} page={page_size} lens={lens} extra={extra} "
        f"bad={bad_entries}")
    h, h_kv = 8, 2
    gen = torch.Generator().manual_seed(31)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    total = cu[-1]
    ks = [_rand(total, h_kv, d, dtype, gen) for _ in range(cp)]
    vs = [_rand(total, h_kv, d, dtype, gen) for _ in range(cp)]
    q = _rand(total, h, d, dtype, gen)
    kc, pt = host_pages(ks, cu, page_size, spare=2, seed=3, extra_cols=extra)
    vc, _ = host_pages(vs, cu, page_size, spare=2, seed=3, extra_cols=extra)  # the same tables
    if bad_entries:
        num_pages = kc[0].shape[0]
        j = max(range(len(lens)), key=lambda i: lens[i])  # the longest sequence
        npg = (lens[j] + page_size - 1) // page_size
        for src in range(cp):
            col = (src + 1) % npg
            pt[src][j, col] = -7 if src % 2 else num_pages + src
            r0 = cu[j] + col * page_size
            r1 = min(r0 + page_size, cu[j + 1])
            ks[src] = ks[src].clone()
            vs[src] = vs[src].clone()
            ks[src][r0:r1] = 0
            vs[src][r0:r1] = 0
    paged = PagedKVRing([c.to(DEV) for c in kc], [c.to(DEV) for c in vc], [t.to(DEV) for t in pt])
    ring = LocalKVRing([x.to(DEV) for x in ks], [x.to(DEV) for x in vs])
    packed = len(lens) > 1
    cu_dev = torch.tensor(cu, dtype=torch.int32, device=DEV) if packed else None
    mx = max(lens) if packed else None
    desc = None
    if dtype == torch.float8_e4m3fn:
        desc = Descales(q=torch.tensor(0.8, device=DEV),
                        k=[torch.full((h_kv,), 0.4 + 0.1 * r, device=DEV) for r in range(cp)],
                        v=[torch.full((h_kv,), 1.3 - 0.1 * r, device=DEV) for r in range(cp)])
    cfg = RingConfig(cp_size=cp, cp_rank=rank)
    qd = q.to(DEV)
    want, want_lse = ring_flash_attn(qd, ring.k[rank], ring.v[rank], cfg, group=ring, descales=desc,
                                     cu_seqlens=cu_dev, max_seqlen=mx, fused=True, return_lse=True)
    got, got_lse = ring_flash_attn(qd, None, None, cfg, group=paged, descales=desc, cu_seqlens=cu_dev,
                                   max_seqlen=mx, fused=True, return_lse=True)
    assert torch.isfinite(want.float()).all()
    assert torch.equal(bits(got), bits(want))
    assert torch.equal(bits(got_lse), bits(want_lse))


def test_paged_sweep_full_size_e4m3_rank3():
    """N=131072, cp=8, H 32/8, D=128 in OCP e4m3 with per-source descales, rank 3, pages of
    256 rows in a random order: the in-kernel page walk is bit-identical to the contiguous
    sweep."""
    say("paged sweep e4m3 N=131072 cp=8 rank 3 page 256")
    n, cp, rank, d = 131072, 8, 3, 128
    gen = torch.Generator(device=DEV).manual_seed(6)
    e4 = torch.float8_e4m3fn
    q = (torch.randn(n // cp, 32, d, generator=gen, device=DEV) * 2).to(e4)
    ks = [(torch.randn(n // cp, 8, d, generator=gen, device=DEV) * 2).to(e4) for _ in range(cp)]
    vs = [(torch.randn(n // cp, 8, d, generator=gen, device=DEV) * 2).to(e4) for _ in range(cp)]
    desc = Descales(q=torch.tensor(0.02, device=DEV), k=[torch.tensor(0.01 + 0.002 * r, device=DEV) for r in range(cp)],
                    v=[torch.tensor(0.03 - 0.001 * r, device=DEV) for r in range(cp)])
    ring = LocalKVRing(ks, vs)
    paged = PagedKVRing.from_shards(ks, vs, 256, spare_pages=5, generator=torch.Generator().manual_seed(4))
    cfg = RingConfig(cp_size=cp, cp_rank=rank)
    want, want_lse = ring_flash_attn(q, ks[rank], vs[rank], cfg, group=ring, descales=desc, return_lse=True)
    got, got_lse = ring_flash_attn(q, None, None, cfg, group=paged, descales=desc, return_lse=True)
    assert torch.equal(bits(got), bits(want))
    assert torch.equal(bits(got_lse), bits(want_lse))
