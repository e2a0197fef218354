"""GPU parity of the ring sweep's backward (fa4cp_ring_sweep_bwd) against the oracle.

Every rank of small rings: dq and each source's dk / dv contribution against the oracle's
ring backward (oracle forward out / LSE, same rounded inputs).  All ranks together, their
contributions summed into shared buffers (accumulate=True): the stitched gradients against
float64 autograd of dense causal attention.  The autograd function: the same gradients as the
functional call.  Tolerance: max |err| <= 2e-2 * max(1, max |reference|) for bf16 inputs (5e-3
for fp16): the probabilities and dS enter the products rounded to the input type, and the
gradients grow with the number of keys, so the bound is relative to their magnitude.
"""

import math

import pytest
import torch

from fa4_ring import LocalKVRing, RingConfig, ring_flash_attn, zigzag_shard
from fa4_ring.backward import ring_flash_attn_backward, ring_flash_attn_func
from fa4_ring.zigzag import zigzag_shard_varlen
from gpu_helpers import DEV, rounded, say, scale_for
from oracle import ring_oracle as O

pytestmark = pytest.mark.gpu


def _tol(dtype):
    return 2e-2 if dtype == torch.bfloat16 else 5e-3


def _rel_err(got, want):
    g, w = got.float().cpu(), want.float().cpu()
    return float((g - w).abs().max()) / max(1.0, float(w.abs().max()))


def _full_cu(lens):
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    return cu


CASES = [  # (lens, H, H_kv, D, cp, dtype)
    ([512], 4, 2, 128, 2, torch.bfloat16),
    ([1024], 8, 2, 128, 4, torch.bfloat16),
    ([1024], 4, 4, 64, 4, torch.float16),
    ([2048], 8, 1, 128, 8, torch.bfloat16),
    ([1024], 8, 8, 64, 1, torch.bfloat16),
    ([320, 640, 192], 4, 2, 128, 4, torch.bfloat16),  # packed: sequences of 80, 160 and 48 local rows
    ([400, 208], 8, 4, 64, 2, torch.float16),  # local lengths not multiples of 32
    ([1024], 16, 2, 128, 4, torch.bfloat16),  # 8 query heads per kv head
    ([320, 144], 4, 4, 128, 2, torch.bfloat16),  # one query head per kv head: dk/dv workgroups of one block
    ([1024], 8, 2, 256, 4, torch.bfloat16),  # head dim 256
    ([512, 384], 4, 2, 256, 2, torch.float16),  # head dim 256, packed, two query heads per kv head
    ([512], 2, 2, 256, 2, torch.bfloat16),  # head dim 256, one query head per kv head
]


@pytest.mark.parametrize("lens,h,hkv,d,cp,dtype", CASES)
def test_backward_every_rank_against_oracle(lens, h, hkv, d, cp, dtype):
    say(f"ring backward lens={lens} h={h}/{hkv} d={d} cp={cp} {dtype}")
    full_cu = _full_cu(lens)
    packed = len(lens) > 1
    q, k, v = O.random_qkv(full_cu[-1], h, hkv, d, seed=31)
    q, k, v = (rounded(x, dtype) for x in (q, k, v))
    dout = rounded(torch.randn(full_cu[-1], h, d, generator=torch.Generator().manual_seed(32)), dtype)
    scale = scale_for(d)
    qd, kd, vd, dod = (x.to(dtype).to(DEV) for x in (q, k, v, dout))
    ring = LocalKVRing.from_full(kd, vd, cp, full_cu if packed else None)
    ks = [O.zigzag_shard_varlen(k, full_cu, r, cp)[0] for r in range(cp)]
    vs = [O.zigzag_shard_varlen(v, full_cu, r, cp)[0] for r in range(cp)]
    for rank in range(cp):
        cfg = RingConfig(cp_size=cp, cp_rank=rank)
        if packed:
            lq, lcu = zigzag_shard_varlen(qd, full_cu, rank, cp)
            ldo = zigzag_shard_varlen(dod, full_cu, rank, cp)[0]
            mx = int((lcu[1:] - lcu[:-1]).max())
            kw = dict(cu_seqlens=lcu, max_seqlen=mx)
        else:
            lq, ldo, kw = zigzag_shard(qd, rank, cp), zigzag_shard(dod, rank, cp), {}
        out, lse = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, return_lse=True, **kw)
        dq, dk, dv = ring_flash_attn_backward(ldo, lq, ring.k[rank], ring.v[rank], out, lse, cfg, group=ring, **kw)
        oq, ocu = O.zigzag_shard_varlen(q, full_cu, rank, cp)
        odo = O.zigzag_shard_varlen(dout, full_cu, rank, cp)[0]
        oo, ol = O.ring_rank(oq, ks, vs, rank, cp, scale, cu=ocu)
        eq, ek, ev = O.ring_rank_backward(oq, ks, vs, odo, oo, ol, rank, cp, scale, cu=ocu)
        assert dq.dtype == torch.float32 and dq.shape == lq.shape
        errs = [_rel_err(dq, eq)] + [_rel_err(dk[i], ek[i]) for i in range(cp)] + \
               [_rel_err(dv[i], ev[i]) for i in range(cp)]
        say(f"  rank {rank}: max relative |err| dq {errs[0]:.2e} dk {max(errs[1:cp + 1]):.2e} "
            f"dv {max(errs[cp + 1:]):.2e} (bar {_tol(dtype)})")
        assert max(errs) <= _tol(dtype), f"rank {rank}: {errs}"


@pytest.mark.parametrize("lens,cp", [([1024], 4), ([256, 512, 128], 2)])
def test_backward_all_ranks_accumulate_equals_dense_autograd(lens, cp):
    """Every rank's backward adds into one set of buffers (accumulate=True, as a ring's
    backward sums the contributions at each source): dq stitched and every source's dk / dv
    equal float64 autograd of dense causal attention over the whole sequences."""
    h, hkv, d, dtype = 8, 2, 128, torch.bfloat16
    say(f"ring backward all ranks accumulated lens={lens} cp={cp}")
    full_cu = _full_cu(lens)
    packed = len(lens) > 1
    q, k, v = O.random_qkv(full_cu[-1], h, hkv, d, seed=41)
    q, k, v = (rounded(x, dtype) for x in (q, k, v))
    dout = rounded(torch.randn(full_cu[-1], h, d, generator=torch.Generator().manual_seed(42)), dtype)
    scale = scale_for(d)
    q64, k64, v64 = (x.double().requires_grad_(True) for x in (q, k, v))
    outs = []
    for j in range(len(lens)):
        s, e = full_cu[j], full_cu[j + 1]
        sc = torch.einsum("qhd,khd->hqk", q64[s:e], k64[s:e].repeat_interleave(h // hkv, 1)) * scale
        sc = sc.masked_fill(torch.triu(torch.ones(e - s, e - s, dtype=torch.bool), 1), float("-inf"))
        outs.append(torch.einsum("hqk,khd->qhd", torch.softmax(sc, -1), v64[s:e].repeat_interleave(h // hkv, 1)))
    torch.cat(outs).backward(dout.double())

    qd, kd, vd, dod = (x.to(dtype).to(DEV) for x in (q, k, v, dout))
    ring = LocalKVRing.from_full(kd, vd, cp, full_cu if packed else None)
    t = full_cu[-1] // cp
    dk = [torch.zeros(t, hkv, d, device=DEV) for _ in range(cp)]
    dv = [torch.zeros(t, hkv, d, device=DEV) for _ in range(cp)]
    dq_full = torch.zeros(full_cu[-1], h, d)
    for rank in range(cp):
        cfg = RingConfig(cp_size=cp, cp_rank=rank)
        lq, lcu = zigzag_shard_varlen(qd, full_cu, rank, cp)
        ldo = zigzag_shard_varlen(dod, full_cu, rank, cp)[0]
        kw = dict(cu_seqlens=lcu, max_seqlen=int((lcu[1:] - lcu[:-1]).max())) if packed else {}
        out, lse = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, return_lse=True, **kw)
        dq, _, _ = ring_flash_attn_backward(ldo, lq, ring.k[rank], ring.v[rank], out, lse, cfg, group=ring, dk=dk,
                                            dv=dv, accumulate=True, **kw)
        dq_full[torch.from_numpy(O.zigzag_rows_varlen(full_cu, rank, cp))] = dq.cpu()
    dk_full = torch.zeros(full_cu[-1], hkv, d)
    dv_full = torch.zeros(full_cu[-1], hkv, d)
    for src in range(cp):
        rows = torch.from_numpy(O.zigzag_rows_varlen(full_cu, src, cp))
        dk_full[rows] = dk[src].cpu()
        dv_full[rows] = dv[src].cpu()
    errs = (_rel_err(dq_full, q64.grad), _rel_err(dk_full, k64.grad), _rel_err(dv_full, v64.grad))
    say(f"  max relative |err| dq {errs[0]:.2e} dk {errs[1]:.2e} dv {errs[2]:.2e} (bar {_tol(dtype)})")
    assert max(errs) <= _tol(dtype)


def test_backward_autograd_function_matches_functional():
    """ring_flash_attn_func under torch.autograd gives the functional backward's gradients
    (in the input dtype) for the local q and for every source's K / V shard."""
    say("ring backward through torch.autograd")
    n, h, hkv, d, cp, rank = 1024, 8, 2, 128, 4, 2
    g = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn(n // cp, h, d, device=DEV, generator=g).to(torch.bfloat16)
    ks = [torch.randn(n // cp, hkv, d, device=DEV, generator=g).to(torch.bfloat16) for _ in range(cp)]
    vs = [torch.randn(n // cp, hkv, d, device=DEV, generator=g).to(torch.bfloat16) for _ in range(cp)]
    dout = torch.randn(n // cp, h, d, device=DEV, generator=g).to(torch.bfloat16)
    cfg = RingConfig(cp_size=cp, cp_rank=rank)
    ring = LocalKVRing(ks, vs)
    out, lse = ring_flash_attn(q, ks[rank], vs[rank], cfg, group=ring, return_lse=True)
    dq, dk, dv = ring_flash_attn_backward(dout, q, ks[rank], vs[rank], out, lse, cfg, group=ring)

    qa = q.clone().requires_grad_(True)
    ka = [x.clone().requires_grad_(True) for x in ks]
    va = [x.clone().requires_grad_(True) for x in vs]
    oa = ring_flash_attn_func(qa, LocalKVRing(ka, va), cfg)
    assert torch.equal(oa.detach(), out)
    oa.backward(dout)
    assert torch.equal(qa.grad, dq.to(torch.bfloat16))
    for i in range(cp):
        assert torch.equal(ka[i].grad, dk[i].to(torch.bfloat16)), f"dk[{i}]"
        assert torch.equal(va[i].grad, dv[i].to(torch.bfloat16)), f"dv[{i}]"


def test_backward_is_deterministic():
    """No atomics: two backward calls give the same bits."""
    say("ring backward run-to-run")
    n, h, hkv, d, cp, rank = 2048, 8, 2, 128, 4, 1
    g = torch.Generator(device=DEV).manual_seed(6)
    q = torch.randn(n // cp, h, d, device=DEV, generator=g).to(torch.bfloat16)
    ks = [torch.randn(n // cp, hkv, d, device=DEV, generator=g).to(torch.bfloat16) for _ in range(cp)]
    vs = [torch.randn(n // cp, hkv, d, device=DEV, generator=g).to(torch.bfloat16) for _ in range(cp)]
    dout = torch.randn(n // cp, h, d, device=DEV, generator=g).to(torch.bfloat16)
    cfg = RingConfig(cp_size=cp, cp_rank=rank)
    ring = LocalKVRing(ks, vs)
    out, lse = ring_flash_attn(q, ks[rank], vs[rank], cfg, group=ring, return_lse=True)
    a = ring_flash_attn_backward(dout, q, ks[rank], vs[rank], out, lse, cfg, group=ring)
    b = ring_flash_attn_backward(dout, q, ks[rank], vs[rank], out, lse, cfg, group=ring)
    assert torch.equal(a[0], b[0])
    assert all(torch.equal(x, y) for x, y in zip(a[1], b[1]))
    assert all(torch.equal(x, y) for x, y in zip(a[2], b[2]))


def test_backward_full_size_sampled_rows_and_keys():
    """The headline shape (N=131072, cp 8, rank 3, H 32/8, D 128, bf16), where the oracle's
    whole ring backward is out of reach: dq of sampled rows (every 1024th local row and the
    last, every head) and the rank's dk / dv contributions for sampled keys of its own source,
    an earlier one and a later one, against float64 sums on the host over every key (row)
    each attends in the dense causal sequence, from the same inputs and the forward's out and
    LSE.  Keys of an earlier source that no row of the rank attends (its back half) must get
    exact zeros."""
    n, cp, rank, hq, hkv, d = 131072, 8, 3, 32, 8, 128
    group = hq // hkv
    say(f"ring backward full size n={n} cp={cp} rank={rank} h={hq}/{hkv} d={d}")
    gen = torch.Generator(device=DEV).manual_seed(8)
    q = torch.randn(n, hq, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    k = torch.randn(n, hkv, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    v = torch.randn(n, hkv, d, device=DEV, generator=gen, dtype=torch.bfloat16)
    ring = LocalKVRing.from_full(k, v, cp)
    lq = zigzag_shard(q, rank, cp)
    del q
    ldo = torch.randn(lq.shape, device=DEV, generator=gen, dtype=torch.bfloat16)
    cfg = RingConfig(cp_size=cp, cp_rank=rank)
    out, lse = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, return_lse=True)
    dq, dk, dv = ring_flash_attn_backward(ldo, lq, ring.k[rank], ring.v[rank], out, lse, cfg, group=ring)
    scale = scale_for(d)
    t = lq.shape[0]
    grow = torch.from_numpy(O.zigzag_rows(n, rank, cp))  # global position of each local row
    kf, vf = k.float().cpu(), v.float().cpu()
    qf, dof, of = lq.double().cpu(), ldo.double().cpu(), out.double().cpu()
    lsef = lse.double().cpu()
    delta = (dof * of).sum(-1)  # [t, hq]

    # dq of sampled rows: dq[r, h] = scale sum_j P_j (dO.v_j - delta) k_j over keys j <= row
    rows = sorted(set(range(0, t, 1024)) | {t // 2 - 1, t - 1})
    got = dq[torch.tensor(rows, device=DEV)].double().cpu()
    exp = torch.empty_like(got)
    for i, r in enumerate(rows):
        g = int(grow[r])
        for kh in range(hkv):
            hs = slice(kh * group, (kh + 1) * group)
            kk, vv = kf[:g + 1, kh].double(), vf[:g + 1, kh].double()
            p = torch.exp(qf[r, hs] @ kk.T * scale - lsef[r, hs, None])  # [group, g + 1]
            ds = p * (dof[r, hs] @ vv.T - delta[r, hs, None])
            exp[i, hs] = scale * (ds @ kk)
    err = float((got - exp).abs().max()) / max(1.0, float(exp.abs().max()))
    say(f"  dq: {len(rows)} rows x {hq} heads: max relative |err| {err:.2e} (bar 2e-2)")
    assert err <= 2e-2, err

    # dk / dv of sampled keys: this rank's rows r with position >= the key's, every head of
    # the key's group: dv_j = sum P dO_r, dk_j = scale sum dS q_r
    half = t // 2
    for src in (rank, (rank - 1) % cp, (rank + 2) % cp):
        kpos = torch.from_numpy(O.zigzag_rows(n, src, cp))
        keys = [0, half // 3, half - 1, half, half + half // 2, t - 1]
        gk_, gv_ = dk[src][torch.tensor(keys, device=DEV)].double().cpu(), dv[src][torch.tensor(keys, device=DEV)].double().cpu()
        ek, ev = torch.zeros_like(gk_), torch.zeros_like(gv_)
        kcpu, vcpu = ring.k[src][torch.tensor(keys, device=DEV)].double().cpu(), \
            ring.v[src][torch.tensor(keys, device=DEV)].double().cpu()
        for kh in range(hkv):
            hs = slice(kh * group, (kh + 1) * group)
            qh, doh, lh, dh = qf[:, hs], dof[:, hs], lsef[:, hs], delta[:, hs]
            for i, kj in enumerate(keys):
                m = grow >= int(kpos[kj])  # the rank's rows that attend this key
                if not bool(m.any()):
                    continue
                qm, dom = qh[m], doh[m]  # [rows, group, d]
                p = torch.exp(qm @ kcpu[i, kh] * scale - lh[m])  # [rows, group]
                ds = p * (dom @ vcpu[i, kh] - dh[m])
                ev[i, kh] = (p[..., None] * dom).sum((0, 1))
                ek[i, kh] = scale * (ds[..., None] * qm).sum((0, 1))
        for name, gt, ex in (("dk", gk_, ek), ("dv", gv_, ev)):
            e = float((gt - ex).abs().max()) / max(1.0, float(ex.abs().max()))
            say(f"  {name}[{src}]: {len(keys)} keys x {hkv} heads: max relative |err| {e:.2e} (bar 2e-2)")
            assert e <= 2e-2, (name, src, e)
        if src == (rank - 1) % cp:  # an earlier source: only its front half is attended
            assert float(gk_[3:].abs().max()) == 0.0 and float(gv_[3:].abs().max()) == 0.0
