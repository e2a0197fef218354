"""GPU parity of the individual HIP kernels against the CPU oracle, through the C ABI
(zig-zag gather/scatter bit-exact, merges within 1e-5 in fp32, attention per step pattern)."""

import math

import pytest
import torch

from fa4_ring import zigzag as Z
from fa4_ring.fa4_backend import SEL_ALL, SEL_BACK_HALF, SEL_FRONT_HALF, fa4_attn
from fa4_ring.merge import make_merger, merge_state, merge_state_in_place, merge_states, merge_states_list
from gpu_helpers import (DEV, TOL_BF16_OUT, TOL_FP8_OUT, TOL_LSE, TOL_MERGE_FP32, lse_err, max_err,
                         oracle_attn, rounded, say, scale_for, seq_bounds)
from oracle import ring_oracle as O

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------------- zig-zag

@pytest.mark.parametrize("shape,dtype", [((96, 3, 8), torch.bfloat16), ((64, 5), torch.uint8),
                                         ((128, 8, 128), torch.float16), ((48, 7), torch.float32),
                                         ((256, 2, 64), torch.float8_e4m3fn)])
@pytest.mark.parametrize("cp", [1, 2, 4, 8])
def test_zigzag_shard_unshard_bit_exact(shape, dtype, cp):
    n = shape[0]
    if n % (2 * cp):
        pytest.skip("length not shardable")
    say(f"zigzag shape={shape} dtype={dtype} cp={cp}")
    g = torch.Generator().manual_seed(cp)
    x = torch.randint(0, 255, shape, generator=g, dtype=torch.uint8)
    if dtype != torch.uint8:
        x = torch.randn(shape, generator=g).to(dtype)
    xd = x.to(DEV)
    shards = []
    for r in range(cp):
        s = Z.zigzag_shard(xd, r, cp)
        exp = x[torch.from_numpy(O.zigzag_rows(n, r, cp))]
        assert torch.equal(s.cpu().view(torch.uint8), exp.contiguous().view(torch.uint8))
        shards.append(s)
    back = Z.zigzag_unshard(shards, cp)
    assert torch.equal(back.cpu().view(torch.uint8), x.view(torch.uint8))


@pytest.mark.parametrize("lens,cp", [([16, 32], 2), ([32, 16, 48], 4), ([64, 64], 8),
                                     ([4856, 9720, 8592, 4864, 1832, 15456, 2784, 1576], 4)])
def test_zigzag_varlen_bit_exact(lens, cp):
    say(f"zigzag varlen lens={lens} cp={cp}")
    full_cu = [0]
    for n in lens:
        full_cu.append(full_cu[-1] + n)
    x = torch.randn(full_cu[-1], 2, 64).to(torch.bfloat16)
    xd = x.to(DEV)
    shards = []
    for r in range(cp):
        loc, lcu = Z.zigzag_shard_varlen(xd, full_cu, r, cp)
        exp, ecu = O.zigzag_shard_varlen(x.float(), full_cu, r, cp)
        assert lcu.cpu().tolist() == ecu
        assert lcu.dtype == torch.int32
        assert torch.equal(loc.cpu().float(), exp)
        shards.append(loc)
    back = Z.zigzag_unshard_varlen(shards, full_cu, cp)
    assert torch.equal(back.cpu(), x)


# ------------------------------------------------------------------------- merges

_HALF_ULP = {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}


def assert_rounded_close(got, exp, dtype, mask=None):
    """fp32 math within 1e-5, plus one rounding of the result to the storage type."""
    g, e = got.float().cpu(), exp.float()
    bound = TOL_MERGE_FP32 + _HALF_ULP[dtype] * e.abs()
    bad = (g - e).abs() > bound
    if mask is not None:
        bad &= mask
    assert not bad.any(), f"{int(bad.sum())} elements off, max err {max_err(g, e, mask)}"

def _states(t, h, d, seed, dtype, inf_frac=0.0):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(t, h, d, generator=g)
    s = torch.randn(t, h, generator=g) * 4
    if inf_frac:
        s[torch.rand(t, h, generator=g) < inf_frac] = float("-inf")
    return rounded(v, dtype), s


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("t,h,d", [(37, 3, 64), (256, 8, 128), (100, 2, 256), (8, 1, 8)])
def test_merge_state_in_place(dtype, t, h, d):
    say(f"merge_state_in_place dtype={dtype} t={t} h={h} d={d}")
    va, sa = _states(t, h, d, 1, dtype, inf_frac=0.1)
    vb, sb = _states(t, h, d, 2, dtype, inf_frac=0.1)
    sa[0, 0] = sb[0, 0] = float("-inf")  # at least one row empty on both sides
    both = torch.isinf(sa) & torch.isinf(sb)
    vd, sd = va.to(dtype).to(DEV), sa.to(DEV)
    merge_state_in_place(vd, sd, vb.to(dtype).to(DEV), sb.to(DEV))
    eo, el = O.merge(va, sa, vb, sb)
    ok = ~both
    assert_rounded_close(vd, eo, dtype, ok.unsqueeze(-1).expand_as(eo))
    assert lse_err(sd.cpu()[ok], el[ok]) <= TOL_MERGE_FP32
    # rows where both sides are empty: the oracle's (the reference formula's) NaN out and
    # -inf LSE
    assert both.any()
    assert torch.isnan(eo[both]).all() and torch.isnan(vd.cpu().float()[both]).all()
    assert lse_err(sd.cpu()[both], el[both]) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_merge_state_out_of_place(dtype):
    """merge_state writes a new state equal bit for bit to the in-place merge and leaves its
    inputs alone."""
    say(f"merge_state out of place dtype={dtype}")
    t, h, d = 300, 4, 128
    va, sa = _states(t, h, d, 5, dtype, inf_frac=0.1)
    vb, sb = _states(t, h, d, 6, dtype, inf_frac=0.1)
    a_v, a_s, b_v, b_s = va.to(dtype).to(DEV), sa.to(DEV), vb.to(dtype).to(DEV), sb.to(DEV)
    keep = [x.clone() for x in (a_v, a_s, b_v, b_s)]
    ov, os_ = merge_state(a_v, a_s, b_v, b_s)
    for x, y in zip((a_v, a_s, b_v, b_s), keep):
        assert torch.equal(x, y), "an input was modified"
    iv, is_ = a_v.clone(), a_s.clone()
    merge_state_in_place(iv, is_, b_v, b_s)
    torch.cuda.synchronize()
    assert torch.equal(ov.cpu().view(torch.uint8), iv.cpu().view(torch.uint8))
    assert torch.equal(os_.cpu().view(torch.uint8), is_.cpu().view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("t,ns,h,d", [(50, 8, 4, 128), (17, 3, 2, 64), (64, 1, 1, 256), (40, 16, 2, 128),
                                      (33, 21, 3, 64)])
def test_merge_states_list(dtype, t, ns, h, d):
    """The S-way merge over separate tensors equals the oracle's merge_states of their stack;
    -inf states are not read (their v is NaN); more states than one launch takes are merged
    in groups."""
    say(f"merge_states_list dtype={dtype} t={t} S={ns} h={h} d={d}")
    g = torch.Generator().manual_seed(100 + ns)
    v = rounded(torch.randn(t, ns, h, d, generator=g), dtype)
    s = torch.randn(t, ns, h, generator=g) * 3
    s[torch.rand(t, ns, h, generator=g) < 0.2] = float("-inf")
    s[0] = float("-inf")
    vn = v.clone()
    vn[torch.isinf(s)] = float("nan")
    vs = [vn[:, i].contiguous().to(dtype).to(DEV) for i in range(ns)]
    ss = [s[:, i].contiguous().to(DEV) for i in range(ns)]
    out, so = merge_states_list(vs, ss)
    eo, el = O.merge_states(v, s)
    if ns <= 16:
        assert_rounded_close(out, eo, dtype)
    else:
        # the first group's result is stored in the v type before the second merge: one more
        # rounding, of a value no larger than max |v|
        bound = TOL_MERGE_FP32 + 2 * _HALF_ULP[dtype] * float(v.abs().max())
        assert max_err(out, eo) <= bound
    assert lse_err(so, el) <= TOL_MERGE_FP32


def _ring_partials(n, h, hkv, d, cp, rank, dtype=torch.bfloat16):
    """Full-size per-step partials of one rank's small ring, as the reference's loop builds
    them (fa4_ring/ring_attention.py:112-172, the late-Q steps padded with zeros / -inf),
    from this library's attention kernel, plus the oracle's partials of the same steps."""
    from fa4_ring.fa4_backend import SEL_BACK_HALF as BACK, SEL_FRONT_HALF as FRONT, fa4_attn

    q, k, v = O.random_qkv(n, h, hkv, d, seed=7)
    q, k, v = (rounded(x, dtype) for x in (q, k, v))
    ks = [O.zigzag_shard(k, r, cp) for r in range(cp)]
    vs = [O.zigzag_shard(v, r, cp) for r in range(cp)]
    lq = O.zigzag_shard(q, rank, cp)
    lqd = lq.to(dtype).to(DEV)
    parts = []
    for step in range(cp):
        src = (rank - step) % cp
        kd, vd = ks[src].to(dtype).to(DEV), vs[src].to(dtype).to(DEV)
        if step == 0:
            o, l = fa4_attn(lqd, kd, vd, causal=True)
        elif step <= rank:
            o, l = fa4_attn(lqd, kd, vd, causal=False, k_sel=FRONT)
        else:
            o = torch.zeros_like(lqd)
            l = torch.full(lqd.shape[:2], float("-inf"), device=DEV)
            fa4_attn(lqd, kd, vd, causal=False, q_sel=BACK, out=o, lse=l)
        parts.append((o, l))
    oracle_parts = [O.ring_rank(lq, ks, vs, rank, cp, scale_for(d), steps=[st]) for st in range(cp)]
    return parts, oracle_parts


@pytest.mark.parametrize("mode", ["incremental", "batched"])
@pytest.mark.parametrize("rank", [0, 2, 3])
def test_mergers_on_device_ring_partials(mode, rank):
    """IncrementalMerger / BatchedMerger (via make_merger) fed one rank's device partials
    step by step, as the reference's ring loop feeds them: the result equals the oracle's
    merge of the oracle's partials, and the caller's partials are never modified."""
    say(f"merger {mode} on device ring partials rank={rank}")
    n, h, hkv, d, cp = 1024, 8, 2, 128, 4
    parts, oparts = _ring_partials(n, h, hkv, d, cp, rank)
    keep = [(o.clone(), l.clone()) for o, l in parts]
    m = make_merger(mode)
    for o, l in parts:
        m.add(o, l)
    out = m.result()
    torch.cuda.synchronize()
    for (o, l), (ko, kl) in zip(parts, keep):
        assert torch.equal(o, ko) and torch.equal(l, kl), "a partial was modified"
    if mode == "incremental":
        eo, el = oparts[0]
        for o, l in oparts[1:]:
            eo, el = O.merge(eo, el, o, l)
        assert lse_err(m.lse, el) <= TOL_LSE
    else:
        eo, el = O.merge_states(torch.stack([p[0] for p in oparts], 1), torch.stack([p[1] for p in oparts], 1))
        _, lse = m.result_with_lse()
        assert lse_err(lse, el) <= TOL_LSE
    assert out.dtype == torch.bfloat16 and out.shape == (n // cp, h, d)
    assert max_err(out, eo) <= TOL_BF16_OUT


def test_incremental_merger_reused_buffer():
    """A caller that writes every step's partial into one preallocated buffer (as
    fa4_attn(..., out=part) invites) gets the same merge as with separate buffers: the
    first add copies the partial before the buffer is overwritten."""
    say("incremental merger, one partial buffer reused across add() calls")
    n, h, hkv, d, cp, rank = 1024, 8, 2, 128, 4, 3
    parts, oparts = _ring_partials(n, h, hkv, d, cp, rank)
    buf_o, buf_l = torch.empty_like(parts[0][0]), torch.empty_like(parts[0][1])
    m = make_merger("incremental")
    for o, l in parts:
        buf_o.copy_(o)
        buf_l.copy_(l)
        m.add(buf_o, buf_l)
    buf_o.fill_(float("nan"))  # the merger must hold nothing of the caller's buffer
    out = m.result()
    torch.cuda.synchronize()
    eo, el = oparts[0]
    for o, l in oparts[1:]:
        eo, el = O.merge(eo, el, o, l)
    assert lse_err(m.lse, el) <= TOL_LSE
    assert max_err(out, eo) <= TOL_BF16_OUT


@pytest.mark.parametrize("mode", ["incremental", "batched"])
def test_merger_single_partial(mode):
    """One partial: the incremental merger returns a copy (later changes to the caller's
    tensor do not reach it), the batched one the partial itself, as the reference's."""
    say(f"merger {mode} single partial")
    o = torch.randn(64, 2, 64, device=DEV).to(torch.bfloat16)
    l = torch.randn(64, 2, device=DEV)
    m = make_merger(mode)
    m.add(o, l)
    r = m.result()
    assert torch.equal(r, o)
    if mode == "incremental":
        assert r.data_ptr() != o.data_ptr()
    else:
        assert r is o


@pytest.mark.parametrize("cu", [None, [0, 8, 20, 64], [0, 8, 8, 20, 64, 64]])
@pytest.mark.parametrize("sel", [SEL_BACK_HALF, SEL_FRONT_HALF])
def test_merge_state_in_place_half_rows(cu, sel):
    say(f"merge half rows cu={cu} sel={sel}")
    t, h, d = 64, 4, 128
    va, sa = _states(t, h, d, 3, torch.float32)
    vb, sb = _states(t, h, d, 4, torch.float32)
    vd, sd = va.to(DEV), sa.to(DEV)
    cud = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=DEV)
    merge_state_in_place(vd, sd, vb.to(DEV), sb.to(DEV), cu_seqlens=cud, row_sel=sel)
    rows = O.get_half_index(cu if cu is not None else [0, t], front=(sel == SEL_FRONT_HALF))
    eo, el = va.clone(), sa.clone()
    mo, ml = O.merge(va[rows], sa[rows], vb[rows], sb[rows])
    eo[rows], el[rows] = mo, ml
    assert max_err(vd, eo) <= TOL_MERGE_FP32
    assert lse_err(sd, el) <= TOL_MERGE_FP32


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("t,ns,h,d", [(50, 8, 4, 128), (17, 3, 2, 64), (64, 1, 1, 256)])
def test_merge_states(dtype, t, ns, h, d):
    say(f"merge_states dtype={dtype} t={t} S={ns} h={h} d={d}")
    g = torch.Generator().manual_seed(ns)
    v = rounded(torch.randn(t, ns, h, d, generator=g), dtype)
    s = torch.randn(t, ns, h, generator=g) * 3
    s[torch.rand(t, ns, h, generator=g) < 0.2] = float("-inf")
    s[0] = float("-inf")  # one row with every state empty
    vd = v.clone()
    vd[torch.isinf(s)] = float("nan")  # never read when its LSE is -inf
    out, so = merge_states(vd.to(dtype).to(DEV), s.to(DEV))
    eo, el = O.merge_states(v, s)
    assert_rounded_close(out, eo, dtype)
    assert lse_err(so, el) <= TOL_MERGE_FP32


# ------------------------------------------------------------------------- V^T layout

@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float16, 64),
                                     (torch.float8_e4m3fn, 128), (torch.bfloat16, 256)])
@pytest.mark.parametrize("cu,sel", [(None, SEL_ALL), (None, SEL_FRONT_HALF), ([0, 64, 64, 330, 402], SEL_ALL),
                                    ([0, 64, 64, 330, 402], SEL_FRONT_HALF),
                                    ([0, 200, 456], SEL_BACK_HALF)])
def test_transpose_v_layout_bit_exact(dtype, d, cu, sel):
    """V^T positions: sequence j's selected keys at P_j + i, P_j = sum of the earlier
    sequences' selected lengths rounded up to 128, zeros up to the next multiple of 128."""
    from fa4_ring.fa4_backend import transpose_v
    say(f"transpose_v {dtype} d={d} cu={cu} sel={sel}")
    total = cu[-1] if cu is not None else 300
    hkv = 3
    g = torch.Generator().manual_seed(5)
    v = torch.randn(total, hkv, d, generator=g).to(dtype)
    cud = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=DEV)
    mx = None if cu is None else max(b - a for a, b in zip(cu[:-1], cu[1:]))
    vt, stride = transpose_v(v.to(DEV), cu_seqlens_k=cud, max_seqlen_k=mx, k_sel=sel)
    got = vt.cpu().view(torch.uint8 if dtype == torch.float8_e4m3fn else torch.int16).reshape(hkv, d, stride)
    raw = v.view(torch.uint8 if dtype == torch.float8_e4m3fn else torch.int16)
    pos = 0
    for (s0, e0) in seq_bounds(cu, total, sel):
        n = e0 - s0
        pad = (n + 127) // 128 * 128
        assert torch.equal(got[:, :, pos:pos + n], raw[s0:e0].permute(1, 2, 0))
        assert (got[:, :, pos + n:pos + pad] == 0).all()
        pos += pad


def _many_seq_cu(nseq, seed):
    """cu of nseq packed sequences with even lengths in [0, 300], some empty, some 2 rows."""
    g = torch.Generator().manual_seed(seed)
    lens = (torch.randint(0, 151, (nseq,), generator=g) * 2).tolist()
    lens[3] = 0
    lens[70 % nseq] = 2
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    return cu


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float8_e4m3fn, 128)])
@pytest.mark.parametrize("sel", [SEL_ALL, SEL_FRONT_HALF, SEL_BACK_HALF])
def test_transpose_v_layout_many_sequences(dtype, d, sel):
    """150 packed sequences: the V^T start of sequence j sums more than 64 earlier padded
    lengths (the kernels sum them 64 at a time across a wavefront)."""
    from fa4_ring.fa4_backend import transpose_v
    cu = _many_seq_cu(150, 9)
    say(f"transpose_v {dtype} d={d} 150 sequences sel={sel}")
    total, hkv = cu[-1], 2
    v = torch.randn(total, hkv, d, generator=torch.Generator().manual_seed(6)).to(dtype)
    cud = torch.tensor(cu, dtype=torch.int32, device=DEV)
    mx = max(b - a for a, b in zip(cu[:-1], cu[1:]))
    vt, stride = transpose_v(v.to(DEV), cu_seqlens_k=cud, max_seqlen_k=mx, k_sel=sel)
    got = vt.cpu().view(torch.uint8 if dtype == torch.float8_e4m3fn else torch.int16).reshape(hkv, d, stride)
    raw = v.view(torch.uint8 if dtype == torch.float8_e4m3fn else torch.int16)
    pos = 0
    for (s0, e0) in seq_bounds(cu, total, sel):
        n = e0 - s0
        pad = (n + 127) // 128 * 128
        assert torch.equal(got[:, :, pos:pos + n], raw[s0:e0].permute(1, 2, 0))
        assert (got[:, :, pos + n:pos + pad] == 0).all()
        pos += pad


@pytest.mark.parametrize("dtype,d,count", [(torch.bfloat16, 128, 8), (torch.float8_e4m3fn, 256, 3),
                                           (torch.float16, 64, 16), (torch.bfloat16, 128, 1)])
@pytest.mark.parametrize("cu", [None, [0, 200, 200, 713]])
def test_transpose_v_many_equals_one_by_one(dtype, d, count, cu):
    """One launch over `count` tensors writes what `count` single transposes write."""
    from fa4_ring.fa4_backend import transpose_v, transpose_v_many
    say(f"transpose_v_many {dtype} d={d} count={count} cu={cu}")
    total = cu[-1] if cu is not None else 300
    g = torch.Generator().manual_seed(6)
    vs = [torch.randn(total, 2, d, generator=g).to(dtype).to(DEV) for _ in range(count)]
    cud = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=DEV)
    mx = None if cu is None else max(b - a for a, b in zip(cu[:-1], cu[1:]))
    many, stride = transpose_v_many(vs, cu_seqlens_k=cud, max_seqlen_k=mx)
    for v, got in zip(vs, many):
        one, s1 = transpose_v(v, cu_seqlens_k=cud, max_seqlen_k=mx)
        assert s1 == stride
        iv = torch.uint8 if dtype == torch.float8_e4m3fn else torch.int16
        # positions past the last sequence's padding are never written (workspace)
        used = sum((b - a + 127) // 128 * 128 for a, b in seq_bounds(cu, total, 0))
        a_ = one.view(iv).reshape(2, d, stride)[:, :, :used]
        b_ = got.view(iv).reshape(2, d, stride)[:, :, :used]
        assert torch.equal(a_.cpu(), b_.cpu())


# ------------------------------------------------------------------------- attention

def _qkv(tq, tk, h, hkv, d, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(tq, h, d, generator=g)
    k = torch.randn(tk, hkv, d, generator=g)
    v = torch.randn(tk, hkv, d, generator=g)
    return rounded(q, dtype), rounded(k, dtype), rounded(v, dtype)


ATTN_CASES = [
    # tq, tk, h, hkv, d, causal, q_sel, k_sel, cu
    (256, 256, 4, 1, 128, True, SEL_ALL, SEL_ALL, None),
    (200, 200, 8, 2, 128, True, SEL_ALL, SEL_ALL, None),         # tail rows/keys
    (512, 256, 8, 8, 128, False, SEL_ALL, SEL_ALL, None),        # plain non-causal
    (512, 512, 8, 2, 128, False, SEL_ALL, SEL_FRONT_HALF, None),  # step s <= rank
    (512, 512, 8, 2, 128, False, SEL_BACK_HALF, SEL_ALL, None),   # step s > rank
    (300, 300, 6, 3, 64, True, SEL_ALL, SEL_ALL, None),
    (130, 130, 2, 2, 256, True, SEL_ALL, SEL_ALL, None),
    (160, 160, 16, 2, 256, False, SEL_BACK_HALF, SEL_ALL, None),
    (192, 192, 8, 1, 64, False, SEL_ALL, SEL_FRONT_HALF, None),
    (None, None, 8, 2, 128, True, SEL_ALL, SEL_ALL, [0, 64, 200, 202, 460]),
    (None, None, 8, 2, 128, False, SEL_ALL, SEL_FRONT_HALF, [0, 64, 200, 202, 460]),
    (None, None, 4, 4, 128, False, SEL_BACK_HALF, SEL_ALL, [0, 96, 100, 612]),
    (64, 96, 4, 2, 128, True, SEL_ALL, SEL_ALL, None),            # bottom-right causal
    (None, None, 8, 2, 128, True, SEL_ALL, SEL_ALL, [0, 64, 64, 200, 200]),         # empty seqs
    (None, None, 8, 2, 64, False, SEL_BACK_HALF, SEL_ALL, [0, 0, 130, 131, 260]),   # 1-row seq
    (None, None, 4, 1, 128, False, SEL_ALL, SEL_FRONT_HALF, [0, 1, 1, 67]),         # no keys
    # head dim 256 (32-key tiles when V^T is given)
    (512, 512, 8, 2, 256, False, SEL_ALL, SEL_FRONT_HALF, None),
    (72, 100, 4, 2, 256, True, SEL_ALL, SEL_ALL, None),           # bottom-right causal, tails
    (None, None, 4, 2, 256, True, SEL_ALL, SEL_ALL, [0, 64, 200, 202, 460]),
    (None, None, 8, 1, 256, False, SEL_BACK_HALF, SEL_ALL, [0, 0, 130, 131, 260]),
]


@pytest.mark.parametrize("use_vt", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", ATTN_CASES)
def test_attention_16bit(dtype, case, use_vt):
    tq, tk, h, hkv, d, causal, q_sel, k_sel, cu = case
    if cu is not None:
        tq = tk = cu[-1]
    say(f"attn {dtype} tq={tq} tk={tk} h={h}/{hkv} d={d} causal={causal} sel={q_sel},{k_sel} "
        f"cu={cu} vt={use_vt}")
    q, k, v = _qkv(tq, tk, h, hkv, d, 7, dtype)
    scale = scale_for(d)
    cud = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=DEV)
    mx = None if cu is None else max(b - a for a, b in zip(cu[:-1], cu[1:]))
    out = torch.full((tq, h, d), float("nan"), dtype=dtype, device=DEV)
    lse = torch.full((tq, h), float("nan"), device=DEV)
    fa4_attn(q.to(dtype).to(DEV), k.to(dtype).to(DEV), v.to(dtype).to(DEV), causal=causal,
             softmax_scale=scale, cu_seqlens_q=cud, cu_seqlens_k=cud, max_seqlen_q=mx,
             max_seqlen_k=mx, q_sel=q_sel, k_sel=k_sel, out=out, lse=lse, use_vt=use_vt)
    eo, el = oracle_attn(q, k, v, causal, scale, cu, cu, q_sel, k_sel)
    sel = ~torch.isnan(el)
    # rows outside the selection are left untouched
    assert torch.isnan(out.cpu().float()[~sel]).all() and torch.isnan(lse.cpu()[~sel]).all()
    assert max_err(out, eo, sel.unsqueeze(-1).expand_as(eo)) <= TOL_BF16_OUT
    assert lse_err(lse.cpu()[sel], el[sel]) <= TOL_LSE


def test_attention_default_layout_and_gqa_strided_views():
    """Reference calling convention: no cu_seqlens, default scale, fresh outputs; q given
    as a strided view of a larger buffer."""
    say("attn strided views")
    q, k, v = _qkv(256, 256, 8, 2, 128, 9, torch.bfloat16)
    big = torch.zeros(256, 12, 128, dtype=torch.bfloat16)
    big[:, 2:10] = q.to(torch.bfloat16)
    qd = big.to(DEV)[:, 2:10]
    out, lse = fa4_attn(qd, k.to(torch.bfloat16).to(DEV), v.to(torch.bfloat16).to(DEV), causal=True)
    eo, el = O.cpu_attn(q, k, v, True, 1 / math.sqrt(128))
    assert out.shape == (256, 8, 128) and lse.shape == (256, 8) and lse.dtype == torch.float32
    assert max_err(out, eo) <= TOL_BF16_OUT and lse_err(lse, el) <= TOL_LSE


FP8_CASES = [
    (512, 512, 8, 2, 128, True, SEL_ALL, SEL_ALL, None),
    (600, 600, 8, 2, 128, True, SEL_ALL, SEL_ALL, None),
    (512, 512, 8, 2, 128, False, SEL_ALL, SEL_FRONT_HALF, None),
    (512, 512, 8, 2, 128, False, SEL_BACK_HALF, SEL_ALL, None),
    (384, 384, 16, 2, 256, True, SEL_ALL, SEL_ALL, None),
    (384, 384, 16, 2, 256, False, SEL_BACK_HALF, SEL_ALL, None),
    (None, None, 8, 8, 128, True, SEL_ALL, SEL_ALL, [0, 128, 136, 520]),
    (None, None, 8, 2, 128, False, SEL_BACK_HALF, SEL_ALL, [0, 0, 256, 256, 390]),
    (333, 333, 8, 4, 128, True, SEL_ALL, SEL_ALL, None),          # 2 heads per kv head, tails
    (64, 200, 4, 4, 128, True, SEL_ALL, SEL_ALL, None),           # bottom-right causal, MHA
    (700, 700, 4, 1, 128, False, SEL_ALL, SEL_FRONT_HALF, None),  # MQA, partial key tile
    (1100, 1100, 4, 1, 128, True, SEL_ALL, SEL_ALL, None),        # rows past the precise block
]


@pytest.mark.parametrize("use_vt", [True, False])
@pytest.mark.parametrize("case", FP8_CASES)
def test_attention_e4m3(case, use_vt):
    tq, tk, h, hkv, d, causal, q_sel, k_sel, cu = case
    if cu is not None:
        tq = tk = cu[-1]
    say(f"attn e4m3 tq={tq} h={h}/{hkv} d={d} causal={causal} sel={q_sel},{k_sel} cu={cu}")
    g = torch.Generator().manual_seed(21)
    qf = torch.randn(tq, h, d, generator=g)
    kf = torch.randn(tk, hkv, d, generator=g)
    vf = torch.randn(tk, hkv, d, generator=g)
    sq, sk, sv = O.amax_scale(qf), O.amax_scale(kf), O.amax_scale(vf)
    q8, k8, v8 = O.quantize_e4m3(qf, sq), O.quantize_e4m3(kf, sk), O.quantize_e4m3(vf, sv)
    scale = scale_for(d)
    cud = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=DEV)
    mx = None if cu is None else max(b - a for a, b in zip(cu[:-1], cu[1:]))
    out = torch.full((tq, h, d), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse = torch.full((tq, h), float("nan"), device=DEV)
    fa4_attn(q8.to(DEV), k8.to(DEV), v8.to(DEV), causal=causal, softmax_scale=scale,
             cu_seqlens_q=cud, cu_seqlens_k=cud, max_seqlen_q=mx, max_seqlen_k=mx,
             q_descale=torch.tensor(sq, device=DEV), k_descale=torch.tensor([sk] * hkv, device=DEV),
             v_descale=torch.tensor(sv, device=DEV).reshape(1, 1).expand(1, hkv),
             q_sel=q_sel, k_sel=k_sel, out=out, lse=lse, use_vt=use_vt)
    eo, el = oracle_attn(O.dequantize_e4m3(q8, sq), O.dequantize_e4m3(k8, sk),
                         O.dequantize_e4m3(v8, sv), causal, scale, cu, cu, q_sel, k_sel)
    sel = ~torch.isnan(el)
    assert max_err(out, eo, sel.unsqueeze(-1).expand_as(eo)) <= TOL_FP8_OUT
    assert lse_err(lse.cpu()[sel], el[sel]) <= TOL_LSE


PAD_CASES = [
    # tq, tk, h, hkv, d, causal, q_sel, k_sel, cu: head dims without a kernel of their own
    (200, 200, 8, 2, 32, True, SEL_ALL, SEL_ALL, None),
    (256, 256, 4, 1, 80, False, SEL_ALL, SEL_FRONT_HALF, None),
    (256, 256, 8, 2, 96, False, SEL_BACK_HALF, SEL_ALL, None),
    (None, None, 4, 2, 96, True, SEL_ALL, SEL_ALL, [0, 64, 200, 202, 460]),
    (130, 130, 4, 2, 192, True, SEL_ALL, SEL_ALL, None),
    (64, 96, 4, 4, 160, True, SEL_ALL, SEL_ALL, None),  # bottom-right causal
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", PAD_CASES)
def test_attention_padded_head_dims(dtype, case):
    """Head dims without a kernel run at the next supported one on zero-padded copies, with
    the selection semantics intact: rows outside a q selection keep what out held."""
    tq, tk, h, hkv, d, causal, q_sel, k_sel, cu = case
    if cu is not None:
        tq = tk = cu[-1]
    say(f"attn padded head dim {dtype} tq={tq} tk={tk} h={h}/{hkv} d={d} causal={causal} sel={q_sel},{k_sel} cu={cu}")
    q, k, v = _qkv(tq, tk, h, hkv, d, 13, dtype)
    scale = scale_for(d)
    cud = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=DEV)
    mx = None if cu is None else max(b - a for a, b in zip(cu[:-1], cu[1:]))
    out = torch.full((tq, h, d), float("nan"), dtype=dtype, device=DEV)
    lse = torch.full((tq, h), float("nan"), device=DEV)
    got, glse = fa4_attn(q.to(dtype).to(DEV), k.to(dtype).to(DEV), v.to(dtype).to(DEV), causal=causal,
                         cu_seqlens_q=cud, cu_seqlens_k=cud, max_seqlen_q=mx, max_seqlen_k=mx,
                         q_sel=q_sel, k_sel=k_sel, out=out, lse=lse)
    assert got is out and glse is lse
    eo, el = oracle_attn(q, k, v, causal, scale, cu, cu, q_sel, k_sel)  # default scale: 1/sqrt(d)
    sel = ~torch.isnan(el)
    assert torch.isnan(out.cpu().float()[~sel]).all() and torch.isnan(lse.cpu()[~sel]).all()
    assert max_err(out, eo, sel.unsqueeze(-1).expand_as(eo)) <= TOL_BF16_OUT
    assert lse_err(lse.cpu()[sel], el[sel]) <= TOL_LSE
    if q_sel == SEL_ALL:  # fresh outputs
        o2, l2 = fa4_attn(q.to(dtype).to(DEV), k.to(dtype).to(DEV), v.to(dtype).to(DEV), causal=causal,
                          cu_seqlens_q=cud, cu_seqlens_k=cud, max_seqlen_q=mx, max_seqlen_k=mx, k_sel=k_sel)
        assert o2.shape == (tq, h, d) and o2.is_contiguous()
        assert torch.equal(o2, out) and torch.equal(l2, lse)


@pytest.mark.parametrize("d", [64, 96, 200])
def test_attention_e4m3_padded_head_dims(d):
    say(f"attn e4m3 padded head dim d={d}")
    tq, h, hkv = 384, 8, 2
    g = torch.Generator().manual_seed(31)
    qf, kf, vf = (torch.randn(tq, hh, d, generator=g) for hh in (h, hkv, hkv))
    sq, sk, sv = O.amax_scale(qf), O.amax_scale(kf), O.amax_scale(vf)
    q8, k8, v8 = O.quantize_e4m3(qf, sq), O.quantize_e4m3(kf, sk), O.quantize_e4m3(vf, sv)
    out, lse = fa4_attn(q8.to(DEV), k8.to(DEV), v8.to(DEV), causal=True, q_descale=torch.tensor(sq, device=DEV),
                        k_descale=torch.tensor(sk, device=DEV), v_descale=torch.tensor(sv, device=DEV))
    assert out.dtype == torch.bfloat16 and out.shape == (tq, h, d)
    eo, el = O.cpu_attn(O.dequantize_e4m3(q8, sq), O.dequantize_e4m3(k8, sk), O.dequantize_e4m3(v8, sv), True,
                        scale_for(d))
    assert max_err(out, eo) <= TOL_FP8_OUT and lse_err(lse, el) <= TOL_LSE


def test_attention_inputs_not_contiguous_in_d():
    """q, k and v whose head dim is strided are copied to contiguous rows first (as the
    reference's .contiguous() before FA4): same result as contiguous inputs."""
    say("attn inputs strided in D")
    q, k, v = _qkv(256, 256, 8, 2, 128, 17, torch.bfloat16)
    qb, kb, vb = (t.to(torch.bfloat16).to(DEV) for t in (q, k, v))
    qs, ks, vs = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (qb, kb, vb))  # stride(2) != 1
    assert qs.stride(2) != 1 and torch.equal(qs, qb)
    o1, l1 = fa4_attn(qs, ks, vs, causal=True)
    o2, l2 = fa4_attn(qb, kb, vb, causal=True)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    eo, el = O.cpu_attn(q, k, v, True, scale_for(128))
    assert max_err(o1, eo) <= TOL_BF16_OUT and lse_err(l1, el) <= TOL_LSE


def test_attention_rejects_unsupported():
    say("attn rejects")
    x = torch.zeros(64, 2, 320, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(AssertionError, match="head dim"):
        fa4_attn(x, x, x, causal=True)
    y = torch.zeros(64, 2, 288, dtype=torch.float8_e4m3fn, device=DEV)
    with pytest.raises(AssertionError, match="head dim"):
        fa4_attn(y, y, y, causal=True)
    z = torch.zeros(64, 3, 128, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(AssertionError, match="multiple"):
        fa4_attn(z, w, w, causal=True)
