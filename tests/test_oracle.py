"""Pins the CPU oracle before anything is compared against it.

Every oracle function is checked against something other than its own formula: the
reference's known-answer lists, torch SDPA, brute-force float64 loops, the merge
identity attention(K1 u K2) == merge(attention(K1), attention(K2)), the reference's
end-to-end invariant unshard(ring) == dense causal attention (with a planted one-hop
source lag that must fail it), and a bit-level e4m3 decoder.
"""

import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ring_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _kat():
    with open(os.path.join(GOLDEN, "zigzag_kat.json")) as f:
        return json.load(f)


# ---------------------------------------------------------------- zig-zag index math


def test_zigzag_pairs_early_and_late_kat():
    kat = _kat()["pairs_early_late"]
    x = torch.arange(kat["n"]).reshape(-1, 1).float()
    for r, rows in kat["rows"].items():
        got = O.zigzag_shard(x, int(r), kat["cp_size"]).flatten().long().tolist()
        assert got == rows
        assert O.zigzag_rows(kat["n"], int(r), kat["cp_size"]).tolist() == rows


def test_zigzag_each_rank_holds_2h():
    kat = _kat()["each_rank_2h"]
    for r in range(kat["cp_size"]):
        assert len(O.zigzag_rows(kat["n"], r, kat["cp_size"])) == kat["rows_per_rank"]


def test_zigzag_roundtrip_and_partition():
    for cp in _kat()["roundtrip_cp_sizes"]:
        n = 4 * cp * 3
        x = torch.arange(n).reshape(n, 1).float()
        shards = [O.zigzag_shard(x, r, cp) for r in range(cp)]
        assert torch.equal(O.zigzag_unshard(shards, cp), x)
        # the ranks' rows partition 0..n-1
        allrows = np.concatenate([O.zigzag_rows(n, r, cp) for r in range(cp)])
        assert sorted(allrows.tolist()) == list(range(n))


def test_half_index_kats():
    kat = _kat()
    first, second = O.half_indices(kat["half_indices"]["local_len"])
    assert first.tolist() == kat["half_indices"]["first"]
    assert second.tolist() == kat["half_indices"]["second"]
    g = kat["get_half_index"]
    assert O.get_half_index(g["cu"], front=True).tolist() == g["front"]
    assert O.get_half_index(g["cu"], front=False).tolist() == g["back"]
    assert [c // 2 for c in g["cu"]] == g["half_cu"]


def test_shard_varlen_kat():
    g = _kat()["shard_varlen"]
    x = torch.arange(g["full_cu"][-1]).reshape(-1, 1).float()
    for rank in range(g["cp_size"]):
        local, local_cu = O.zigzag_shard_varlen(x, g["full_cu"], rank, g["cp_size"])
        assert local_cu == g["local_cu"]
        assert local.shape[0] == g["local_rows"]
        # each sequence is sharded on its own
        for j in range(len(g["full_cu"]) - 1):
            s, e = g["full_cu"][j], g["full_cu"][j + 1]
            seg = O.zigzag_shard(x[s:e], rank, g["cp_size"])
            assert torch.equal(local[local_cu[j]:local_cu[j + 1]], seg)


def test_c4_lengths_fixture():
    with open(os.path.join(GOLDEN, "c4_lengths.json")) as f:
        fx = json.load(f)
    lens = O.varlen_lengths(fx["seed"])
    assert lens == fx["lengths"]
    assert all(l % 8 == 0 and 1024 <= l <= 16384 for l in lens) and sum(lens) <= 65536
    assert all(l % (2 * 4) == 0 for l in lens)  # shardable at cp_size = 4


# ---------------------------------------------------------------- attention + lse


def _brute_attn(q, k, v, causal, scale, align=None):
    """float64 triple loop: the textbook definition.  Causal: query i sees the keys
    j <= i + align, align = Tk - Tq (bottom-right) unless given; a query that sees no key
    gets out 0 and lse -inf."""
    tq, h, d = q.shape
    tk, hkv, _ = k.shape
    g = h // hkv
    align = tk - tq if align is None else align
    out = np.zeros((tq, h, v.shape[2]))
    lse = np.zeros((tq, h))
    qn, kn, vn = q.double().numpy(), k.double().numpy(), v.double().numpy()
    for i in range(tq):
        for hh in range(h):
            keys = range(tk) if not causal else range(min(tk, max(0, i + align + 1)))
            if len(keys) == 0:
                lse[i, hh] = -math.inf
                continue
            sc = np.array([scale * float(np.dot(qn[i, hh], kn[j, hh // g])) for j in keys])
            m = sc.max()
            w = np.exp(sc - m)
            lse[i, hh] = m + math.log(w.sum())
            out[i, hh] = sum(w[t] * vn[j, hh // g] for t, j in enumerate(keys)) / w.sum()
    return torch.from_numpy(out), torch.from_numpy(lse)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("h,hkv", [(4, 4), (4, 2), (4, 1), (6, 3)])
def test_cpu_attn_vs_brute_force(causal, h, hkv):
    g = torch.Generator().manual_seed(3)
    t, d = 9, 8
    q, k, v = (torch.randn(t, hh, d, generator=g) for hh in (h, hkv, hkv))
    scale = 0.37
    out, lse = O.cpu_attn(q, k, v, causal, scale)
    bo, bl = _brute_attn(q, k, v, causal, scale)
    assert (out.double() - bo).abs().max() < 1e-5
    assert (lse.double() - bl).abs().max() < 1e-5


@pytest.mark.parametrize("tq,tk", [(5, 11), (11, 5), (1, 7), (7, 1), (8, 8)])
def test_cpu_attn_bottom_right_causal(tq, tk):
    """Causal with Tq != Tk is bottom-right aligned (query i sees key j <= i + Tk - Tq), the
    mask the kernel-level tests use for packed query / key lengths that differ.  Rows that
    see no key give (0, -inf).  A mask aligned top-left instead (a planted mistake) must
    fail the same comparison."""
    g = torch.Generator().manual_seed(11)
    h, hkv, d = 4, 2, 8
    q = torch.randn(tq, h, d, generator=g)
    k = torch.randn(tk, hkv, d, generator=g)
    v = torch.randn(tk, hkv, d, generator=g)
    scale = 0.41
    out, lse = O.cpu_attn(q, k, v, True, scale)
    bo, bl = _brute_attn(q, k, v, True, scale)
    assert (out.double() - bo).abs().max() < 1e-5
    fin = torch.isfinite(bl)
    assert torch.equal(torch.isfinite(lse), fin)
    assert (lse.double()[fin] - bl[fin]).abs().max() < 1e-5
    if tq > tk:  # the first Tq - Tk queries see no key
        assert torch.all(out[: tq - tk] == 0) and torch.all(lse[: tq - tk] == -math.inf)
    if tq != tk:
        po, pl = _brute_attn(q, k, v, True, scale, align=0)  # planted: top-left alignment
        bad = (out.double() - po).abs().max() > 1e-3 or not torch.equal(torch.isfinite(lse), torch.isfinite(pl))
        assert bad, "a top-left aligned mask went unnoticed"


def test_cpu_attn_vs_sdpa_and_chunking():
    g = torch.Generator().manual_seed(5)
    t, h, hkv, d = 300, 8, 2, 32
    q, k, v = (torch.randn(t, hh, d, generator=g) for hh in (h, hkv, hkv))
    scale = 1 / math.sqrt(d)
    out, _ = O.cpu_attn(q, k, v, True, scale, row_chunk=64)  # chunked
    out_full, _ = O.cpu_attn(q, k, v, True, scale, row_chunk=4096)
    kk = k.repeat_interleave(h // hkv, 1).transpose(0, 1)[None].double()
    vv = v.repeat_interleave(h // hkv, 1).transpose(0, 1)[None].double()
    ref = F.scaled_dot_product_attention(q.transpose(0, 1)[None].double(), kk, vv,
                                         is_causal=True, scale=scale)[0].transpose(0, 1)
    assert (out.double() - ref).abs().max() < 1e-5
    assert torch.equal(out, out_full)


def test_lse_is_log_of_softmax_denominator():
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(20, 2, 16, generator=g) for _ in range(3))
    scale = 0.25
    _, lse = O.cpu_attn(q, k, v, False, scale)
    s = torch.einsum("qhd,khd->hqk", q.double(), k.double()) * scale
    assert (lse.double() - torch.log(torch.exp(s).sum(-1)).T).abs().max() < 1e-5


# ---------------------------------------------------------------- merges


def _split_keys(seed, t=24, tk=40, h=4, hkv=2, d=16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(t, h, d, generator=g)
    k = torch.randn(tk, hkv, d, generator=g) * 2
    v = torch.randn(tk, hkv, d, generator=g)
    return q, k, v


@pytest.mark.parametrize("cut", [1, 13, 39])
def test_merge_equals_attention_over_union(cut):
    q, k, v = _split_keys(cut)
    scale = 0.3
    full_o, full_l = O.cpu_attn(q, k, v, False, scale)
    oa, la = O.cpu_attn(q, k[:cut], v[:cut], False, scale)
    ob, lb = O.cpu_attn(q, k[cut:], v[cut:], False, scale)
    mo, ml = O.merge(oa, la, ob, lb)
    assert (mo - full_o).abs().max() < 1e-5
    assert (ml - full_l).abs().max() < 1e-5
    # merge is symmetric
    mo2, ml2 = O.merge(ob, lb, oa, la)
    assert (mo2 - mo).abs().max() < 1e-6 and (ml2 - ml).abs().max() < 1e-6


def test_merge_neg_inf_is_identity_and_both_neg_inf_is_nan():
    q, k, v = _split_keys(2)
    o, l = O.cpu_attn(q, k, v, False, 0.3)
    z = torch.zeros_like(o)
    ninf = torch.full_like(l, float("-inf"))
    mo, ml = O.merge(o, l, z, ninf)
    assert torch.allclose(mo, o, atol=1e-6) and torch.equal(ml, l)
    mo, ml = O.merge(z, ninf, z, ninf)
    assert torch.isnan(mo).all()  # the reference's merge NaN-poisons such rows


def test_merge_states_equals_attention_over_union():
    q, k, v = _split_keys(9, tk=50)
    scale = 0.3
    cuts = [0, 7, 20, 21, 50]
    parts = [O.cpu_attn(q, k[a:b], v[a:b], False, scale) for a, b in zip(cuts[:-1], cuts[1:])]
    vs = torch.stack([p[0] for p in parts], 1)
    ss = torch.stack([p[1] for p in parts], 1)
    mo, ml = O.merge_states(vs, ss)
    fo, fl = O.cpu_attn(q, k, v, False, scale)
    assert (mo - fo).abs().max() < 1e-5 and (ml - fl).abs().max() < 1e-5
    # a -inf state is skipped, an all -inf row gives (0, -inf)
    ss2 = ss.clone()
    ss2[:, 1] = float("-inf")
    vs2 = vs.clone()
    vs2[:, 1] = float("nan")
    mo2, _ = O.merge_states(vs2, ss2)
    assert torch.isfinite(mo2).all()
    mo3, ml3 = O.merge_states(vs, torch.full_like(ss, float("-inf")))
    assert (mo3 == 0).all() and torch.isinf(ml3).all()


# ---------------------------------------------------------------- the ring sweep

RING_CASES = [  # tests/test_algorithm_cpu.py:202-211
    (16, 4, 4, 8, 2), (32, 8, 2, 16, 4), (64, 8, 8, 16, 4), (64, 4, 1, 32, 8),
    (128, 8, 2, 64, 8), (48, 6, 3, 16, 2), (96, 8, 8, 16, 4),
]
VARLEN_CASES = [  # tests/test_algorithm_cpu.py:217-223
    ([16, 32], 4, 4, 8, 2), ([32, 16, 48], 8, 2, 16, 4), ([64, 64], 4, 1, 16, 8),
    ([48, 24], 6, 3, 16, 2),
]


@pytest.mark.parametrize("n,h,hkv,d,cp", RING_CASES)
def test_ring_equals_dense_causal(n, h, hkv, d, cp):
    torch.manual_seed(0)
    q, k, v = torch.randn(n, h, d), torch.randn(n, hkv, d), torch.randn(n, hkv, d)
    scale = 1 / math.sqrt(d)
    ref = O.dense_causal(q, k, v, scale)
    got = O.simulate_ring(q, k, v, cp, scale)
    assert torch.allclose(got, ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("n,h,hkv,d,cp", [c for c in RING_CASES if c[4] > 1])
def test_ring_with_planted_source_lag_fails(n, h, hkv, d, cp):
    """The one-hop lag of the reference GPU loop (step s attending rank - s + 1) must
    break the dense-causal invariant; this guards the oracle's source indexing."""
    torch.manual_seed(0)
    q, k, v = torch.randn(n, h, d), torch.randn(n, hkv, d), torch.randn(n, hkv, d)
    scale = 1 / math.sqrt(d)
    ref = O.dense_causal(q, k, v, scale)
    bad = O.simulate_ring(q, k, v, cp, scale, src_lag=1)
    assert (bad - ref).abs().max() > 1e-2


@pytest.mark.parametrize("lens,h,hkv,d,cp", VARLEN_CASES)
@pytest.mark.parametrize("mode", ["incremental", "batched"])
def test_ring_varlen_equals_dense_causal(lens, h, hkv, d, cp, mode):
    torch.manual_seed(0)
    seqs = [(torch.randn(n, h, d), torch.randn(n, hkv, d), torch.randn(n, hkv, d)) for n in lens]
    scale = 1 / math.sqrt(d)
    recon = O.simulate_ring_varlen(seqs, cp, scale, merge_mode=mode)
    for (q, k, v), got in zip(seqs, recon):
        assert torch.allclose(got, O.dense_causal(q, k, v, scale), atol=1e-4, rtol=1e-4)


def test_ring_rank_batched_equals_incremental_and_lse_is_dense():
    n, h, hkv, d, cp = 64, 4, 2, 16, 4
    q, k, v = O.random_qkv(n, h, hkv, d, seed=1)
    scale = 1 / math.sqrt(d)
    ks = [O.zigzag_shard(k, r, cp) for r in range(cp)]
    vs = [O.zigzag_shard(v, r, cp) for r in range(cp)]
    _, dense_lse = O.cpu_attn(q, k, v, True, scale)
    for rank in range(cp):
        lq = O.zigzag_shard(q, rank, cp)
        oi, li = O.ring_rank(lq, ks, vs, rank, cp, scale)
        ob, lb = O.ring_rank(lq, ks, vs, rank, cp, scale, merge_mode="batched")
        assert (oi - ob).abs().max() < 1e-5 and (li - lb).abs().max() < 1e-5
        assert (li - O.zigzag_shard(dense_lse, rank, cp)).abs().max() < 1e-4


def test_dense_causal_rows_matches_full():
    q, k, v = O.random_qkv(80, 4, 2, 16, seed=4)
    scale = 0.25
    full, lse = O.cpu_attn(q, k, v, True, scale)
    rows, heads = [0, 5, 79, 40], [0, 3, 2, 1]
    o, l = O.dense_causal_rows(q, k, v, rows, heads, scale)
    for i, (r, hh) in enumerate(zip(rows, heads)):
        assert (o[i] - full[r, hh]).abs().max() < 1e-5
        assert abs(float(l[i] - lse[r, hh])) < 1e-5


@pytest.mark.parametrize("key_block", [7, 64, 1000])
def test_dense_causal_rows_all_heads_matches_per_pair(key_block):
    """The batched row checker equals the per-(row, head) one on every head, for packed
    sequences (rows of the first and second sequence, the first and last row of each), with
    key blocks that split sequences unevenly."""
    lens = [56, 90, 34]
    cu = [0, 56, 146, 180]
    q, k, v = O.random_qkv(cu[-1], 6, 2, 16, seed=12)
    scale = 0.3
    rows = [0, 1, 55, 56, 57, 100, 145, 146, 179, 30]
    starts = [cu[int(np.searchsorted(cu, r, side="right")) - 1] for r in rows]
    o, l = O.dense_causal_rows_all_heads(q[rows], rows, starts, k, v, scale, key_block=key_block)
    for i, (r, s) in enumerate(zip(rows, starts)):
        eo, el = O.dense_causal_rows(q, k, v, [r] * 6, list(range(6)), scale, seq_start=s)
        assert (o[i] - eo).abs().max() < 2e-5, (r, key_block)
        assert (l[i] - el).abs().max() < 2e-5, (r, key_block)
    # a planted off-by-one (row i also seeing key i + 1) must be caught
    bad, _ = O.dense_causal_rows_all_heads(q[rows], [r + 1 for r in rows[:3]] + rows[3:], starts, k, v, scale)
    assert (bad[:3] - o[:3]).abs().max() > 1e-2


def _dense_grads_fp64(q, k, v, dout, scale, full_cu):
    """torch autograd of block-diagonal causal attention in float64 (GQA by repetition)."""
    q64, k64, v64 = (x.double().requires_grad_(True) for x in (q, k, v))
    h = q.shape[1]
    g = h // k.shape[1]
    outs = []
    for j in range(len(full_cu) - 1):
        s, e = full_cu[j], full_cu[j + 1]
        kq = k64[s:e].repeat_interleave(g, dim=1)
        vq = v64[s:e].repeat_interleave(g, dim=1)
        sc = torch.einsum("qhd,khd->hqk", q64[s:e], kq) * scale
        n = e - s
        sc = sc.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool), 1), float("-inf"))
        outs.append(torch.einsum("hqk,khd->qhd", torch.softmax(sc, -1), vq))
    torch.cat(outs).backward(dout.double())
    return q64.grad, k64.grad, v64.grad


def _ring_grads(q, k, v, dout, cp, scale, full_cu, drop_delta=False):
    """Every rank's oracle backward; dK / dV contributions summed per source shard and all
    shards stitched back to the full sequence."""
    ks = [O.zigzag_shard_varlen(k, full_cu, r, cp)[0] for r in range(cp)]
    vs = [O.zigzag_shard_varlen(v, full_cu, r, cp)[0] for r in range(cp)]
    dqs, dk_sum, dv_sum = [], [torch.zeros_like(x) for x in ks], [torch.zeros_like(x) for x in vs]
    for rank in range(cp):
        lq, lcu = O.zigzag_shard_varlen(q, full_cu, rank, cp)
        ldo = O.zigzag_shard_varlen(dout, full_cu, rank, cp)[0]
        out, lse = O.ring_rank(lq, ks, vs, rank, cp, scale, cu=lcu)
        dq, dk, dv = O.ring_rank_backward(lq, ks, vs, ldo, out, lse, rank, cp, scale, cu=lcu, drop_delta=drop_delta)
        dqs.append(dq)
        for i in range(cp):
            dk_sum[i] += dk[i]
            dv_sum[i] += dv[i]

    def stitch(parts):
        full = torch.zeros(q.shape[0], *parts[0].shape[1:])
        for r in range(cp):
            full[torch.from_numpy(O.zigzag_rows_varlen(full_cu, r, cp))] = parts[r]
        return full

    return stitch(dqs), stitch(dk_sum), stitch(dv_sum)


@pytest.mark.parametrize("lens,h,hkv,d,cp", [([64], 4, 2, 16, 4), ([96], 2, 1, 8, 2), ([32, 48, 16], 4, 2, 8, 2),
                                             ([128], 4, 4, 16, 8), ([64, 128], 8, 2, 8, 4)])
def test_ring_backward_equals_dense_autograd(lens, h, hkv, d, cp):
    """Summed over every rank (dq stitched, each source's dK / dV contributions added), the
    oracle's ring backward equals torch autograd of dense causal attention in float64, per
    packed sequence; the same with delta dropped (a plausible mistake) does not."""
    full_cu = [0]
    for n in lens:
        full_cu.append(full_cu[-1] + n)
    q, k, v = O.random_qkv(full_cu[-1], h, hkv, d, seed=21)
    dout = torch.randn(full_cu[-1], h, d, generator=torch.Generator().manual_seed(22))
    scale = 1 / math.sqrt(d)
    gq, gk, gv = _dense_grads_fp64(q, k, v, dout, scale, full_cu)
    dq, dk, dv = _ring_grads(q, k, v, dout, cp, scale, full_cu)
    for got, want in ((dq, gq), (dk, gk), (dv, gv)):
        assert (got.double() - want).abs().max() < 1e-4 * max(1.0, float(want.abs().max()))
    bq, bk, _ = _ring_grads(q, k, v, dout, cp, scale, full_cu, drop_delta=True)
    assert (bq.double() - gq).abs().max() > 1e-2 and (bk.double() - gk).abs().max() > 1e-2


# ---------------------------------------------------------------- e4m3


def _e4m3_bits(code: int) -> float:
    """Independent decoder: interpret the byte through its bit fields via integer math."""
    s = -1 if (code >> 7) & 1 else 1
    e = (code >> 3) & 15
    m = code & 7
    if e == 15 and m == 7:
        return float("nan")
    mant = m if e == 0 else (8 + m)
    exp = -6 if e == 0 else e - 7
    return s * mant * 2.0 ** (exp - 3)


def test_e4m3_decoder_against_torch_all_codes():
    codes = torch.arange(256, dtype=torch.uint8)
    tv = codes.view(torch.float8_e4m3fn).float().tolist()
    for c in range(256):
        a, b, t = O.e4m3_decode(c), _e4m3_bits(c), tv[c]
        if math.isnan(t):
            assert math.isnan(a) and math.isnan(b)
        else:
            assert a == b == t, (c, a, b, t)
    assert O.e4m3_decode(0x7E) == 448.0 and O.e4m3_decode(0x01) == 2.0 ** -9


def test_quantize_e4m3_round_trip_and_saturation():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(4096, generator=g) * 3
    s = O.amax_scale(x)
    x8 = O.quantize_e4m3(x, s)
    back = O.dequantize_e4m3(x8, s)
    # amax maps to 448 exactly, relative error of e4m3 is <= 2^-4 for normals
    assert abs(float(back.abs().max()) - float(x.abs().max())) < 1e-6 * float(x.abs().max())
    normal = x.abs() / s >= 2 ** -6
    rel = ((back - x).abs() / x.abs())[normal]
    assert rel.max() <= 2 ** -4 + 1e-7
    # values past the range saturate instead of turning into NaN
    big = O.quantize_e4m3(torch.tensor([1000.0, -1e6]), 1.0).float()
    assert big.tolist() == [448.0, -448.0]
