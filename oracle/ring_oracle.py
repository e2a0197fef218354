"""CPU oracle for the per-rank zig-zag ring-attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the ``fa4_ring`` package and its HIP
library) may import, call or link this module; only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` use it, to check results or as the timed CPU
baseline.

It restates the reference's own CPU algorithm (hxy0118/fa4-cp) in fp32 torch on the CPU:

* zig-zag index math          fa4_ring/zigzag.py:26-97
* per-chunk attention + LSE   tests/test_algorithm_cpu.py:28-48 (einsum + logsumexp)
* online-softmax merge        tests/test_algorithm_cpu.py:51-59
* one rank's ring sweep       tests/test_algorithm_cpu.py:62-90 and :114-168, i.e. with the
                              correct source ``src = (rank - step) % cp_size`` at step ``step``
                              (the GPU path of fa4_ring/ring_attention.py:125-171 lags one hop)
* batched merge               flashinfer.cascade.merge_states, as used by
                              fa4_ring/merge.py:67-86 (not vendored in the reference; restated
                              from its published semantics: an S-way max-shifted LSE merge)
* dense causal reference      fa4_ring/reference.py:20-54 and tests/test_algorithm_cpu.py:93-95
* OCP e4m3fn quantisation     the FP8 recipe of the benchmark configs: scale = amax / 448,
                              x8 = clamp(x / scale, +-448) cast to float8_e4m3fn, and
                              dequantisation x8 * scale (the descale of fa4_ring/fa4_backend.py:45-55)

Attention is computed in query-row chunks so that full-size shapes fit in host memory; the
chunking does not change the arithmetic of a row.

How each function is pinned (tests/test_oracle.py):
  zig-zag / half index / local_cu  the reference's known-answer lists (tests/golden/zigzag_kat.json,
                                   copied from tests/test_zigzag.py:21-78) and closed forms
  cpu_attn / lse                   torch SDPA, brute-force float64 loops (square and bottom-right
                                   causal, with a planted alignment error that must fail),
                                   softmax invariants
  merge / merge_states             attention over K1 u K2 == merge(attention over K1, over K2)
  ring sweep                       unshard(all ranks) == dense causal attention for the eleven
                                   cases of tests/test_algorithm_cpu.py:202-223, plus a planted
                                   one-hop source lag that must fail the same check
  e4m3                             an independent bit-level decoder over all 256 codes
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

E4M3_MAX = 448.0

# --------------------------------------------------------------------------------------
# zig-zag index math (fa4_ring/zigzag.py:26-97)
# --------------------------------------------------------------------------------------


def local_seqlen(n: int, cp_size: int) -> int:
    """zigzag.py:26-28."""
    assert n % (2 * cp_size) == 0
    return n // cp_size


def zigzag_rows(n: int, cp_rank: int, cp_size: int) -> np.ndarray:
    """Rows of a length-n sequence held by cp_rank, in local order (zigzag.py:31-39):
    chunk cp_rank then chunk 2*cp_size-1-cp_rank, chunks of h = n / (2*cp_size)."""
    assert n % (2 * cp_size) == 0
    h = n // (2 * cp_size)
    j = 2 * cp_size - 1 - cp_rank
    return np.concatenate([np.arange(cp_rank * h, (cp_rank + 1) * h),
                           np.arange(j * h, (j + 1) * h)]).astype(np.int64)


def zigzag_shard(x: torch.Tensor, cp_rank: int, cp_size: int) -> torch.Tensor:
    """zigzag.py:31-39."""
    idx = torch.from_numpy(zigzag_rows(x.shape[0], cp_rank, cp_size))
    return x.index_select(0, idx.to(x.device)).contiguous()


def zigzag_unshard(local_shards: Sequence[torch.Tensor], cp_size: int) -> torch.Tensor:
    """zigzag.py:42-50: inverse of zigzag_shard over all ranks."""
    assert len(local_shards) == cp_size
    n = local_shards[0].shape[0] * cp_size
    out = local_shards[0].new_empty((n,) + tuple(local_shards[0].shape[1:]))
    for r, loc in enumerate(local_shards):
        out[torch.from_numpy(zigzag_rows(n, r, cp_size))] = loc
    return out


def half_indices(local_len: int) -> Tuple[np.ndarray, np.ndarray]:
    """zigzag.py:53-62."""
    h = local_len // 2
    return np.arange(0, h), np.arange(h, local_len)


def get_half_index(cu: Sequence[int], *, front: bool) -> np.ndarray:
    """zigzag.py:65-79: front (early) or back (late) half rows of every packed sequence."""
    parts = []
    for i in range(len(cu) - 1):
        s, e = int(cu[i]), int(cu[i + 1])
        assert (e - s) % 2 == 0
        mid = (s + e) // 2
        parts.append(np.arange(s, mid) if front else np.arange(mid, e))
    return np.concatenate(parts).astype(np.int64) if parts else np.zeros(0, np.int64)


def local_cu_from_full(full_cu: Sequence[int], cp_size: int) -> List[int]:
    """Local cu_seqlens of every rank (zigzag.py:82-97): each sequence contributes
    2 * N_j / (2 * cp_size) rows."""
    out = [0]
    for j in range(len(full_cu) - 1):
        n = int(full_cu[j + 1]) - int(full_cu[j])
        assert n % (2 * cp_size) == 0
        out.append(out[-1] + n // cp_size)
    return out


def zigzag_rows_varlen(full_cu: Sequence[int], cp_rank: int, cp_size: int) -> np.ndarray:
    """Rows of the packed full tensor held by cp_rank, in local order (zigzag.py:82-97)."""
    parts = []
    for j in range(len(full_cu) - 1):
        s, e = int(full_cu[j]), int(full_cu[j + 1])
        parts.append(s + zigzag_rows(e - s, cp_rank, cp_size))
    return np.concatenate(parts) if parts else np.zeros(0, np.int64)


def zigzag_shard_varlen(x: torch.Tensor, full_cu: Sequence[int], cp_rank: int, cp_size: int):
    """zigzag.py:82-97 -> (local packed rows, local cu_seqlens as a python list)."""
    idx = torch.from_numpy(zigzag_rows_varlen(full_cu, cp_rank, cp_size))
    return x.index_select(0, idx).contiguous(), local_cu_from_full(full_cu, cp_size)


# --------------------------------------------------------------------------------------
# attention and merge (tests/test_algorithm_cpu.py:28-59)
# --------------------------------------------------------------------------------------


def expand_kv(k: torch.Tensor, n_q_heads: int) -> torch.Tensor:
    """GQA/MQA head expansion (reference.py:20-27, test_algorithm_cpu.py:28-33): query head
    j reads kv head j // (H_q / H_kv)."""
    h_kv = k.shape[1]
    if h_kv == n_q_heads:
        return k
    assert n_q_heads % h_kv == 0
    return k.repeat_interleave(n_q_heads // h_kv, dim=1)


def cpu_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, scale: float,
             row_chunk: int = 2048, heads: Optional[Sequence[int]] = None):
    """q [Tq,H,D], k/v [Tk,Hkv,D] -> out [Tq,H,D] fp32, lse [Tq,H] fp32 natural log
    (test_algorithm_cpu.py:36-48).  The causal mask is the one the ring uses (query i sees
    key j <= i) when Tq == Tk, and bottom-right aligned otherwise, as FA4's varlen causal
    mask (the call of fa4_ring/fa4_backend.py:106-120): query i sees key j <= i + Tk - Tq.
    A row that sees no key gets out 0 and lse -inf.  ``heads`` restricts the computation
    to those query heads (the other rows are left NaN)."""
    tq, h, d = q.shape
    tk = k.shape[0]
    off = tk - tq  # bottom-right alignment (0 for the ring's square causal step)
    kq = expand_kv(k.float(), h)
    vq = expand_kv(v.float(), h)
    out = torch.full((tq, h, v.shape[2]), float("nan"), dtype=torch.float32)
    lse = torch.full((tq, h), float("nan"), dtype=torch.float32)
    head_list = list(range(h)) if heads is None else list(heads)
    qf = q.float()
    for hh in head_list:
        kh = kq[:, hh, :]  # [Tk, D]
        vh = vq[:, hh, :]
        for r0 in range(0, tq, row_chunk):
            r1 = min(tq, r0 + row_chunk)
            sc = (qf[r0:r1, hh, :] @ kh.T) * scale  # [rows, Tk]
            if causal:
                qi = torch.arange(r0, r1).unsqueeze(1) + off
                kj = torch.arange(tk).unsqueeze(0)
                sc = sc.masked_fill(kj > qi, float("-inf"))
            l = torch.logsumexp(sc, dim=-1)
            # a row without keys (all -inf) has a NaN softmax: it gets out 0, lse -inf
            p = torch.nan_to_num(torch.softmax(sc, dim=-1), nan=0.0)
            out[r0:r1, hh, :] = p @ vh
            lse[r0:r1, hh] = l
    return out, lse


def cpu_attn_varlen(q, k, v, cu_q: Sequence[int], cu_k: Sequence[int], causal: bool, scale: float):
    """Per-sequence attention over packed sequences (test_algorithm_cpu.py:100-111)."""
    h, dv = q.shape[1], v.shape[2]
    out = torch.zeros(q.shape[0], h, dv)
    lse = torch.full((q.shape[0], h), float("-inf"))
    for j in range(len(cu_q) - 1):
        qs, qe, ks, ke = int(cu_q[j]), int(cu_q[j + 1]), int(cu_k[j]), int(cu_k[j + 1])
        if qe == qs:
            continue
        o, l = cpu_attn(q[qs:qe], k[ks:ke], v[ks:ke], causal=causal, scale=scale)
        out[qs:qe] = o
        lse[qs:qe] = l
    return out, lse


def merge(out_a, lse_a, out_b, lse_b):
    """Online-softmax merge of two (out, lse) states (test_algorithm_cpu.py:51-59).
    A -inf row in b contributes nothing; -inf in both gives NaN, as in the reference."""
    m = torch.maximum(lse_a, lse_b)
    ea = torch.exp(lse_a - m)
    eb = torch.exp(lse_b - m)
    denom = (ea + eb).clamp_min(1e-20)
    out = (out_a * ea.unsqueeze(-1) + out_b * eb.unsqueeze(-1)) / denom.unsqueeze(-1)
    return out, torch.logaddexp(lse_a, lse_b)


def merge_states(v: torch.Tensor, s: torch.Tensor):
    """S-way merge: v [T,S,H,D], s [T,S,H] -> ([T,H,D], [T,H]) (flashinfer merge_states
    semantics as used by merge.py:79-85).  States with s = -inf are skipped; all -inf rows
    give (0, -inf)."""
    v = v.float()
    s = s.float()
    m = s.max(dim=1).values  # [T,H]
    m_safe = torch.where(torch.isinf(m) & (m < 0), torch.zeros_like(m), m)
    w = torch.exp(s - m_safe.unsqueeze(1))  # [T,S,H]; -inf -> 0
    wsum = w.sum(dim=1)
    vw = torch.where(w.unsqueeze(-1) > 0, v * w.unsqueeze(-1), torch.zeros_like(v)).sum(dim=1)
    out = torch.where(wsum.unsqueeze(-1) > 0, vw / wsum.clamp_min(1e-30).unsqueeze(-1),
                      torch.zeros_like(vw))
    lse = torch.where(wsum > 0, m_safe + torch.log(wsum.clamp_min(1e-30)),
                      torch.full_like(wsum, float("-inf")))
    return out, lse


# --------------------------------------------------------------------------------------
# one rank's ring sweep (test_algorithm_cpu.py:62-90, :114-168)
# --------------------------------------------------------------------------------------


def ring_rank(lq: torch.Tensor, k_shards: Sequence[torch.Tensor], v_shards: Sequence[torch.Tensor],
              rank: int, cp_size: int, scale: float, cu: Optional[Sequence[int]] = None,
              merge_mode: str = "incremental", steps: Optional[Sequence[int]] = None,
              src_lag: int = 0):
    """Local output and LSE of one rank's causal zig-zag sweep, in fp32.

    Step 0 is local causal attention; step s <= rank attends all local Q to the front
    (early) half of source (rank - s) % cp_size; step s > rank attends the back (late) half
    of Q to all of that source's KV and merges into the back rows only.  ``cu`` is the
    local cu_seqlens (packed varlen), None for one sequence.  ``merge_mode`` "batched"
    merges all partials at the end with merge_states instead of step by step.
    ``src_lag`` plants a one-hop source lag (for the oracle's own negative test only)."""
    t = lq.shape[0]
    if cu is None:
        cu = [0, t]
    cu = [int(c) for c in cu]
    half_cu = [c // 2 for c in cu]
    front = torch.from_numpy(get_half_index(cu, front=True))
    back = torch.from_numpy(get_half_index(cu, front=False))
    partials = []
    steps = range(cp_size) if steps is None else steps
    for step in steps:
        src = (rank - step + src_lag) % cp_size if step > 0 else rank
        k, v = k_shards[src].float(), v_shards[src].float()
        if step == 0:
            o, l = cpu_attn_varlen(lq, k, v, cu, cu, causal=True, scale=scale)
        elif step <= rank:
            o, l = cpu_attn_varlen(lq, k[front], v[front], cu, half_cu, causal=False, scale=scale)
        else:
            ob, lb = cpu_attn_varlen(lq[back], k, v, half_cu, cu, causal=False, scale=scale)
            o = torch.zeros(t, lq.shape[1], v.shape[2])
            l = torch.full((t, lq.shape[1]), float("-inf"))
            o[back] = ob
            l[back] = lb
        partials.append((o, l))
    if merge_mode == "batched":
        if len(partials) == 1:
            return partials[0]
        return merge_states(torch.stack([p[0] for p in partials], 1),
                            torch.stack([p[1] for p in partials], 1))
    acc_o, acc_l = partials[0]
    for o, l in partials[1:]:
        acc_o, acc_l = merge(acc_o, acc_l, o, l)
    return acc_o, acc_l


def ring_rank_backward(lq: torch.Tensor, k_shards: Sequence[torch.Tensor], v_shards: Sequence[torch.Tensor],
                       dout: torch.Tensor, out: torch.Tensor, lse: torch.Tensor, rank: int, cp_size: int,
                       scale: float, cu: Optional[Sequence[int]] = None, drop_delta: bool = False):
    """One rank's gradients in fp32, given its ring output ``out`` and natural-log ``lse``
    (from ring_rank) and the gradient ``dout`` of ``out``: (dq [T,H,D], dk per source rank,
    dv per source rank), the dk / dv entries being this rank's contributions to that
    source's K / V gradient.  The reference has no backward; this restates the gradient of
    its forward schedule (ring_rank above): every (row, key) pair of a step contributes with
    P = exp(scale q.k - lse) against the final lse, dS = P (dO.v - delta) with
    delta = rowsum(dO * out), dq += scale dS k, dk += scale dS^T q, dv += P^T dO.
    ``drop_delta`` plants a mistake (delta taken as 0) for the oracle's own negative test."""
    t, h, d = lq.shape
    cu = [0, t] if cu is None else [int(c) for c in cu]
    hkv = k_shards[0].shape[1]
    g = h // hkv
    qf, dof = lq.float(), dout.float()
    delta = torch.zeros(t, h) if drop_delta else (dof * out.float()).sum(-1)
    dq = torch.zeros(t, h, d)
    dks = [torch.zeros(t, hkv, d) for _ in range(cp_size)]
    dvs = [torch.zeros(t, hkv, v_shards[0].shape[2]) for _ in range(cp_size)]
    for step in range(cp_size):
        src = (rank - step) % cp_size
        k, v = k_shards[src].float(), v_shards[src].float()
        for j in range(len(cu) - 1):
            s0, e0 = cu[j], cu[j + 1]
            n = e0 - s0
            if n == 0:
                continue
            half = n // 2
            if step == 0:
                rows, keys = torch.arange(s0, e0), torch.arange(s0, e0)
            elif step <= rank:
                rows, keys = torch.arange(s0, e0), torch.arange(s0, s0 + half)
            else:
                rows, keys = torch.arange(s0 + half, e0), torch.arange(s0, e0)
            if rows.numel() == 0 or keys.numel() == 0:
                continue
            for hh in range(h):
                kvh = hh // g
                qh, kh, vh, dh = qf[rows, hh], k[keys, kvh], v[keys, kvh], dof[rows, hh]
                sc = (qh @ kh.T) * scale
                if step == 0:
                    sc = sc.masked_fill(keys.unsqueeze(0) > rows.unsqueeze(1), float("-inf"))
                p = torch.exp(sc - lse[rows, hh].unsqueeze(1))
                ds = p * (dh @ vh.T - delta[rows, hh].unsqueeze(1))
                dq[rows, hh] += scale * (ds @ kh)
                dks[src][keys, kvh] += scale * (ds.T @ qh)
                dvs[src][keys, kvh] += p.T @ dh
    return dq, dks, dvs


def dense_causal(q, k, v, scale):
    """test_algorithm_cpu.py:93-95."""
    return cpu_attn(q, k, v, causal=True, scale=scale)[0]


def simulate_ring(q, k, v, cp_size, scale, src_lag: int = 0):
    """All ranks in sequence, outputs stitched back to [N,H,D] (test_algorithm_cpu.py:62-90)."""
    n = q.shape[0]
    ks = [zigzag_shard(k, r, cp_size) for r in range(cp_size)]
    vs = [zigzag_shard(v, r, cp_size) for r in range(cp_size)]
    outs = []
    for rank in range(cp_size):
        o, _ = ring_rank(zigzag_shard(q, rank, cp_size), ks, vs, rank, cp_size, scale,
                         src_lag=src_lag)
        outs.append(o)
    return zigzag_unshard(outs, cp_size)


def simulate_ring_varlen(seqs, cp_size, scale, merge_mode="incremental"):
    """Packed varlen version (test_algorithm_cpu.py:114-168); returns per-sequence outputs."""
    lens = [s[0].shape[0] for s in seqs]
    full_cu = [0]
    for n in lens:
        full_cu.append(full_cu[-1] + n)
    Q = torch.cat([s[0] for s in seqs])
    K = torch.cat([s[1] for s in seqs])
    V = torch.cat([s[2] for s in seqs])
    ks, vs, outs = [], [], []
    for r in range(cp_size):
        lk, _ = zigzag_shard_varlen(K, full_cu, r, cp_size)
        lv, _ = zigzag_shard_varlen(V, full_cu, r, cp_size)
        ks.append(lk)
        vs.append(lv)
    local_cu = None
    for rank in range(cp_size):
        lq, local_cu = zigzag_shard_varlen(Q, full_cu, rank, cp_size)
        o, _ = ring_rank(lq, ks, vs, rank, cp_size, scale, cu=local_cu, merge_mode=merge_mode)
        outs.append(o)
    recon = []
    for j in range(len(lens)):
        shards = [outs[r][local_cu[j]:local_cu[j + 1]] for r in range(cp_size)]
        recon.append(zigzag_unshard(shards, cp_size))
    return recon


def dense_causal_rows(q_full, k_full, v_full, rows: Sequence[int], heads: Sequence[int],
                      scale: float, seq_start: int = 0):
    """Exact fp32 causal attention for selected (row, head) pairs of one full sequence that
    starts at row seq_start: row i sees keys seq_start..i.  Returns (out [n, D], lse [n])."""
    outs, lses = [], []
    h_q = q_full.shape[1]
    g = h_q // k_full.shape[1]
    for r, hh in zip(rows, heads):
        qv = q_full[r, hh].float()
        kk = k_full[seq_start:r + 1, hh // g].float()
        vv = v_full[seq_start:r + 1, hh // g].float()
        sc = (kk @ qv) * scale
        lse = torch.logsumexp(sc, 0)
        outs.append(torch.softmax(sc, 0) @ vv)
        lses.append(lse)
    return torch.stack(outs), torch.stack(lses)


def dense_causal_rows_all_heads(q_rows: torch.Tensor, positions: Sequence[int], seq_starts: Sequence[int],
                                k_full: torch.Tensor, v_full: torch.Tensor, scale: float,
                                key_block: int = 8192):
    """Exact fp32 causal attention of many query rows, every head: query row i (q_rows[i],
    [H_q, D]) sits at packed position positions[i] of a sequence that starts at
    seq_starts[i], so it sees keys seq_starts[i] .. positions[i] of k_full / v_full
    [N, H_kv, D].  Returns (out [R, H_q, Dv], lse [R, H_q]).

    The same arithmetic as dense_causal_rows (one row, one head at a time), batched: the
    query heads of a kv head are stacked, and keys go in blocks of ``key_block`` folded with
    the online-softmax merge (merge(), the identity this oracle's merge tests pin), each
    block only for the rows that see part of it."""
    r_count, h_q, d = q_rows.shape
    h_kv = k_full.shape[1]
    g = h_q // h_kv
    pos = torch.as_tensor(list(positions), dtype=torch.int64)
    start = torch.as_tensor(list(seq_starts), dtype=torch.int64)
    out = torch.zeros(r_count, h_q, v_full.shape[2])
    lse = torch.full((r_count, h_q), float("-inf"))
    if r_count == 0:
        return out, lse
    qf = q_rows.float()
    k0 = int(start.min())
    k1 = int(pos.max()) + 1
    for b0 in range(k0, k1, key_block):
        b1 = min(k1, b0 + key_block)
        rows = ((start < b1) & (pos >= b0)).nonzero().flatten()
        if rows.numel() == 0:
            continue
        kb = k_full[b0:b1].float()  # [B, H_kv, D]
        vb = v_full[b0:b1].float()
        kpos = torch.arange(b0, b1)
        visible = (kpos.unsqueeze(0) >= start[rows].unsqueeze(1)) & (kpos.unsqueeze(0) <= pos[rows].unsqueeze(1))
        for gi in range(h_kv):
            qh = qf[rows, gi * g:(gi + 1) * g, :]  # [r, g, D]
            sc = torch.einsum("rgd,kd->rgk", qh, kb[:, gi]) * scale
            sc = sc.masked_fill(~visible.unsqueeze(1), float("-inf"))
            bl = torch.logsumexp(sc, dim=-1)  # [r, g]
            p = torch.exp(sc - torch.where(torch.isinf(bl), torch.zeros_like(bl), bl).unsqueeze(-1))
            bo = torch.einsum("rgk,kd->rgd", p, vb[:, gi])
            mo, ml = merge(out[rows, gi * g:(gi + 1) * g], lse[rows, gi * g:(gi + 1) * g], bo, bl)
            # a row with no visible key in this block keeps its state (merge would NaN it
            # only if both were -inf, which happens before the first visible block)
            keep = torch.isinf(bl) & (bl < 0)
            mo = torch.where(keep.unsqueeze(-1), out[rows, gi * g:(gi + 1) * g], mo)
            ml = torch.where(keep, lse[rows, gi * g:(gi + 1) * g], ml)
            out[rows, gi * g:(gi + 1) * g] = mo
            lse[rows, gi * g:(gi + 1) * g] = ml
    return out, lse


# --------------------------------------------------------------------------------------
# OCP e4m3fn
# --------------------------------------------------------------------------------------


def e4m3_decode(code: int) -> float:
    """Value of an OCP float8_e4m3fn byte: 1 sign, 4 exponent (bias 7), 3 mantissa bits;
    exponent 0 is subnormal (m/8 * 2^-6); S.1111.111 is NaN; no infinities."""
    sign = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return sign * (m / 8.0) * 2.0 ** -6
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def quantize_e4m3(x: torch.Tensor, scale: float) -> torch.Tensor:
    """x8 = clamp(x / scale, +-448) cast to float8_e4m3fn (round to nearest even)."""
    return (x.float() / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)


def dequantize_e4m3(x8: torch.Tensor, scale: float) -> torch.Tensor:
    return x8.float() * scale


def amax_scale(x: torch.Tensor) -> float:
    """Per-tensor scale amax / 448 (1.0 for an all-zero tensor)."""
    a = float(x.float().abs().max()) if x.numel() else 0.0
    return a / E4M3_MAX if a > 0 else 1.0


# --------------------------------------------------------------------------------------
# workloads
# --------------------------------------------------------------------------------------

# the five benchmark configurations (causal zig-zag ring, one rank's share)
CONFIGS = {
    "c1": dict(n=2048, cp=4, hq=8, hkv=2, d=128, dtype="fp32"),
    "c2": dict(n=131072, cp=8, hq=32, hkv=8, d=128, dtype="bf16"),
    "c3": dict(n=131072, cp=8, hq=32, hkv=8, d=128, dtype="e4m3"),
    "c4": dict(n=None, cp=4, hq=32, hkv=8, d=128, dtype="bf16"),
    "c5": dict(n=262144, cp=8, hq=16, hkv=2, d=256, dtype="e4m3"),
}


def varlen_lengths(seed: int = 0, count: int = 8, lo: int = 128, hi: int = 2049,
                   total_max: int = 65536) -> List[int]:
    """Packed-varlen sequence lengths: 8 * randint(lo, hi) per sequence from a seeded CPU
    generator, redrawn until the total is <= total_max (multiples of 8 in [1024, 16384])."""
    g = torch.Generator().manual_seed(seed)
    while True:
        lens = (8 * torch.randint(lo, hi, (count,), generator=g)).tolist()
        if sum(lens) <= total_max:
            return [int(x) for x in lens]


def random_qkv(n: int, hq: int, hkv: int, d: int, seed: int = 0):
    """Full-sequence q, k, v ~ N(0,1) in fp32, drawn in that order from one seeded CPU
    generator."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n, hq, d, generator=g)
    k = torch.randn(n, hkv, d, generator=g)
    v = torch.randn(n, hkv, d, generator=g)
    return q, k, v
