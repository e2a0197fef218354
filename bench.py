"""Benchmark of one rank's causal zig-zag ring sweep on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--rank 3] [--no-cpu-baseline]

A step is one rank's full ring sweep over inputs already resident in HBM, at the bf16
benchmark configuration: N = 131072 tokens, cp_size = 8 (local Q, K, V of 16384 tokens
each), H_q = 32, H_kv = 8, D = 128, causal, rank 3 (all source ranks' KV shards in HBM).
The default sweep transposes every source shard's V once (fa4cp_transpose_v) and runs one
fused kernel over all cp_size sources (fa4cp_ring_sweep_fwd); both are inside the timed
step.  The reference's per-step form (one attention launch plus one LSE merge per step) is
timed beside it as `per_step_bf16`.

Prints one JSON line.  `value` is causal-adjusted attention TFLOP/s of the sweep:
F = sum over steps of 4 * Tq * Tk * D * H_q (halved for the causal step) = 17.592 TFLOP per
sweep, divided by the measured sweep time.  Also reported: the same sweep in OCP e4m3
with per-source-rank descales, the incremental and batched merge kernels and the zig-zag
gather in GB/s against the 8 TB/s HBM peak, and the CPU oracle timed on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "fa4-cp_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "ring-sweep attn TFLOP/s + % MFMA peak (bf16/fp8); merge GB/s, 1×MI355X"
PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 dense bf16 FLOP/clk/CU
PEAK_FP8_TFLOPS = 5033.2
PEAK_HBM_GBS = 8000.0

N, CP, HQ, HKV, D = 131072, 8, 32, 8, 128

# HBM bytes per attention launch of the rank-3 sweep (mean over its 8 launches), from two
# rocprofv3 counter passes over this script: FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000, the
# factors being what those counters read for the zig-zag gather (a plain copy of known size).
# The summary with both commands is under profiles/.
ATTN_TRAFFIC_BYTES_RANK3 = 467355 * 1024
# The same for the fused sweep kernel (one launch per sweep).
SWEEP_TRAFFIC_BYTES_RANK3 = 2436944 * 1024
# ... for the packed-sequence sweep (cp_size 4, rank 3) and the e4m3 head-dim-256 sweep
# (N = 262144, rank 3), and for merge_states in their batched per-step forms (same factors,
# counter passes over `bench.py --workload c4` / `--workload c5`).
C4_SWEEP_TRAFFIC_BYTES = (2 * 162099 + 102521) * 1024
C5_SWEEP_TRAFFIC_BYTES = (2 * 2595454 + 266600) * 1024
C4_MERGE_STATES_TRAFFIC_BYTES = (2 * 204965 + 100913) * 1024
# ... for the e4m3 sweep at the headline shape (rank 3), counter passes over `--workload c3`
C3_SWEEP_TRAFFIC_BYTES_RANK3 = (2 * 567996 + 135355) * 1024
C5_MERGE_STATES_TRAFFIC_BYTES = (2 * 802850 + 264192) * 1024


def sweep_flops(t_local: int, cp: int, hq: int, d: int) -> float:
    """Causal-adjusted FLOPs of one rank's sweep: every step is 4 * (T*T/2) * D * H_q
    (causal T x T, front-half T x T/2, back-half T/2 x T), i.e. cp * 8 * h^2 * D * H_q."""
    h = t_local // 2
    return cp * 8.0 * h * h * d * hq


class KernelClock:
    """Records torch.cuda events around every attention / merge launch of the sweep (the
    launches go to torch's current stream, where the events are recorded too)."""

    def __init__(self):
        self.events = {}

    def wrap(self, name, fn):
        import torch

        def inner(*a, **k):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            r = fn(*a, **k)
            e.record()
            self.events.setdefault(name, []).append((s, e))
            return r

        return inner

    def mean_ms(self, name):
        ev = self.events.get(name, [])
        return sum(s.elapsed_time(e) for s, e in ev) / len(ev) if ev else float("nan")

    def count(self, name):
        return len(self.events.get(name, []))


def make_bf16_inputs(rank: int, seed: int = 0):
    import torch

    from fa4_ring import LocalKVRing, zigzag_shard

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(N, HQ, D, device=dev, generator=g, dtype=torch.bfloat16)
    k = torch.randn(N, HKV, D, device=dev, generator=g, dtype=torch.bfloat16)
    v = torch.randn(N, HKV, D, device=dev, generator=g, dtype=torch.bfloat16)
    ring = LocalKVRing.from_full(k, v, CP)
    lq = zigzag_shard(q, rank, CP)
    return q, lq, ring


def make_fp8_inputs(rank: int, seed: int = 1):
    """q scale = amax(local q) / 448; k / v scales per source rank = amax(shard) / 448,
    quantised by the library's FP8 producer (fa4cp_quantize_e4m3)."""
    import torch

    from fa4_ring import LocalKVRing, quantize_ring, zigzag_shard

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(N, HQ, D, device=dev, generator=g)
    k = torch.randn(N, HKV, D, device=dev, generator=g)
    v = torch.randn(N, HKV, D, device=dev, generator=g)
    lq = zigzag_shard(q, rank, CP)
    del q
    ks = [zigzag_shard(k, r, CP) for r in range(CP)]
    vs = [zigzag_shard(v, r, CP) for r in range(CP)]
    q8, k8, v8, desc = quantize_ring(lq, ks, vs)
    return q8, LocalKVRing(k8, v8), desc


def timed_sweeps(fn, steps: int, warmup: int, clock: KernelClock = None):
    import torch

    from fa4_ring import ring_attention as RA

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    saved = (RA.fa4_attn, RA.merge_state_in_place, RA.merge_states, RA.transpose_v, RA.launch_sweep,
             RA.transpose_v_many)
    if clock is not None:
        RA.fa4_attn = clock.wrap("attn", saved[0])
        RA.merge_state_in_place = clock.wrap("merge_inplace", saved[1])
        RA.merge_states = clock.wrap("merge_states", saved[2])
        RA.transpose_v = clock.wrap("transpose_v", saved[3])
        RA.launch_sweep = clock.wrap("sweep_kernel", saved[4])
        RA.transpose_v_many = clock.wrap("transpose_v_many", saved[5])
    try:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
    finally:
        (RA.fa4_attn, RA.merge_state_in_place, RA.merge_states, RA.transpose_v, RA.launch_sweep,
         RA.transpose_v_many) = saved
    return dt


def merge_bytes_inplace(rows: int, h: int, d: int, bv: int) -> float:
    """Read v, v_other, s, s_other; write v, s."""
    return rows * h * (3 * d * bv + 3 * 4)


def merge_bytes_batched(rows: int, s: int, h: int, d: int, bv: int) -> float:
    return rows * h * (s * (d * bv + 4) + d * bv + 4)


def merge_counter_rate(traffic, ms: float) -> dict:
    """merge_states GB/s and fraction of HBM peak on counter bytes (None off the profiled rank):
    the algorithmic figure counts -inf states the kernel does not read."""
    if traffic is None:
        return {"merge_states_counter_GBs": None, "merge_states_counter_frac": None}
    gbs = traffic / (ms * 1e-3) / 1e9
    return {"merge_states_counter_GBs": round(gbs, 1), "merge_states_counter_frac": round(gbs / PEAK_HBM_GBS, 4)}


def cpu_baseline(rank: int, rows: int) -> dict:
    """The CPU oracle (fp32 torch on the host cores) on a bounded sample of the same
    workload: step 1 of the rank's sweep (all local Q x front half of source rank-1's KV)
    restricted to the first `rows` local query rows, all heads."""
    import torch

    from oracle import ring_oracle as O

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    t = N // CP
    q = torch.randn(rows, HQ, D, generator=g).to(torch.bfloat16).float()
    k = torch.randn(t // 2, HKV, D, generator=g).to(torch.bfloat16).float()
    v = torch.randn(t // 2, HKV, D, generator=g).to(torch.bfloat16).float()
    O.cpu_attn(q[:64], k, v, False, 1 / math.sqrt(D))  # warm the BLAS
    t0 = time.perf_counter()
    O.cpu_attn(q, k, v, False, 1 / math.sqrt(D))
    dt = time.perf_counter() - t0
    flops = 4.0 * rows * (t // 2) * D * HQ
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": (f"oracle cpu_attn fp32, ring step {1} of rank {rank} (all Q x front half of "
                       f"source {rank - 1}'s KV) on the first {rows} of {t} local query rows, "
                       f"{HQ} heads, Tk={t // 2}, D={D}: {flops / 1e12:.3f} TFLOP in {dt:.2f} s on {cpu}"),
            "full_sweep_s_extrapolated": round(sweep_flops(t, CP, HQ, D) / (flops / dt), 1)}


C4_LENGTHS = [4856, 9720, 8592, 4864, 1832, 15456, 2784, 1576]  # 8 * randint(128, 2049), seed 0


def _cpu_threads() -> int:
    import torch

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
    torch.set_num_threads(threads)
    return threads


def _cpu_model() -> str:
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


def _event_ms(fn, n=10):
    """Mean HIP-event time of `fn` on torch's current stream (where the library launches)."""
    import torch

    for _ in range(3):
        fn()
    evs = []
    for _ in range(n):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        evs.append((s, e))
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in evs) / n


def c4_block(rank: int, steps: int, warmup: int, with_cpu: bool) -> dict:
    """Packed sequences: the 8 lengths above (49680 tokens), cp_size = 4, H_q = 32, H_kv = 8,
    D = 128, bf16, one rank's sweep in the fused form and in both per-step merge modes; the
    zig-zag shard of the packed q; and the oracle's whole fp32 sweep of the same rank on the
    host cores (the complete job, not a sample)."""
    import torch

    from fa4_ring import LocalKVRing, RingConfig, ring_flash_attn
    from fa4_ring.zigzag import _shard, zigzag_shard_varlen

    cp, hq, hkv, d = 4, HQ, HKV, D
    full_cu = [0]
    for n in C4_LENGTHS:
        full_cu.append(full_cu[-1] + n)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn(full_cu[-1], hq, d, device=dev, generator=g, dtype=torch.bfloat16)
    k = torch.randn(full_cu[-1], hkv, d, device=dev, generator=g, dtype=torch.bfloat16)
    v = torch.randn(full_cu[-1], hkv, d, device=dev, generator=g, dtype=torch.bfloat16)
    ring = LocalKVRing.from_full(k, v, cp, full_cu)
    lq, local_cu = zigzag_shard_varlen(q, full_cu, rank, cp)
    max_local = int((local_cu[1:] - local_cu[:-1]).max())
    flops = sum(cp * 8.0 * (n // (2 * cp)) ** 2 * d * hq for n in C4_LENGTHS)

    def run(fused, mode="incremental"):
        return ring_flash_attn(lq, ring.k[rank], ring.v[rank], RingConfig(cp_size=cp, cp_rank=rank, merge_mode=mode),
                               group=ring, cu_seqlens=local_cu, max_seqlen=max_local, fused=fused)

    clock = KernelClock()
    sec = timed_sweeps(lambda: run(True), steps, warmup, clock)
    sw_ms = clock.mean_ms("sweep_kernel")
    seci = timed_sweeps(lambda: run(False, "incremental"), steps, warmup)
    secb = timed_sweeps(lambda: run(False, "batched"), steps, warmup)
    clockb = KernelClock()
    timed_sweeps(lambda: run(False, "batched"), max(3, steps // 2), 1, clockb)
    ms_ms = clockb.mean_ms("merge_states")
    t_local = lq.shape[0]
    bb = merge_bytes_batched(t_local, cp, hq, d, 2)
    # zig-zag shard of the packed full q (per-sequence chunks r and 2cp-1-r), device cu
    cu_dev = torch.tensor(full_cu, dtype=torch.int32, device=dev)
    zms = _event_ms(lambda: _shard(q, rank, cp, cu_dev, len(C4_LENGTHS)))
    zbytes = 2.0 * t_local * hq * d * 2
    kt = flops / (sw_ms * 1e-3) / 1e12
    out = {
        "workload": f"bf16 causal zig-zag ring sweep over packed sequences {C4_LENGTHS} ({full_cu[-1]} tokens), "
                    f"cp_size={cp}, rank {rank}, H_q={hq}, H_kv={hkv}, D={d}",
        "flop_per_sweep": flops,
        "fused": {"ms_per_step": round(sec * 1e3, 3), "TFLOP/s": round(flops / sec / 1e12, 2),
                  "frac_of_peak": round(flops / sec / 1e12 / PEAK_BF16_TFLOPS, 4)},
        "roofline": {"bound": "mfma", "kernel": "attn_fwd_16bit_sweep<bf16,128,4> (packed)", "achieved": round(kt, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(kt / PEAK_BF16_TFLOPS, 4),
                     "traffic": C4_SWEEP_TRAFFIC_BYTES if rank == 3 else None,
                     "algorithmic_per_launch": f"{flops / 1e12:.4f} TFLOP (the whole sweep)",
                     "avg_launch_ms": round(sw_ms, 4), "launches": clock.count("sweep_kernel")},
        "per_step_incremental": {"ms_per_step": round(seci * 1e3, 3), "TFLOP/s": round(flops / seci / 1e12, 2)},
        "per_step_batched": {"ms_per_step": round(secb * 1e3, 3), "TFLOP/s": round(flops / secb / 1e12, 2),
                             "merge_states_ms": round(ms_ms, 4), "merge_states_bytes": round(bb),
                             "merge_states_GBs": round(bb / (ms_ms * 1e-3) / 1e9, 1),
                             "merge_states_frac": round(bb / (ms_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                             "merge_states_traffic": C4_MERGE_STATES_TRAFFIC_BYTES if rank == 3 else None,
                             **merge_counter_rate(C4_MERGE_STATES_TRAFFIC_BYTES if rank == 3 else None, ms_ms)},
        "zigzag_varlen": {"kernel": "shard_kernel<u32x4> (packed sequences, full q)", "avg_launch_ms": round(zms, 4),
                          "bytes": round(zbytes), "achieved_GBs": round(zbytes / (zms * 1e-3) / 1e9, 1),
                          "frac": round(zbytes / (zms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
    }
    if with_cpu:
        from oracle import ring_oracle as O

        threads = _cpu_threads()
        qc, kc, vc = q.float().cpu(), k.float().cpu(), v.float().cpu()
        ks = [O.zigzag_shard_varlen(kc, full_cu, r, cp)[0] for r in range(cp)]
        vs = [O.zigzag_shard_varlen(vc, full_cu, r, cp)[0] for r in range(cp)]
        oq, ocu = O.zigzag_shard_varlen(qc, full_cu, rank, cp)
        t0 = time.perf_counter()
        O.ring_rank(oq, ks, vs, rank, cp, 1 / math.sqrt(d), cu=ocu)
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
                               "kind": "port",
                               "sample": f"the whole job: the oracle's fp32 sweep of rank {rank} over the 8 packed "
                                         f"sequences ({flops / 1e12:.4f} TFLOP) in {dt:.2f} s on {_cpu_model()}"}
    return out


def c5_block(rank: int, steps: int, warmup: int, with_cpu: bool, cpu_rows: int = 4096) -> dict:
    """The e4m3 head-dim-256 sweep: N = 262144, cp_size = 8 (local 32768 tokens), H_q = 16,
    H_kv = 2, D = 256, q scale per local shard and k / v scales per source shard (the FP8
    producer), bf16 out.  The fused sweep, the per-step form with the batched merge (8
    stashed partials, one merge_states) and with the incremental merge; the oracle on the
    host cores on a bounded sample (step 1 for the first `cpu_rows` local query rows)."""
    import torch

    from fa4_ring import LocalKVRing, RingConfig, quantize_ring, ring_flash_attn, zigzag_shard

    n, cp, hq, hkv, d = 262144, 8, 16, 2, 256
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(2)
    q = torch.randn(n, hq, d, device=dev, generator=g, dtype=torch.bfloat16)
    k = torch.randn(n, hkv, d, device=dev, generator=g, dtype=torch.bfloat16)
    v = torch.randn(n, hkv, d, device=dev, generator=g, dtype=torch.bfloat16)
    lq = zigzag_shard(q, rank, cp)
    del q
    ks = [zigzag_shard(k, r, cp) for r in range(cp)]
    vs = [zigzag_shard(v, r, cp) for r in range(cp)]
    del k, v
    q8, k8, v8, desc = quantize_ring(lq, ks, vs)
    ring = LocalKVRing(k8, v8)
    t_local = n // cp
    flops = sweep_flops(t_local, cp, hq, d)

    def run(fused, mode="incremental"):
        return ring_flash_attn(q8, ring.k[rank], ring.v[rank], RingConfig(cp_size=cp, cp_rank=rank, merge_mode=mode),
                               group=ring, descales=desc, fused=fused)

    clock = KernelClock()
    sec = timed_sweeps(lambda: run(True), steps, warmup, clock)
    sw_ms = clock.mean_ms("sweep_kernel")
    psteps = max(3, steps // 2)
    secb = timed_sweeps(lambda: run(False, "batched"), psteps, 2)
    seci = timed_sweeps(lambda: run(False, "incremental"), psteps, 2)
    clockb = KernelClock()
    timed_sweeps(lambda: run(False, "batched"), psteps, 1, clockb)
    ms_ms = clockb.mean_ms("merge_states")
    a_ms = clockb.mean_ms("attn")
    bb = merge_bytes_batched(t_local, cp, hq, d, 2)
    kt = flops / (sw_ms * 1e-3) / 1e12
    out = {
        "workload": f"e4m3 causal zig-zag ring sweep, one rank's share of cp_size={cp} over N={n} (local {t_local} "
                    f"tokens), H_q={hq}, H_kv={hkv}, D={d}, rank {rank}, per-source-rank k/v descales, bf16 out",
        "flop_per_sweep": flops,
        "fused": {"ms_per_step": round(sec * 1e3, 3), "TFLOP/s": round(flops / sec / 1e12, 2),
                  "frac_of_fp8_peak": round(flops / sec / 1e12 / PEAK_FP8_TFLOPS, 4)},
        "roofline": {"bound": "mfma", "kernel": "attn_fwd_e4m3_sweep<256,4>", "achieved": round(kt, 2),
                     "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s", "frac": round(kt / PEAK_FP8_TFLOPS, 4),
                     "traffic": C5_SWEEP_TRAFFIC_BYTES if rank == 3 else None,
                     "algorithmic_per_launch": f"{flops / 1e12:.4f} TFLOP (the whole sweep)",
                     "avg_launch_ms": round(sw_ms, 4), "launches": clock.count("sweep_kernel")},
        "per_step_batched": {"ms_per_step": round(secb * 1e3, 3), "TFLOP/s": round(flops / secb / 1e12, 2),
                             "attn_avg_launch_ms": round(a_ms, 4),
                             "merge_states_ms": round(ms_ms, 4), "merge_states_bytes": round(bb),
                             "merge_states_GBs": round(bb / (ms_ms * 1e-3) / 1e9, 1),
                             "merge_states_frac": round(bb / (ms_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                             "merge_states_traffic": C5_MERGE_STATES_TRAFFIC_BYTES if rank == 3 else None,
                             **merge_counter_rate(C5_MERGE_STATES_TRAFFIC_BYTES if rank == 3 else None, ms_ms)},
        "per_step_incremental": {"ms_per_step": round(seci * 1e3, 3), "TFLOP/s": round(flops / seci / 1e12, 2)},
    }
    if with_cpu:
        from oracle import ring_oracle as O

        threads = _cpu_threads()
        half = t_local // 2
        src = (rank - 1) % cp
        qf = (q8[:cpu_rows].float() * desc.q.float()).cpu()
        kf = (ring.k[src][:half].float() * desc.k[src].float()).cpu()
        vf = (ring.v[src][:half].float() * desc.v[src].float()).cpu()
        O.cpu_attn(qf[:64], kf, vf, False, 1 / math.sqrt(d))  # warm the BLAS
        t0 = time.perf_counter()
        O.cpu_attn(qf, kf, vf, False, 1 / math.sqrt(d))
        dt = time.perf_counter() - t0
        sflops = 4.0 * cpu_rows * half * d * hq
        out["cpu_baseline"] = {"value": round(sflops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
                               "kind": "port",
                               "sample": f"oracle cpu_attn fp32 on the dequantised e4m3 inputs, ring step 1 of rank "
                                         f"{rank} (all Q x front half of source {src}'s KV) for the first {cpu_rows} "
                                         f"of {t_local} local query rows, {hq} heads, Tk={half}, D={d}: "
                                         f"{sflops / 1e12:.3f} TFLOP in {dt:.2f} s on {_cpu_model()}",
                               "full_sweep_s_extrapolated": round(flops / (sflops / dt), 1)}
    del ring, q8, k8, v8
    return out


def _single_line(args, block: dict, dtype: str, peak: float, config: dict) -> dict:
    """A stand-alone JSON line for one of the extra workloads (``--workload``)."""
    sec = block["fused"]["ms_per_step"] * 1e-3
    value = block["flop_per_sweep"] / sec / 1e12
    line = {"metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": block["fused"]["ms_per_step"], "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype,
            "data": "synthetic (q/k/v ~ N(0,1), seeded on the GPU)", "config": config,
            "frac_of_peak": round(value / peak, 4)}
    line.update({k: v for k, v in block.items() if k not in ("fused", "flop_per_sweep")})
    line.setdefault("cpu_baseline", None)
    return line


def c3_block(rank: int, steps: int, warmup: int, paged: bool = False) -> dict:
    """The e4m3 sweep at the bf16 shape (N = 131072, cp_size = 8, H_q = 32, H_kv = 8, D = 128):
    OCP e4m3 q/k/v, q scale amax/448 of the local shard, k / v scales per source shard
    (quantised by the library's producer), bf16 out; fused (the sweep kernel clocked) and per
    step (attention per launch, clocked in a second pass).  `paged`: also the fused sweep
    over paged caches of the same K/V (256-row pages), K read through the page tables."""
    from fa4_ring import RingConfig, ring_flash_attn

    flops = sweep_flops(N // CP, CP, HQ, D)
    per_launch = flops / CP
    q8, ring8, desc = make_fp8_inputs(rank)
    cfg8 = RingConfig(cp_size=CP, cp_rank=rank)
    clock8 = KernelClock()
    sec8 = timed_sweeps(lambda: ring_flash_attn(q8, ring8.k[rank], ring8.v[rank], cfg8, group=ring8,
                                                descales=desc), steps, warmup, clock8)
    s8 = clock8.mean_ms("sweep_kernel")
    per_step8 = lambda: ring_flash_attn(q8, ring8.k[rank], ring8.v[rank], cfg8, group=ring8,  # noqa: E731
                                        descales=desc, fused=False)
    sec8p = timed_sweeps(per_step8, max(3, steps // 2), 2)  # unclocked wall time
    clock8p = KernelClock()
    timed_sweeps(per_step8, max(3, steps // 2), 1, clock8p)
    a8 = clock8p.mean_ms("attn")
    extra = {}
    if paged:
        import torch

        from fa4_ring import PagedKVRing
        pring = PagedKVRing.from_shards(ring8.k, ring8.v, 256, spare_pages=8,
                                        generator=torch.Generator().manual_seed(rank))
        clockpg = KernelClock()
        secpg = timed_sweeps(lambda: ring_flash_attn(q8, None, None, cfg8, group=pring, descales=desc),
                             max(3, steps // 2), 2, clockpg)
        spg = clockpg.mean_ms("sweep_kernel")
        extra["paged"] = {"workload": "the fused sweep over paged caches (256-row pages, random order), K read in "
                                      "place through the page tables",
                          "ms_per_step": round(secpg * 1e3, 3), "TFLOP/s": round(flops / secpg / 1e12, 2),
                          "sweep_kernel": {"kernel": "attn_fwd_e4m3_sweep<128,4,paged K>",
                                           "avg_launch_ms": round(spg, 4),
                                           "TFLOP/s": round(flops / (spg * 1e-3) / 1e12, 2),
                                           "frac": round(flops / (spg * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4)}}
        del pring
    return {**extra, "workload": "same shape, OCP e4m3 q/k/v, per-source-rank k/v descales, bf16 out",
            "ms_per_step": round(sec8 * 1e3, 3), "TFLOP/s": round(flops / sec8 / 1e12, 2),
            "frac_of_fp8_peak": round(flops / sec8 / 1e12 / PEAK_FP8_TFLOPS, 4),
            "sweep_kernel": {"kernel": "attn_fwd_e4m3_sweep<128,4>", "avg_launch_ms": round(s8, 4),
                             "TFLOP/s": round(flops / (s8 * 1e-3) / 1e12, 2),
                             "frac": round(flops / (s8 * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4)},
            "per_step": {"ms_per_step": round(sec8p * 1e3, 3),
                         "TFLOP/s": round(flops / sec8p / 1e12, 2),
                         "attn_kernel": "attn_fwd_e4m3_vt<128,4>",
                         "attn_avg_launch_ms": round(a8, 4),
                         "attn_TFLOP/s": round(per_launch / (a8 * 1e-3) / 1e12, 2),
                         "attn_frac": round(per_launch / (a8 * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4)}}


def bench_c3(args) -> int:
    import torch

    block = c3_block(args.rank, args.steps, args.warmup)
    torch.cuda.synchronize()
    if args.rank != 7:
        b7 = c3_block(7, max(3, args.steps // 2), 2)
        block["rank7"] = {k: b7[k] for k in ("ms_per_step", "TFLOP/s", "frac_of_fp8_peak", "sweep_kernel")}
    block["flop_per_sweep"] = sweep_flops(N // CP, CP, HQ, D)
    block["fused"] = {"ms_per_step": block["ms_per_step"]}
    config = {"workload": f"e4m3 causal zig-zag ring sweep, one rank's share of cp_size={CP} over N={N} (local "
                          f"{N // CP} tokens), H_q={HQ}, H_kv={HKV}, D={D}, rank {args.rank}, per-source-rank k/v "
                          "descales, fused sweep kernel",
              "global_batch": 1, "seq_len": N, "cp_size": CP, "cp_rank": args.rank, "h_q": HQ, "h_kv": HKV,
              "head_dim": D, "parallelism": "cp8 (one rank's share on 1 GPU)"}
    line = _single_line(args, block, "e4m3", PEAK_FP8_TFLOPS, config)
    line["roofline"] = {"bound": "mfma", "kernel": block["sweep_kernel"]["kernel"],
                        "achieved": block["sweep_kernel"]["TFLOP/s"], "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                        "frac": block["sweep_kernel"]["frac"],
                        "traffic": C3_SWEEP_TRAFFIC_BYTES_RANK3 if args.rank == 3 else None,
                        "avg_launch_ms": block["sweep_kernel"]["avg_launch_ms"]}
    print(json.dumps(line), flush=True)
    return 0


def bwd_block(rank: int, steps: int, warmup: int) -> dict:
    """The backward of the bf16 sweep at the headline shape (N = 131072, cp_size = 8, H_q = 32,
    H_kv = 8, D = 128): dq and every source's dk / dv contribution for one rank, from the
    forward's out and LSE.  FLOPs counted as 2.5 x the forward's (the usual five products of
    a flash-attention backward against the forward's two: 43.98 TFLOP); the kernels compute
    seven (dq recomputes the scores and dP)."""
    import torch

    from fa4_ring import RingConfig, ring_flash_attn
    from fa4_ring.backward import ring_flash_attn_backward

    _, lq, ring = make_bf16_inputs(rank)
    cfg = RingConfig(cp_size=CP, cp_rank=rank)
    out, lse = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, return_lse=True)
    g = torch.Generator(device=lq.device).manual_seed(7)
    dout = torch.randn(lq.shape, device=lq.device, generator=g, dtype=torch.bfloat16)
    t = lq.shape[0]
    dq = torch.empty(lq.shape, dtype=torch.float32, device=lq.device)
    dk = [torch.empty((t, HKV, D), dtype=torch.float32, device=lq.device) for _ in range(CP)]
    dv = [torch.empty((t, HKV, D), dtype=torch.float32, device=lq.device) for _ in range(CP)]

    def bwd():
        return ring_flash_attn_backward(dout, lq, ring.k[rank], ring.v[rank], out, lse, cfg, group=ring, dq=dq, dk=dk,
                                        dv=dv)

    ms = _event_ms(bwd, n=max(3, steps // 2))
    flops = 2.5 * sweep_flops(t, CP, HQ, D)
    return {"workload": f"backward of the bf16 sweep (rank {rank}): dq and the dk / dv contributions to all {CP} "
                        "source shards, fp32 gradients",
            "ms_per_step": round(ms, 3), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
            "frac_of_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "flop_per_step": flops, "kernels": "bwd_pack_kernel + bwd_pack_kv_kernel + bwd_dq_pp_kernel<bf16,128,4> + bwd_dkdv_kernel<bf16,128>"}


def bench_bwd(args) -> int:
    block = bwd_block(args.rank, args.steps, args.warmup)
    value = block["TFLOP/s"]
    print(json.dumps({
        "metric": METRIC, "value": value, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": block["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (q/k/v/dout ~ N(0,1) bf16, seeded on the GPU)",
        "config": {"workload": block["workload"] + f", N={N}, cp_size={CP}, H_q={HQ}, H_kv={HKV}, D={D}",
                   "global_batch": 1, "seq_len": N, "cp_size": CP, "cp_rank": args.rank, "h_q": HQ, "h_kv": HKV,
                   "head_dim": D, "parallelism": "cp8 (one rank's share on 1 GPU)"},
        "frac_of_peak": block["frac_of_peak"], "cpu_baseline": None}), flush=True)
    return 0


def bench_c4(args) -> int:
    rank = args.rank % 4
    block = c4_block(rank, args.steps, args.warmup, not args.no_cpu_baseline)
    config = {"workload": block["workload"] + ", fused sweep kernel", "global_batch": len(C4_LENGTHS),
              "seq_len": max(C4_LENGTHS), "cp_size": 4, "cp_rank": rank, "h_q": HQ, "h_kv": HKV, "head_dim": D,
              "parallelism": "cp4 (one rank's share on 1 GPU)"}
    print(json.dumps(_single_line(args, block, "bf16", PEAK_BF16_TFLOPS, config)), flush=True)
    return 0


def c5_bf16_block(rank: int, steps: int, warmup: int) -> dict:
    """The head-dim-256 shape of c5_block in bf16 (no quantisation): the fused sweep
    (attn_fwd_16bit_sweep<bf16,256,4>, 32-key tiles) with its kernel clocked, the per-step
    form with the incremental merge, and the backward (FLOPs counted as 2.5 x the forward's)."""
    import torch

    from fa4_ring import LocalKVRing, RingConfig, ring_flash_attn, zigzag_shard

    n, cp, hq, hkv, d = 262144, 8, 16, 2, 256
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(2)
    q = torch.randn(n, hq, d, device=dev, generator=g, dtype=torch.bfloat16)
    k = torch.randn(n, hkv, d, device=dev, generator=g, dtype=torch.bfloat16)
    v = torch.randn(n, hkv, d, device=dev, generator=g, dtype=torch.bfloat16)
    lq = zigzag_shard(q, rank, cp)
    del q
    ring = LocalKVRing.from_full(k, v, cp)
    del k, v
    t_local = n // cp
    flops = sweep_flops(t_local, cp, hq, d)

    def run(fused):
        return ring_flash_attn(lq, ring.k[rank], ring.v[rank], RingConfig(cp_size=cp, cp_rank=rank),
                               group=ring, fused=fused)

    clock = KernelClock()
    sec = timed_sweeps(lambda: run(True), steps, warmup, clock)
    sw_ms = clock.mean_ms("sweep_kernel")
    seci = timed_sweeps(lambda: run(False), max(3, steps // 2), 2)
    kt = flops / (sw_ms * 1e-3) / 1e12
    # the backward of the same sweep (dq and every source's dk / dv contribution, fp32)
    from fa4_ring.backward import ring_flash_attn_backward

    cfg = RingConfig(cp_size=cp, cp_rank=rank)
    o, lse = ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, return_lse=True)
    dout = torch.randn(lq.shape, device=dev, generator=g, dtype=torch.bfloat16)
    dq = torch.empty(lq.shape, dtype=torch.float32, device=dev)
    dk = [torch.empty((t_local, hkv, d), dtype=torch.float32, device=dev) for _ in range(cp)]
    dv = [torch.empty((t_local, hkv, d), dtype=torch.float32, device=dev) for _ in range(cp)]
    bms = _event_ms(lambda: ring_flash_attn_backward(dout, lq, ring.k[rank], ring.v[rank], o, lse, cfg, group=ring,
                                                     dq=dq, dk=dk, dv=dv), n=max(3, steps // 2))
    bflops = 2.5 * flops
    del o, lse, dout, dq, dk, dv
    out = {
        "workload": f"bf16 causal zig-zag ring sweep, one rank's share of cp_size={cp} over N={n} (local {t_local} "
                    f"tokens), H_q={hq}, H_kv={hkv}, D={d}, rank {rank}",
        "ms_per_step": round(sec * 1e3, 3), "TFLOP/s": round(flops / sec / 1e12, 2),
        "frac_of_peak": round(flops / sec / 1e12 / PEAK_BF16_TFLOPS, 4),
        "sweep_kernel": {"kernel": "attn_fwd_16bit_sweep<bf16,256,4>", "avg_launch_ms": round(sw_ms, 4),
                         "TFLOP/s": round(kt, 2), "frac": round(kt / PEAK_BF16_TFLOPS, 4)},
        "per_step_incremental": {"ms_per_step": round(seci * 1e3, 3), "TFLOP/s": round(flops / seci / 1e12, 2)},
        "backward": {"ms_per_step": round(bms, 3), "TFLOP/s": round(bflops / (bms * 1e-3) / 1e12, 2),
                     "frac_of_peak": round(bflops / (bms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                     "flop_per_step": bflops,
                     "kernels": "bwd_pack_kernel + bwd_pack_kv_kernel + bwd_dq_pair_kernel<bf16,256,4> + bwd_dkdv_kernel<bf16,256>"},
    }
    del ring, lq
    return out


def bench_c5(args) -> int:
    block = c5_block(args.rank, args.steps, args.warmup, not args.no_cpu_baseline)
    block["bf16_d256"] = c5_bf16_block(args.rank, max(3, args.steps // 2), 2)
    config = {"workload": block["workload"] + ", fused sweep kernel", "global_batch": 1, "seq_len": 262144,
              "cp_size": 8, "cp_rank": args.rank, "h_q": 16, "h_kv": 2, "head_dim": 256,
              "parallelism": "cp8 (one rank's share on 1 GPU)"}
    print(json.dumps(_single_line(args, block, "e4m3", PEAK_FP8_TFLOPS, config)), flush=True)
    return 0


def bench_c1(args) -> int:
    """The reference's CPU-runnable case (N = 2048, cp_size = 4, H_q = 8, H_kv = 2, D = 128,
    seed 0): every rank's sweep on the GPU in bf16 (fused; the per-step form beside it), and
    as cpu_baseline the oracle's fp32 restatement of the reference CPU ring algorithm timed
    in full, all four ranks, on the host cores."""
    import torch

    from fa4_ring import LocalKVRing, RingConfig, ring_flash_attn, zigzag_shard

    n, cp, hq, hkv, d = 2048, 4, 8, 2, 128
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    q = torch.randn(n, hq, d, generator=g)
    k = torch.randn(n, hkv, d, generator=g)
    v = torch.randn(n, hkv, d, generator=g)
    qd, kd, vd = (t.to(torch.bfloat16).to(dev) for t in (q, k, v))
    ring = LocalKVRing.from_full(kd, vd, cp)
    lqs = [zigzag_shard(qd, r, cp) for r in range(cp)]
    cfgs = [RingConfig(cp_size=cp, cp_rank=r) for r in range(cp)]
    flops = cp * sweep_flops(n // cp, cp, hq, d)  # all four ranks' sweeps

    def job(fused):
        return [ring_flash_attn(lqs[r], ring.k[r], ring.v[r], cfgs[r], group=ring, fused=fused) for r in range(cp)]

    sec = timed_sweeps(lambda: job(None), args.steps, args.warmup)
    secp = timed_sweeps(lambda: job(False), args.steps, args.warmup)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import ring_oracle as O

        threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
        threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
        torch.set_num_threads(threads)
        ks = [O.zigzag_shard(k, r, cp) for r in range(cp)]
        vs = [O.zigzag_shard(v, r, cp) for r in range(cp)]
        lq = [O.zigzag_shard(q, r, cp) for r in range(cp)]
        O.ring_rank(lq[0], ks, vs, 0, cp, 1 / math.sqrt(d))  # warm the BLAS
        t0 = time.perf_counter()
        for r in range(cp):
            O.ring_rank(lq[r], ks, vs, r, cp, 1 / math.sqrt(d))
        dt = time.perf_counter() - t0
        cpu = {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
               "sample": f"the whole job: the oracle's fp32 ring sweep of all {cp} ranks "
                         f"({flops / 1e9:.3f} GFLOP) in {dt:.3f} s"}
    value = flops / sec / 1e12
    print(json.dumps({
        "metric": METRIC, "value": round(value, 4), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (q/k/v ~ N(0,1) fp32 from a seed-0 CPU generator, "
                                                      "rounded to bf16 for the GPU)",
        "config": {"workload": f"the reference's CPU case: causal zig-zag ring sweep of all {cp} ranks of "
                               f"N={n}, H_q={hq}, H_kv={hkv}, D={d}, one after another on one GPU, fused sweep",
                   "global_batch": 1, "seq_len": n, "cp_size": cp, "h_q": hq, "h_kv": hkv, "head_dim": d,
                   "parallelism": "cp4 (every rank's share on 1 GPU)"},
        "frac_of_peak": round(value / PEAK_BF16_TFLOPS, 6),
        "note": "launch-bound: 2.1 GFLOP per rank",
        "per_step": {"ms_per_step": round(secp * 1e3, 4), "TFLOP/s": round(flops / secp / 1e12, 4)},
        "cpu_baseline": cpu}), flush=True)
    return 0


def bench_paged(args) -> int:
    """The fused sweep over paged K/V caches (256-row pages in a random order, 8 spare pages)
    against the same sweep over contiguous shards, bf16 and e4m3, at the headline shape
    (N = 131072, cp_size = 8, H_q = 32, H_kv = 8, D = 128, rank ``--rank``).  The two forms
    alternate in one process; the sweep kernels are clocked with HIP events."""
    import torch

    from fa4_ring import PagedKVRing, RingConfig, ring_flash_attn

    rank = args.rank
    flops = sweep_flops(N // CP, CP, HQ, D)
    cfg = RingConfig(cp_size=CP, cp_rank=rank)

    def kernel_ms(fn):
        clock = KernelClock()
        timed_sweeps(fn, args.steps, args.warmup, clock)
        return clock.mean_ms("sweep_kernel")

    def pair(lq, ring, desc, peak, name):
        paged = PagedKVRing.from_shards(ring.k, ring.v, 256, spare_pages=8,
                                        generator=torch.Generator().manual_seed(rank))
        cont = lambda: ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, descales=desc)  # noqa: E731
        pg = lambda: ring_flash_attn(lq, None, None, cfg, group=paged, descales=desc)  # noqa: E731
        c_ms, p_ms = [], []
        for _ in range(2):
            c_ms.append(kernel_ms(cont))
            p_ms.append(kernel_ms(pg))
        c, p = sum(c_ms) / 2, sum(p_ms) / 2
        del paged
        return {"contiguous": {"kernel": name, "avg_launch_ms": round(c, 4),
                               "frac": round(flops / (c * 1e-3) / 1e12 / peak, 4)},
                "paged": {"kernel": name.replace(">", ",paged K>"), "avg_launch_ms": round(p, 4),
                          "frac": round(flops / (p * 1e-3) / 1e12 / peak, 4)},
                "paged_over_contiguous": round(p / c - 1, 4)}

    q, lq, ring = make_bf16_inputs(rank)
    del q
    bf = pair(lq, ring, None, PEAK_BF16_TFLOPS, "attn_fwd_16bit_sweep<bf16,128,4>")
    del lq, ring
    torch.cuda.synchronize()
    q8, ring8, desc = make_fp8_inputs(rank)
    e8 = pair(q8, ring8, desc, PEAK_FP8_TFLOPS, "attn_fwd_e4m3_sweep<128,4>")
    sec = bf["paged"]["avg_launch_ms"] * 1e-3
    line = {"metric": METRIC, "value": round(flops / sec / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": bf["paged"]["avg_launch_ms"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (q/k/v ~ N(0,1), seeded on the GPU)",
            "config": {"workload": f"bf16 causal zig-zag ring sweep (N={N}, cp_size={CP}, H_q={HQ}, H_kv={HKV}, "
                                   f"D={D}, rank {rank}) with every source's K/V in a paged cache (256-row pages, "
                                   "random order), K read in place; ms_per_step is the sweep kernel alone",
                       "seq_len": N, "cp_size": CP, "cp_rank": rank},
            "frac_of_peak": bf["paged"]["frac"], "bf16": bf, "e4m3": e8, "cpu_baseline": None}
    print(json.dumps(line), flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--rank", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=16384)
    ap.add_argument("--skip-extra", action="store_true", help="only the headline bf16 sweep")
    ap.add_argument("--workload", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "bwd", "paged"],
                    help="c2 (default): the bf16 N=131072 sweep with its extras; c1: the reference's "
                         "CPU case (N=2048, cp_size 4) on every rank, with the oracle's CPU time; c3: "
                         "the e4m3 sweep at the c2 shape (ranks 3 and 7); c4: "
                         "packed bf16 sequences (8 lengths, cp_size 4); c5: the e4m3 N=262144, H_q=16, "
                         "H_kv=2, D=256 sweep (and the same shape in bf16); paged: the c2 and c3 sweeps over paged K/V caches against "
                         "contiguous shards")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (one rank's sweep with every source "
              f"rank's KV resident in HBM); --gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    if args.workload == "c5":
        return bench_c5(args)
    if args.workload == "c3":
        return bench_c3(args)
    if args.workload == "bwd":
        return bench_bwd(args)
    if args.workload == "c4":
        return bench_c4(args)
    if args.workload == "c1":
        return bench_c1(args)
    if args.workload == "paged":
        return bench_paged(args)

    import torch

    from fa4_ring import RingConfig, ring_flash_attn
    from fa4_ring.merge import merge_states
    from fa4_ring.zigzag import zigzag_shard

    rank = args.rank
    t_local = N // CP
    flops = sweep_flops(t_local, CP, HQ, D)
    per_launch = flops / CP

    # ---------------- headline: bf16 sweep, one fused launch (V transposes + sweep kernel)
    q_full, lq, ring = make_bf16_inputs(rank)
    cfg = RingConfig(cp_size=CP, cp_rank=rank, merge_mode="incremental")

    def sweep():
        return ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring)

    clock = KernelClock()
    sec = timed_sweeps(sweep, args.steps, args.warmup, clock)
    value = flops / sec / 1e12
    sw_ms = clock.mean_ms("sweep_kernel")
    sw_tflops = flops / (sw_ms * 1e-3) / 1e12
    # V -> V^T: every source's whole shard, read and written once, all 8 in one launch
    tr_ms = clock.mean_ms("transpose_v_many")
    tr_bytes = CP * 2.0 * t_local * HKV * D * 2

    # ---------------- the reference's per-step sweep (attention + LSE merge per step)
    # the per-step form: its wall time unclocked (two events around each of its ~23 launches
    # per step would add host time), then a clocked pass for the per-launch figures
    per_step = lambda: ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfg, group=ring, fused=False)  # noqa: E731
    secp = timed_sweeps(per_step, args.steps, args.warmup)
    clockp = KernelClock()
    timed_sweeps(per_step, args.steps, 1, clockp)
    attn_ms = clockp.mean_ms("attn")
    merge_ms = clockp.mean_ms("merge_inplace")
    attn_tflops = per_launch / (attn_ms * 1e-3) / 1e12
    # merge bytes: steps 1..rank merge every row, steps rank+1.. only the back half
    n_full = min(rank, CP - 1)
    n_back = CP - 1 - n_full
    mbytes = (n_full * merge_bytes_inplace(t_local, HQ, D, 2) +
              n_back * merge_bytes_inplace(t_local // 2, HQ, D, 2)) / (CP - 1)
    merge_gbs = mbytes / (merge_ms * 1e-3) / 1e9

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (q/k/v ~ N(0,1) bf16, seeded on the GPU)",
        "config": {"workload": "bf16 causal zig-zag ring sweep, one rank's share of cp_size=8 over "
                               "N=131072 (local Q/K/V 16384 tokens), H_q=32, H_kv=8, D=128, "
                               f"rank {rank}, all 8 source KV shards in HBM, fused sweep kernel",
                   "global_batch": 1, "seq_len": N, "cp_size": CP, "cp_rank": rank,
                   "h_q": HQ, "h_kv": HKV, "head_dim": D, "parallelism": "cp8 (one rank's share on 1 GPU)"},
        "frac_of_peak": round(value / PEAK_BF16_TFLOPS, 4),
        "roofline": {"bound": "mfma", "kernel": "attn_fwd_16bit_sweep<bf16,128,4>",
                     "achieved": round(sw_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(sw_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": SWEEP_TRAFFIC_BYTES_RANK3 if rank == 3 else None,
                     "algorithmic_per_launch": f"{flops / 1e12:.4f} TFLOP (the whole sweep: "
                                               "4*Tq*Tk*D*H_q per step, halved for the causal step)",
                     "avg_launch_ms": round(sw_ms, 4), "launches": clock.count("sweep_kernel")},
        "transpose_v": {"kernel": "transpose_reg_kernel<u16,128> (8 shards per launch)", "avg_launch_ms": round(tr_ms, 4),
                        "algorithmic_bytes_per_launch": round(tr_bytes),
                        "achieved_GBs": round(tr_bytes / (tr_ms * 1e-3) / 1e9, 1),
                        "frac": round(tr_bytes / (tr_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                        "launches": clock.count("transpose_v_many")},
        "per_step_bf16": {
            "workload": "same sweep as the reference runs it: one attention launch per step "
                        "(V transposed first) and an in-place LSE merge after each",
            "ms_per_step": round(secp * 1e3, 3), "TFLOP/s": round(flops / secp / 1e12, 2),
            "attn": {"kernel": "attn_fwd_16bit_vt<bf16,128,4>", "avg_launch_ms": round(attn_ms, 4),
                     "TFLOP/s": round(attn_tflops, 2), "frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": ATTN_TRAFFIC_BYTES_RANK3 if rank == 3 else None,
                     "launches": clockp.count("attn")},
            "merge": {"kernel": "merge_inplace_kernel<bf16>", "avg_launch_ms": round(merge_ms, 4),
                      "algorithmic_bytes_per_launch": round(mbytes),
                      "achieved_GBs": round(merge_gbs, 1), "peak_GBs": PEAK_HBM_GBS,
                      "frac": round(merge_gbs / PEAK_HBM_GBS, 4), "launches": clockp.count("merge_inplace")}},
    }

    # zig-zag gather of the full q (bf16, 1 GiB -> 128 MiB)
    zz = []
    for _ in range(3):
        zigzag_shard(q_full, rank, CP)
    for _ in range(10):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        zigzag_shard(q_full, rank, CP)
        e.record()
        zz.append((s, e))
    torch.cuda.synchronize()
    zms = sum(s.elapsed_time(e) for s, e in zz) / len(zz)
    zbytes = 2.0 * t_local * HQ * D * 2
    # FP8 producer on the local q (bf16 -> e4m3, one scale): amax pass + quantise pass
    from fa4_ring import quantize_e4m3
    for _ in range(3):
        quantize_e4m3(lq)
    qev = []
    for _ in range(10):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        quantize_e4m3(lq)
        e.record()
        qev.append((s, e))
    torch.cuda.synchronize()
    qms = sum(s.elapsed_time(e) for s, e in qev) / len(qev)
    qbytes = t_local * HQ * D * (2 + 2 + 1)
    result["fp8_producer"] = {"kernels": "amax_kernel<bf16> + quant_kernel<bf16>", "avg_call_ms": round(qms, 4),
                              "bytes": round(qbytes), "note": "reads x twice (amax, then quantise), writes e4m3",
                              "achieved_GBs": round(qbytes / (qms * 1e-3) / 1e9, 1),
                              "frac": round(qbytes / (qms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    result["zigzag"] = {"kernel": "shard_kernel<u32x4>", "avg_launch_ms": round(zms, 4),
                        "bytes": round(zbytes), "achieved_GBs": round(zbytes / (zms * 1e-3) / 1e9, 1),
                        "frac": round(zbytes / (zms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    if not args.skip_extra:
        # rank 7 (only front-half steps)
        lq7 = zigzag_shard(q_full, 7, CP)
        cfg7 = RingConfig(cp_size=CP, cp_rank=7)
        sec7 = timed_sweeps(lambda: ring_flash_attn(lq7, ring.k[7], ring.v[7], cfg7, group=ring),
                            max(3, args.steps // 2), 2)
        result["rank7_bf16"] = {"ms_per_step": round(sec7 * 1e3, 3), "TFLOP/s": round(flops / sec7 / 1e12, 2)}
        # batched merge mode and one merge_states launch at S = 8
        cfgb = RingConfig(cp_size=CP, cp_rank=rank, merge_mode="batched")
        clockb = KernelClock()
        secb = timed_sweeps(lambda: ring_flash_attn(lq, ring.k[rank], ring.v[rank], cfgb, group=ring, fused=False),
                            max(3, args.steps // 2), 2, clockb)
        ms_ms = clockb.mean_ms("merge_states")
        bb = merge_bytes_batched(t_local, CP, HQ, D, 2)
        result["batched_bf16"] = {"ms_per_step": round(secb * 1e3, 3), "TFLOP/s": round(flops / secb / 1e12, 2),
                                  "merge_states_ms": round(ms_ms, 4), "merge_states_bytes": round(bb),
                                  "merge_states_GBs": round(bb / (ms_ms * 1e-3) / 1e9, 1)}
        del lq7
        # fp8 sweep: fused (default) and per step
        result["fp8"] = c3_block(rank, args.steps, args.warmup, paged=True)
        # rank 7 (only front-half steps) in e4m3, its own inputs and descales
        b7 = c3_block(7, max(3, args.steps // 2), 2)
        result["fp8"]["rank7"] = {k: b7[k] for k in ("ms_per_step", "TFLOP/s", "frac_of_fp8_peak", "sweep_kernel")}
        result["fp8"]["cpu_baseline"] = ("the oracle computes e4m3 inputs dequantised in fp32: the same CPU work "
                                         "per FLOP as the bf16 sweep's cpu_baseline below")
        # paged K/V caches (pages of 256 rows in a random order): paged V^T, then the sweep
        # kernel reading K through the page tables
        from fa4_ring import PagedKVRing
        from fa4_ring.paged import transpose_v_paged_many
        paged = PagedKVRing.from_shards(ring.k, ring.v, 256, spare_pages=8,
                                        generator=torch.Generator().manual_seed(rank))
        clockpg = KernelClock()
        secpg = timed_sweeps(lambda: ring_flash_attn(lq, None, None, cfg, group=paged), args.steps, 2, clockpg)
        pk_ms = clockpg.mean_ms("sweep_kernel")
        pt_ms = _event_ms(lambda: transpose_v_paged_many(paged, t_local))
        pbytes = CP * 2.0 * t_local * HKV * D * 2  # every source's V: read once, written once (as V^T)
        result["paged_bf16"] = {
            "workload": "same sweep with every source's K/V in a paged cache (256-row pages, random "
                        "page order): one paged V^T launch, then the sweep kernel reading K in place "
                        "through the page tables (no K copy)",
            "ms_per_step": round(secpg * 1e3, 3), "TFLOP/s": round(flops / secpg / 1e12, 2),
            "sweep_kernel": {"kernel": "attn_fwd_16bit_sweep<bf16,128,4,paged K>", "avg_launch_ms": round(pk_ms, 4),
                             "TFLOP/s": round(flops / (pk_ms * 1e-3) / 1e12, 2),
                             "frac": round(flops / (pk_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)},
            "transpose_v_paged": {"kernel": "transpose_reg_kernel<u16,128>, paged (8 caches per launch)",
                                  "avg_launch_ms": round(pt_ms, 4), "bytes": round(pbytes),
                                  "achieved_GBs": round(pbytes / (pt_ms * 1e-3) / 1e9, 1),
                                  "frac": round(pbytes / (pt_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}}
        del paged
    del ring, lq, q_full
    torch.cuda.synchronize()
    if not args.skip_extra:
        # the packed-sequence and head-dim-256 configurations, every form they name
        result["c4_varlen_bf16"] = c4_block(3, args.steps, args.warmup, not args.no_cpu_baseline)
        torch.cuda.synchronize()
        result["c5_fp8_d256"] = c5_block(3, max(3, args.steps // 2), 2, not args.no_cpu_baseline)
        torch.cuda.synchronize()
        result["c5_bf16_d256"] = c5_bf16_block(3, max(3, args.steps // 2), 2)
        torch.cuda.synchronize()
        result["backward_bf16"] = bwd_block(rank, args.steps, args.warmup)
        torch.cuda.synchronize()

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(rank, args.cpu_rows)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
