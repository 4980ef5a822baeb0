"""Benchmark: one OrthoCache decode layer (score + compact + attend) on one MI355X.

Workload: Gemma-style global-attention decode,
batch 1, 32 query heads over 16 kv heads, head_dim 256, 65,536 tokens (128
blocks of 512), bf16 K/V, 90% of blocks evicted by the tau quantile.  Inputs
are synthetic (seeded, generated on the GPU) and resident in HBM before the
timed region.  A step is one layer (oc_decode_layer): the scoring kernel
(band statistics, bound, two-gate mask and attention logits in one pass over
the keys), the attention over the retained blocks (which derives the
compacted list from the mask) and its combine, launched on one stream with no
host synchronisation between steps.

Prints one JSON line.  ``value`` is microseconds per layer (lower is better).
``roofline`` is for the dominant kernel (block scoring) from HIP events on
its own launch stream; ``cpu_baseline`` times the C/OpenMP restatement of the
reference algorithm (oracle/oc_port.c) on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "µs per layer score+compact+attend @64K tok, 90% evict; HBM GB/s (% peak)"
PEAK_HBM_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--evict", type=float, default=0.9)
    p.add_argument("--seq", type=int, default=65536)
    p.add_argument("--kernel-reps", type=int, default=100)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="first run a plain device copy of this many MiB (reference for HBM counters)")
    p.add_argument("--workload", choices=("c2", "c2-cached", "c3", "c4", "c5"), default="c2",
                   help="c2: the headline decode layer (default); c2-cached: C2 with the scoring hoisted to "
                        "cache-write time; c3: ragged batched decode; c4: chunked prefill on the matrix cores; "
                        "c5: 60-layer scoring sweep")
    return p.parse_args()


def settle(fn, torch, seconds=0.5, batch=50):
    """Run fn until the GPU has been busy for about `seconds` (clocks reach
    their steady state under a continuous decode loop); not timed."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(batch):
            fn()
        torch.cuda.synchronize()


def event_time_us(fn, reps, torch):
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) * 1000.0 / reps


def copy_bandwidth(torch, dev, mib=1024, reps=20):
    """The box's achievable copy bandwidth, reported beside the published
    peak: a device-to-device copy of `mib` MiB (torch's copy kernel), read +
    write bytes over the HIP-event time of `reps` copies, after two untimed
    ones.  A copy mixes reads and writes and runs below what the read-dominated
    scoring pass reaches, so the published peak stays the roofline's."""
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    us = event_time_us(lambda: dst.copy_(src), reps, torch)
    del src, dst
    moved = 2 * mib * (1 << 20)
    return {"gbps": round(moved / (us * 1e-6) / 1e9, 1), "bytes_per_copy": moved, "us_per_copy": round(us, 2),
            "method": f"torch copy_ of {mib} MiB fp32 on the device (read + write bytes), HIP events, "
                      f"mean over {reps} copies"}


def _score_kernel_name(d: int, hkv: int, nq_pad: int) -> str:
    """The scoring kernel instantiation the library launches for bf16 keys and
    queries (oc_score.hip launch_score_dt): heads with 128- or 256-byte rows go
    two per tile when the head count is even."""
    lanes, hpt = d // 8, 1
    if lanes in (8, 16) and hkv % 2 == 0:
        lanes, hpt = 2 * lanes, 2
    return f"score_kernel<bf16, {lanes}, bf16, {nq_pad}, {hpt}>"


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.machine()


def _host_bf16(t):
    """A bf16 device tensor as a host uint16 array of its bit patterns."""
    import numpy as np
    import torch

    return t.view(dtype=torch.int16).cpu().numpy().view(np.uint16)


def _time_host(step, budget_s, min_reps=20, max_reps=200):
    """Median wall time of step() over at least min_reps runs after one
    untimed run (the reference's bench() convention: median after warmup,
    benchmarks/phase_d_indirect_dma.py:39-47); as many more runs as fit in
    budget_s, up to max_reps.  Returns (median_s, reps, last result)."""
    t0 = time.perf_counter()
    res = step()
    est = time.perf_counter() - t0
    reps = max(min_reps, min(max_reps, int(budget_s / max(est, 1e-6))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        res = step()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], reps, res


def _baseline(value_us, reps, sample):
    from oracle import native as ON

    return {"value": round(value_us, 1), "unit": "us", "cores": int(ON.port().oc_port_threads()), "kind": "port",
            "sample": f"{sample}; median of {reps} after one warmup run; oracle/oc_port.c (the reference "
                      f"algorithm in C/OpenMP: full 9-stage FWHT, band sums, bound, mask, stable partition, "
                      f"fp32 online-softmax loop), {_cpu_model()}"}


def cpu_baseline(wl, tau, zmax, budget_s, gpu_mask=None):
    """Time oracle/oc_port.c (the reference algorithm in C/OpenMP) on this
    host over the full C2 layer; the port's mask is compared with the GPU's."""
    import numpy as np

    from oracle import native as ON
    from oracle import oc_oracle as O

    ON.port()
    k, v = _host_bf16(wl.k), _host_bf16(wl.v)
    q = wl.q.float().cpu().numpy()
    qf = O.fold_gqa(q, k.shape[1])
    nb = k.shape[0] // 512

    def layer():
        tm, z = ON.port_score(k, qf)
        mask, idx, n = ON.port_compact(tm, z, tau, zmax)
        ON.port_attend(q, k, v, idx, n)
        return mask, n

    t_one = time.perf_counter()
    layer()
    t_one = time.perf_counter() - t_one
    if t_one * 20 <= 3 * budget_s:
        med, reps, (mask, n) = _time_host(layer, budget_s)
        sample = f"full C2 layer ({nb} blocks), num_active={n}"
        if gpu_mask is not None:
            sample += ", mask " + ("equal to" if np.array_equal(mask, gpu_mask) else "DIFFERENT from") + " the GPU's"
        return _baseline(med * 1e6, reps, sample)
    # A slow host: time the first blocks and scale to the layer.
    nblk = max(8, min(nb, int(nb * budget_s / (20 * t_one))))
    kk, vv = k[: nblk * 512], v[: nblk * 512]

    def part():
        tm, z = ON.port_score(kk, qf)
        _, idx, n = ON.port_compact(tm, z, tau, zmax)
        ON.port_attend(q, kk, vv, idx, n)

    med, reps, _ = _time_host(part, budget_s)
    return _baseline(med * 1e6 * nb / nblk, reps, f"first {nblk} of {nb} C2 blocks, scaled by {nb}/{nblk}")


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "bench.py measures one GPU only: every box in this run has one GPU and "
                                   "the path's multi-GPU exchange is not built; run with --gpus 1"}))
        sys.exit(2)

    import torch

    from orthocache_amd import _native, _ops, workloads

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm device"}))
        sys.exit(1)
    dev = torch.device("cuda:0")
    print(f"bench: lib {_native.LIB_PATH}", file=sys.stderr, flush=True)

    if args.workload != "c2":
        {"c2-cached": run_c2_cached, "c3": run_c3, "c4": run_c4, "c5": run_c5}[args.workload](args, torch, dev)
        return

    if args.copy_probe_mib:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    wl = workloads.c2(dev, seq=args.seq)
    sc = _ops.score(wl.k, wl.q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max[0], sc.zeta, args.evict)
    layer = _ops.DecodeLayer(wl.q, wl.k, wl.v, tau, zmax)
    score_fn, compact_fn, attend_fn = layer.phases()

    settle(layer.run, torch)
    for _ in range(args.warmup):
        layer.run()
    torch.cuda.synchronize()
    num_active = int(layer.num_active[0].item())
    print(f"bench: warmup done, num_active={num_active}", file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        layer.run()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    us_per_layer = wall * 1e6 / args.steps
    layer_event_us = event_time_us(layer.run, args.steps, torch)

    # The configuration's eviction sweep (50/75/90% by the tau quantile),
    # each a separate layer over the same inputs, timed with HIP events.
    sweep = {}
    for ev in (0.5, 0.75, 0.9):
        t_ev, z_ev = workloads.calibrate_unified(sc.tau_max[0], sc.zeta, ev)
        lay = _ops.DecodeLayer(wl.q, wl.k, wl.v, t_ev, z_ev)
        for _ in range(args.warmup):
            lay.run()
        sweep[str(ev)] = {"us": round(event_time_us(lay.run, args.steps, torch), 2),
                          "num_active": int(lay.num_active[0].item())}
        del lay

    score_us = event_time_us(score_fn, args.kernel_reps, torch)
    # One segment: no compaction launch (the attention derives the list).
    compact_us = event_time_us(compact_fn, args.kernel_reps, torch) if compact_fn else 0.0
    attend_us = event_time_us(attend_fn, args.kernel_reps, torch)
    print(f"bench: timed {args.steps} steps", file=sys.stderr, flush=True)
    copy = copy_bandwidth(torch, dev)

    s, hkv, d = wl.k.shape
    nb = s // 512
    esz = wl.k.element_size()
    q_bytes = wl.q.numel() * wl.q.element_size()
    out_bytes = wl.q.numel() * 2
    nq = wl.q.shape[-3] * (wl.q.shape[-2] // hkv)
    # The layer's byte model (the metric's): keys read once by the scoring,
    # then the retained blocks' keys and values read by the attention.
    kv_retained = num_active * 512 * hkv * d * esz
    compact_bytes = nb * hkv * 8 + nb * 4 + 4
    layer_bytes = (s * hkv * d * esz + q_bytes + nb * hkv * 8) + compact_bytes + (2 * kv_retained + q_bytes + out_bytes)
    # What this build's kernels move: with scoring-pass logits the scoring
    # kernel also writes the fp32 logits of every key row, and the attention
    # reads the retained values and logits instead of keys and values.
    logits = _ops.layer_uses_logits(wl.k.dtype, d, nq, wl.q.dtype)
    nqp = _ops.logits_nq_pad(nq)
    logit_bytes = nb * hkv * 512 * nqp * 4 if logits else 0
    score_bytes = s * hkv * d * esz + q_bytes + nb * hkv * 8 + logit_bytes
    if logits:
        attend_bytes = kv_retained + num_active * hkv * 512 * nqp * 4 + out_bytes
    else:
        attend_bytes = 2 * kv_retained + q_bytes + out_bytes
    moved_bytes = score_bytes + compact_bytes + attend_bytes
    # The roofline counts the scoring kernel's algorithmic bytes of the
    # metric's model (keys once, queries, 8 B of scores per tile); the logits
    # it also stores for the attention are listed on their own.
    score_model_bytes = s * hkv * d * esz + q_bytes + nb * hkv * 8
    score_gbs = score_model_bytes / (score_us * 1e-6) / 1e9
    # score_kernel<key dtype, lanes per row, query dtype, logit query slots>
    kernel = f"score_kernel<bf16, 32, bf16, {nqp if logits else 0}>"
    traffic = None
    traffic_src = None
    tpath = os.path.join(ROOT, "profiles", "score_kernel_c2_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        # Counters measured for this very kernel variant only.
        if tj.get("kernel") == kernel:
            traffic = tj.get("bytes_per_launch")
            traffic_src = ("profiles/score_kernel_c2_traffic.json: rocprofv3 FETCH_SIZE + WRITE_SIZE of this "
                           "kernel variant at this workload, scaled by a plain copy kernel's counters; "
                           "not measured by this run")

    result = {
        "metric": METRIC,
        "value": round(us_per_layer, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_layer / 1000.0, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V + block offsets, 10% noise blocks, generated on the GPU)",
        "config": {"workload": wl.name, "batch": 1, "q_heads": 32, "kv_heads": hkv, "head_dim": d,
                   "seq_len": s, "blocks": nb, "evict": args.evict, "num_active": num_active,
                   "tau": tau, "zeta_max": zmax},
        "layer_gbps": round(layer_bytes / (us_per_layer * 1e-6) / 1e9, 1),
        "layer_frac_of_peak": round(layer_bytes / (us_per_layer * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
        "layer_event_us": round(layer_event_us, 2),
        "evict_sweep": sweep,
        "algorithmic_bytes": {"score": score_bytes, "compact": compact_bytes, "attend": attend_bytes,
                              "layer": moved_bytes, "layer_model": layer_bytes},
        "scoring_pass_logits": logits,
        "kernels_us": {"score": round(score_us, 2), "mask_compact": round(compact_us, 2),
                       "attend_and_combine": round(attend_us, 2)},
        "roofline": {"bound": "hbm", "kernel": kernel, "achieved": round(score_gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(score_gbs / PEAK_HBM_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_src,
                     "algorithmic_bytes": score_model_bytes, "logits_store_bytes": logit_bytes,
                     "kernel_us": round(score_us, 2)},
        "hbm_copy": copy,
    }
    if not args.no_cpu:
        try:
            gm = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, tau_max=layer.tau_max,
                                   zeta=layer.zeta, tau=tau, zeta_max=zmax, want_mask=True, want_indices=False)
            result["cpu_baseline"] = cpu_baseline(wl, tau, zmax, args.cpu_budget, gpu_mask=gm.mask.cpu().numpy())
        except Exception as e:  # the GPU result stands without it
            result["cpu_baseline"] = {"error": f"{type(e).__name__}: {e}"}
    print(json.dumps(result), flush=True)


def run_c4(args, torch, dev):
    """C4: 512 queries x 131072 keys (256 blocks),
    8 kv heads, head_dim 128, bf16, 75% of blocks evicted.  A step is one
    chunk: scoring, the bound of every query, mask + compaction and the
    matrix-core attention over the 64 retained blocks."""
    from orthocache_amd import _ops, workloads

    evict = 0.75
    wl = workloads.c4(dev)
    sc = _ops.score(wl.k, wl.q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max.amax(dim=0), sc.zeta, evict)
    layer = _ops.PrefillLayer(wl.q, wl.k, wl.v, tau, zmax)
    plan = _ops.attend_plan(wl.q, wl.k, wl.v, layer.indices, layer.num_active)
    score_fn, bound_fn, compact_fn, attend_fn = layer.phases()
    settle(layer.run, torch)
    for _ in range(args.warmup):
        layer.run()
    torch.cuda.synchronize()
    num_active = int(layer.num_active[0].item())
    print(f"bench: c4 warmup done, num_active={num_active}, plan={plan}", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        layer.run()
    torch.cuda.synchronize()
    us_step = (time.perf_counter() - t0) * 1e6 / args.steps
    kus = {name: event_time_us(fn, args.kernel_reps, torch)
           for name, fn in (("score", score_fn), ("bounds", bound_fn), ("mask_compact", compact_fn),
                            ("attend_prefill_and_combine", attend_fn))}
    print(f"bench: timed {args.steps} steps", file=sys.stderr, flush=True)
    s, hkv, d = wl.k.shape
    sq, hq, _ = wl.q.shape
    rows = sq * hq
    keys = num_active * 512
    flops = 4.0 * rows * keys * d  # Q K^T and P V, 2 flops per multiply-add
    tflops = flops / (kus["attend_prefill_and_combine"] * 1e-6) / 1e12
    peak = 2500.0
    result = {
        "metric": "us per prefill chunk score+bounds+compact+attend, C4 512q x 128K keys, 75% evict",
        "value": round(us_step, 2), "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(us_step / 1000.0, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V + block offsets, 10% noise blocks, generated on the GPU)",
        "config": {"workload": wl.name, "queries": sq, "q_heads": hq, "kv_heads": hkv, "head_dim": d,
                   "seq_len": s, "blocks": s // 512, "evict": evict, "num_active": num_active,
                   "attend_plan": list(plan)},
        "kernels_us": {k: round(v, 2) for k, v in kus.items()},
        "attend_flops": flops,
        "roofline": {"bound": "mfma", "kernel": "attend_prefill_kernel<bf16, 128> + prefill_combine_half_kernel<128>",
                     "achieved": round(tflops, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 4), "traffic": None},
    }
    if not args.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline_c4(wl, tau, zmax, args.cpu_budget, num_active)
        except Exception as e:
            result["cpu_baseline"] = {"error": f"{type(e).__name__}: {e}"}
    print(json.dumps(result), flush=True)


def cpu_baseline_c4(wl, tau, zmax, budget_s, gpu_active):
    """The C/OpenMP port over the whole C4 chunk: scores with the bound of all
    512 queries, mask + compaction, attention of every query row."""
    from oracle import native as ON
    from oracle import oc_oracle as O

    k, v = _host_bf16(wl.k), _host_bf16(wl.v)
    q = wl.q.float().cpu().numpy()
    qf = O.fold_gqa(q, k.shape[1])

    def step():
        tm, z = ON.port_score(k, qf)
        _, idx, n = ON.port_compact(tm, z, tau, zmax)
        ON.port_attend(q, k, v, idx, n)
        return n

    # About 2 s per chunk on 16 EPYC threads: at least 10 runs, not 20.
    med, reps, n = _time_host(step, budget_s, min_reps=10)
    return _baseline(med * 1e6, reps, f"full C4 chunk (512 queries x 256 blocks), num_active={n} "
                                      f"(GPU {gpu_active})")


def _line(metric, us, args, config, extra):
    r = {"metric": metric, "value": round(us, 2), "unit": "us", "n_gpus": 1, "steps": args.steps,
         "warmup": args.warmup, "ms_per_step": round(us / 1000.0, 5), "higher_is_better": False,
         "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
         "data": "synthetic (seeded N(0,1) K/V + block offsets, 10% noise blocks, generated on the GPU)",
         "config": config}
    r.update(extra)
    return r


def _per_segment_thresholds(torch, tm, z, cu_blocks, evicts):
    from orthocache_amd import workloads

    taus, zmaxs = [], []
    for s, ev in enumerate(evicts):
        lo, hi = int(cu_blocks[s]), int(cu_blocks[s + 1])
        t, zm = workloads.calibrate_unified(tm[lo:hi], z[lo:hi], ev)
        taus.append(t)
        zmaxs.append(zm)
    dev = tm.device
    return (torch.tensor(taus, dtype=torch.float32, device=dev), torch.tensor(zmaxs, dtype=torch.float32, device=dev))


def run_c2_cached(args, torch, dev):
    """C2 with the scoring hoisted to cache-write time (the reference's
    docs/mathematical_framework.md:242-250): per step, bounds from the cached
    (dc, E_AC) of every block, the two-gate mask on the cached zeta,
    compaction and attention.  Also times the write-time cost: the statistics
    of one newly filled block (once per 512 decode steps)."""
    import orthocache_amd as oc
    from orthocache_amd import _ops, workloads

    wl = workloads.c2(dev, seq=args.seq)
    sc = _ops.score(wl.k, wl.q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max[0], sc.zeta, args.evict)
    st = oc.block_stats(wl.k)
    layer = oc.CachedDecodeLayer(wl.q, wl.k, wl.v, st, tau, zmax)
    settle(layer.run, torch)
    for _ in range(args.warmup):
        layer.run()
    torch.cuda.synchronize()
    num_active = int(layer.num_active[0].item())
    us = event_time_us(layer.run, args.steps, torch)
    s, hkv, d = wl.k.shape
    nb = s // 512
    us_block = event_time_us(lambda: st.update(wl.k, nb - 1, 1), args.kernel_reps, torch)
    stats_bytes = nb * hkv * (d + 2) * 4
    q_bytes = wl.q.numel() * wl.q.element_size()
    attend_bytes = num_active * 512 * hkv * d * 2 * 2 + q_bytes + wl.q.numel() * 2
    step_bytes = stats_bytes + q_bytes + nb * hkv * 8 + attend_bytes
    gbs = step_bytes / (us * 1e-6) / 1e9
    print(json.dumps(_line("us per decode step bounds(cached stats)+compact+attend, C2 64K tok, 90% evict", us, args,
                           {"workload": wl.name + "_cached_stats", "batch": 1, "q_heads": 32, "kv_heads": hkv,
                            "head_dim": d, "seq_len": s, "blocks": nb, "evict": args.evict,
                            "num_active": num_active},
                           {"algorithmic_bytes": step_bytes, "step_gbps": round(gbs, 1),
                            "write_time_us_per_new_block": round(us_block, 2)})), flush=True)


def run_c3(args, torch, dev):
    """C3: batch 32 ragged decode, 32 query / 8 kv
    heads, d=128, lengths uniform in [4096, 32768] (multiples of 512), each
    sequence with its own eviction rate in [30%, 95%].  A step is one fused
    layer over the whole batch (one scoring launch, one compaction launch with
    one workgroup per sequence, attention + combine)."""
    from orthocache_amd import _ops, varlen, workloads

    wl = workloads.c3(dev)
    cu_b = (wl.cu_seqlens // 512).cpu().numpy()
    tm, z = varlen.score_varlen(wl.q, wl.k, wl.cu_seqlens)
    tau_t, zmax_t = _per_segment_thresholds(torch, tm, z, cu_b, wl.meta["evict"])
    nseg = len(wl.meta["lens"])
    layer = _ops.DecodeLayer(wl.q, wl.k, wl.v, tau_t, zmax_t, cu_blocks=varlen.cu_blocks_from_seqlens(wl.cu_seqlens),
                             num_segments=nseg)
    settle(layer.run, torch)
    for _ in range(args.warmup):
        layer.run()
    torch.cuda.synchronize()
    active = layer.num_active.cpu().numpy()
    us = event_time_us(layer.run, args.steps, torch)
    # Each phase alone, with the kernels the layer runs (scoring with logits,
    # mask + compaction, attention + combine).
    kus = {name: event_time_us(fn, args.kernel_reps, torch)
           for name, fn in zip(("score", "mask_compact", "attend_and_combine"), layer.phases()) if fn is not None}
    s, hkv, d = wl.k.shape
    hq = wl.q.shape[-2]
    kept = int(active.sum())
    q_bytes = wl.q.numel() * 2
    score_bytes = s * hkv * d * 2 + q_bytes + (s // 512) * hkv * 8
    attend_bytes = kept * 512 * hkv * d * 2 * 2 + q_bytes + wl.q.numel() * 2
    total = score_bytes + attend_bytes
    gbs = total / (us * 1e-6) / 1e9
    score_gbs = score_bytes / (kus["score"] * 1e-6) / 1e9
    nq = wl.q.shape[-3] * (hq // hkv)
    extra = {"algorithmic_bytes": total, "layer_gbps": round(gbs, 1),
             "layer_frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
             "kernels_us": {k: round(v, 2) for k, v in kus.items()},
             "roofline": {"bound": "hbm",
                          "kernel": _score_kernel_name(wl.k.shape[-1], hkv, _ops.logits_nq_pad(nq)) + " (segments)",
                          "achieved": round(score_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(score_gbs / PEAK_HBM_GBS, 4), "traffic": None,
                          "algorithmic_bytes": score_bytes, "kernel_us": round(kus["score"], 2)}}
    extra["hbm_copy"] = copy_bandwidth(torch, dev)
    if not args.no_cpu:
        try:
            extra["cpu_baseline"] = cpu_baseline_segments(wl, tau_t.cpu().numpy(), zmax_t.cpu().numpy(),
                                                          args.cpu_budget, attend=True, gpu_active=kept)
        except Exception as e:
            extra["cpu_baseline"] = {"error": f"{type(e).__name__}: {e}"}
    print(json.dumps(_line("us per batched decode layer score+compact+attend, C3 ragged batch 32",
                           us, args,
                           {"workload": wl.name, "batch": nseg, "q_heads": hq, "kv_heads": hkv, "head_dim": d,
                            "tokens": s, "blocks": s // 512, "retained_blocks": kept,
                            "evict_range": [0.30, 0.95]}, extra)), flush=True)


def cpu_baseline_segments(wl, taus, zmaxs, budget_s, attend, gpu_active):
    """The C/OpenMP port over every segment of a ragged batch (C3) or layer of
    a sweep (C5): per segment its scores, mask + compaction and (C3) attention,
    as the reference runs one sequence per call."""
    import numpy as np

    from oracle import native as ON
    from oracle import oc_oracle as O

    cu = (wl.cu_seqlens.cpu().numpy() // 512).astype(np.int64)
    k = _host_bf16(wl.k)
    v = _host_bf16(wl.v) if attend else None
    q = wl.q.float().cpu().numpy()
    hkv = k.shape[1]
    segs = [(int(cu[i]) * 512, int(cu[i + 1]) * 512, O.fold_gqa(q[i], hkv)) for i in range(len(cu) - 1)]

    def step():
        kept = 0
        for i, (lo, hi, qf) in enumerate(segs):
            tm, z = ON.port_score(k[lo:hi], qf)
            _, idx, n = ON.port_compact(tm, z, float(taus[i]), float(zmaxs[i]))
            kept += n
            if attend:
                ON.port_attend(q[i], k[lo:hi], v[lo:hi], idx, n)
        return kept

    med, reps, kept = _time_host(step, budget_s)
    what = "attention" if attend else "no attention"
    return _baseline(med * 1e6, reps, f"all {len(segs)} segments, one port call per segment ({what}), "
                                      f"{kept} blocks kept (GPU {gpu_active})")


def run_c5(args, torch, dev):
    """C5: 60-layer scoring sweep with no attention:
    50 sliding-window layers of 1024 tokens and 10 global layers of 65536, 16
    kv heads, d=256, bf16 keys.  A step is one sweep: one scoring launch over
    all layers as segments (FWHT bands, zeta, inline bound of each layer's 32
    query heads) and one mask + compaction launch, at 90% eviction."""
    from orthocache_amd import varlen, workloads

    wl = workloads.c5(dev)
    cu_b = (wl.cu_seqlens // 512).cpu().numpy()
    tm, z = varlen.score_varlen(wl.q, wl.k, wl.cu_seqlens)
    nl = len(wl.meta["lens"])
    tau_t, zmax_t = _per_segment_thresholds(torch, tm, z, cu_b, [0.9] * nl)

    def sweep():
        t2, z2 = varlen.score_varlen(wl.q, wl.k, wl.cu_seqlens)
        return varlen.mask_compact_varlen(t2, z2, wl.cu_seqlens, tau_t, zmax_t)

    settle(sweep, torch, batch=5)
    for _ in range(args.warmup):
        sweep()
    torch.cuda.synchronize()
    us = event_time_us(sweep, args.steps, torch)
    kept = int(sweep()[2].sum().item())
    score_us = event_time_us(lambda: varlen.score_varlen(wl.q, wl.k, wl.cu_seqlens), args.kernel_reps, torch)
    s, hkv, d = wl.k.shape
    score_bytes = s * hkv * d * 2 + wl.q.numel() * 2 + (s // 512) * hkv * 8
    gbs = score_bytes / (us * 1e-6) / 1e9
    score_gbs = score_bytes / (score_us * 1e-6) / 1e9
    extra = {"algorithmic_bytes": score_bytes, "sweep_gbps": round(gbs, 1),
             "sweep_frac_of_peak": round(gbs / PEAK_HBM_GBS, 4), "retained_blocks": kept,
             "roofline": {"bound": "hbm", "kernel": "score_kernel<bf16, 32, bf16, 0> (60 layers as segments)",
                          "achieved": round(score_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(score_gbs / PEAK_HBM_GBS, 4), "traffic": None,
                          "algorithmic_bytes": score_bytes, "kernel_us": round(score_us, 2)}}
    extra["hbm_copy"] = copy_bandwidth(torch, dev)
    if not args.no_cpu:
        try:
            extra["cpu_baseline"] = cpu_baseline_segments(wl, tau_t.cpu().numpy(), zmax_t.cpu().numpy(),
                                                          args.cpu_budget, attend=False, gpu_active=kept)
        except Exception as e:
            extra["cpu_baseline"] = {"error": f"{type(e).__name__}: {e}"}
    print(json.dumps(_line("us per 60-layer scoring sweep (score + mask + compaction), C5", us, args,
                           {"workload": wl.name, "layers": nl, "kv_heads": hkv, "head_dim": d, "tokens": s,
                            "blocks": s // 512, "evict": 0.9}, extra)), flush=True)


if __name__ == "__main__":
    main()
