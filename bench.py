#!/usr/bin/env python3
"""Flash-DMLA benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--secondary decode,bwd,onthefly] [--no-cpu-baseline]

Primary line (headline metric, config 2): cache-latent DMLA prefill forward, bf16, causal,
B=4, H=16, S=2048, Q [B,H,S,576], shared K_lat [B,S,576], V_lat = K_lat[..., :512], scale
1/sqrt(192), inputs N(0,1)*0.5 (synthetic, seeded).  One step = one forward launch over the
whole batch with inputs resident in HBM.  value = algorithmic TFLOP/s over the K timed steps,
counting B*H*S(S+1)*(576+512) flops (unmasked causal pairs only).

Before its W warmup launches, each workload runs untimed for clock_settle_s (0.1 s), so that
the K timed launches see the settled shader clock rather than its ramp (see _settle).
The K timed steps carry one HIP event pair around all of them on the launch stream (no
per-launch events, which add GPU time between launches); `roofline.achieved` divides the
algorithmic work by that GPU time per step, and K further launches with HIP events around each
give the per-launch median, mean and spread beside it;
`traffic` comes from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary when present.
`cpu_baseline` times the fp32 PyTorch eager oracle (oracle/dmla_ref.py) on the host cores
(at most 16 threads) over the same workload, repeated for about --cpu-seconds seconds.
`secondary` carries the paged decode (config 3) in KV GB/s with its own HBM roofline, timed
the same way with rotating KV pools larger than the 256 MB MALL, the cache-latent backward
(config 5) in TFLOP/s, counting B*H*S(S+1)*(3*576+2*512) flops, and the on-the-fly forward
(config 4) in TFLOP/s, counting B*H*S(S+1)*128 + 4*B*S*H*128*64 flops (projection once),
and the on-the-fly backward at the config-4 shapes, counting B*H*S(S+1)*320 + 8*B*S*H*128*64
flops (five products per causal pair plus the four projection gradients).
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ds-flashdmla-moe_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk/CU)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
SCALE = 1.0 / math.sqrt(192.0)


def _seeded(shape, seed, scale, dtype):
    import torch

    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _load_traffic(name):
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


SETTLE_S = 0.1   # untimed load before each workload's warmup (seconds of wall time)


def _settle(fn):
    """Runs fn() untimed for SETTLE_S seconds (synchronizing every 8 launches); returns the
    number of launches.  The shader clock ramps over the first tens of milliseconds of load:
    the prefill kernel measured 323 us (median of 40) after 5 warmup launches, 285 us after 30
    and 276-281 us once settled.  Every workload here also follows seconds of host-only work
    (its input generation, the previous workload's CPU baseline) in which the clock drops
    again.  Without this, a short --warmup would time the ramp instead of the kernel."""
    import torch

    t0 = time.perf_counter()
    n = 0
    while True:
        for _ in range(8):
            fn()
        n += 8
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= SETTLE_S:
            return n


class _Roctx:
    """ROCTx ranges around each workload's timed launches (libroctx64 through ctypes; a no-op
    where the library is absent).  Under `rocprofv3 --marker-trace --kernel-trace` they let
    --trace-summary average exactly the timed launches, not the settle and warm-up ones."""

    _lib = None

    @classmethod
    def _load(cls):
        if cls._lib is None:
            import ctypes

            cls._lib = False
            # rocprofv3 traces the ROCTx of rocprofiler-sdk; the older libroctx64 is the fallback
            for name in ("librocprofiler-sdk-roctx.so", "/opt/rocm/lib/librocprofiler-sdk-roctx.so",
                         "libroctx64.so", "/opt/rocm/lib/libroctx64.so"):
                try:
                    lib = ctypes.CDLL(name)
                except OSError:
                    continue
                lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
                lib.roctxRangePushA.restype = ctypes.c_int
                lib.roctxRangePop.restype = ctypes.c_int
                cls._lib = lib
                break
        return cls._lib

    @classmethod
    def push(cls, msg):
        lib = cls._load()
        if lib:
            lib.roctxRangePushA(msg.encode())

    @classmethod
    def pop(cls):
        lib = cls._load()
        if lib:
            lib.roctxRangePop()


def _time_launches(fn, steps, warmup, tag=None):
    """Settles the clock (_settle), runs fn() warmup times, then `steps` timed times, then
    `steps` more with an event pair around each launch.  Returns (wall ms/step, kernel stats).
    `tag` (workload, work per launch, unit) names the ROCTx range around the timed steps.

    The timed steps are bracketed by torch.cuda.synchronize() on both sides and by one HIP
    event pair on the launch stream (the current stream, which the C ABI receives), with
    nothing recorded between the steps: an event pair around every launch adds 4-7 us per
    step on the GPU (prefill 283 against 278-281 us per step, decode 127-129 against 121-123
    us, same box).  The per-launch durations come from the second pass of `steps` launches
    with events around each; the kernel figure is their median, the mean rides along, and
    `region_ms` is the timed steps' own GPU time per step.
    """
    import torch

    settle = _settle(fn)
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    if tag is not None:
        _Roctx.push("bench:%s:%d:%.6g:%s" % (tag[0], steps, tag[1], tag[2]))
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    if tag is not None:
        _Roctx.pop()
    region_ms = e0.elapsed_time(e1) / steps

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(stream)
        fn(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) for a, b in ev)
    mid = len(per) // 2
    median = per[mid] if len(per) % 2 else 0.5 * (per[mid - 1] + per[mid])
    return wall_ms, {"median": median, "mean": sum(per) / len(per), "min": per[0], "max": per[-1],
                     "launches": len(per), "settle_launches": settle, "region_ms": region_ms}


def _roofline(bound, work, stats, peak, unit, traffic, kernel, work_key):
    """roofline object: achieved from the timed steps' GPU time per step (one event pair around
    all K of them); the per-launch median, mean and spread of the evented pass ride along."""
    achieved = work / (stats["region_ms"] * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
    return {"bound": bound, "achieved": achieved, "peak": peak, "unit": unit, "frac": achieved / peak,
            "traffic": traffic, "kernel": kernel, "kernel_ms": stats["median"], "kernel_ms_mean": stats["mean"],
            "kernel_ms_min": stats["min"], "kernel_ms_max": stats["max"], "launches_timed": stats["launches"],
            "region_ms": stats["region_ms"], "clock_settle_launches": stats["settle_launches"], work_key: work}


def bench_prefill(steps, warmup, cpu_baseline):
    import torch

    from python import ops

    B, H, S = 4, 16, 2048
    dev = torch.device("cuda:0")
    q = _seeded((B, H, S, 576), 0, 0.5, torch.bfloat16).to(dev)
    k = _seeded((B, S, 576), 1, 0.5, torch.bfloat16).to(dev)
    flops = B * H * S * (S + 1) * (576 + 512)

    def step(i=0):
        ops.flash_dmla_fwd(q, k, 512, SCALE, True)

    wall_ms, ks = _time_launches(step, steps, warmup, ("prefill", flops, "TFLOP/s"))
    res = {
        "metric": "DMLA prefill TFLOP/s (cache-latent fwd, config 2)",
        "value": flops / (wall_ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "ms_per_step": wall_ms,
        "config": {"workload": "cache-latent prefill fwd (benchmark config 2)", "batch": B, "heads": H,
                   "seq_len": S, "d_qk": 576, "d_v": 512, "causal": True, "softmax_scale": SCALE},
        "roofline": _roofline("mfma", flops, ks, PEAK_BF16_TFLOPS, "TFLOP/s", _load_traffic("prefill"),
                              "mqa_fwd_kernel<false>", "algorithmic_flops_per_launch"),
    }
    if cpu_baseline:
        res["cpu_baseline"] = cpu_prefill(q.cpu(), k.cpu(), cpu_baseline)
    return res


def _cpu_threads():
    """Host threads for the CPU baseline: the cores this process may run on, at most 16 (the
    GPU box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _host_info():
    """The GPU box's host as the CPU baseline saw it: logical CPUs, the affinity set this process
    may use, the threads torch used and the CPU model name."""
    import torch

    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_count": os.cpu_count(), "affinity": affinity, "torch_threads": torch.get_num_threads(),
            "cpu_model": model}


def _time_repeated(fn, budget_s):
    """Calls fn() until at least budget_s seconds have passed; returns (calls, seconds)."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        t = time.perf_counter() - t0
        if t >= budget_s:
            return n, t


def cpu_prefill(q, k, budget_s):
    """fp32 eager oracle over the whole config-2 batch, repeated for about budget_s seconds."""
    import torch

    from oracle import dmla_ref as R

    torch.set_num_threads(_cpu_threads())
    qs, ks = q.float(), k.float()
    B, H, S = qs.shape[0], qs.shape[1], qs.shape[2]
    flops = B * H * S * (S + 1) * (576 + 512)
    R.dmla_fwd_cache_latent(qs[:1, :, :256], ks[:1, :256], 512, SCALE, True)  # warm-up
    n, t = _time_repeated(lambda: R.dmla_fwd_cache_latent(qs, ks, 512, SCALE, True), budget_s)
    return {"value": n * flops / t / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port", "host": _host_info(),
            "sample": f"all of config 2 ({B}x{H} heads x {S} causal) through the fp32 eager oracle, "
                      f"{n} passes in {t:.1f} s",
            "seconds": t}


def bench_decode(steps, warmup, cpu_baseline):
    import torch

    from python import ops

    B, H, P = 64, 128, 64
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(1024, 8193, (B,), generator=g)
    n_pages = (lens + P - 1) // P
    total = int(n_pages.sum())
    max_pages = int(n_pages.max())
    # Three rotating pools (each ~340 MB) so every step streams KV that is not in the 256 MB MALL.
    pools, tables = [], []
    for r in range(3):
        gr = torch.Generator().manual_seed(100 + r)
        pools.append((torch.randn(total, P, 576, generator=gr) * 0.5).to(torch.bfloat16).to(dev))
        perm = torch.randperm(total, generator=gr)
        table = torch.zeros(B, max_pages, dtype=torch.int32)
        c = 0
        for b in range(B):
            n = int(n_pages[b])
            table[b, :n] = perm[c:c + n].to(torch.int32)
            c += n
        tables.append(table.to(dev))
    q = _seeded((B, H, 576), 4, 0.5, torch.bfloat16).to(dev)
    sl = lens.to(torch.int32).to(dev)
    kv_bytes = int(lens.sum()) * 576 * 2
    bytes_total = kv_bytes + q.numel() * 2 + B * H * 512 * 2 + tables[0].numel() * 4 + B * 4

    def step(i=0):
        r = i % 3
        ops.flash_dmla_decode_paged(q, pools[r], tables[r], sl, 512, SCALE)

    wall_ms, ks = _time_launches(step, steps, warmup, ("decode", bytes_total, "GB/s"))
    res = {
        "metric": "DMLA paged decode KV GB/s (config 3)",
        "value": bytes_total / (wall_ms * 1e-3) / 1e9,
        "unit": "GB/s",
        "ms_per_step": wall_ms,
        "config": {"workload": "paged decode (benchmark config 3)", "batch": B, "heads": H, "page": P,
                   "ctx_sum": int(lens.sum()), "ctx_min": int(lens.min()), "ctx_max": int(lens.max())},
        "roofline": _roofline("hbm", bytes_total, ks, PEAK_HBM_GBS, "GB/s", _load_traffic("decode"),
                              "mqa_fwd_kernel<true> + lse_combine_kernel", "algorithmic_bytes_per_launch"),
    }
    if cpu_baseline:
        res["cpu_baseline"] = cpu_decode(q.cpu(), pools[0].cpu(), tables[0].cpu(), lens.to(torch.int32), bytes_total,
                                         cpu_baseline)
    return res


def cpu_decode(q, pool, table, lens, bytes_total, budget_s):
    """fp32 eager oracle (gather through the block table + attention) over all 64 sequences,
    repeated for about budget_s seconds."""
    import torch

    from oracle import dmla_ref as R

    torch.set_num_threads(_cpu_threads())
    qf = q.float()
    R.dmla_decode_paged(qf[:1], pool, table[:1], lens[:1], 512, SCALE)  # warm-up
    n, t = _time_repeated(lambda: R.dmla_decode_paged(qf, pool, table, lens, 512, SCALE), budget_s)
    return {"value": n * bytes_total / t / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port", "host": _host_info(),
            "sample": f"all of config 3 ({q.shape[0]} sequences, ctx sum {int(lens.sum())}) through the fp32 "
                      f"eager oracle, {n} passes in {t:.1f} s",
            "seconds": t}


def bench_onthefly(steps, warmup, cpu_baseline):
    """Config 4: on-the-fly forward, projections inside the kernel."""
    import torch

    from python import ops

    B, H, S = 2, 32, 4096
    dev = torch.device("cuda:0")
    q = _seeded((B, H, S, 64), 10, 1.0, torch.bfloat16).to(dev)
    k = _seeded((B, S, H, 128), 11, 1.0, torch.bfloat16).to(dev)
    v = _seeded((B, S, H, 128), 12, 1.0, torch.bfloat16).to(dev)
    bound = math.sqrt(6.0 / (128 + 64))
    g = torch.Generator().manual_seed(13)
    wk = ((torch.rand(H, 128, 64, generator=g) * 2 - 1) * bound).to(torch.bfloat16).to(dev)
    wv = ((torch.rand(H, 128, 64, generator=g) * 2 - 1) * bound).to(torch.bfloat16).to(dev)
    # Attention B*H*S(S+1)*128 plus the projections counted once, 2 * (2*B*S*H*128*64).
    flops = B * H * S * (S + 1) * 128 + 2 * (2 * B * S * H * 128 * 64)

    def step(i=0):
        ops.flash_dmla_fwd_onthefly(q, k, v, wk, wv, 0.125, True)

    wall_ms, ks = _time_launches(step, steps, warmup, ("onthefly", flops, "TFLOP/s"))
    res = {
        "metric": "DMLA on-the-fly prefill TFLOP/s (config 4)",
        "value": flops / (wall_ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "ms_per_step": wall_ms,
        "config": {"workload": "on-the-fly prefill fwd (benchmark config 4)", "batch": B, "heads": H, "seq_len": S,
                   "d_in": 128, "d_lat": 64, "causal": True, "softmax_scale": 0.125},
        "roofline": _roofline("mfma", flops, ks, PEAK_BF16_TFLOPS, "TFLOP/s", _load_traffic("onthefly"),
                              "otf_fwd_kernel", "algorithmic_flops_per_launch"),
    }
    if cpu_baseline:
        res["cpu_baseline"] = cpu_onthefly(q.cpu(), k.cpu(), v.cpu(), wk.cpu(), wv.cpu(), flops, cpu_baseline)
    return res


def cpu_onthefly(q, k, v, wk, wv, flops, budget_s):
    """fp32 eager oracle (projection + exact attention) on batch element 0, repeated ~budget_s."""
    import torch

    from oracle import dmla_ref as R

    torch.set_num_threads(_cpu_threads())
    qf, kf, vf, wkf, wvf = q[:1].float(), k[:1].float(), v[:1].float(), wk.float(), wv.float()
    n, t = _time_repeated(lambda: R.dmla_fwd_onthefly(qf, kf, vf, wkf, wvf, 0.125, True), budget_s)
    return {"value": n * flops / q.shape[0] / t / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "host": _host_info(), "sample": f"config 4 batch element 0 through the fp32 eager oracle, {n} passes in {t:.1f} s",
            "seconds": t}


def bench_bwd(steps, warmup, cpu_baseline):
    """Config 5: cache-latent backward (all its kernels) from one forward's saved o, m, l."""
    import torch

    from python import ops

    B, H, S = 4, 16, 2048
    dev = torch.device("cuda:0")
    q = _seeded((B, H, S, 576), 0, 0.5, torch.bfloat16).to(dev)
    k = _seeded((B, S, 576), 1, 0.5, torch.bfloat16).to(dev)
    do = _seeded((B, H, S, 512), 2, 1.0, torch.bfloat16).to(dev)
    o, m, l = ops.flash_dmla_fwd(q, k, 512, SCALE, True)
    flops = B * H * S * (S + 1) * (3 * 576 + 2 * 512)

    def step(i=0):
        ops.flash_dmla_bwd(q, k, o, do, m, l, 512, SCALE, True)

    wall_ms, ks = _time_launches(step, steps, warmup, ("bwd", flops, "TFLOP/s"))
    res = {
        "metric": "DMLA backward TFLOP/s (cache-latent, config 5)",
        "value": flops / (wall_ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "ms_per_step": wall_ms,
        "config": {"workload": "cache-latent backward (benchmark config 5)", "batch": B, "heads": H, "seq_len": S,
                   "d_qk": 576, "d_v": 512, "causal": True, "softmax_scale": SCALE},
        "roofline": _roofline("mfma", flops, ks, PEAK_BF16_TFLOPS, "TFLOP/s", _load_traffic("bwd"),
                              "bwd_prep + bwd_kt + bwd_dkdv + bwd_dq (dK_lat reduction in its trailing workgroups)", "algorithmic_flops_per_launch"),
    }
    if cpu_baseline:
        res["cpu_baseline"] = cpu_bwd(q.cpu(), k.cpu(), o.cpu(), do.cpu(), m.cpu(), l.cpu(), flops, cpu_baseline)
    return res


def cpu_bwd(q, k, o, do, m, l, flops, budget_s):
    """fp32 eager closed-form oracle backward over all of config 5, repeated for ~budget_s s."""
    import torch

    from oracle import dmla_ref as R

    torch.set_num_threads(_cpu_threads())
    qf, kf, of, dof = q.float(), k.float(), o.float(), do.float()
    n, t = _time_repeated(lambda: R.dmla_bwd_cache_latent(qf, kf, of, dof, m, l, 512, SCALE, True), budget_s)
    return {"value": n * flops / t / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port", "host": _host_info(),
            "sample": f"all of config 5 through the fp32 eager oracle backward, {n} passes in {t:.1f} s",
            "seconds": t}


def bench_onthefly_bwd(steps, warmup, cpu_baseline):
    """On-the-fly backward (all six kernels) at the config-4 shapes from one forward's o, m, l."""
    import torch

    from python import ops

    B, H, S = 2, 32, 4096
    dev = torch.device("cuda:0")
    q = _seeded((B, H, S, 64), 10, 1.0, torch.bfloat16).to(dev)
    k = _seeded((B, S, H, 128), 11, 1.0, torch.bfloat16).to(dev)
    v = _seeded((B, S, H, 128), 12, 1.0, torch.bfloat16).to(dev)
    do = _seeded((B, H, S, 64), 14, 1.0, torch.bfloat16).to(dev)
    bound = math.sqrt(6.0 / (128 + 64))
    g = torch.Generator().manual_seed(13)
    wk = ((torch.rand(H, 128, 64, generator=g) * 2 - 1) * bound).to(torch.bfloat16).to(dev)
    wv = ((torch.rand(H, 128, 64, generator=g) * 2 - 1) * bound).to(torch.bfloat16).to(dev)
    o, m, l = ops.flash_dmla_fwd_onthefly(q, k, v, wk, wv, 0.125, True, return_stats=True)
    # Five products per unmasked (row, key) pair (S, dP, dV_lat, dK_lat, dQ: 2 * 64 flops each)
    # plus the projection gradients dK, dV, dWK, dWV (2 * B*S*H*128*64 each); the recomputed
    # K_lat / V_lat are not credited.
    flops = B * H * S * (S + 1) * 5 * 64 + 4 * (2 * B * S * H * 128 * 64)

    def step(i=0):
        ops.flash_dmla_bwd_onthefly(q, k, v, wk, wv, o, do, m, l, 0.125, True)

    wall_ms, ks = _time_launches(step, steps, warmup, ("onthefly_bwd", flops, "TFLOP/s"))
    res = {
        "metric": "DMLA on-the-fly backward TFLOP/s (config-4 shapes)",
        "value": flops / (wall_ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "ms_per_step": wall_ms,
        "config": {"workload": "on-the-fly backward at the benchmark config 4 shapes", "batch": B, "heads": H,
                   "seq_len": S, "d_in": 128, "d_lat": 64, "causal": True, "softmax_scale": 0.125},
        "roofline": _roofline("mfma", flops, ks, PEAK_BF16_TFLOPS, "TFLOP/s", _load_traffic("onthefly_bwd"),
                              "otf_bwd_prep + proj + dkdv + dq + wgrad + wreduce", "algorithmic_flops_per_launch"),
    }
    if cpu_baseline:
        res["cpu_baseline"] = cpu_onthefly_bwd([t.cpu() for t in (q, k, v, wk, wv, o, do, m, l)], flops,
                                               cpu_baseline)
    return res


def cpu_onthefly_bwd(ts, flops, budget_s):
    """fp32 eager closed-form oracle backward on batch element 0, repeated for ~budget_s s."""
    import torch

    from oracle import dmla_ref as R

    torch.set_num_threads(_cpu_threads())
    q, k, v, wk, wv, o, do, m, l = ts
    B = q.shape[0]
    xs = [q[:1].float(), k[:1].float(), v[:1].float(), wk.float(), wv.float(), o[:1].float(), do[:1].float(),
          m[:1], l[:1]]
    n, t = _time_repeated(lambda: R.dmla_bwd_onthefly(*xs, 0.125, True), budget_s)
    return {"value": n * flops / B / t / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port", "host": _host_info(),
            "sample": f"batch element 0 of the config-4 shapes through the fp32 eager oracle backward, "
                      f"{n} passes in {t:.1f} s",
            "seconds": t}


def copy_calibration(mib):
    """Streaming copies of `mib` MiB for calibrating the HBM byte counters.  torch's elementwise
    negation kernel is a plain copy (it reads N bytes and writes N bytes), so FETCH_SIZE and
    WRITE_SIZE of its dispatches give the counters' scale for the kernels' traffic figures."""
    import torch

    n = mib * 1024 * 1024
    src = torch.randn(n // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "launches": 5}))


def _read_csv(path):
    import csv

    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def trace_summary(trace_dir):
    """Per workload, the kernels rocprofv3 traced inside the ROCTx range around its timed launches
    (`rocprofv3 --kernel-trace --marker-trace --output-format csv`): calls, mean / min / max
    duration, their GPU time per step and the achieved rate that time gives.  Returns a list of
    dicts, one per workload."""
    import glob

    def one(pattern):
        hits = sorted(glob.glob(os.path.join(trace_dir, "**", pattern), recursive=True))
        if not hits:
            raise SystemExit(f"no {pattern} under {trace_dir}")
        return _read_csv(hits[0])

    kernels = one("*kernel_trace.csv")
    markers = one("*marker_api_trace.csv")
    ranges = []
    for row in markers:
        text = next((v for v in row.values() if isinstance(v, str) and v.startswith("bench:")), None)
        if text is None:
            continue
        _, name, steps, work, unit = text.split(":", 4)
        ranges.append((name, int(steps), float(work), unit, int(row["Start_Timestamp"]), int(row["End_Timestamp"])))
    out = []
    for name, steps, work, unit, t0, t1 in ranges:
        per = {}
        for k in kernels:
            ks, ke = int(k["Start_Timestamp"]), int(k["End_Timestamp"])
            if t0 <= ks and ke <= t1:
                per.setdefault(k["Kernel_Name"], []).append((ke - ks) * 1e-3)   # us
        total_us = sum(sum(v) for v in per.values())
        gpu_ms = total_us * 1e-3 / steps
        scale = 1e12 if unit == "TFLOP/s" else 1e9
        peak = PEAK_BF16_TFLOPS if unit == "TFLOP/s" else PEAK_HBM_GBS
        achieved = work / (gpu_ms * 1e-3) / scale if gpu_ms > 0 else None
        out.append({"workload": name, "steps": steps, "kernel_ms_per_step": gpu_ms, "achieved": achieved,
                    "unit": unit, "frac": achieved / peak if achieved else None,
                    "kernels": {kn: {"calls": len(v), "mean_us": sum(v) / len(v), "min_us": min(v), "max_us": max(v)}
                                for kn, v in sorted(per.items(), key=lambda kv: -sum(kv[1]))}})
    return out


def shape_sweep(steps, warmup):
    """One JSON line per (workload, shape): the prefill, the paged decode and the cache-latent
    backward around their benchmark configurations, with the same timing (GPU time of the
    timed steps per step) and work accounting as the main lines.  Not part of the driver's
    contract; it shows how the kernels behave away from the one benchmarked shape."""
    import torch

    from python import ops

    dev = torch.device("cuda:0")
    out = []
    for B, S in ((16, 512), (8, 1024), (4, 2048), (2, 4096), (1, 8192)):
        H = 16
        q = _seeded((B, H, S, 576), 0, 0.5, torch.bfloat16).to(dev)
        k = _seeded((B, S, 576), 1, 0.5, torch.bfloat16).to(dev)
        flops = B * H * S * (S + 1) * (576 + 512)
        _, ks = _time_launches(lambda i=0: ops.flash_dmla_fwd(q, k, 512, SCALE, True), steps, warmup)
        rate = flops / (ks["region_ms"] * 1e-3) / 1e12
        out.append({"workload": "prefill", "B": B, "H": H, "S": S, "ms": ks["region_ms"], "TFLOP/s": rate,
                    "frac": rate / PEAK_BF16_TFLOPS})
        del q, k
    P, H = 64, 128
    for B in (16, 64, 256):
        g = torch.Generator().manual_seed(3)
        lens = torch.randint(1024, 8193, (B,), generator=g)
        n_pages = (lens + P - 1) // P
        total, max_pages = int(n_pages.sum()), int(n_pages.max())
        pools, tables = [], []
        for r in range(3):
            gr = torch.Generator().manual_seed(100 + r)
            pools.append((torch.randn(total, P, 576, generator=gr) * 0.5).to(torch.bfloat16).to(dev))
            perm = torch.randperm(total, generator=gr)
            table = torch.zeros(B, max_pages, dtype=torch.int32)
            c = 0
            for bb in range(B):
                n = int(n_pages[bb])
                table[bb, :n] = perm[c:c + n].to(torch.int32)
                c += n
            tables.append(table.to(dev))
        q = _seeded((B, H, 576), 4, 0.5, torch.bfloat16).to(dev)
        sl = lens.to(torch.int32).to(dev)
        nbytes = int(lens.sum()) * 576 * 2 + q.numel() * 2 + B * H * 512 * 2 + tables[0].numel() * 4 + B * 4
        _, ks = _time_launches(
            lambda i=0: ops.flash_dmla_decode_paged(q, pools[i % 3], tables[i % 3], sl, 512, SCALE), steps, warmup)
        rate = nbytes / (ks["region_ms"] * 1e-3) / 1e9
        out.append({"workload": "decode", "B": B, "H": H, "ctx": "1024..8192", "ms": ks["region_ms"], "GB/s": rate,
                    "frac": rate / PEAK_HBM_GBS})
        del pools, tables, q
    for B, S in ((8, 1024), (4, 2048), (2, 4096), (1, 8192)):
        H = 16
        q = _seeded((B, H, S, 576), 0, 0.5, torch.bfloat16).to(dev)
        k = _seeded((B, S, 576), 1, 0.5, torch.bfloat16).to(dev)
        do = _seeded((B, H, S, 512), 2, 1.0, torch.bfloat16).to(dev)
        o, m, l = ops.flash_dmla_fwd(q, k, 512, SCALE, True)
        flops = B * H * S * (S + 1) * (3 * 576 + 2 * 512)
        _, ks = _time_launches(lambda i=0: ops.flash_dmla_bwd(q, k, o, do, m, l, 512, SCALE, True), steps, warmup)
        rate = flops / (ks["region_ms"] * 1e-3) / 1e12
        out.append({"workload": "bwd", "B": B, "H": H, "S": S, "ms": ks["region_ms"], "TFLOP/s": rate,
                    "frac": rate / PEAK_BF16_TFLOPS})
        del q, k, do, o, m, l
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--secondary", default="decode,bwd,onthefly,onthefly_bwd",
                    help="comma list of extra workloads: decode, bwd, onthefly, onthefly_bwd")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline time budget per workload")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run MIB-sized device copies (HBM counter calibration) and exit")
    ap.add_argument("--sweep", action="store_true",
                    help="only time prefill, decode and backward over a range of shapes (one JSON line each) and exit")
    ap.add_argument("--trace-summary", metavar="DIR", default=None,
                    help="summarise a rocprofv3 --kernel-trace --marker-trace CSV output directory of a bench run "
                         "(the kernels inside each workload's timed range) and exit; needs no GPU")
    args = ap.parse_args()
    if args.trace_summary:
        for rec in trace_summary(args.trace_summary):
            print(json.dumps(rec))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): every box here has a single GPU, "
              "so this build runs and reports the single-GPU path", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.sweep:
        for rec in shape_sweep(args.steps, args.warmup):
            print(json.dumps(rec), flush=True)
        return
    cpu = 0.0 if args.no_cpu_baseline else args.cpu_seconds
    primary = bench_prefill(args.steps, args.warmup, cpu)
    secondary = {}
    for name in [s for s in args.secondary.split(",") if s]:
        if name == "decode":
            secondary["decode"] = bench_decode(args.steps, args.warmup, cpu)
        elif name == "bwd":
            secondary["bwd"] = bench_bwd(args.steps, args.warmup, cpu)
        elif name == "onthefly":
            secondary["onthefly"] = bench_onthefly(args.steps, args.warmup, cpu)
        elif name == "onthefly_bwd":
            secondary["onthefly_bwd"] = bench_onthefly_bwd(args.steps, args.warmup, cpu)
        else:
            raise SystemExit(f"unknown secondary workload {name}")
    line = {
        "metric": primary["metric"],
        "value": primary["value"],
        "unit": primary["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": primary["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 inputs of the benchmark config 2 shapes)",
        "config": primary["config"],
        "clock_settle_s": SETTLE_S,
        "roofline": primary["roofline"],
        "cpu_baseline": primary.get("cpu_baseline"),
        "secondary": secondary,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
