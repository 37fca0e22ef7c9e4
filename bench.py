"""Sparse-MLA benchmark on one MI355X (the reference's headline table, README.md:22-39).

A "step" is one sparse_mla launch over the whole configuration, preceded
(untimed) by a cache-eviction sweep, as the reference evicts L2 before every
launch and reports the device-task duration (README.md:56-57). Kernel time is
taken with HIP events on the launch stream around the launch alone; the
median over the K timed steps is reported.

Headline (``value``): sparse-MLA prefill, Q 8192 tokens over a 32K context
in effective TFLOPS = 4*H*D*sum(valid rows) / kernel
time (README.md:38). The decode configuration (B64 x 6 queries over 128K,
configs[3]) and the 32K prefill are reported alongside in
``extra``, each with ms, TFLOPS and its roofline fraction.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense bf16
# Published effective TFLOPS of the reference's DSv4.1 sparse-MLA table
# (Ascend 910B3, README.md:33-36): the basis of vs_baseline.
REFERENCE_TFLOPS = {"prefill8k": 100.4, "prefill32k": 99.7, "decode": 78.5, "decode768": 79.5}
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
FLUSH_BYTES = 1 << 30       # > 4x the 256 MiB Infinity Cache


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def time_launches(launch, steps, warmup, flush):
    import torch

    for _ in range(warmup):
        flush()
        launch()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    times = []
    wall0 = time.perf_counter()
    for _ in range(steps):
        flush()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        launch()
        end.record(stream)
        times.append((start, end))
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = [s.elapsed_time(e) for s, e in times]
    return statistics.median(ms), ms, wall


def warm_clocks(launch, flush, seconds=1.0):
    """Run the first workload for about `seconds` before any timing: the GPU
    otherwise reports its first launches at ramping clocks (about 10% slower).
    Each launch is preceded by the same cache flush as a timed launch, so every
    dispatch of the kernel in a profile of this process runs under the timed
    conditions and the profile's average duration matches the timed median."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            flush()
            launch()
        torch.cuda.synchronize()


def host_times(launch, flush, calls=30):
    """Median and max host time in microseconds of one call (the Python entry
    and the launcher, no synchronisation), each call queued behind the cache
    flush so that it never waits for the GPU."""
    import torch

    times = []
    for k in range(calls):
        flush()
        t0 = time.perf_counter()
        launch()
        times.append((time.perf_counter() - t0) * 1e6)
        if k % 10 == 9:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return round(statistics.median(times), 1), round(max(times), 1)


def sparse_config(name, batch, queries, context, steps, warmup, flush, device, prewarm=0.0):
    import torch

    from ascendflow_amd.sparse_attention import sparse_mla
    from ascendflow_amd.sparse_attention.inputs import compulsory_bytes, effective_flops, make_inputs, measurement_policy

    t0 = time.perf_counter()
    policy = measurement_policy(batch=batch, query_tokens=queries, context=context)
    inputs = make_inputs(policy, context, device=device)
    torch.cuda.synchronize()
    log(f"[bench] {name}: inputs ready in {time.perf_counter() - t0:.1f}s")
    args, kwargs = inputs.call_args(), inputs.call_kwargs()
    if prewarm:
        warm_clocks(lambda: sparse_mla(*args, **kwargs), flush, prewarm)
    median, samples, wall = time_launches(lambda: sparse_mla(*args, **kwargs), steps, warmup, flush)
    flops = effective_flops(policy, inputs.host, context)
    nbytes = compulsory_bytes(policy, inputs.touched)
    tflops = flops / (median * 1e-3) / 1e12
    gbs = nbytes / (median * 1e-3) / 1e9
    # The reference's secondary figure: selected KV logical bytes, valid rows x
    # D x 2 over every query (sparse_performance.py:273-275), i.e. flops / (2 H).
    logical = flops // (2 * policy["H"])
    host_us, host_max = host_times(lambda: sparse_mla(*args, **kwargs), flush)
    bound_us, bound_max = host_times(sparse_mla.bind(*args, **kwargs), flush)
    log(f"[bench] {name}: median {median:.4f} ms, {tflops:.1f} TFLOPS, {gbs:.0f} GB/s; host per call {host_us} us "
        f"(bound {bound_us} us)")
    return {
        "workload": name,
        "B": batch,
        "T": policy["T"],
        "context": context,
        "ms": round(median, 5),
        "ms_min": round(min(samples), 5),
        "ms_max": round(max(samples), 5),
        "tflops": round(tflops, 2),
        "flops": flops,
        "compulsory_bytes": nbytes,
        "gbs": round(gbs, 1),
        "mfma_frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "logical_kv_bytes": logical,
        "logical_kv_gbs": round(logical / (median * 1e-3) / 1e9, 1),
        "host_us": host_us,
        "host_us_max": host_max,
        "host_us_bound": bound_us,
        "host_us_bound_max": bound_max,
        "wall_s": round(wall, 3),
        "_inputs": inputs,
    }


def profiled_traffic(key):
    """HBM bytes per launch from the committed rocprofv3 PMC summary of this
    workload (FETCH_SIZE + WRITE_SIZE, each scaled by a known-size copy)."""
    import re

    path = ROOT / "profiles" / f"sparse_mla_{key}.md"
    if not path.exists():
        return None
    match = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", path.read_text(), re.M)
    return int(match.group(1)) if match else None


ATTENTION_KEYS = ("fa_c2", "fa_c2_causal", "simple_c1")


def attention_extras(steps, warmup, flush, device, which=ATTENTION_KEYS, prewarm=0.0):
    """Flash attention C2 (B1 H32 D128 S8192 f16) and teaching attention C1 timings."""
    import torch

    from ascendflow_amd.flash_attention import attention_target, simple_attention

    gen = torch.Generator(device=device)
    gen.manual_seed(9102201)
    out = {}
    q, k, v = (torch.randn((1, 32, 8192, 128), generator=gen, device=device).to(torch.float16) for _ in range(3))
    o = torch.empty_like(q)
    for causal in (False, True):
        if ("fa_c2_causal" if causal else "fa_c2") not in which:
            continue
        if prewarm:
            warm_clocks(lambda: attention_target(q, k, v, o, 8192, 8192, B=1, HQ=32, HKV=32, D=128, CAUSAL=causal),
                        flush, prewarm)
            prewarm = 0.0
        ms, _, _ = time_launches(lambda: attention_target(q, k, v, o, 8192, 8192, B=1, HQ=32, HKV=32, D=128, CAUSAL=causal),
                                 steps, warmup, flush)
        flops = 4 * 32 * 128 * (8192 * 8192 if not causal else 8192 * 8193 // 2)
        tf = flops / (ms * 1e-3) / 1e12
        out["fa_c2_causal" if causal else "fa_c2"] = {"ms": round(ms, 5), "tflops": round(tf, 2),
                                                       "mfma_frac": round(tf / MFMA_PEAK_TFLOPS, 4)}
        log(f"[bench] flash attention B1 H32 S8192 D128 f16 causal={causal}: {ms:.4f} ms, {tf:.1f} TFLOPS")
    del q, k, v, o
    if "simple_c1" not in which:
        return out
    qs = torch.randn((8, 1024, 128), generator=gen, device=device).to(torch.float16)
    ks, vs = (torch.randn((8, 128, 128), generator=gen, device=device).to(torch.float16) for _ in range(2))
    os_ = torch.empty_like(qs)
    ms, _, _ = time_launches(lambda: simple_attention(qs, ks, vs, os_, S=1024, H=8), steps, warmup, flush)
    out["simple_c1"] = {"ms": round(ms, 5), "tflops": round(4 * 8 * 1024 * 128 * 128 / (ms * 1e-3) / 1e12, 2)}
    log(f"[bench] simple attention H8 S1024: {ms:.4f} ms")
    return out


def gather_probe_extras(steps, warmup, flush, device, depths=(1, 2, 4, 8)):
    """The gather probe on the decode configuration (B64 x 6 at 128K): the
    planned rows of all 384 tokens streamed through LDS with no compute, at
    several chunks (16 rows) in flight per workgroup, one workgroup per token
    (as the one-item kernel) or 256 workgroups with equal shares. Rates: the
    listed rows (640 per token, 1 KiB each: the reference's logical KV read
    rate) and the unique KV rows touched (the HBM roofline basis) per second."""
    import torch

    from ascendflow_amd.sparse_attention.inputs import make_inputs, measurement_policy
    from ascendflow_amd.sparse_attention.probe import gather_probe, sparse_mla_plan

    policy = measurement_policy(batch=64, query_tokens=6, context=131072)
    inputs = make_inputs(policy, 131072, device=device)
    workspace = sparse_mla_plan(inputs.tensors, policy)
    torch.cuda.synchronize()
    listed = int(workspace[: 4 * policy["T"]].view(torch.int32).sum().item()) * 1024
    unique = (len(inputs.touched["ori_kv"]) + len(inputs.touched["cmp_kv"])) * 1024
    sums = torch.empty((384, 16), dtype=torch.int32, device=device)
    out = {"listed_bytes": listed, "unique_kv_bytes": unique}
    for depth in depths:
        for grid, balanced in ((384, False), (256, True)):
            ms, _, _ = time_launches(lambda: gather_probe(inputs.tensors, policy, workspace, grid, depth, balanced, sums),
                                     steps, warmup, flush)
            key = f"depth{depth}_{'balanced256' if balanced else 'items384'}"
            out[key] = {"us": round(ms * 1e3, 2), "listed_GB_s": round(listed / (ms * 1e-3) / 1e9, 1),
                        "unique_GB_s": round(unique / (ms * 1e-3) / 1e9, 1)}
            log(f"[bench] gather probe {key}: {ms * 1e3:.1f} us, listed {out[key]['listed_GB_s']} GB/s, "
                f"unique {out[key]['unique_GB_s']} GB/s")
    return out


TOPK_SHAPES = {
    # Index scores over the compressed positions of the sparse configurations:
    # one f32 score per (query token, compressed position), C = context / 2.
    "decode": ("top-k selection B64x6 ctx131072 (C 65536)", 64, 6, 131072),
    "prefill8k": ("top-k selection B1 Q8192 ctx32768 (C 16384)", 1, 8192, 32768),
}


def device_figures(device):
    """The shader clock the GPU runs at under an ALU load (launch_clock_probe:
    shader cycles over the 100 MHz real-time counter while every SIMD runs
    FMAs; MFMA-heavy kernels run lower, as their PMC cycle counts in profiles/
    show) and a measured stream-copy bandwidth (a 1 GiB device-to-device copy,
    read plus write bytes over its HIP-event time, median of 5)."""
    import torch

    from ascendflow_amd import _native

    lib = _native.library()
    stream = torch.cuda.current_stream(device).cuda_stream
    out = torch.zeros(5, dtype=torch.int64, device=device)
    clocks = []
    for _ in range(3):
        _native.check(lib.launch_clock_probe(stream, out.data_ptr(), 200000), "launch_clock_probe")
        torch.cuda.synchronize()
        c0, c1, r0, r1 = (int(v) for v in out[:4].tolist())
        clocks.append(100.0 * (c1 - c0) / max(1, r1 - r0))
    src = torch.ones((1 << 30) // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    times = []
    for _ in range(6):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        dst.copy_(src)
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end))
    copy_ms = statistics.median(times[1:])
    del src, dst
    return {"shader_clock_mhz_valu_load": round(statistics.median(clocks), 1),
            "stream_copy_gbs": round(2 * (1 << 30) / (copy_ms * 1e-3) / 1e9, 1),
            "stream_copy": "1 GiB float32 device-to-device copy (read + write bytes), median of 5 after one warm-up"}


def topk_problem(batch, queries, context, device, seed=4102026):
    """Seeded N(0,1) index scores and the sparse metadata of one shape, with
    the per-token candidate counts (the causal cutoff, as the sparse contract)."""
    import numpy as np
    import torch

    t, c = batch * queries, context // 2
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    scores = torch.randn((t, c), generator=gen, device=device)
    counts = np.full(batch, queries, np.int64)
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    offsets = np.concatenate([np.arange(queries)] * batch)
    cand = np.minimum(c, (context - queries + offsets + 1) // 2)
    meta = {
        "cu_seqlens_q": torch.as_tensor(cu, device=device),
        "seqused_cmp_kv": torch.full((batch,), context // 2, dtype=torch.int32, device=device),
        "cmp_residual_kv": torch.full((batch,), context % 2, dtype=torch.int32, device=device),
    }
    return scores, meta, cand


def topk_extras(steps, warmup, flush, device, keys=("decode", "prefill8k")):
    """Top-k index selection (TOPK 512) on the decode and 8K-prefill shapes.
    Algorithmic bytes: every candidate score read once (4 B) and the index rows
    written (4 B x TOPK per token)."""
    import torch

    from ascendflow_amd.sparse_attention import sparse_topk_indices

    out = {}
    for key in keys:
        name, b, q, ctx = TOPK_SHAPES[key]
        scores, meta, cand = topk_problem(b, q, ctx, device)
        indices = torch.empty((b * q, 1, 512), dtype=torch.int32, device=device)
        launch = lambda: sparse_topk_indices(scores, meta["cu_seqlens_q"], meta["seqused_cmp_kv"],
                                             meta["cmp_residual_kv"], TOPK=512, RATIO=2, out=indices)
        ms, _, _ = time_launches(launch, steps, warmup, flush)
        nbytes = int(4 * cand.sum() + 4 * b * q * 512)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[key] = {"workload": name, "us": round(ms * 1e3, 2), "algorithmic_bytes": nbytes,
                    "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"[bench] {name}: {ms * 1e3:.1f} us, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM)")
        del scores, indices
    return out


def cpu_topk(key, sample_tokens=48):
    """The oracle's brute-force selection (one stable lexsort per token, NumPy,
    one thread) on a token sample of one top-k shape, scaled to all tokens."""
    import numpy as np
    import torch

    from oracle.topk_reference import topk_indices

    name, b, q, ctx = TOPK_SHAPES[key]
    scores, meta, cand = topk_problem(b, q, ctx, torch.device("cpu"))
    t = b * q
    tokens = np.linspace(0, t - 1, min(sample_tokens, t)).astype(int)
    host = scores.numpy()
    # Each sampled token as a one-query request with its own cutoff.
    run = lambda: [topk_indices(host[k : k + 1], np.array([0, 1], np.int32), np.array([cand[k]], np.int32),
                                np.array([0], np.int32), 512, 1) for k in tokens]
    seconds = median_seconds(run, 3)
    fraction = len(tokens) / t
    return {
        "us_full_scaled": round(seconds / fraction * 1e6, 1),
        "gbs": round(4 * float(cand[tokens].sum()) / seconds / 1e9, 3),
        "sample": f"{len(tokens)} of {t} tokens of {name}, NumPy, 1 thread, median of 3 runs {seconds:.3f} s, "
                  f"scaled by {t}/{len(tokens)}",
    }


def cpu_threads():
    """Threads for the CPU baseline: every CPU in this process's affinity mask,
    capped by the cgroup CPU quota when one is set (more threads than the quota
    only time-slice). Returns (threads, affinity CPUs, quota or None)."""
    import math

    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        limit, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if limit != "max":
            quota = int(limit) / int(period)
    except (OSError, ValueError):
        pass
    threads = affinity if quota is None else max(1, min(affinity, math.ceil(quota)))
    return threads, affinity, quota


def cpu_model():
    """The host CPU as /proc/cpuinfo names it (model name, family/model/stepping,
    physical cores per socket, MHz) and the logical CPUs the host has."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                key, value = (part.strip() for part in line.split(":", 1))
                fields.setdefault(key, value)
    except OSError:
        return "unknown"
    name = fields.get("model name", "unknown")
    ident = "/".join(fields.get(k, "?") for k in ("cpu family", "model", "stepping"))
    cores = fields.get("cpu cores", "?")
    mhz = fields.get("cpu MHz", "?")
    return f"{name} (family/model/stepping {ident}, {cores} cores per socket, {mhz} MHz, {os.cpu_count()} logical CPUs on the host)"


def median_seconds(fn, repeats):
    fn()  # warm
    runs = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        runs.append(time.perf_counter() - t0)
    return statistics.median(runs)


def cpu_sparse(result, sample_tokens, seed=0):
    """The oracle's vectorised FP32 PyTorch-CPU sparse MLA (the reference's
    batched FP32 reference, sparse_reference.py:141-171) on a token sample of
    one configuration; the rate is scaled to the whole configuration."""
    import numpy as np

    from oracle.cpu_reference import CpuSparseMla, host_view

    inputs = result["_inputs"]
    policy = inputs.policy
    t = policy["T"]
    rng = np.random.default_rng(seed)
    tokens = list(range(t)) if sample_tokens >= t else sorted(rng.choice(t, sample_tokens, replace=False).tolist())
    data = host_view(inputs, tokens)
    ref = CpuSparseMla(data, policy, np.stack([data["q"][k] for k in tokens]), tokens)
    seconds = median_seconds(ref.run, 3)
    fraction = len(tokens) / t
    return {
        "ms_full_scaled": round(seconds / fraction * 1e3, 2),
        "tflops": round(result["flops"] * fraction / seconds / 1e12, 4),
        "sample": f"{len(tokens)} of {t} tokens of {result['workload']}, median of 3 runs {seconds:.3f} s"
                  + ("" if fraction == 1 else f", scaled by {t}/{len(tokens)}"),
    }


def cpu_flash_c2(heads=2):
    """FP32 PyTorch-CPU softmax attention for FA C2 (B1 H32 S8192 D128, the
    reference's FP32 attention math) on ``heads`` whole heads, in 1024-query
    blocks; the rate is scaled to all 32 heads."""
    import torch

    gen = torch.Generator()
    gen.manual_seed(9102201)
    q, k, v = (torch.randn((heads, 8192, 128), generator=gen).half().float() for _ in range(3))
    scale = 128 ** -0.5

    @torch.inference_mode()
    def run():
        out = torch.empty_like(q)
        for h in range(heads):
            kt = k[h].t().contiguous()
            for first in range(0, 8192, 1024):
                scores = (q[h, first : first + 1024] @ kt) * scale
                out[h, first : first + 1024] = torch.softmax(scores, dim=-1) @ v[h]
        return out

    seconds = median_seconds(run, 3)
    flops = 4 * heads * 128 * 8192 * 8192
    return {
        "ms_full_scaled": round(seconds * 32 / heads * 1e3, 2),
        "tflops": round(flops / seconds / 1e12, 4),
        "sample": f"{heads} of 32 heads of FA B1 H32 S8192 D128 non-causal, median of 3 runs {seconds:.3f} s, "
                  f"scaled by 32/{heads}",
    }


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=30)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--only", choices=["prefill8k", "decode", "prefill32k", "decode768", "gather", "topk",
                                           *ATTENTION_KEYS],
                        default=None,
                        help="time one configuration only (profiling runs; the attention keys print a log only)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-attention", action="store_true", help="skip the flash/teaching attention extras")
    parser.add_argument("--prewarm", type=float, default=1.0,
                        help="seconds of untimed launches before the first timed configuration (clock ramp)")
    parser.add_argument("--cpu-sample", type=int, default=2048,
                        help="tokens in the CPU-baseline sample of each prefill configuration")
    parser.add_argument("--no-flush", action="store_true", help="keep caches warm between launches")
    parser.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                        help="also run a plain device copy of MIB MiB (PMC byte-counter calibration)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the sparse-MLA path shards by query token with no exchange, so N GPUs run N independent "
              "token shards; only the one-GPU share is measured here)", file=sys.stderr)
        return 2

    import torch

    from ascendflow_amd import _native

    device = torch.device("cuda:0")
    lib = _native.library()
    flush_buf = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device=device)
    stream = lambda: torch.cuda.current_stream(device).cuda_stream

    def flush():
        if not args.no_flush:
            _native.check(lib.launch_cache_flush(stream(), flush_buf.data_ptr(), FLUSH_BYTES), "cache flush")

    if args.copy_calibration:
        src = torch.ones(args.copy_calibration << 18, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)  # one plain elementwise pass: reads and writes MIB MiB
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: 3 neg passes of {args.copy_calibration} MiB")
        del src, dst

    if args.only == "gather":
        extras = gather_probe_extras(args.steps, args.warmup, flush, device)
        print(json.dumps({"gather_probe": extras}), flush=True)
        return 0

    if args.only == "topk":
        extras = topk_extras(args.steps, args.warmup, flush, device)
        print(json.dumps({"topk": extras}), flush=True)
        return 0

    if args.only in ATTENTION_KEYS:
        extras = attention_extras(args.steps, args.warmup, flush, device, which=(args.only,), prewarm=args.prewarm)
        log(f"[bench] {args.only}: {json.dumps(extras[args.only])}")
        return 0

    configs = {
        "prefill8k": ("sparse_mla prefill B1 Q8192 ctx32768", 1, 8192, 32768),
        "decode": ("sparse_mla decode B64x6 ctx131072", 64, 6, 131072),
        "prefill32k": ("sparse_mla prefill B1 Q32768 ctx32768", 1, 32768, 32768),
        # README.md:36's second decode row (not a BASELINE config): B128 x 6 at 128K.
        "decode768": ("sparse_mla decode B128x6 ctx131072", 128, 6, 131072),
    }
    order = [args.only] if args.only else ["prefill8k", "decode", "prefill32k", "decode768"]
    # CPU-baseline samples per configuration (tokens): about a second of CPU work each.
    cpu_samples = {"prefill8k": args.cpu_sample, "decode": 384, "prefill32k": args.cpu_sample, "decode768": 768}
    threads, affinity, quota = cpu_threads()
    torch.set_num_threads(threads)
    results, cpu = {}, {}
    for key in order:
        name, b, q, ctx = configs[key]
        results[key] = sparse_config(name, b, q, ctx, args.steps, args.warmup, flush, device,
                                     prewarm=args.prewarm if key == order[0] else 0.0)
        if not args.no_cpu_baseline:
            log(f"[bench] timing the CPU baseline of {key}")
            cpu[key] = cpu_sparse(results[key], cpu_samples[key])
            log(f"[bench] CPU {key}: {cpu[key]['ms_full_scaled']} ms (scaled), {cpu[key]['tflops']} TFLOPS")
        results[key].pop("_inputs")  # free device memory before the next configuration
        torch.cuda.empty_cache()

    extras = {}
    if not args.only:
        extras["device"] = device_figures(device)
        log(f"[bench] device: {extras['device']['shader_clock_mhz_valu_load']} MHz shader clock under ALU load, "
            f"{extras['device']['stream_copy_gbs']} GB/s stream copy")
        extras["gather_probe"] = gather_probe_extras(args.steps, args.warmup, flush, device)
        extras["topk"] = topk_extras(args.steps, args.warmup, flush, device)
        if not args.no_cpu_baseline:
            for key in TOPK_SHAPES:
                cpu[f"topk_{key}"] = cpu_topk(key)
                log(f"[bench] CPU topk_{key}: {cpu[f'topk_{key}']['us_full_scaled']} us (scaled)")
    if not args.only and not args.no_attention:
        extras.update(attention_extras(args.steps, args.warmup, flush, device))
        if not args.no_cpu_baseline:
            cpu["fa_c2"] = cpu_flash_c2()
            log(f"[bench] CPU fa_c2: {cpu['fa_c2']['ms_full_scaled']} ms (scaled)")

    head_key = order[0]
    head = results[head_key]
    baseline = None
    host = f"FP32 torch CPU, {threads} threads ({affinity} CPUs in the affinity mask" + (
        f", cgroup quota {quota:g} CPUs)" if quota is not None else ", no cgroup quota)") + f", {cpu_model()}"
    if head_key in cpu:
        baseline = {
            "value": cpu[head_key]["tflops"],
            "unit": "TFLOPS",
            "cores": threads,
            "kind": "port",
            "sample": f"{cpu[head_key]['sample']}; {host}",
        }

    bound = "hbm" if head_key == "decode" else "mfma"
    # Over the whole call: for prefill its two kernels (the plan kernel, ~2.5%
    # of it, and the persistent attention kernel), as launched back to back.
    achieved = head["gbs"] if bound == "hbm" else head["tflops"]
    peak = HBM_PEAK_GBS if bound == "hbm" else MFMA_PEAK_TFLOPS
    record = {
        "metric": "sparse-MLA kernel ms + TFLOPS (prefill Q8K/32K; decode B64x6 @128K), 1 GPU",
        "value": head["tflops"],
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        # The reference's published effective TFLOPS for the same configuration
        # (Ascend 910B3, README.md:33-36; the same FLOP convention, README.md:38).
        "vs_baseline": (round(head["tflops"] / REFERENCE_TFLOPS[head_key], 3) if head_key in REFERENCE_TFLOPS else None),
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.1 Q/KV, sorted top-k without replacement, zero caches with touched rows patched)",
        "config": {
            "workload": head["workload"],
            "H": 64, "kv_heads": 1, "D": 512, "window": 128, "topk": 512, "ratio": 2, "page": 128,
            "T": head["T"], "context": head["context"], "B": head["B"],
            "timing": "HIP events around each launch, cache-eviction sweep before each, median",
        },
        "roofline": {
            "bound": bound,
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": "GB/s" if bound == "hbm" else "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": profiled_traffic(head_key),
        },
        "cpu_baseline": baseline,
        "extra": {k: {kk: vv for kk, vv in v.items() if kk != "_inputs"} for k, v in results.items()},
        "reference_ascend_910b3_ms": {"prefill8k": 6.847, "prefill32k": 27.225, "decode": 0.410, "decode768": 0.810},
        "reference_ascend_910b3_tflops": REFERENCE_TFLOPS,
    }
    record["extra"].update(extras)
    if cpu:
        record["extra"]["cpu_baseline_per_config"] = dict(cpu, host=host)
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
