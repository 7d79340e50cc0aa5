#!/usr/bin/env python3
"""Benchmark: fused paged-attention decode on one MI355X.

One "step" = one decode-attention call over the whole batch (one layer) of the
Qwen3-8B-shaped GQA workload (B=32, Hq=32, Hkv=8, D=128, BS=128, context
lengths U[1024, 8192], seeded), inputs resident in HBM. Prints ONE JSON line:
value = algorithmic KV-read GB/s (K+V of valid tokens + Q + out + tables,
divided by the step time: the main and merge kernels, back to back), plus
µs/step, the roofline of the main kernel (its time over back-to-back
launches) and the CPU baseline (the C restatement of the reference kernels,
timed on the host).

    python bench.py [--steps K] [--warmup W] [--config NAME] [--no-cpu-baseline] [--no-other-configs]

The default run also times every other config (cfg1, cfg3-5, cfg2_fp8 and the
reference's unroll Case1) on the GPU, and reports their main-kernel µs, HBM
and MFMA fractions and step µs under "other_configs".

The synthetic K and V caches share one allocation laid out by
kv_cache.alloc_kv_pools (V an odd multiple of 256 bytes from K), the layout
the library recommends; --kv-layout separate allocates them apart, which
costs the GQA main kernel 1-4%.

Only one GPU is used; --gpus N with N > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak
DEFAULT_CONFIG = "cfg2_qwen3_8b"
# The headline metric, quoted on the default workload; other --config runs
# carry their workload name after it.
METRIC = "decode-attn KV-read GB/s & % HBM peak; µs/step at Qwen3-8B shape bs=32"
KV_LAYOUTS = {
    "pool": "K and V caches in one allocation, V 256 bytes past K's end rounded to 512 (kv_cache.alloc_kv_pools)",
    "separate": "K and V caches in two allocations",
}


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", default=DEFAULT_CONFIG)
    p.add_argument("--tg-mode", default="graph", choices=["eager", "graph"],
                   help="--op taskgraph: launch tasks as submitted, or as one hipGraph per step")
    p.add_argument("--op", default="decode",
                   choices=["decode", "decode_append", "decode_prelude", "kv_append", "prelude", "taskgraph"],
                   help="decode (the headline path); kv_append / prelude: the cache-write step before it")
    p.add_argument("--tokens", type=int, default=32768,
                   help="--op kv_append: tokens written per call (32 = one decode step of bs=32)")
    p.add_argument("--workers", type=int, default=0, help="worker wavefronts; 0 = one per wave slot")
    p.add_argument("--kv-layout", default="pool", choices=["pool", "separate"],
                   help="pool: K and V caches in one allocation from kv_cache.alloc_kv_pools (V an odd multiple "
                        "of 256 bytes from K); separate: two allocations")
    p.add_argument("--out-dtype", default="bf16", choices=["bf16", "f32"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-other-configs", action="store_true",
                   help="default config only: skip timing the other configs in the same run")
    p.add_argument("--q-len", type=int, default=0, help="shape variant: query tokens per sequence (0 = the config's)")
    p.add_argument("--num-heads", type=int, default=0, help="shape variant: query heads (0 = the config's)")
    p.add_argument("--causal", type=int, default=-1, choices=[-1, 0, 1],
                   help="shape variant: causal multi-token decode (-1 = the config's)")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU-baseline sample duration")
    p.add_argument("--cpu-threads", type=int, default=0,
                   help="0 = every CPU this process may use, capped at OMP_NUM_THREADS when set (the box's share)")
    p.add_argument("--traffic-file", default=str(ROOT / "profiles" / "traffic.json"),
                   help="measured HBM bytes per launch (from rocprofv3 --pmc), if present")
    p.add_argument("--calibrate-copy-mib", type=int, default=0,
                   help="before the timed region, run 3 device copies of this many MiB (a kernel of known "
                        "traffic that calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE in the same run)")
    return p.parse_args()


def variant_config(cfg, args):
    """The config with the shape overrides of --q-len / --num-heads / --causal
    (same seed and draw order, so the context lengths and block table stay
    the config's); its name records them."""
    import dataclasses

    changes, tags = {}, []
    if args.q_len > 0 and args.q_len != cfg.q_len:
        changes["q_len"], tags = args.q_len, tags + [f"q_len={args.q_len}"]
    if args.num_heads > 0 and args.num_heads != cfg.num_heads:
        changes["num_heads"], tags = args.num_heads, tags + [f"heads={args.num_heads}"]
    if args.causal >= 0 and bool(args.causal) != cfg.causal:
        changes["causal"], tags = bool(args.causal), tags + [f"causal={args.causal}"]
    if not changes:
        return cfg
    name = f"{cfg.name}[{','.join(tags)}]"
    return dataclasses.replace(cfg, name=name, description=f"{cfg.description}; variant {','.join(tags)}", **changes)


def time_decode(case, out, num_workers: int, dev, steps: int, warmup: int) -> dict:
    """Time one decode config on device-resident inputs: `steps` back-to-back
    calls between two events on the launch stream (the step: main + merge
    kernels), then the main kernel alone: `steps` back-to-back main launches
    between two events (each writes the same partials and outputs; one merge
    after them leaves the output complete). Back to back is how a serving loop
    runs it: events around every launch would add their own overhead and let
    the clock recover between launches (the MLA kernel runs 11% faster after
    an idle gap)."""
    import torch

    from simpler_amd import paged_attention as pa

    cfg = case.config
    pargs = pa.make_args(case.query, case.key_cache, case.value_cache, case.block_table, case.context_lens, out,
                         case.scale, causal=cfg.causal, num_workers=num_workers, k_scale=case.k_scale,
                         v_scale=case.v_scale)
    stream = torch.cuda.current_stream(dev)
    print(f"[bench] {cfg.name}: warmup {warmup}", file=sys.stderr, flush=True)
    for _ in range(warmup):
        pa.launch(pargs, dev, stream.cuda_stream)
    torch.cuda.synchronize(dev)
    pa.check_errors(dev)

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        pa.launch(pargs, dev, stream.cuda_stream)
    end.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    step_ms = start.elapsed_time(end) / steps

    pa.launch(pargs, dev, stream.cuda_stream, phases=pa.PHASE_MAIN)  # one untimed split step first
    pa.launch(pargs, dev, stream.cuda_stream, phases=pa.PHASE_MERGE)
    torch.cuda.synchronize(dev)
    m0, m1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    m0.record(stream)
    for _ in range(steps):
        pa.launch(pargs, dev, stream.cuda_stream, phases=pa.PHASE_MAIN)
    m1.record(stream)
    pa.launch(pargs, dev, stream.cuda_stream, phases=pa.PHASE_MERGE)
    torch.cuda.synchronize(dev)
    pa.check_errors(dev)
    main_ms = m0.elapsed_time(m1) / steps
    print(f"[bench] {cfg.name}: {step_ms * 1e3:.1f} us/step, main kernel {main_ms * 1e3:.1f} us, "
          f"wall {wall:.3f} s", file=sys.stderr, flush=True)
    return {"step_ms": step_ms, "main_ms": main_ms, "wall_s": wall, "workers": pa.plan(pargs),
            "kernel": pa.kernel_name(pargs)}


def other_configs(args, dev, skip: str) -> dict:
    """Every other benchmark config, timed in this same run (fewer steps, no CPU
    baseline): main-kernel µs and its fraction of HBM peak (and of the dense
    bf16 MFMA peak), and the step µs."""
    import torch

    from simpler_amd.workloads import CONFIGS, algorithmic_bytes, algorithmic_flops, make_case

    res = {}
    steps, warmup = max(1, min(args.steps, 50)), max(1, min(args.warmup, 5))
    out_dtype = torch.bfloat16 if args.out_dtype == "bf16" else torch.float32
    for name in CONFIGS:
        if name == skip:
            continue
        case_cpu = make_case(name)
        case = case_cpu.to(dev, kv_pool=args.kv_layout == "pool")
        out = torch.empty(case.out_shape(), dtype=out_dtype, device=dev)
        tm = time_decode(case, out, args.workers, dev, steps, warmup)
        nbytes = algorithmic_bytes(case_cpu, out_bytes=2 if out_dtype == torch.bfloat16 else 4)
        res[name] = {"kernel": tm["kernel"], "workers": tm["workers"], "main_us": round(tm["main_ms"] * 1e3, 2),
                     "frac": round(nbytes / (tm["main_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "step_us": round(tm["step_ms"] * 1e3, 2),
                     "step_frac": round(nbytes / (tm["step_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": nbytes, "steps": steps,
                     # the MFMA side of the roofline (MLA sits near the ridge)
                     "mfma_frac": round(algorithmic_flops(case_cpu) / (tm["main_ms"] * 1e-3) / 1e12
                                        / MFMA_BF16_PEAK_TFLOPS, 4)}
        del case, out
        torch.cuda.empty_cache()
    return res


def api_time(case, out, cfg, steps: int, warmup: int) -> dict | None:
    """µs per `Worker(level=2).run` of the reference paged-attention callable on
    the same device-resident inputs: the API time of a call, i.e. the
    simpler_run host path through libsimpler_hip.so, its argument checks and
    both kernels, up to the stream synchronisation it ends with."""
    import ctypes

    from simpler_amd import Worker
    from simpler_amd import paged_attention as pa
    from simpler_amd.task_interface import ChipStorageTaskArgs, ChipTensor
    from simpler_amd.torch_interop import torch_dtype_to_datatype

    def chip(t):
        return ChipTensor.make(t.data_ptr(), tuple(int(x) for x in t.shape), torch_dtype_to_datatype(t.dtype),
                               child_memory=True, strides=tuple(int(x) for x in t.stride()))

    w = Worker(level=2, platform="mi355x", device_id=out.device.index or 0)
    w.init()
    try:
        handle = w.register(pa.reference_chain_callable())
        targs = ChipStorageTaskArgs()
        for t in (case.query, case.key_cache, case.value_cache, case.block_table, case.context_lens, out):
            targs.add_tensor(chip(t))
        if case.fp8:
            targs.add_tensor(chip(case.k_scale))
            targs.add_tensor(chip(case.v_scale))
        targs.add_scalar(ctypes.c_float(case.scale))
        if cfg.causal:
            targs.add_scalar(1)
        for _ in range(warmup):
            w.chip_worker.run(handle, targs)
        t0 = time.perf_counter()
        for _ in range(steps):
            w.chip_worker.run(handle, targs)
        us = (time.perf_counter() - t0) / steps * 1e6
    finally:
        w.close()
    return {"us_per_call": round(us, 2), "calls": steps,
            "path": "Worker(level=2).run -> simpler_run (libsimpler_hip.so), device-resident tensors, "
                    "reference QK/SF/PV/UP callable"}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the baseline's record."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads(requested: int) -> tuple[int, int]:
    """(threads to use, CPUs this process may run on). The GPU box grants one
    GPU's share of its host, 16 CPUs, and says so in OMP_NUM_THREADS; the
    baseline uses every CPU of that share (all of nproc where no share is set)."""
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    if requested > 0:
        return requested, nproc
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return (min(nproc, share) if share > 0 else nproc), nproc


def cpu_baseline(case, args) -> dict | None:
    """Time the C restatement of the reference kernels on this host (kind "port"):
    2 warm-up steps, then at least 10 timed steps and at least --cpu-seconds of
    work; the median step time is the figure."""
    try:
        import numpy as np

        from oracle import pa_oracle_c
        from simpler_amd.workloads import algorithmic_bytes
    except Exception as e:  # pragma: no cover - reported, never fatal
        return {"value": None, "error": f"oracle unavailable: {e}"}
    threads, nproc = cpu_threads(args.cpu_threads)
    c = case.config

    def bits(t):
        return t.contiguous().view(__import__("torch").int16).numpy().view(np.uint16)

    kc, vc = case.key_cache, case.value_cache
    if case.fp8:  # power-of-two scales: the dequantised caches are exactly bf16
        from simpler_amd.workloads import dequantize_kv_fp8
        kc = dequantize_kv_fp8(kc, case.k_scale).to(__import__("torch").bfloat16)
        vc = dequantize_kv_fp8(vc, case.v_scale).to(__import__("torch").bfloat16)
    q, k = bits(case.query), bits(kc)
    v = None if c.mla else bits(vc)
    bt, cl = case.block_table.numpy(), case.context_lens.numpy()
    out = np.zeros((c.batch, c.q_len, c.num_heads, c.head_dim_v), dtype=np.float32)

    def step():
        pa_oracle_c.decode(q, k, v, bt, cl, case.scale, causal=c.causal, v_dim=c.head_dim_v if c.mla else None,
                           n_threads=threads, out=out)

    for _ in range(2):
        step()
    times, t0 = [], time.perf_counter()
    while len(times) < 10 or (time.perf_counter() - t0 < args.cpu_seconds and len(times) < 1000):
        s0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - s0)
    el = time.perf_counter() - t0
    times.sort()
    median = times[len(times) // 2] if len(times) % 2 else 0.5 * (times[len(times) // 2 - 1] + times[len(times) // 2])
    nbytes = algorithmic_bytes(case, out_bytes=2 if args.out_dtype == "bf16" else 4)
    return {
        "value": round(nbytes / median / 1e9, 3),
        "unit": "GB/s",
        "us_per_step": round(median * 1e6, 1),
        "median_us": round(median * 1e6, 1),
        "mean_us": round(sum(times) / len(times) * 1e6, 1),
        "runs": len(times),
        "warmup": 2,
        "cores": threads,
        "nproc": nproc,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"full {c.name} decode step (all {c.batch}x{c.kv_heads} sequence/kv-head items), median of "
                  f"{len(times)} steps after 2 warm-ups ({el:.1f} s), C restatement of the reference QK/SF/PV/UP "
                  f"kernels (oracle/pa_oracle.c), {threads} pthreads on {nproc} CPUs available"
                  + ("; fp8 caches given to it dequantised (bf16-exact), bytes counted as fp8" if case.fp8 else ""),
    }


def bench_kv(args) -> int:
    """Time the KV-cache append or the fused decode prelude (Qwen3-8B layer shape)."""
    import numpy as np
    import torch

    from simpler_amd import kv_cache as kvc

    dev = torch.device("cuda", 0)
    hq, hkv, d, bs = 32, 8, 128, 128
    g = torch.Generator().manual_seed(20261210)
    stream = torch.cuda.current_stream(dev)
    if args.op == "kv_append":
        n = args.tokens
        nblk = (2 * n + bs - 1) // bs
        kc = torch.zeros(nblk, bs, hkv, d, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        key = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16).to(dev)
        val = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16).to(dev)
        slots = torch.randperm(nblk * bs, generator=g)[:n].to(torch.int32).to(dev)
        pargs = kvc.append_args(key, val, slots, kc, vc)
        call = lambda: kvc.launch_append(pargs, stream=stream.cuda_stream)
        nbytes = n * (4 * hkv * d * 2 + 4)
        workload = f"kv_append: {n} tokens, Hkv={hkv}, D={d}, block_size={bs}, random slots in a {nblk}-block pool"
        kernel = "kv_append_kernel"
        metric = "kv-append GB/s (K+V rows read and written)"
    else:
        b = 32
        seq = torch.randint(1024, 8192, (b,), generator=g, dtype=torch.int32)
        max_blocks = 64
        table = torch.arange(b * max_blocks, dtype=torch.int32).reshape(b, max_blocks)
        from simpler_amd.workloads import current_token_slots, rope_tables
        cos, sin = (t.to(dev) for t in rope_tables(max_blocks * bs, d))
        slots = current_token_slots(table, seq, bs).to(dev)
        rn = lambda *sh: torch.randn(*sh, generator=g).to(dev)
        qp, kp, vp = rn(b, hq * d), rn(b, hkv * d), rn(b, hkv * d)
        ir = rn(b).abs() + 0.5
        qw, kw = rn(d) * 0.1 + 1, rn(d) * 0.1 + 1
        kc = torch.zeros(b * max_blocks, bs, hkv, d, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        q_out = torch.empty(b, hq, d, dtype=torch.bfloat16, device=dev)
        seq_d = seq.to(dev)
        pargs = kvc.prelude_args(qp, kp, vp, ir, qw, kw, cos, sin, seq_d, slots, kc, vc, hq, q_out)
        call = lambda: kvc.launch_prelude(pargs, stream=stream.cuda_stream)
        nbytes = b * ((hq + 2 * hkv) * d * 4 + 4 + 2 * d * 4 + 8 + hq * d * 2 + 2 * hkv * d * 2) + 2 * d * 4
        workload = f"prelude: B={b}, Hq={hq}, Hkv={hkv}, D={d}: q/k RMS norm + RoPE + K/V append"
        kernel = "qk_norm_rope_append_kernel"
        metric = "decode prelude (q/k norm + RoPE + KV append) GB/s"
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        call()
    e1.record(stream)
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / args.steps
    gbs = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline and args.op == "kv_append":
        from oracle import kv_oracle as ko
        sample = min(n, 4096)
        kcn = np.zeros((nblk, bs, hkv, d), np.uint16)
        kn = np.ones((sample, hkv, d), np.uint16)
        sl = slots[:sample].cpu().numpy()
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < min(args.cpu_seconds, 5.0):
            ko.kv_append(kcn, kcn, kn, kn, sl)
            reps += 1
        el = (time.perf_counter() - t0) / reps
        cpu = {"value": round(sample * (4 * hkv * d * 2 + 4) / el / 1e9, 3), "unit": "GB/s", "cores": 1,
               "kind": "port", "sample": f"oracle kv_append of {sample} tokens ({reps} repetitions, numpy, 1 thread; "
                                         "includes the oracle's cache copies)"}
    line = {
        "metric": metric, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "us_per_step": round(ms * 1e3, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": workload, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": kernel,
                     "kernel_us": round(ms * 1e3, 2), "algorithmic_bytes": nbytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_decode_prelude(args) -> int:
    """The decode prelude (q/k RMS norm + RoPE, v scaling), the KV append and
    the decode in one call (simpler_hip_pa_decode_prelude: the prelude's launch
    at the slots the block table gives, then the decode's two) on a bf16 GQA
    config with 128-dim heads, beside the same work as two calls:
    simpler_hip_qk_norm_rope_append with a caller-built slot mapping, then
    simpler_hip_pa_decode on its query (and the decode alone)."""
    import torch

    from simpler_amd import kv_cache as kvc
    from simpler_amd import paged_attention as pa
    from simpler_amd.workloads import CONFIGS, algorithmic_bytes, make_case, rope_tables

    dev = torch.device("cuda", 0)
    cfg = CONFIGS[args.config]
    if cfg.mla or cfg.kv_format != "bf16" or cfg.head_dim_k != 128 or cfg.head_dim_v != 128:
        print("bench.py: --op decode_prelude times bf16 GQA configs with 128-dim heads", file=sys.stderr)
        return 2
    case_cpu = make_case(cfg)
    case = case_cpu.to(dev, kv_pool=args.kv_layout == "pool")
    g = torch.Generator().manual_seed(20261212)
    b, ql, hq, hkv, d = cfg.batch, cfg.q_len, cfg.num_heads, cfg.kv_heads, cfg.head_dim_k
    rn = lambda *shape, std=0.5: (torch.randn(*shape, generator=g) * std).to(dev)  # noqa: E731
    q_proj, k_proj, v_proj = rn(b, ql, hq, d), rn(b, ql, hkv, d), rn(b, ql, hkv, d)
    inv_rms = (1.0 + torch.rand(b, ql, generator=g) * 0.2).to(dev)
    q_w, k_w = (1.0 + rn(d, std=0.1)), (1.0 + rn(d, std=0.1))
    cos, sin = (t.to(dev) for t in rope_tables(int(case_cpu.context_lens.max()) + 1, d))
    qp = lambda t: t if ql > 1 else t[:, 0].contiguous()  # noqa: E731
    out = torch.empty(case.out_shape(), dtype=torch.bfloat16, device=dev)
    fargs, pre = pa.prelude_args(qp(q_proj), qp(k_proj), qp(v_proj), inv_rms, q_w, k_w, cos, sin, case.key_cache,
                                 case.value_cache, case.block_table, case.context_lens, out, case.scale,
                                 eps=kvc.EPS, causal=cfg.causal, num_workers=args.workers)
    # the two-step form: the standalone prelude over every new token, then the decode on its query
    pos = case.context_lens.long()[:, None] - ql + torch.arange(ql, device=dev)[None, :]
    phys = case.block_table.long().gather(1, pos.clamp(min=0) // cfg.block_size)
    slots = torch.where(pos >= 0, phys * cfg.block_size + pos % cfg.block_size, -1).to(torch.int32).reshape(-1)
    q_out = torch.empty(b * ql, hq, d, dtype=torch.bfloat16, device=dev)
    sargs = kvc.prelude_args(q_proj.reshape(b * ql, hq * d), k_proj.reshape(b * ql, hkv * d),
                             v_proj.reshape(b * ql, hkv * d), inv_rms.reshape(-1), q_w, k_w, cos, sin,
                             (pos + 1).reshape(-1).to(torch.int32), slots, case.key_cache, case.value_cache, hq, q_out)
    query = q_out.reshape(b, ql, hq, d) if ql > 1 else q_out
    dargs = pa.make_args(query, case.key_cache, case.value_cache, case.block_table, case.context_lens, out,
                         case.scale, causal=cfg.causal, num_workers=args.workers)
    stream = torch.cuda.current_stream(dev)
    sid = stream.cuda_stream
    variants = {
        "one_call": lambda: pa.launch(fargs, dev, sid, prelude=pre),
        "separate": lambda: (kvc.launch_prelude(sargs, stream=sid), pa.launch(dargs, dev, sid)),
        "decode_only": lambda: pa.launch(dargs, dev, sid),
    }
    runs = {name: [] for name in variants}
    for rnd in range(5):
        for name, call in variants.items():
            for _ in range(args.warmup):
                call()
            torch.cuda.synchronize(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(args.steps):
                call()
            e1.record(stream)
            torch.cuda.synchronize(dev)
            runs[name].append(e0.elapsed_time(e1) / args.steps * 1e3)
            print(f"[bench] round {rnd} {name}: {runs[name][-1]:.2f} us/step", file=sys.stderr, flush=True)
    us = {name: sorted(r)[len(r) // 2] for name, r in runs.items()}
    pa.check_errors(dev)
    # decode bytes plus the projections read (fp32 q, k, v) and the new K/V rows written
    proj = b * ql * (hq + 2 * hkv) * d * 4
    nbytes = algorithmic_bytes(case_cpu, out_bytes=2) + proj + b * ql * hkv * 2 * d * 2
    gbs = nbytes / (us["one_call"] * 1e-6) / 1e9
    line = {
        "metric": f"decode with prelude and KV append in one call GB/s [{cfg.name}]", "value": round(gbs, 2),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(us["one_call"] / 1e3, 5), "us_per_step": round(us["one_call"], 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.description}; q/k RMS norm + RoPE and the append of {ql} new "
                               "token(s) per sequence, then the decode", "parallelism": "single GPU"},
        "us_per_step_separate": round(us["separate"], 2), "us_per_step_decode_only": round(us["decode_only"], 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "qk_norm_rope_append_kernel + pa_decode_kernel + pa_merge_kernel",
                     "kernel_us": round(us["one_call"], 2), "algorithmic_bytes": nbytes},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_decode_append(args) -> int:
    """The KV append and the decode in one call (simpler_hip_pa_decode_append:
    fused into the decode's launches where a worker runs one row tile, else the
    append's launch first) on a decode config, beside the same work as two
    calls: simpler_hip_kv_append at caller-built slots, then
    simpler_hip_pa_decode (and the decode alone)."""
    import torch

    from simpler_amd import kv_cache as kvc
    from simpler_amd import paged_attention as pa
    from simpler_amd.workloads import CONFIGS, algorithmic_bytes, make_case

    dev = torch.device("cuda", 0)
    cfg = CONFIGS[args.config]
    if cfg.mla or cfg.kv_format != "bf16":
        print("bench.py: --op decode_append times bf16 GQA configs", file=sys.stderr)
        return 2
    case_cpu = make_case(cfg)
    case = case_cpu.to(dev, kv_pool=args.kv_layout == "pool")
    g = torch.Generator().manual_seed(20261211)
    shape = (cfg.batch, cfg.q_len, cfg.kv_heads)
    k_new = torch.randn(*shape, cfg.head_dim_k, generator=g).to(torch.bfloat16).to(dev)
    v_new = torch.randn(*shape, cfg.head_dim_v, generator=g).to(torch.bfloat16).to(dev)
    out = torch.empty(case.out_shape(), dtype=torch.bfloat16, device=dev)
    pargs = pa.make_args(case.query, case.key_cache, case.value_cache, case.block_table, case.context_lens, out,
                         case.scale, causal=cfg.causal, num_workers=args.workers)
    pa.append_tensors(pargs, case.query, case.key_cache, case.value_cache, k_new, v_new)
    pos = case.context_lens.long()[:, None] - cfg.q_len + torch.arange(cfg.q_len, device=dev)[None, :]
    phys = case.block_table.long().gather(1, pos.clamp(min=0) // cfg.block_size)
    slots = torch.where(pos >= 0, phys * cfg.block_size + pos % cfg.block_size, -1).to(torch.int32).reshape(-1)
    aargs = kvc.append_args(k_new.reshape(-1, cfg.kv_heads, cfg.head_dim_k),
                            v_new.reshape(-1, cfg.kv_heads, cfg.head_dim_v), slots, case.key_cache, case.value_cache)
    stream = torch.cuda.current_stream(dev)
    sid = stream.cuda_stream
    variants = {
        "one_call": lambda: pa.launch(pargs, dev, sid, key_new=k_new, value_new=v_new),
        "separate": lambda: (kvc.launch_append(aargs, stream=sid), pa.launch(pargs, dev, sid)),
        "decode_only": lambda: pa.launch(pargs, dev, sid),
    }
    # the variants take turns (five rounds); each one's figure is its median round
    runs = {name: [] for name in variants}
    for rnd in range(5):
        for name, call in variants.items():
            for _ in range(args.warmup):
                call()
            torch.cuda.synchronize(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(args.steps):
                call()
            e1.record(stream)
            torch.cuda.synchronize(dev)
            runs[name].append(e0.elapsed_time(e1) / args.steps * 1e3)
            print(f"[bench] round {rnd} {name}: {runs[name][-1]:.2f} us/step", file=sys.stderr, flush=True)
    us = {name: sorted(r)[len(r) // 2] for name, r in runs.items()}
    pa.check_errors(dev)
    # decode bytes plus the appended rows (read from key_new/value_new, written to the caches)
    new_rows = cfg.batch * cfg.q_len * cfg.kv_heads * (cfg.head_dim_k + cfg.head_dim_v) * 2
    nbytes = algorithmic_bytes(case_cpu, out_bytes=2) + 2 * new_rows
    gbs = nbytes / (us["one_call"] * 1e-6) / 1e9
    line = {
        "metric": f"decode with KV append in one call GB/s [{cfg.name}]", "value": round(gbs, 2), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(us["one_call"] / 1e3, 5),
        "us_per_step": round(us["one_call"], 2), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.description}; {cfg.q_len} new token(s) per sequence appended",
                   "parallelism": "single GPU"},
        "us_per_step_separate": round(us["separate"], 2), "us_per_step_decode_only": round(us["decode_only"], 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "pa_decode_kernel (append) + pa_merge_kernel (one row tile per worker; else "
                               "kv_append_kernel first)", "kernel_us": round(us["one_call"], 2),
                     "algorithmic_bytes": nbytes},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_taskgraph(args) -> int:
    """The reference's unfused paged-attention chain on the task-graph backend.

    A step = one run of the reference orchestration (paged_attention_orch.cpp:
    one alloc task + QK, SF, PV, UP per KV block and 16-row head tile), from
    the host-side DAG build (dependency inference, allocation) to the last task
    finishing; eager launches each task as it is submitted, graph launches one
    hipGraph with the inferred edges. The workload is the reference's own
    runnable case (cfg1: B=2, Hq=16, Hkv=1, D=128, BS=128, L=512)."""
    import torch

    from simpler_amd import paged_attention as pa
    from simpler_amd.task_graph import TaskGraph
    from simpler_amd.task_interface import ChipTensor, DataType
    from simpler_amd.workloads import CONFIGS, algorithmic_bytes, make_case

    cfg = CONFIGS[args.config if args.config != DEFAULT_CONFIG else "cfg1_small"]
    dev = torch.device("cuda", 0)
    case_cpu = make_case(cfg)
    case = case_cpu.to(dev, kv_pool=args.kv_layout == "pool")
    out_dtype = torch.bfloat16 if args.out_dtype == "bf16" else torch.float32
    out = torch.zeros(case.out_shape(), dtype=out_dtype, device=dev)
    dt = {torch.bfloat16: DataType.BFLOAT16, torch.float32: DataType.FLOAT32, torch.int32: DataType.INT32}
    tensors = [ChipTensor.make(t.data_ptr(), tuple(t.shape), dt[t.dtype], child_memory=True)
               for t in (case.query, case.key_cache, case.value_cache, case.block_table, case.context_lens, out)]
    stream = torch.cuda.current_stream(dev)
    g = TaskGraph(args.tg_mode, stream=stream.cuda_stream)

    def step():
        g.reset()
        g.orchestrate_paged_attention(tensors, case.scale)
        g.launch()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize(dev)
    ntasks = g.task_count
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize(dev)
    wall = (time.perf_counter() - t0) / args.steps
    ev_ms = start.elapsed_time(end) / args.steps
    ms = max(ev_ms, wall * 1e3)  # the host builds each step's DAG: the wall clock bounds the step
    # the fused kernel on the same inputs, for comparison
    pargs = pa.make_args(case.query, case.key_cache, case.value_cache, case.block_table, case.context_lens, out,
                         case.scale)
    for _ in range(args.warmup):
        pa.launch(pargs, dev, stream.cuda_stream)
    torch.cuda.synchronize(dev)
    f0 = time.perf_counter()
    for _ in range(args.steps):
        pa.launch(pargs, dev, stream.cuda_stream)
    torch.cuda.synchronize(dev)
    fused_us = (time.perf_counter() - f0) / args.steps * 1e6
    g.close()
    nbytes = algorithmic_bytes(case_cpu, out_bytes=2 if args.out_dtype == "bf16" else 4)
    gbs = nbytes / (ms * 1e-3) / 1e9
    cpu = None if args.no_cpu_baseline else cpu_baseline(case_cpu, args)
    others = None
    if cfg.name == DEFAULT_CONFIG and not args.no_other_configs:
        others = other_configs(args, dev, skip=cfg.name)
    line = {
        "metric": f"{METRIC} [{cfg.name}, task graph {args.tg_mode}]",
        "value": round(gbs, 3), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "us_per_step": round(ms * 1e3, 2),
        "event_us_per_step": round(ev_ms * 1e3, 2), "wall_us_per_step": round(wall * 1e6, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: {cfg.description}; reference orchestration, {ntasks} tasks per step",
                   "tasks_per_step": ntasks, "tg_mode": args.tg_mode, "out_dtype": args.out_dtype,
                   "fused_us_per_step": round(fused_us, 2), "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 6), "traffic": None,
                     "kernel": f"task graph step ({ntasks} launches: QK/SF/PV/UP incore kernels)",
                     "kernel_us": round(ms * 1e3, 2), "algorithmic_bytes": nbytes,
                     "note": "launch-bound: per-kernel durations are in profiles/task_graph_cfg1_small.md"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path shards by batch / kv head with no exchange, see DESIGN.md", file=sys.stderr)
        return 2
    if args.op == "taskgraph":
        return bench_taskgraph(args)
    if args.op == "decode_append":
        return bench_decode_append(args)
    if args.op == "decode_prelude":
        return bench_decode_prelude(args)
    if args.op != "decode":
        return bench_kv(args)

    import torch

    from simpler_amd.workloads import CONFIGS, algorithmic_bytes, algorithmic_flops, kv_bytes, make_case

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    cfg = variant_config(CONFIGS[args.config], args)
    print(f"[bench] generating {cfg.name}: {cfg.description}", file=sys.stderr, flush=True)
    case_cpu = make_case(cfg)
    case = case_cpu.to(dev, kv_pool=args.kv_layout == "pool")
    out_dtype = torch.bfloat16 if args.out_dtype == "bf16" else torch.float32
    out = torch.empty(case.out_shape(), dtype=out_dtype, device=dev)

    if args.calibrate_copy_mib > 0:
        src = torch.empty(args.calibrate_copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        del src, dst

    tm = time_decode(case, out, args.workers, dev, args.steps, args.warmup)
    workers, kernel_name = tm["workers"], tm["kernel"]
    kernel_ms, main_ms, wall = tm["step_ms"], tm["main_ms"], tm["wall_s"]

    out_bytes = 2 if out_dtype == torch.bfloat16 else 4
    nbytes = algorithmic_bytes(case_cpu, out_bytes=out_bytes)
    gbs = nbytes / (kernel_ms * 1e-3) / 1e9  # whole step (main + merge kernels)
    main_gbs = nbytes / (main_ms * 1e-3) / 1e9
    flops = algorithmic_flops(case_cpu)
    traffic = None
    tf = Path(args.traffic_file)
    if tf.exists():
        try:
            t = json.loads(tf.read_text()).get(cfg.name)
            traffic = t.get("hbm_bytes_per_launch") if isinstance(t, dict) else None
        except Exception:
            traffic = None

    try:
        api = api_time(case, out, cfg, steps=min(args.steps, 100), warmup=min(args.warmup, 5))
    except Exception as exc:  # reported, not fatal: the kernel figures above stand on their own
        print(f"[bench] API timing skipped: {exc}", file=sys.stderr, flush=True)
        api = None
    cpu = None if args.no_cpu_baseline else cpu_baseline(case_cpu, args)
    others = None
    if cfg.name == DEFAULT_CONFIG and not args.no_other_configs:
        others = other_configs(args, dev, skip=cfg.name)
    line = {
        "metric": METRIC if cfg.name == DEFAULT_CONFIG else f"{METRIC} [{cfg.name}]",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(kernel_ms, 5),
        "us_per_step": round(kernel_ms * 1e3, 2),
        "wall_ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{cfg.name}: {cfg.description}",
            "seed": case_cpu.seed,
            "batch": cfg.batch,
            "q_len": cfg.q_len,
            "num_heads": cfg.num_heads,
            "kv_heads": cfg.kv_heads,
            "head_dim": [cfg.head_dim_k, cfg.head_dim_v],
            "block_size": cfg.block_size,
            "context_tokens": int(case_cpu.context_lens.sum()),
            "out_dtype": args.out_dtype,
            "kv_format": "fp8_e4m3fn + fp32 scale per (block, kv head); bf16 MFMA" if case_cpu.fp8 else "bf16",
            "kv_layout": KV_LAYOUTS[args.kv_layout] if not cfg.mla else "one latent cache; V is its first Dv columns",
            "workers": workers,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(main_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(main_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": kernel_name,
            "kernel_us": round(main_ms * 1e3, 2),
            "algorithmic_bytes": nbytes,
            "kv_bytes": kv_bytes(case_cpu),
            "step_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tflops": round(flops / (main_ms * 1e-3) / 1e12, 3),
            "mfma_frac": round(flops / (main_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        },
        "api": api,
        "cpu_baseline": cpu,
        "other_configs": others,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
