"""Benchmark: minidist's gradient-communication path on one MI355X.

Default workload (the headline metric, cfg1): the per-rank path over
GPT-2-124M's fp32 gradients with W = 8 data-parallel replicas resident in HBM
(rank 0 live, peers' packed contributions staged before timing), 25 MB
buckets in reverse parameter order, loss scale 2^16.  One step is

    DistributedDataParallel.finish_gradient_sync()
        pack + 1/W + W-way SUM + unpack + unscale + found-inf
                         -> mdx_pack_allreduce_unpack_planned (all 148 gradients, 18 buckets,
                            one dispatch: each gradient is read, packed into this rank's
                            contribution row, summed with the 7 peers' rows in rank order;
                            the average is written to the bucket and into every .grad)
    DistributedGradScaler.unscale_(opt) -> the found-inf flag read (the path's one host sync)
    DistributedGradScaler.update()

value = the bytes the step's dispatch actually reads and writes, 44*N for fp32
at W = 8 (gradients read, W-1 peer rows read, this rank's packed row, the
bucket and the gradients written), divided by the median step time -- the
traffic the rocprofv3 FETCH_SIZE / WRITE_SIZE counters measure.  The
configuration's staged accounting, 52*N (pack 8N, W-way 36N, unpack 8N: the
pipeline as three passes, which the fused kernel does not need), is reported
beside it as config.alg_gbs.  The roofline object is for the dominant (and
only) kernel, timed by HIP events recorded on its own stream around every
dispatch of the timed region: ``achieved`` is the configuration's algorithmic
bytes of the step that one dispatch performs (52*N) over its average time,
``hbm_achieved`` the 44*N it actually moves, and ``traffic`` what the PMC
counters read.  ``--no-bucket-average`` measures keep_bucket_average=False
(40*N moved: the average is not copied into the buckets).
The CPU baseline (reference op chain on torch CPU + gloo, W processes) runs
first, before anything touches the GPU.

The other benchmark configurations are parity cases; ``--workload`` measures
them too (one JSON line each, same fields; the CPU baseline for cfg0 and cfg2,
whose replicas fit in host memory):

    cfg0  tiny GPT fp32, W = 4, one 13 MiB bucket      (staged bytes 36*N)
    cfg2  GPT-2-medium fp32, W = 4, 25 MB buckets       (staged bytes 36*N)
    cfg3  FSDP units of GPT-2-XL (48 blocks), W = 8: bf16 gather cast + fp32
          reduce-scatter share per unit                  (26*S per unit)
    cfg4  Llama-7B bf16 grads, W = 8, fp32 buckets (reduce_dtype widening)
                                                         (26*N)
    cfg3-f16, cfg4-f16   the same with fp16 in place of bf16 (the reference
          trainer's --fsdp-param-dtype fp16; fp16 gradients)

    python bench.py [--gpus 1] [--steps 200] [--warmup 10] [--no-cpu-baseline] [--workload cfg1]

Three probes print their own JSON line instead: ``--calibrate-copy`` (the known-size copy that
scales the PMC traffic counters), ``--dispatch-floor`` (cfg3 issued one unit at a time) and
``--op-rates`` (the MAX / MIN / PRODUCT all-reduce beside the SUM kernel).
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import subprocess
import sys
import time
from contextlib import contextmanager
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "distributed-training-framework_amd"))

METRIC = "grad-bucket pipeline HBM GB/s (% of 8 TB/s) GPT-2-124M W=8; ms/step"
HBM_PEAK_GBS = 8000.0
W_CFG1 = 8
CAP_MB = 25.0
LOSS_SCALE = 2.0**16


# The reference's CPU path (oracle/gloo_path.py) for each workload: the configuration, W, and
# the runner's arguments that bound it to about 10-30 s of CPU work.  cfg3 times 2 of its 48
# FSDP units per step and cfg4 (~324 GB of host memory at W = 8) its first decoder layer and
# final norm; both are scaled to the whole step and say so.
CPU_BASELINE = {
    "cfg0": ("tiny", 4, []),
    "cfg1": ("gpt2-small", W_CFG1, []),
    "cfg2": ("gpt2-medium", 4, []),
    "cfg3": (None, 8, ["--fsdp", "--units", "2"]),
    "cfg4": ("llama-7b", 8, ["--layers", "1", "--layers-only", "--scale", str(2.0**12)]),
}


def cpu_baseline(workload: str, steps: int, threads: int) -> dict | None:
    """Time the reference's CPU path (oracle/gloo_path.py) in a child process."""
    config, world, extra = CPU_BASELINE[workload]
    cmd = [sys.executable, "-m", "oracle.gloo_path", "--world", str(world), "--steps", str(steps), "--warmup", "1",
           "--threads", str(threads), *extra]
    if config is not None:
        cmd += ["--config", config]
    res = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=600)
    if res.returncode != 0:
        print(res.stderr[-2000:], file=sys.stderr, flush=True)
        return None
    line = [ln for ln in res.stdout.splitlines() if ln.startswith("{")][-1]
    return json.loads(line)


@contextmanager
def gc_paused():
    """Python's cyclic garbage collector paused over a timed region, as ``timeit`` does: a full
    collection in a process that holds torch takes 10-50 ms and would otherwise land inside one
    step -- or between a HIP event and the dispatch it brackets, inflating that launch's time."""
    was_enabled = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        if was_enabled:
            gc.enable()


def affinity_cpus() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def cgroup_cpus() -> float | None:
    """CPUs the cgroup's CPU quota grants (cgroup v2 ``cpu.max``), or None without a quota."""
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
    except (OSError, ValueError):
        return None
    return None if quota == "max" else int(quota) / int(period)


def granted_cpus() -> int | None:
    """The CPU share the environment grants this job (``OMP_NUM_THREADS``; 16 per GPU on the
    GPU boxes, whatever the machine's own CPU count), or None when unset."""
    try:
        return int(os.environ["OMP_NUM_THREADS"])
    except (KeyError, ValueError):
        return None


def host_cores() -> int:
    """Cores the CPU baseline may keep busy: the affinity set, capped by the cgroup quota and
    by the granted share."""
    cores = affinity_cpus()
    for cap in (cgroup_cpus(), granted_cpus()):
        if cap is not None:
            cores = min(cores, int(cap))
    return max(1, cores)


def host_description() -> dict:
    """The host the CPU baseline ran on: logical CPUs, the affinity set, the CPU model."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:  # pragma: no cover
        pass
    if model is None:
        try:
            out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
            model = next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")), None)
        except (OSError, subprocess.SubprocessError):  # pragma: no cover
            pass
    return {"os_cpu_count": os.cpu_count(), "affinity_cpus": affinity_cpus(), "cgroup_quota_cpus": cgroup_cpus(),
            "granted_cpus_OMP_NUM_THREADS": granted_cpus(),
            "cores_used": host_cores(), "model": model}


def calibrate_copy() -> int:
    import torch

    from minidist import _native

    dev = torch.device("cuda", 0)
    n = 1 << 28  # 1 GiB of fp32 read, 1 GiB written per dispatch
    src = torch.ones(n, device=dev)
    dst = torch.empty(n, device=dev)
    spans = _native.spans_array([(src.data_ptr(), dst.data_ptr(), n)])
    s = torch.cuda.current_stream(dev).cuda_stream
    for _ in range(10):
        _native.pack(spans, _native.MDX_F32, _native.MDX_F32, 1.0, False, s)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "mdx_pack f32 copy", "bytes_read": 4 * n, "bytes_written": 4 * n,
                      "dispatches": 10}))
    return 0


def dispatch_floor() -> int:
    """cfg3 issued per unit (the reference's order): how fast can two stream-ordered dispatches
    per unit -- the unshard cast and the reduce-scatter share -- possibly be?

    Measured with the library entry points FSDP calls per unit (mdx_cast_f32_bf16 and
    mdx_reduce_scatter_share, W = 8, one piece), each sequence enqueued behind a spin kernel and
    timed on the GPU from first to last dispatch:

    * the stream's cost of one dispatch that moves nothing: a one-workgroup cast, 400 back to back;
    * per-dispatch times of the cast and the share at shard sizes from 2^20 to 2^25 elements,
      rotating over up to 48 units (every sequence's data exceeds the 256 MB Infinity Cache), and
      their sustained rates: the slope between the two largest sizes.

    The floor of a unit is then two empty dispatches plus its 26*S bytes at the sustained rates;
    it is compared with the time per unit that 70% of 8 TB/s allows."""
    import torch

    from minidist import _native

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    s_ptr = stream.cuda_stream
    W, n_units, S_cfg3 = 8, 48, 3_842_600

    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    torch.cuda._sleep(1_000_000)
    c1.record()
    torch.cuda.synchronize()
    hold = int(1_000_000 * 20.0 / max(c0.elapsed_time(c1), 1e-3))  # ~20 ms

    def gpu_ms(enqueue, reps: int = 5) -> float:
        """Median GPU time of the enqueued sequence (the host enqueues it while a spin holds the stream)."""
        out = []
        for _ in range(reps + 1):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(hold)
            e0.record()
            enqueue()
            e1.record()
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1))
        return sorted(out[1:])[reps // 2]

    tiny_src = torch.ones(8, device=dev)
    tiny_dst = torch.empty(8, dtype=torch.bfloat16, device=dev)
    n_tiny = 400

    def tiny():
        for _ in range(n_tiny):
            _native.cast_f32_bf16(tiny_src.data_ptr(), tiny_dst.data_ptr(), 8, s_ptr)

    empty_us = gpu_ms(tiny) * 1e3 / n_tiny
    sweep = []
    for S in (1 << 20, 1 << 21, 1 << 22, S_cfg3, 1 << 23, 1 << 24, 1 << 25):
        n = max(4, min(n_units, (4 << 30) // (26 * S)))
        src = torch.randn(n, S, device=dev) * 0.02
        dst = torch.empty(n, S, dtype=torch.bfloat16, device=dev)
        rows = (torch.randn(W, n, S, device=dev) * 1e-3).to(torch.bfloat16)
        out = torch.empty(n, S, device=dev)
        pieces = [_native.pieces_array([(rows[0, k].data_ptr(), 0, S)]) for k in range(n)]
        peers = [[rows[r, k].data_ptr() for r in range(W)] for k in range(n)]

        def casts():
            for k in range(n):
                _native.cast_f32_bf16(src[k].data_ptr(), dst[k].data_ptr(), S, s_ptr)

        def shares():
            for k in range(n):
                _native.reduce_scatter_share(pieces[k], peers[k], 0, _native.MDX_BF16, _native.MDX_F32, True,
                                             out[k].data_ptr(), _native.MDX_F32, False, 1.0, None, s_ptr)

        def units():
            for k in range(n):
                _native.cast_f32_bf16(src[k].data_ptr(), dst[k].data_ptr(), S, s_ptr)
                _native.reduce_scatter_share(pieces[k], peers[k], 0, _native.MDX_BF16, _native.MDX_F32, True,
                                             out[k].data_ptr(), _native.MDX_F32, False, 1.0, None, s_ptr)

        cast_us, share_us, unit_us = (gpu_ms(f) * 1e3 / n for f in (casts, shares, units))
        sweep.append({"S": S, "units": n, "cast_us": round(cast_us, 3), "share_us": round(share_us, 3),
                      "unit_us": round(unit_us, 3), "cast_gbs": round(6 * S / (cast_us * 1e-6) / 1e9, 1),
                      "share_gbs": round(20 * S / (share_us * 1e-6) / 1e9, 1)})
        print(f"[bench] dispatch floor: {sweep[-1]}", file=sys.stderr, flush=True)
        del src, dst, rows, out
        torch.cuda.empty_cache()
    big = sorted(sweep, key=lambda r: r["S"])[-2:]
    dS = big[1]["S"] - big[0]["S"]
    cast_rate = 6 * dS / ((big[1]["cast_us"] - big[0]["cast_us"]) * 1e-6) / 1e9
    share_rate = 20 * dS / ((big[1]["share_us"] - big[0]["share_us"]) * 1e-6) / 1e9
    floor_unit_us = 2 * empty_us + (6 * S_cfg3 / (cast_rate * 1e9) + 20 * S_cfg3 / (share_rate * 1e9)) * 1e6
    bar_unit_us = 26 * S_cfg3 / (0.7 * HBM_PEAK_GBS * 1e9) * 1e6
    measured = next(r for r in sweep if r["S"] == S_cfg3)
    print(json.dumps({
        "probe": "cfg3 per-unit dispatch floor (mdx_cast_f32_bf16 + mdx_reduce_scatter_share, W=8)",
        "empty_dispatch_us": round(empty_us, 3),
        "sustained_cast_gbs": round(cast_rate, 1),
        "sustained_share_gbs": round(share_rate, 1),
        "cfg3_unit_measured_us": measured["unit_us"],
        "cfg3_unit_floor_us": round(floor_unit_us, 3),
        "cfg3_unit_bar_us": round(bar_unit_us, 3),
        "cfg3_step_floor_ms": round(n_units * floor_unit_us * 1e-3, 4),
        "cfg3_step_measured_ms": round(n_units * measured["unit_us"] * 1e-3, 4),
        "cfg3_step_bar_ms": round(n_units * bar_unit_us * 1e-3, 4),
        "sweep": sweep,
    }), flush=True)
    return 0


def op_rates() -> int:
    """The non-SUM all-reduce (mdx_allreduce_op: MAX, MIN, PRODUCT) beside the SUM kernel
    (mdx_allreduce_sum) on the same fp32 rows: W = 8 over 2^26 elements and W = 4 over 2^27, one
    run each, (W+1)*4 bytes per element moved.  HIP events around each dispatch on the stream it
    is launched on, median of 20 after 3 untimed."""
    import torch

    from minidist import _native

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    s_ptr = stream.cuda_stream
    out = {"probe": "mdx_allreduce_op (MAX, MIN, PRODUCT) beside mdx_allreduce_sum, fp32, one run", "cases": []}
    for W, N in ((8, 1 << 26), (4, 1 << 27)):
        rows = torch.randn(W, N, device=dev)
        res = torch.empty(N, device=dev)
        ptrs = [rows[r].data_ptr() for r in range(W)]
        launches = {
            "sum": lambda: _native.allreduce_sum(ptrs, _native.MDX_F32, [0], [N], res.data_ptr(), s_ptr),
            **{name: (lambda op=op: _native.allreduce_op(ptrs, _native.MDX_F32, op, [0], [N], res.data_ptr(), s_ptr))
               for name, op in (("max", _native.MDX_OP_MAX), ("min", _native.MDX_OP_MIN),
                                ("product", _native.MDX_OP_PRODUCT))},
        }
        for name, launch in launches.items():
            for _ in range(3):
                launch()
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(20)]
            for e0, e1 in ev:
                e0.record(stream)
                launch()
                e1.record(stream)
            torch.cuda.synchronize()
            us = sorted(e0.elapsed_time(e1) for e0, e1 in ev)[10] * 1e3
            out["cases"].append({"W": W, "numel": N, "op": name, "us": round(us, 1),
                                 "gbs": round((W + 1) * 4 * N / (us * 1e-6) / 1e9, 1)})
            print(f"[bench] op rates: {out['cases'][-1]}", file=sys.stderr, flush=True)
        del rows, res
        torch.cuda.empty_cache()
    print(json.dumps(out), flush=True)
    return 0


# Committed rocprofv3 FETCH_SIZE + WRITE_SIZE summaries of each workload's dominant kernel: the
# pack fused into the all-reduce + unpack (default), or the two-dispatch pipeline's fused
# all-reduce + unpack (--two-dispatch).
TRAFFIC_FILES = {
    ("cfg0", True): "pack_allreduce_tiny_gpt_w4_traffic.json",
    ("cfg1", True): "pack_allreduce_gpt2_124m_w8_traffic.json",
    ("cfg1", True, "no-bucket-average"): "pack_allreduce_gpt2_124m_w8_no_bucket_average_traffic.json",
    ("cfg2", True): "pack_allreduce_gpt2_medium_w4_traffic.json",
    ("cfg4", True): "pack_allreduce_llama7b_w8_traffic.json",
    ("cfg0", False): "allreduce_unpack_tiny_gpt_w4_traffic.json",
    ("cfg1", False): "allreduce_unpack_gpt2_124m_w8_traffic.json",
    ("cfg2", False): "allreduce_unpack_gpt2_medium_w4_traffic.json",
    ("cfg4", False): "allreduce_wide_llama7b_w8_traffic.json",
    ("cfg3", False): "share_cast_gpt2_xl_fsdp_w8_traffic.json",
    ("cfg3", True): "share_multi_cast_batch_gpt2_xl_fsdp_w8_traffic.json",
}


def measured_traffic(workload: str, fused_pack: bool = False, keep_bucket: bool = True) -> int | None:
    """HBM bytes per dispatch of the dominant kernel, from the committed PMC summary."""
    key = (workload, fused_pack) if keep_bucket else (workload, fused_pack, "no-bucket-average")
    path = ROOT / "profiles" / TRAFFIC_FILES.get(key, "")
    if not path.is_file():
        return None
    return json.loads(path.read_text()).get("bytes_per_launch")


# ---------------------------------------------------------------------------
# DDP workloads (cfg0, cfg1, cfg2, cfg4)
# ---------------------------------------------------------------------------

DDP_WORKLOADS = {
    "cfg1": dict(model="GPT2_SMALL", W=8, grad_scale=1e-3, dtype="f32", reduce_dtype=None,
                 desc="cfg1: GPT-2-124M fp32 grads (148 tensors, N=124,439,808), W=8 replicas on one GPU, "
                      "25 MB buckets in reverse parameter order (18 buckets), loss scale 2^16"),
    "cfg0": dict(model="TINY_GPT", W=4, grad_scale=1e-2, dtype="f32", reduce_dtype=None,
                 desc="cfg0: tiny GPT (4L, h256, V1024, ctx128) fp32 grads (52 tensors, N=3,454,464), W=4, "
                      "25 MB cap (one bucket), loss scale 2^16"),
    "cfg2": dict(model="GPT2_MEDIUM", W=4, grad_scale=1e-3, dtype="f32", reduce_dtype=None,
                 desc="cfg2: GPT-2-medium fp32 grads (292 tensors, N=354,823,168), W=4, 25 MB buckets "
                      "(74 buckets), loss scale 2^16"),
    "cfg4": dict(model="LLAMA_7B", W=8, grad_scale=1e-3, dtype="bf16", reduce_dtype="f32",
                 desc="cfg4: Llama-7B bf16 grads (291 tensors, N=6,738,415,616), W=8 bf16 contributions "
                      "(~108 GB) summed in fp32 into fp32 25 MB buckets (291), unpacked to bf16, loss scale 2^12"),
    "cfg4-f16": dict(model="LLAMA_7B", W=8, grad_scale=1e-3, dtype="f16", reduce_dtype="f32",
                     desc="cfg4-f16: Llama-7B fp16 grads (291 tensors, N=6,738,415,616), W=8 fp16 contributions "
                          "(~108 GB) summed in fp32 into fp32 25 MB buckets (291), unpacked to fp16, loss scale "
                          "2^12"),
}
TORCH_DTYPE_NAMES = {"f32": "float32", "bf16": "bfloat16", "f16": "float16"}
KERNEL_TYPE_NAMES = {"f32": "float", "bf16": "bf16", "f16": "f16"}


def bench_ddp(name: str, args) -> dict:
    import torch

    from minidist import DDP, DistributedGradScaler, ResidentGroup
    from minidist import workloads as wl

    cfg = DDP_WORKLOADS[name]
    W = cfg["W"]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if cfg["model"] == "LLAMA_7B":
        specs = wl.llama_specs(**wl.LLAMA_7B, dtype=getattr(torch, TORCH_DTYPE_NAMES[cfg["dtype"]]))
        loss_scale = 2.0**12
    else:
        specs = wl.gpt_specs(**getattr(wl, cfg["model"]))
        loss_scale = LOSS_SCALE
    N = wl.total_numel(specs)
    reduce_dtype = torch.float32 if cfg["reduce_dtype"] == "f32" else None

    model = wl.SpecModule(specs, dev)
    scaler = DistributedGradScaler(init_scale=loss_scale)
    group = ResidentGroup(W, 0, dev)
    # --dropin: DDP built exactly as the reference's callers build it (no grad_scaler=, no
    # reduce_dtype=), so the scaler's unscale_ makes its own pass over every gradient.
    fused_unscale = not args.dropin
    if args.dropin and reduce_dtype is not None:
        raise SystemExit("--dropin covers the same-dtype workloads (cfg0, cfg1, cfg2)")
    # --no-bucket-average: the fused launch leaves the bucket out (keep_bucket_average=False)
    keep_bucket = not args.no_bucket_average
    ddp = DDP(model, process_group=group, bucket_cap_mb=CAP_MB, grad_scaler=scaler if fused_unscale else None,
              reduce_dtype=reduce_dtype, capture_graphs=args.graphs, keep_bucket_average=keep_bucket)
    # --two-dispatch: pack, then the fused all-reduce + unpack (the pipeline before the pack was fused in)
    ddp._fuse_pack = not (args.two_dispatch or args.staged)
    fused_pack = ddp._fuse_pack
    ddp.allocate_buckets()
    gen = torch.Generator(device=dev).manual_seed(1234)
    scale = cfg["grad_scale"] * loss_scale
    for p in model.parameters():
        g = (torch.randn(p.shape, device=dev, generator=gen) * scale).to(p.dtype)
        if args.misaligned:
            # the gradient is a view one element into its own allocation: its address is 4 bytes
            # (fp32) or 2 bytes (16-bit) past the 16-byte alignment the bucket rows have
            holder = torch.empty(p.numel() + 1, dtype=p.dtype, device=dev)
            holder[1:].copy_(g.reshape(-1))
            g = holder[1:].view(p.shape)
        p.grad = g
    n_buckets = len(ddp._buckets)
    for b in range(n_buckets):
        rows = ddp.bucket_replicas(b)
        wire_dtype, prescaled = ddp.bucket_wire_format(b)
        for r in range(1, W):
            x = torch.randn(rows[r].shape, device=dev, generator=gen) * (scale / W if prescaled else scale)
            rows[r].copy_(x.to(wire_dtype))
            del x
        if (b + 1) % 32 == 0 or b + 1 == n_buckets:  # staging cfg4's 108 GB takes a while under a profiler
            print(f"[bench] staged the peers' contributions of {b + 1}/{n_buckets} buckets", file=sys.stderr,
                  flush=True)

    class _Opt:  # the scaler only reads param_groups
        param_groups = [{"params": list(model.parameters())}]

    opt = _Opt()

    # Dominant kernel timing: HIP events around the fused W-way reduction
    # dispatch, recorded on the stream it is launched on (the caller's: these
    # workloads use no communication stream).  The stream object and the event
    # pairs are made before the timed region, so each dispatch adds only its two
    # event records to the host's work.
    red_events: list = []
    timing: dict = {"on": False, "stream": None, "pool": []}
    hook_name = "pack_all_reduce_unpack_planned" if fused_pack else "all_reduce_unpack_planned"
    orig = getattr(ResidentGroup, hook_name)

    def event_pair():
        if timing["pool"]:
            return timing["pool"].pop()
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed_all_reduce(self, *a, **k):
        if not timing["on"]:
            return orig(self, *a, **k)
        s = timing["stream"]
        e0, e1 = event_pair()
        e0.record(s)
        work = orig(self, *a, **k)
        e1.record(s)
        red_events.append((e0, e1))
        return work

    # With --graphs the dispatch is replayed from a captured graph, where no host code runs
    # around it: the events then come from a separate pass of eager steps.
    setattr(ResidentGroup, hook_name, timed_all_reduce)

    def staged_sum() -> None:
        """--staged: the W-way sum of the contribution rows into the buckets (one mdx_allreduce_sum)."""
        from minidist import _native

        wire, flat = ddp._arenas[(ddp._buckets[0].wire_dtype, ddp._buckets[0].dtype, 0)]
        rows = group.replicas(wire)
        _native.allreduce_sum(
            [r.data_ptr() for r in rows], _native.dtype_code(wire.dtype), [b.arena_offset for b in ddp._buckets],
            [b.numel for b in ddp._buckets], flat.data_ptr(), torch.cuda.current_stream(dev).cuda_stream,
        )

    def timed_sum():
        """--staged: the W-way sum dispatch, with HIP events like the fused reduction's."""
        if not timing["on"]:
            return staged_sum()
        s = timing["stream"]
        e0, e1 = event_pair()
        e0.record(s)
        staged_sum()
        e1.record(s)
        red_events.append((e0, e1))

    def step() -> bool:
        ddp.finish_gradient_sync()
        found = scaler.unscale_(opt)
        scaler.update()
        return found

    if args.staged:
        # The reference's three stages as separate dispatches over the same data: pack (x 1/W) into the
        # buckets, the W-way sum written back into this rank's buckets (one mdx_allreduce_sum), then
        # unpack from the buckets into the gradients with the scaler's unscale + found-inf.
        if cfg["reduce_dtype"] is not None:
            raise SystemExit("--staged covers the same-dtype workloads (cfg0, cfg1, cfg2)")
        if len({(b.wire_dtype, b.dtype) for b in ddp._buckets}) != 1:
            raise SystemExit("--staged needs every bucket in one dtype")
        plan = ddp._plan(0, len(ddp._buckets))

        def step() -> bool:  # noqa: F811 - the staged variant of the step above
            plan.refresh()
            plan.pack(1.0 / W)
            inv_scale, flag = scaler._begin_fused_unscale(dev, plan.param_ids)
            timed_sum()
            plan.unpack(inv_scale, flag)
            found = scaler.unscale_(opt)
            scaler.update()
            return found

    steps = args.steps if not name.startswith("cfg4") else min(args.steps, 20)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Timed region, with HIP events around every fused reduction dispatch on its
    # own stream (two event records per step cost ~0.8% of a cfg1 step).  Every
    # step ends in the scaler's flag read (a host synchronisation), so the host
    # clock between step ends is each step's own time.
    timing["stream"] = torch.cuda.current_stream(dev)
    timing["pool"] = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                      for _ in range(steps + (min(steps, 50) if args.graphs else 0))]
    with gc_paused():
        timing["on"] = not args.graphs
        t0 = time.perf_counter()
        found_any = False
        ends = []
        for _ in range(steps):
            found_any |= step()
            ends.append(time.perf_counter())
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        step_ms = sorted((b - a) * 1e3 for a, b in zip([t0] + ends[:-1], ends))
        if args.graphs:
            ddp._capture_graphs = False
            timing["on"] = True
            for _ in range(min(steps, 50)):
                step()
            torch.cuda.synchronize()
        timing["on"] = False
    setattr(ResidentGroup, hook_name, orig)

    b0 = ddp._buckets[0]
    s_w = b0.wire.element_size()
    s_b = b0.buffer.element_size()
    s_g = b0.params[0].element_size()
    ms_per_step = step_ms[len(step_ms) // 2]  # median of the timed steps
    mean_ms = elapsed / steps * 1e3
    # Fused pack: the gradient read, W-1 peer rows read, this rank's packed row, the bucket and
    # the gradient written -- one dispatch.  Two-dispatch pipeline: the pack (gradient read, row
    # written), then W rows read, bucket and gradient written.
    red_bytes = (N * (2 * s_g + W * s_w + (s_b if keep_bucket else 0)) if fused_pack
                 else N * (W * s_w + s_b + s_g))
    if b0.widening:
        alg_bytes = N * (W * s_w + s_b + s_b + s_g)  # the configuration's accounting (26*N)
        hbm_bytes = red_bytes if fused_pack else N * (2 * s_g) + red_bytes
        alg_note = "W*N*2 + N*4 + N*4 + N*2 = 26*N (bf16 contributions, fp32 bucket, bf16 grads)"
    else:
        alg_bytes = N * (2 * s_g + (W + 3) * s_b)  # pack + W-way + unpack, staged
        hbm_bytes = red_bytes if fused_pack else N * (s_g + s_b) + red_bytes
        alg_note = f"staged pack + W-way + unpack: N*(2*s_g + (W+3)*s_b) = {2 * s_g + (W + 3) * s_b}*N"
    if not fused_unscale:
        hbm_bytes += N * 2 * s_g  # unscale_'s own pass: every gradient read and written again
    # The headline is the bytes the step's kernels actually move (what the PMC
    # counters read); the configuration's staged accounting is reported beside it.
    value = hbm_bytes / (ms_per_step * 1e-3) / 1e9
    alg_gbs = alg_bytes / (ms_per_step * 1e-3) / 1e9
    red_ms = sorted(e0.elapsed_time(e1) for e0, e1 in red_events)
    red_avg_ms = sum(red_ms) / len(red_ms)
    t16 = KERNEL_TYPE_NAMES[cfg["dtype"]]
    if fused_pack:
        kname = (f"allreduce_pack_kernel_dev<{t16}, float, {W}>" if b0.widening
                 else f"allreduce_pack_kernel_dev<float, float, {W}>")
    else:
        kname = (f"allreduce_wide_kernel_dev<{t16}, float, {t16}, {W}>" if b0.widening
                 else f"allreduce_unpack_kernel_dev<float, float, {W}>")
    if args.staged:
        red_bytes = N * (W + 1) * s_b  # W buckets read, the sum written
        hbm_bytes = N * (s_g + s_b) + red_bytes + N * (s_b + s_g)
        kname = f"allreduce_kernel<float, float, {W}, false> (mdx_allreduce_sum)"
    red_gbs = red_bytes / (red_avg_ms * 1e-3) / 1e9
    # The roofline's algorithmic bytes per launch: when the one dispatch is the whole step (the
    # pack fused in), the configuration's accounting of the step (52*N for fp32 at W = 8, 26*N
    # for cfg4); otherwise what the timed kernel itself must move.
    roof_bytes = alg_bytes if fused_pack and not args.staged else red_bytes
    roof_gbs = roof_bytes / (red_avg_ms * 1e-3) / 1e9

    traffic = None if args.staged else measured_traffic(name, fused_pack, keep_bucket)

    return {
        "metric": (METRIC if name == "cfg1" else f"grad-bucket pipeline HBM GB/s (% of 8 TB/s) {name}; ms/step")
                  + "".join(f" [{tag}]" for tag, on in (("staged", args.staged), ("two-dispatch", args.two_dispatch),
                                                        ("graphs", args.graphs), ("dropin", args.dropin),
                                                        ("misaligned", args.misaligned),
                                                        ("no-bucket-average", not keep_bucket)) if on),
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": f"synthetic (seeded randn grads x {cfg['grad_scale']:g} x loss scale; peers' contributions staged "
                "in HBM)",
        "config": {
            "workload": cfg["desc"],
            "world": W,
            "numel": N,
            "buckets": len(ddp._buckets),
            "value_bytes": "hbm_bytes_per_step: the bytes the step's dispatches read and write (PMC-backed)",
            "hbm_bytes_per_step": hbm_bytes,
            "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
            "alg_bytes_per_step": alg_bytes,
            "alg_bytes_formula": alg_note,
            "alg_gbs": round(alg_gbs, 2),
            "alg_frac_of_peak": round(alg_gbs / HBM_PEAK_GBS, 4),
            "ms_per_step_stat": f"median of {steps} timed steps (Python's garbage collector paused)",
            "ms_per_step_mean": round(mean_ms, 4),
            "ms_per_step_min": round(step_ms[0], 4),
            # a full 25 MiB bucket's share of the measured step (one bucket alone would sit in the
            # 256 MB Infinity Cache, so it is not timed on its own)
            "us_per_25MiB_bucket": round(ms_per_step * 1e3 * (25 * 2**20 // b0.buffer.element_size()) / N, 2),
            "found_inf": bool(found_any),
            "launch": "hip graph replay (capture_graphs=True)" if args.graphs else "eager dispatches",
            "api": "drop-in: DDP(module, process_group, bucket_cap_mb) then scaler.unscale_(opt) as its own pass "
                   "(the reference's call sequence)" if args.dropin
                   else "DDP(..., grad_scaler=scaler): unscale + found-inf fused into the unpack",
            "gradients": "views one element into their allocations (no common 16-byte alignment with the rows)"
                         if args.misaligned else "tensors of their own (16-byte aligned)",
            "pipeline": "staged: pack, W-way sum, unpack (three dispatches)" if args.staged
                        else "pack + fused W-way sum / unpack / unscale (two dispatches)" if not fused_pack
                        else "pack fused into the W-way sum / unpack / unscale (one dispatch)",
            "bucket_average": "written into every bucket (the reference's bucket state)" if keep_bucket
                              else "not written (keep_bucket_average=False)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kname if args.staged else
                      f"{kname} ({'mdx_pack_allreduce_unpack_planned' if fused_pack else 'mdx_allreduce_unpack_planned'}"
                      f", all {len(ddp._buckets)} buckets in one dispatch)",
            "achieved": round(roof_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(roof_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": roof_bytes,
            "bytes_formula": alg_note if roof_bytes == alg_bytes else "the timed kernel's own reads and writes",
            "hbm_bytes_per_launch": red_bytes,
            "hbm_achieved": round(red_gbs, 2),
            "hbm_frac": round(red_gbs / HBM_PEAK_GBS, 4),
            "avg_launch_ms": round(red_avg_ms, 4),
        },
        "cpu_baseline": None,
    }


# ---------------------------------------------------------------------------
# FSDP workload (cfg3)
# ---------------------------------------------------------------------------


def bench_fsdp(args, param_dtype_name: str = "bf16") -> dict:
    """48 FSDP units of GPT-2-XL blocks, W = 8: per unit the fp32 -> bf16 (or
    fp16) gather cast into this rank's slot and the reduce-scatter share of 8
    16-bit full-size contributions into the fp32 shard gradient.

    The two kernels of a unit take ~20 us together, far less than the Python
    around them, so the step's dispatches are enqueued behind a spin kernel and
    the step is timed on the GPU (first to last dispatch, HIP events): the
    number is the dispatch sequence's own throughput, as when FSDP's launches
    overlap forward/backward compute.

    ``--fsdp-mode`` picks how the 48 units' work is issued:

    * ``batched`` (default): as FSDP issues it for units that are ready
      together -- the gather casts of all units in one dispatch (the batched
      unshard of ``summon_full_params``, without the peers' gather copies,
      which are the all-gather's own traffic) and the reduce-scatter shares
      of all units in one multi-unit dispatch (``finish_gradient_sync``
      flushing units whose gradients are ready);
    * ``per-unit``: per unit its cast and its share, as the forward and
      backward hooks issue them, on the caller's stream;
    * ``per-unit-streams``: the same with ``comm_streams=True`` (casts on the
      gather stream, shares on the reduce stream);
    * ``unit-batch``: as the hooks issue it with ``unit_batch=K``
      (``--unit-batch``, default 8): the forward gathers K units per batched
      unshard (cast dispatch), the backward holds reduce-scatters until K
      units are ready and sends them as one multi-unit share, last units
      first.

    The per-kernel times of the roofline come from a separate pass with the
    step's dispatches on one stream and HIP events around each."""
    import torch
    from torch import nn

    from minidist import FSDP, MixedPrecisionPolicy, ResidentGroup
    from minidist import workloads as wl

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    W, n_units = 8, wl.GPT2_XL["n_layer"]
    specs = wl.gpt_block_specs(0, wl.GPT2_XL["n_embd"])

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.ps = nn.ParameterList([nn.Parameter(torch.empty(s.shape, device=dev)) for s in specs])

    class Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = nn.ModuleList([Block() for _ in range(n_units)])

    gen = torch.Generator(device=dev).manual_seed(33)
    model = Model()
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, device=dev, generator=gen) * 0.02)
    name = "cfg3" if param_dtype_name == "bf16" else f"cfg3-{param_dtype_name}"
    pdt = getattr(torch, TORCH_DTYPE_NAMES[param_dtype_name])
    policy = MixedPrecisionPolicy(param_dtype=pdt, reduce_dtype=torch.float32)
    mode = args.fsdp_mode
    K = args.unit_batch
    streams = mode == "per-unit-streams"
    # reshard_after_forward=False: the gather buffers stay allocated (the step re-casts into them),
    # and finish_gradient_sync's flush does not free them
    fsdp = FSDP(model, unit_types=(Block,), process_group=ResidentGroup(W, 0, dev), mixed_precision=policy,
                reshard_after_forward=False, comm_streams=streams)
    units = fsdp._units
    assert len(units) == n_units
    own_grads = []
    for u in units:
        u.unshard()  # keep the gather buffers allocated: the step re-casts into them
        peers = u.peer_grad_contributions()
        for r in range(1, W):
            peers[r].copy_((torch.randn(u.padded_numel, device=dev, generator=gen) * 1e-3).to(pdt))
        own_grads.append([(torch.randn(p.shape, device=dev, generator=gen) * 1e-3).to(pdt)
                          for p in u.params])
    S = units[0].shard_numel

    def timed(events, kind, work):
        """``work()``, between two events appended to ``events[kind]`` when events are taken."""
        if events is None:
            work()
            return
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        work()
        e1.record()
        events[kind].append((e0, e1))

    def give_grads(group):
        for u in group:
            i = units.index(u)
            u.flat_shard.grad = None  # the shard gradient is set, not accumulated
            for p, g in zip(u.params, own_grads[i], strict=True):
                p.grad = g

    def step(events=None):
        if mode == "batched":
            timed(events, "cast", lambda: fsdp._cast_own_slots(units))
            give_grads(units)
            # every unit holds gradients: one multi-unit share
            timed(events, "share", fsdp.finish_gradient_sync)
            return
        if mode == "unit-batch":
            for g0 in range(0, n_units, K):  # forward: K units per batched unshard
                timed(events, "cast", lambda g0=g0: fsdp._cast_own_slots(units[g0 : g0 + K]))
            for g1 in range(n_units, 0, -K):  # backward: K held reduce-scatters at a time, last units first
                group = units[max(0, g1 - K) : g1][::-1]
                give_grads(group)
                fsdp._held_reductions = list(group)
                timed(events, "share", fsdp._reduce_held)
            return
        for u in units:
            timed(events, "cast", u._cast_into_own_slot)
            give_grads([u])
            timed(events, "share", u.reduce_scatter_grads)
        fsdp.finish_gradient_sync()  # with side streams: the caller's stream joins both

    def one_stream(on: bool) -> None:
        """Route the units' work to the caller's stream (the per-kernel event pass) or back."""
        for u in units:
            u.streams = None if on else fsdp._streams

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Spin-kernel length that holds the stream ~30 ms (calibrated: its clock rate is the device's).
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    torch.cuda._sleep(1_000_000)
    c1.record()
    torch.cuda.synchronize()
    hold_cycles = int(1_000_000 * 30.0 / max(c0.elapsed_time(c1), 1e-3))
    steps = min(args.steps, 20)
    # Step pass: one event before the first dispatch and one after the last
    # (an event between two dispatches costs a few microseconds of its own).
    per_step = []
    cast_ms, share_ms = [], []
    with gc_paused():
        for _ in range(steps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(hold_cycles)  # hold the stream while the host enqueues the whole step
            e0.record()
            step()
            e1.record()
            torch.cuda.synchronize()
            per_step.append(e0.elapsed_time(e1))
        # Kernel pass: the same steps on one stream with events around every dispatch.
        one_stream(True)
        for _ in range(min(steps, 5)):
            ev = {"cast": [], "share": []}
            torch.cuda._sleep(hold_cycles)
            step(ev)
            torch.cuda.synchronize()
            cast_ms += [e0.elapsed_time(e1) for e0, e1 in ev["cast"]]
            share_ms += [e0.elapsed_time(e1) for e0, e1 in ev["share"]]
        one_stream(False)
    # units one timed launch covers (unit-batch: the mean over its groups)
    per_launch = {"batched": n_units, "unit-batch": n_units / -(-n_units // K)}.get(mode, 1)
    ms_per_step = sorted(per_step)[len(per_step) // 2]
    alg_bytes = n_units * 26 * S  # cast 6S (fp32 read, bf16 write) + share 20S (8 bf16 reads, fp32 write)
    value = alg_bytes / (ms_per_step * 1e-3) / 1e9
    share_avg = sum(share_ms) / len(share_ms)
    cast_avg = sum(cast_ms) / len(cast_ms)
    share_gbs = 20 * S * per_launch / (share_avg * 1e-3) / 1e9
    return {
        "metric": f"FSDP unit gather-cast + reduce-scatter share HBM GB/s (% of 8 TB/s) {name}; ms/step",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{param_dtype_name}->f32",
        "data": f"synthetic (master randn x 0.02, {param_dtype_name} grads randn x 1e-3; peers' contributions staged "
                "in HBM)",
        "config": {
            "workload": f"{name}: 48 FSDP units of GPT-2-XL blocks (12 tensors, 30,740,800 elements each, shard "
                        f"S=3,842,600), W=8, param {param_dtype_name} / reduce fp32; per unit the gather cast and "
                        "the reduce-scatter share ("
                        + ("mdx_pack over the 48 units' master shards + mdx_reduce_scatter_share_multi_planned"
                           if mode == "batched" else
                           f"mdx_pack over {K} units' master shards + mdx_reduce_scatter_share_multi over {K} units"
                           if mode == "unit-batch" else
                           ("mdx_cast_f32_bf16" if param_dtype_name == "bf16" else "mdx_pack, fp32 -> fp16")
                           + " + mdx_reduce_scatter_share per unit")
                        + "); GPU time of the step's dispatches",
            "issue": {"batched": "all units' casts in one dispatch, all units' shares in one multi-unit dispatch "
                                 "(finish_gradient_sync's flush)",
                      "per-unit": "per unit a cast and a share dispatch (the hooks' order), one stream",
                      "per-unit-streams": "per unit a cast on the gather stream and a share on the reduce stream "
                                          "(comm_streams=True)",
                      "unit-batch": f"unit_batch={K}: a cast dispatch per {K} units in forward order, a multi-unit "
                                    f"share per {K} units in backward order"}[mode],
            "ms_per_step_stat": f"median of {steps} steps (Python's garbage collector paused)",
            "world": W,
            "units": n_units,
            "shard_numel": S,
            "alg_bytes_per_step": alg_bytes,
            "alg_bytes_formula": "per unit 6*S (cast) + 20*S (share: W*S*2 read, S*4 written)",
            "cast_avg_ms": round(cast_avg, 5),
            "cast_gbs": round(6 * S * per_launch / (cast_avg * 1e-3) / 1e9, 1),
            "alg_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": (f"share_kernel_dev<{KERNEL_TYPE_NAMES[param_dtype_name]}, float, float, 8> "
                       "(mdx_reduce_scatter_share_multi_planned: 48 units' shares, ~150 pieces, one dispatch)")
                      if mode == "batched" else
                      (f"share_kernel<{KERNEL_TYPE_NAMES[param_dtype_name]}, float, float, 8> "
                       f"(mdx_reduce_scatter_share_multi: {K} units' shares, {3 * K} pieces, one dispatch)")
                      if mode == "unit-batch" else
                      (f"share_kernel_few<{KERNEL_TYPE_NAMES[param_dtype_name]}, float, float, 8> "
                       "(mdx_reduce_scatter_share; rank 0's shard is 3 parameter pieces)"),
            "achieved": round(share_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(share_gbs / HBM_PEAK_GBS, 4),
            "traffic": (measured_traffic(name, mode == "batched") if mode != "unit-batch" else None),
            "bytes_per_launch": 20 * S * per_launch,
            "avg_launch_ms": round(share_avg, 5),
        },
        "cpu_baseline": None,
    }


# ---------------------------------------------------------------------------
# Overlap with backward (cfg1 parameters, a real backward)
# ---------------------------------------------------------------------------


def bench_overlap(args) -> dict:
    """The cfg1 path inside a real training step: forward + backward of a model
    with GPT-2-124M's 148 parameters, DDP over a W = 8 ResidentGroup with the
    fused unscale, the scaler's flag read and update.

    The model is GPT-2-124M's parameter set driven by an attention-free stack
    (embedding + positions; per block ln1 -> qkv -> gelu, three thirds summed
    -> proj, ln2 -> fc -> gelu -> proj, both residual; ln_f; tied head and
    cross-entropy), fp32 throughout, so every product is a plain 2-D matmul.
    Backward produces the gradients in reverse order and DDP's hooks launch
    each bucket run as it completes.  Three timings of the same step:

        compute  forward + backward under no_sync (no gradient path at all),
                 then a stream sync in place of the scaler's flag read
        serial   DDP with its kernels on the compute stream
        overlap  DDP with comm_stream=True (dedicated stream, waits on events)

    exposed = step - compute is the part of the gradient path backward does not hide."""
    import torch
    import torch.nn.functional as F

    from minidist import DDP, DistributedGradScaler, ResidentGroup
    from minidist import workloads as wl

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    W, B, S = W_CFG1, args.overlap_batch, 1024
    cfg = wl.GPT2_SMALL
    h, L, V = cfg["n_embd"], cfg["n_layer"], cfg["vocab"]
    specs = wl.gpt_specs(**cfg)
    gen = torch.Generator(device=dev).manual_seed(7)
    ids = torch.randint(0, V, (B * S,), device=dev, generator=gen)
    tgt = torch.randint(0, V, (B * S,), device=dev, generator=gen)
    pos = torch.arange(S, device=dev).repeat(B)

    def make_model():
        m = wl.SpecModule(specs, dev)
        g = torch.Generator(device=dev).manual_seed(11)
        with torch.no_grad():
            for sp, p in zip(specs, m.parameters(), strict=True):
                if sp.name.endswith(("ln1.weight", "ln2.weight", "ln_f.weight")):
                    p.fill_(1.0)
                elif len(sp.shape) == 1:
                    p.zero_()
                else:
                    p.copy_(torch.randn(sp.shape, device=dev, generator=g) * 0.02)
        return m

    def forward(m) -> torch.Tensor:
        P = dict(zip((sp.name for sp in specs), m.parameters(), strict=True))
        x = P["embedding.wte.weight"][ids] + P["embedding.wpe"][pos]
        for i in range(L):
            q = f"blocks.{i}."
            a = F.layer_norm(x, (h,), P[q + "ln1.weight"], P[q + "ln1.bias"])
            y = F.gelu(F.linear(a, P[q + "attn.qkv.weight"], P[q + "attn.qkv.bias"]), approximate="tanh")
            y = y[:, :h] + y[:, h : 2 * h] + y[:, 2 * h :]
            x = x + F.linear(y, P[q + "attn.proj.weight"], P[q + "attn.proj.bias"])
            a = F.layer_norm(x, (h,), P[q + "ln2.weight"], P[q + "ln2.bias"])
            y = F.gelu(F.linear(a, P[q + "mlp.fc.weight"], P[q + "mlp.fc.bias"]), approximate="tanh")
            x = x + F.linear(y, P[q + "mlp.proj.weight"], P[q + "mlp.proj.bias"])
        x = F.layer_norm(x, (h,), P["lm_head.ln_f.weight"], P["lm_head.ln_f.bias"])
        return F.cross_entropy(F.linear(x, P["embedding.wte.weight"]), tgt)

    def setup(comm_stream):
        m = make_model()
        scaler = DistributedGradScaler(init_scale=LOSS_SCALE)
        ddp = DDP(m, process_group=ResidentGroup(W, 0, dev), bucket_cap_mb=CAP_MB, grad_scaler=scaler,
                  comm_stream=comm_stream)
        ddp.allocate_buckets()
        for b in range(len(ddp._buckets)):
            rows = ddp.bucket_replicas(b)
            for r in range(1, W):
                rows[r].copy_(torch.randn(rows[r].shape, device=dev, generator=gen) * (1e-3 * LOSS_SCALE / W))

        class _Opt:
            param_groups = [{"params": list(m.parameters())}]

        return m, ddp, scaler, _Opt()

    def timed(step, steps):
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        with gc_paused():
            t0 = time.perf_counter()
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) / steps * 1e3

    steps = min(args.steps, 30)
    results = {}
    modes = [m for m in ("compute", "serial", "overlap") if m in args.overlap_modes.split(",")]
    for mode in modes:
        m, ddp, scaler, opt = setup(mode == "overlap")

        def step(m=m, ddp=ddp, scaler=scaler, opt=opt, mode=mode):
            for p in m.parameters():
                p.grad = None
            if mode == "compute":
                with ddp.no_sync():
                    forward(m).backward()
                # the same per-step host sync as the scaler's flag read in the other modes
                torch.cuda.current_stream(dev).synchronize()
                return
            scaler.scale_loss(forward(m)).backward()
            scaler.unscale_(opt)
            scaler.update()

        results[mode] = timed(step, steps)
        del m, ddp, scaler, opt
        torch.cuda.empty_cache()
    if len(modes) < 3:  # a partial run (e.g. under a profiler): the timings only
        print(json.dumps({"workload": "cfg1-overlap", "ms_per_step": results}), flush=True)
        sys.exit(0)
    comp = results["compute"]
    N = wl.total_numel(specs)
    return {
        "metric": "GPT-2-124M-parameter training step with the W=8 gradient path overlapped with backward; ms/step",
        "value": round(results["overlap"], 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(results["overlap"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic (random token ids, {B}x{S} tokens per step; peers' contributions staged in HBM)",
        "config": {
            "workload": "cfg1 parameters (148 tensors, N=124,439,808) on an attention-free GPT-2-124M-shaped fp32 "
                        "stack; DDP over ResidentGroup(W=8), 25 MB buckets, fused unscale, loss scale 2^16",
            "tokens_per_step": B * S,
            "numel": N,
            "compute_ms": round(comp, 4),
            "serial_ms": round(results["serial"], 4),
            "overlap_ms": round(results["overlap"], 4),
            "exposed_serial_ms": round(results["serial"] - comp, 4),
            "exposed_overlap_ms": round(results["overlap"] - comp, 4),
        },
        "roofline": None,
        "cpu_baseline": None,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="cfg1",
                    choices=["cfg0", "cfg1", "cfg2", "cfg3", "cfg4", "cfg3-f16", "cfg4-f16", "cfg1-overlap"])
    ap.add_argument("--overlap-batch", type=int, default=2, help="sequences of 1024 tokens per cfg1-overlap step")
    ap.add_argument("--overlap-modes", default="compute,serial,overlap",
                    help="cfg1-overlap modes to run (all three for the JSON line)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--staged", action="store_true",
                    help="DDP workloads: time the reference's staged pipeline (pack, W-way sum, unpack as three "
                         "dispatches) instead of the fused one, for comparison")
    ap.add_argument("--two-dispatch", action="store_true",
                    help="DDP workloads: pack, then the fused all-reduce + unpack, as two dispatches (the pipeline "
                         "before the pack was fused into the reduction), for comparison")
    ap.add_argument("--graphs", action="store_true",
                    help="DDP workloads: replay each step's launches from a captured HIP graph (capture_graphs=True)")
    ap.add_argument("--dropin", action="store_true",
                    help="DDP workloads: the reference's call sequence unchanged (no grad_scaler=): the scaler's "
                         "unscale_ runs its own pass over the gradients")
    ap.add_argument("--no-bucket-average", action="store_true",
                    help="DDP workloads: keep_bucket_average=False (the fused launch does not copy the average "
                         "into the buckets)")
    ap.add_argument("--misaligned", action="store_true",
                    help="DDP workloads: every gradient a view one element into its allocation")
    ap.add_argument("--unit-batch", type=int, default=8,
                    help="cfg3 --fsdp-mode unit-batch: units per batched gather and per multi-unit share")
    ap.add_argument("--fsdp-mode", default="batched",
                    choices=["batched", "per-unit", "per-unit-streams", "unit-batch"],
                    help="cfg3: how the units' casts and shares are issued (see bench_fsdp)")
    ap.add_argument("--cpu-steps", type=int, default=20)
    ap.add_argument(
        "--calibrate-copy", action="store_true",
        help="only run a plain 1 GiB fp32 copy (mdx_pack, scale 1) 10 times: the known-size "
             "reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings",
    )
    ap.add_argument(
        "--dispatch-floor", action="store_true",
        help="only measure the per-unit floor of cfg3 issued in the reference's order (two stream-ordered "
             "dispatches per unit; see dispatch_floor)",
    )
    ap.add_argument(
        "--op-rates", action="store_true",
        help="only time the non-SUM all-reduce kernel (MAX, MIN, PRODUCT) beside the SUM kernel (see op_rates)",
    )
    args = ap.parse_args()
    if args.calibrate_copy:
        return calibrate_copy()
    if args.dispatch_floor:
        return dispatch_floor()
    if args.op_rates:
        return op_rates()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: this build emulates the W={W_CFG1} data-parallel replicas on a single "
            f"MI355X (no inter-GPU collectives), so --gpus {args.gpus} is not supported",
            file=sys.stderr,
        )
        return 2

    # ---- CPU baseline first: nothing has touched the GPU yet
    cpu = None
    if args.workload in CPU_BASELINE and not args.no_cpu_baseline:
        world = CPU_BASELINE[args.workload][1]
        threads = max(1, host_cores() // world)  # every core this process may run on, split over the ranks
        # about 10 s of CPU work: a GPT-2-medium step takes ~3x a GPT-2-124M one, the tiny GPT ~1%
        steps = {"cfg0": args.cpu_steps * 10, "cfg1": args.cpu_steps, "cfg2": max(3, args.cpu_steps // 3),
                 "cfg3": 3, "cfg4": 2}
        t0 = time.perf_counter()
        cpu = cpu_baseline(args.workload, steps[args.workload], threads)
        print(f"[bench] cpu baseline done in {time.perf_counter() - t0:.1f}s: {cpu}", file=sys.stderr, flush=True)

    if args.workload in ("cfg3", "cfg3-f16"):
        out = bench_fsdp(args, "f16" if args.workload == "cfg3-f16" else "bf16")
    elif args.workload == "cfg1-overlap":
        out = bench_overlap(args)
    else:
        out = bench_ddp(args.workload, args)
    if cpu is not None:
        # the same byte count as `value`, over the CPU step time: value / cpu value = the speedup
        nbytes = out["config"].get("hbm_bytes_per_step", out["config"]["alg_bytes_per_step"])
        cpu_gbs = nbytes / (cpu["median_ms"] * 1e-3) / 1e9
        out["cpu_baseline"] = {
            "value": round(cpu_gbs, 3),
            "unit": "GB/s",
            "cores": cpu["cores"],
            "kind": "port",
            "sample": f"{cpu['steps']} timed steps (+1 warmup) of the {args.workload} pipeline, reference op "
                      f"chain on torch CPU + gloo, {cpu['world']} processes x {cpu['threads_per_rank']} threads, "
                      f"each step from the same pristine gradients; median {cpu['median_ms']:.1f} ms/step"
                      + (f"; {cpu['note']}" if cpu.get("note") else ""),
            "ms_per_step": round(cpu["median_ms"], 2),
            "speedup": round(cpu["median_ms"] / out["ms_per_step"], 1),
            "host": host_description(),
        }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
