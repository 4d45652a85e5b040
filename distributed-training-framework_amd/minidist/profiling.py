"""Collective breakdowns and communication/compute overlap, for traces of this path.

Same surface as the reference's minidist/profiling.py (``COLLECTIVE_PATTERNS``
:65-71, ``profile_steps`` :99-141, ``summarize_collectives`` :161-180,
``format_collective_table`` :183-195, ``OverlapReport`` :244-294,
``analyze_trace`` :305-362), with the gradient path's own kernels known by
name.  The reference recognises collectives by NCCL / c10d names only; here
the gfx950 kernels that carry the data-parallel exchange are classified too:

    mdx allreduce_unpack / allreduce / allreduce_wide kernels  -> all_reduce
    mdx share_kernel (the reduce-scatter share)                -> reduce_scatter
    mdx copy_kernel (bucket pack / unpack, unscale, gather cast) -> bucket_copy
    mdx clear_flag_kernel (the scaler's found-inf flag)        -> flag_clear
    mdx upload_kernel (a plan copied in by the allocation-free
    launch)                                                    -> plan_upload

A kernel is recognised by its demangled name (``mdx::`` namespace) or its
mangled one (``_ZN3mdx``): which of the two a trace holds depends on the
tracer, not on the kernel.

so "how much of the gradient exchange did backward hide" is answered for a
ResidentGroup run exactly as for an RCCL one.  Besides the profiler's Chrome
trace, :func:`analyze_kernel_trace` reads a ``rocprofv3 --kernel-trace``
CSV (``*_kernel_trace.csv``), whose timestamps come from the GPU itself.

Overlap arithmetic: each category's kernels become a set of busy intervals
(concurrent kernels merged, so nothing is counted twice); ``overlapped`` is
the measure of the intersection of the communication and compute sets, and
``exposed = communication - overlapped`` is the part of the exchange during
which no compute ran.
"""

from __future__ import annotations

import csv
import gzip
import json
from collections.abc import Callable, Iterable, Sequence
from dataclasses import dataclass, field
from pathlib import Path

import torch

__all__ = [
    "COLLECTIVE_PATTERNS",
    "CollectiveRow",
    "OverlapReport",
    "analyze_kernel_trace",
    "analyze_trace",
    "classify",
    "format_collective_table",
    "is_collective",
    "profile_steps",
    "summarize_collectives",
]

# Substrings that mark an event as part of a collective: RCCL/NCCL device
# kernels and host ops, torch.distributed's dispatcher ops and annotations,
# and the gradient path's own kernels (namespace mdx::, demangled or mangled).
COLLECTIVE_PATTERNS: tuple[str, ...] = (
    "nccl",
    "rccl",
    "c10d::",
    "record_param_comms",
    "ProcessGroupNCCL",
    "ProcessGroupGloo",
    "mdx::",
    "_ZN3mdx",
)

# (kind, lower-case substrings), first match wins: the mdx kernel names come
# first because "allreduce_unpack" must not fall through to a copy.
_KINDS: tuple[tuple[str, tuple[str, ...]], ...] = (
    ("all_reduce", ("allreduce", "all_reduce")),
    ("reduce_scatter", ("reducescatter", "reduce_scatter", "share_kernel")),
    ("all_gather", ("allgather", "all_gather")),
    ("broadcast", ("broadcast",)),
    ("send_recv", ("sendrecv", "send", "recv", "p2p")),
    ("barrier", ("barrier",)),
    ("bucket_copy", ("copy_kernel",)),
    ("flag_clear", ("clear_flag_kernel",)),
    ("plan_upload", ("upload_kernel",)),
)


def is_collective(name: str) -> bool:
    low = name.lower()
    return any(p.lower() in low for p in COLLECTIVE_PATTERNS)


def classify(name: str) -> str | None:
    """The collective kind of an event or kernel name; None for a name that is not a collective's
    (torch's own ``direct_copy_kernel_cuda`` is no bucket copy) or matches no kind."""
    if not is_collective(name):
        return None
    low = name.lower()
    for kind, needles in _KINDS:
        if any(n in low for n in needles):
            return kind
    return None


# ---------------------------------------------------------------------------
# Interval sets
# ---------------------------------------------------------------------------

Intervals = list[tuple[float, float]]


def _union(iv: Iterable[tuple[float, float]]) -> Intervals:
    """Disjoint, sorted cover of the given intervals."""
    out: Intervals = []
    for lo, hi in sorted(iv):
        if hi <= lo:
            continue
        if out and lo <= out[-1][1]:
            if hi > out[-1][1]:
                out[-1] = (out[-1][0], hi)
        else:
            out.append((lo, hi))
    return out


def _measure(iv: Intervals) -> float:
    return sum(hi - lo for lo, hi in iv)


def _common(a: Intervals, b: Intervals) -> Intervals:
    """Intersection of two disjoint sorted sets (sweep over both at once)."""
    out: Intervals = []
    i = j = 0
    while i < len(a) and j < len(b):
        lo, hi = max(a[i][0], b[j][0]), min(a[i][1], b[j][1])
        if lo < hi:
            out.append((lo, hi))
        # advance whichever interval ends first; the other may meet the next one
        if a[i][1] <= b[j][1]:
            i += 1
        else:
            j += 1
    return out


def _minus(a: Intervals, b: Intervals) -> Intervals:
    """``a`` with ``b`` removed (both disjoint and sorted)."""
    out: Intervals = []
    j = 0
    for lo, hi in a:
        while j < len(b) and b[j][1] <= lo:
            j += 1
        cur, k = lo, j
        while k < len(b) and b[k][0] < hi:
            if b[k][0] > cur:
                out.append((cur, b[k][0]))
            cur = max(cur, b[k][1])
            k += 1
        if cur < hi:
            out.append((cur, hi))
    return out


# ---------------------------------------------------------------------------
# Reports
# ---------------------------------------------------------------------------


@dataclass
class CollectiveRow:
    kind: str
    count: int
    self_time_us: float
    device_time_us: float

    @property
    def avg_us(self) -> float:
        return (self.device_time_us or self.self_time_us) / max(1, self.count)


@dataclass
class OverlapReport:
    """Communication / compute overlap over one trace, in seconds."""

    device: str
    wall_s: float = 0.0
    compute_s: float = 0.0
    comm_s: float = 0.0
    overlapped_s: float = 0.0
    num_comm_events: int = 0
    num_compute_events: int = 0
    per_kind_s: dict[str, float] = field(default_factory=dict)
    note: str = ""

    @property
    def exposed_comm_s(self) -> float:
        """Communication time during which no compute kernel ran."""
        return max(0.0, self.comm_s - self.overlapped_s)

    @property
    def overlap_fraction(self) -> float:
        return self.overlapped_s / self.comm_s if self.comm_s > 0 else 0.0

    @property
    def exposed_fraction_of_step(self) -> float:
        return self.exposed_comm_s / self.wall_s if self.wall_s > 0 else 0.0

    def as_dict(self) -> dict:
        return {
            "device": self.device,
            "wall_ms": self.wall_s * 1e3,
            "compute_ms": self.compute_s * 1e3,
            "comm_ms": self.comm_s * 1e3,
            "overlapped_ms": self.overlapped_s * 1e3,
            "exposed_comm_ms": self.exposed_comm_s * 1e3,
            "overlap_fraction": self.overlap_fraction,
            "comm_events": self.num_comm_events,
            "compute_events": self.num_compute_events,
            "per_kind_ms": {k: v * 1e3 for k, v in self.per_kind_s.items()},
        }

    def format(self) -> str:
        ms = 1e3
        lines = [
            f"  device            : {self.device}",
            f"  wall              : {self.wall_s * ms:.3f} ms",
            f"  compute (busy)    : {self.compute_s * ms:.3f} ms ({self.num_compute_events} events)",
            f"  communication     : {self.comm_s * ms:.3f} ms ({self.num_comm_events} events)",
            f"  overlapped        : {self.overlapped_s * ms:.3f} ms ({self.overlap_fraction:.1%} of comm hidden)",
            f"  exposed comm      : {self.exposed_comm_s * ms:.3f} ms ({self.exposed_fraction_of_step:.1%} of wall)",
        ]
        for kind, sec in sorted(self.per_kind_s.items(), key=lambda kv: -kv[1]):
            lines.append(f"      {kind:<16}{sec * ms:>10.3f} ms")
        if self.note:
            lines.append(f"  note              : {self.note}")
        return "\n".join(lines)


def _report(device: str, events: Iterable[tuple[str, float, float]], note: str = "",
            cpu_blocking: bool = False) -> OverlapReport:
    """Overlap report of (name, begin_s, end_s) events."""
    comm, compute, kinds = [], [], {}
    for name, lo, hi in events:
        if is_collective(name):
            comm.append((lo, hi))
            kinds.setdefault(classify(name) or "other", []).append((lo, hi))
        else:
            compute.append((lo, hi))
    comm_u, compute_u = _union(comm), _union(compute)
    if cpu_blocking:
        # A blocking CPU collective sits inside its callers' frames: count that
        # time as communication only, so the two categories stay disjoint.
        compute_u = _minus(compute_u, comm_u)
    every = _union(comm + compute)
    return OverlapReport(
        device=device,
        wall_s=(every[-1][1] - every[0][0]) if every else 0.0,
        compute_s=_measure(compute_u),
        comm_s=_measure(comm_u),
        overlapped_s=_measure(_common(comm_u, compute_u)),
        num_comm_events=len(comm),
        num_compute_events=len(compute),
        per_kind_s={k: _measure(_union(v)) for k, v in kinds.items()},
        note=note,
    )


def analyze_kernel_trace(
    path: str | Path, since_ns: int | None = None, until_ns: int | None = None
) -> OverlapReport:
    """Overlap report of a ``rocprofv3 --kernel-trace`` CSV (GPU timestamps, ns).

    ``since_ns`` / ``until_ns`` keep only kernels that start inside the window
    (e.g. the timed steps of a run)."""
    events = []
    with open(path, newline="") as fh:
        for row in csv.DictReader(fh):
            t0, t1 = int(row["Start_Timestamp"]), int(row["End_Timestamp"])
            if since_ns is not None and t0 < since_ns:
                continue
            if until_ns is not None and t0 >= until_ns:
                continue
            events.append((row["Kernel_Name"], t0 * 1e-9, t1 * 1e-9))
    return _report("gpu (rocprofv3 kernel trace)", events)


def _load_json(path: str | Path) -> dict:
    path = Path(path)
    opener = gzip.open if path.suffix == ".gz" else open
    with opener(path, "rt") as fh:
        return json.load(fh)


def analyze_trace(path: str | Path, prefer_device: bool = True) -> OverlapReport:
    """Overlap report of a Chrome trace exported by the torch profiler.

    GPU kernel events are used when the trace has them (``prefer_device``);
    otherwise the CPU operators, where a gloo collective blocks its caller and
    overlap is structurally about zero."""
    raw = [e for e in _load_json(path).get("traceEvents", []) if e.get("ph") == "X"]
    kernels = [e for e in raw if e.get("cat") == "kernel"]
    if prefer_device and kernels:
        pool, device, note, blocking = kernels, "cuda", "", False  # torch's device name, also on ROCm
    else:
        pool = [e for e in raw if e.get("cat") in ("cpu_op", "user_annotation")]
        device, blocking = "cpu", True
        note = "Gloo/CPU operators: a gloo collective blocks its caller, so overlap is ~0 by construction"
    events = [
        (e.get("name", ""), float(e["ts"]) * 1e-6, (float(e["ts"]) + float(e.get("dur", 0.0))) * 1e-6)
        for e in pool
    ]
    return _report(device, events, note, cpu_blocking=blocking)


# ---------------------------------------------------------------------------
# Profiler driving and event tables
# ---------------------------------------------------------------------------


def profile_steps(
    step_fn: Callable[[int], None],
    num_steps: int = 6,
    warmup: int = 2,
    wait: int = 1,
    trace_path: str | Path | None = None,
    record_shapes: bool = True,
    with_stack: bool = False,
    activities: Sequence | None = None,
):
    """Run ``step_fn(i)`` for ``num_steps`` steps under the torch profiler.

    The first ``wait`` steps are not recorded and the next ``warmup`` are
    recorded but discarded (first-step allocations, plan builds and
    communicator set-up are not representative); the rest are kept and,
    with ``trace_path``, exported as a Chrome trace."""
    from torch.profiler import ProfilerActivity, profile, schedule

    if activities is None:
        activities = [ProfilerActivity.CPU]
        if torch.cuda.is_available():
            activities.append(ProfilerActivity.CUDA)
    active = max(1, num_steps - wait - warmup)
    with profile(
        activities=list(activities),
        schedule=schedule(wait=wait, warmup=warmup, active=active, repeat=1),
        record_shapes=record_shapes,
        with_stack=with_stack,
    ) as prof:
        for i in range(num_steps):
            step_fn(i)
            prof.step()
    if trace_path is not None:
        trace_path = Path(trace_path)
        trace_path.parent.mkdir(parents=True, exist_ok=True)
        prof.export_chrome_trace(str(trace_path))
    return prof


def summarize_collectives(prof) -> list[CollectiveRow]:
    """Per-kind totals of the collective events in a finished profile."""
    rows: dict[str, CollectiveRow] = {}
    for ev in prof.key_averages():
        if not is_collective(ev.key):
            continue
        row = rows.setdefault(classify(ev.key) or "other", CollectiveRow(classify(ev.key) or "other", 0, 0.0, 0.0))
        row.count += ev.count
        row.self_time_us += float(getattr(ev, "self_cpu_time_total", 0.0) or 0.0)
        for attr in ("self_device_time_total", "self_cuda_time_total"):
            dev_us = float(getattr(ev, attr, 0.0) or 0.0)
            if dev_us:
                row.device_time_us += dev_us
                break
    return sorted(rows.values(), key=lambda r: -max(r.device_time_us, r.self_time_us))


def format_collective_table(rows: Iterable[CollectiveRow]) -> str:
    rows = list(rows)
    if not rows:
        return "  (no collective events recorded)"
    lines = [f"  {'collective':<16}{'count':>8}{'device ms':>12}{'cpu ms':>10}{'avg us':>10}", "  " + "-" * 56]
    for r in rows:
        lines.append(
            f"  {r.kind:<16}{r.count:>8}{r.device_time_us / 1e3:>12.3f}{r.self_time_us / 1e3:>10.3f}{r.avg_us:>10.1f}"
        )
    return "\n".join(lines)
