"""Cut one training step out of a real rocprofv3 kernel trace, as a fixture for the trace reader.

The raw trace came from the cfg1 path inside a real forward + backward, with DDP's bucket
launches on their own stream (MI355X, ROCm 7.2, repo root):

    rocprofv3 --kernel-trace -d gpurun_out/ovtrace/kt -o run --output-format csv -- \\
        python3 bench.py --workload cfg1-overlap --overlap-modes overlap --steps 3 --warmup 1 --no-cpu-baseline

then, on any machine:

    python3 tests/golden/make_rocprof_fixture.py gpurun_out/ovtrace/kt/run_kernel_trace.csv \\
        tests/golden/rocprof_cfg1_overlap_step.csv.gz

The step kept is the last one: every kernel that starts at or after the last embedding gather
(``vectorized_gather_kernel``) that follows more than 300 us of GPU idle time.  The rows keep
rocprofv3's own columns and kernel names, with timestamps made relative to the step's first
kernel; nothing else is changed.
"""

from __future__ import annotations

import csv
import gzip
import sys

COLUMNS = ("Kind", "Stream_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp")
IDLE_NS = 300_000


def last_step(rows: list[dict]) -> list[dict]:
    rows = sorted(rows, key=lambda r: int(r["Start_Timestamp"]))
    start, busy_until = None, None
    for r in rows:
        s = int(r["Start_Timestamp"])
        if busy_until is not None and s - busy_until > IDLE_NS and "vectorized_gather_kernel" in r["Kernel_Name"]:
            start = s
        busy_until = max(busy_until or 0, int(r["End_Timestamp"]))
    if start is None:
        raise SystemExit("no step boundary found")
    return [r for r in rows if int(r["Start_Timestamp"]) >= start]


def main(src: str, dst: str) -> None:
    with open(src, newline="") as fh:
        step = last_step(list(csv.DictReader(fh)))
    t0 = int(step[0]["Start_Timestamp"])
    with gzip.open(dst, "wt", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(COLUMNS)
        for r in step:
            w.writerow([r["Kind"], r["Stream_Id"], r["Kernel_Name"], int(r["Start_Timestamp"]) - t0,
                        int(r["End_Timestamp"]) - t0])
    print(f"{len(step)} kernels, {(int(step[-1]['End_Timestamp']) - t0) / 1e6:.3f} ms -> {dst}")


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
