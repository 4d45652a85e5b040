"""Overlap analysis (minidist.profiling) on the CPU: the interval arithmetic and the
kernel classification, checked on hand-built traces whose answers can be read off.

Follows the reference's tests/test_profiling.py cases (full overlap, full exposure,
partial overlap with classification, concurrent kernels counted once, the labelled
CPU fallback), adds a brute-force check of the interval operations on a grid, and
the gfx950 path's own kernel names as rocprofv3 prints them.
"""

from __future__ import annotations

import csv
import gzip
import json
from pathlib import Path

import numpy as np
import pytest

from minidist import profiling as P

# Kernel names exactly as rocprofv3 reports them for this path.
FUSED = "void mdx::reduce_impl::allreduce_unpack_kernel_dev<float, float, 8>(mdx::DevTable, mdx::ReduceParams)"
PACK = "void mdx::(anonymous namespace)::copy_kernel_dev<float, float, 1, false>(mdx::DevTable, mdx::CopyParams)"
SHARE = "void mdx::reduce_impl::share_kernel<mdx::bf16, float, float, 8>(mdx::PieceBatch, mdx::ReduceParams)"
WIDE = "void mdx::reduce_impl::allreduce_wide_kernel_dev<mdx::bf16, float, mdx::bf16, 8>(mdx::DevTable, mdx::ReduceParams)"
GEMM = "Cijk_Alik_Bljk_SB_MT128x128x16_MI16x16x1_SN_1LDSB0"
TORCH_COPY = "void at::native::vectorized_elementwise_kernel<4, at::native::bfloat16_copy_kernel_cuda(at::TensorIteratorBase&)>"


def test_kernel_classification():
    assert P.classify(FUSED) == "all_reduce" and P.is_collective(FUSED)
    assert P.classify(WIDE) == "all_reduce"
    assert P.classify(SHARE) == "reduce_scatter" and P.is_collective(SHARE)
    assert P.classify(PACK) == "bucket_copy" and P.is_collective(PACK)
    assert P.classify("ncclDevKernel_ReduceScatter_Sum_f32") == "reduce_scatter"
    assert P.classify("nccl:all_gather") == "all_gather"
    assert not P.is_collective(GEMM) and not P.is_collective(TORCH_COPY)
    assert P.classify(TORCH_COPY) is None and P.classify(GEMM) is None


def test_mangled_kernel_names_and_bookkeeping_kernels():
    """A tracer may record a kernel's mangled name: the path's kernels are recognised in that form
    too (namespace mdx, ``_ZN3mdx``), with the same kinds.  The flag clear and the allocation-free
    launch's plan upload have kinds of their own."""
    mangled = {
        "_ZN3mdx11reduce_impl21allreduce_pack_kernelIffLi8EEEvNS_10PieceBatchENS_12ReduceParamsE": "all_reduce",
        "_ZN3mdx11reduce_impl16share_kernel_fewIN3mdx4bf16EffLi8EEEvNS_8PieceFewENS_12ReduceParamsE":
            "reduce_scatter",
        "_ZN3mdx12_GLOBAL__N_115copy_kernel_oneIfNS_4bf16ELi0ELb0EEEvNS_7SpanOneENS_10CopyParamsE": "bucket_copy",
        "_ZN3mdx12_GLOBAL__N_117clear_flag_kernelEPi": "flag_clear",
        "_ZN3mdx12_GLOBAL__N_113upload_kernelENS0_11UploadChunkEPh": "plan_upload",
    }
    for name, kind in mangled.items():
        assert P.is_collective(name) and P.classify(name) == kind, name
    assert P.classify("void mdx::(anonymous namespace)::clear_flag_kernel(int*)") == "flag_clear"
    assert not P.is_collective("_ZN2at6native29vectorized_elementwise_kernelILi4EEEviT_")


def _grid_measure(intervals, lo=0, hi=80):
    cover = np.zeros(hi - lo, dtype=bool)
    for a, b in intervals:
        cover[a - lo : b - lo] = True
    return cover


@pytest.mark.parametrize("seed", range(20))
def test_interval_operations_match_a_grid(seed):
    """Union / intersection / difference against the same sets painted on integer cells."""
    rng = np.random.default_rng(seed)

    def random_set():
        n = int(rng.integers(0, 8))
        starts = rng.integers(0, 60, n)
        return [(int(s), int(s + rng.integers(0, 10))) for s in starts]

    a, b = random_set(), random_set()
    ua, ub = P._union(a), P._union(b)
    ga, gb = _grid_measure(a), _grid_measure(b)
    assert P._measure(ua) == ga.sum()
    assert all(x[1] < y[0] for x, y in zip(ua, ua[1:])), "union must be disjoint and sorted"
    assert P._measure(P._common(ua, ub)) == (ga & gb).sum()
    assert P._measure(P._minus(ua, ub)) == (ga & ~gb).sum()
    assert np.array_equal(_grid_measure(P._common(ua, ub)), ga & gb)
    assert np.array_equal(_grid_measure(P._minus(ua, ub)), ga & ~gb)


def test_union_merges_touching_intervals():
    assert P._union([(0, 2), (1, 3), (5, 6)]) == [(0, 3), (5, 6)]
    assert P._union([(0, 1), (1, 2)]) == [(0, 2)]
    assert P._union([]) == []


def _trace(tmp_path, events):
    path = tmp_path / "trace.json"
    path.write_text(json.dumps({"traceEvents": events}))
    return path


def _k(name, ts, dur):
    return {"ph": "X", "cat": "kernel", "name": name, "ts": ts, "dur": dur}


def test_fully_hidden_exchange(tmp_path):
    r = P.analyze_trace(_trace(tmp_path, [_k(GEMM, 0, 1000), _k(FUSED, 200, 400)]))
    assert r.device == "cuda"
    assert r.comm_s == pytest.approx(400e-6) and r.overlapped_s == pytest.approx(400e-6)
    assert r.overlap_fraction == 1.0 and r.exposed_comm_s == 0.0


def test_fully_exposed_exchange(tmp_path):
    r = P.analyze_trace(_trace(tmp_path, [_k(GEMM, 0, 500), _k("nccl:all_gather", 500, 500)]))
    assert r.overlapped_s == 0.0 and r.overlap_fraction == 0.0
    assert r.exposed_comm_s == pytest.approx(500e-6)
    assert r.exposed_fraction_of_step == pytest.approx(0.5)


def test_partial_overlap_and_per_kind(tmp_path):
    r = P.analyze_trace(_trace(tmp_path, [_k(GEMM, 0, 600), _k(FUSED, 400, 400), _k(SHARE, 800, 100),
                                          _k(PACK, 950, 50)]))
    assert r.comm_s == pytest.approx(550e-6)
    assert r.overlapped_s == pytest.approx(200e-6), "only 400-600 us has compute alongside"
    assert r.exposed_comm_s == pytest.approx(350e-6)
    assert set(r.per_kind_s) == {"all_reduce", "reduce_scatter", "bucket_copy"}
    assert r.per_kind_s["reduce_scatter"] == pytest.approx(100e-6)
    assert r.num_comm_events == 3 and r.num_compute_events == 1


def test_concurrent_kernels_counted_once(tmp_path):
    r = P.analyze_trace(_trace(tmp_path, [_k(GEMM, 0, 1000), _k(GEMM + "_b", 0, 1000)]))
    assert r.compute_s == pytest.approx(1000e-6)


def test_cpu_fallback_is_labelled(tmp_path):
    r = P.analyze_trace(_trace(tmp_path, [
        {"ph": "X", "cat": "cpu_op", "name": "aten::mm", "ts": 0, "dur": 500},
        {"ph": "X", "cat": "cpu_op", "name": "c10d::allreduce_", "ts": 500, "dur": 300},
        {"ph": "X", "cat": "cpu_op", "name": "step", "ts": 0, "dur": 800},  # a parent frame around both
    ]))
    assert r.device == "cpu" and "Gloo" in r.note
    assert r.comm_s == pytest.approx(300e-6) and r.overlapped_s == 0.0
    assert "exposed comm" in r.format()


def test_rocprof_kernel_trace(tmp_path):
    """A rocprofv3 kernel-trace CSV (ns timestamps): two backward GEMMs, a pack and fused
    reduction overlapping the second, and the last bucket's pair after backward ends."""
    path = tmp_path / "run_kernel_trace.csv"
    rows = [(GEMM, 0, 1000), (GEMM, 1000, 2000), (PACK, 1200, 1300), (FUSED, 1300, 1800),
            (PACK, 2000, 2100), (FUSED, 2100, 2600)]
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        for name, t0, t1 in rows:
            w.writerow(["KERNEL_DISPATCH", name, t0, t1])
    r = P.analyze_kernel_trace(path)
    assert r.comm_s == pytest.approx(1200e-9)
    assert r.overlapped_s == pytest.approx(600e-9)
    assert r.exposed_comm_s == pytest.approx(600e-9)
    assert r.wall_s == pytest.approx(2600e-9)
    assert r.per_kind_s == pytest.approx({"bucket_copy": 200e-9, "all_reduce": 1000e-9})
    late = P.analyze_kernel_trace(path, since_ns=2000)
    assert late.compute_s == 0.0 and late.exposed_comm_s == pytest.approx(600e-9)


def test_real_rocprof_trace_of_an_overlapped_step(tmp_path):
    """One step of the cfg1 path inside a real forward + backward on an MI355X, DDP's bucket runs on
    their own stream, as rocprofv3 recorded it (``tests/golden/rocprof_cfg1_overlap_step.csv.gz``,
    cut from the raw trace by ``tests/golden/make_rocprof_fixture.py``): the names rocprofv3 gave
    this path's kernels are its collectives and no other kernel is (torch's own copy kernels
    included); the report's busy, overlapped and exposed times equal a nanosecond grid over the
    same rows."""
    path = tmp_path / "run_kernel_trace.csv"
    path.write_bytes(gzip.decompress((Path(__file__).parent / "golden" / "rocprof_cfg1_overlap_step.csv.gz").read_bytes()))
    with open(path, newline="") as fh:
        rows = list(csv.DictReader(fh))
    r = P.analyze_kernel_trace(path)
    ours = [row for row in rows if "mdx::" in row["Kernel_Name"]]
    gemms = [row for row in rows if row["Kernel_Name"].startswith("Cijk_")]
    assert len(rows) > 500 and ours and gemms
    assert r.num_comm_events == len(ours) and r.num_compute_events == len(rows) - len(ours)
    assert {P.classify(row["Kernel_Name"]) for row in ours} == {"all_reduce"}
    assert any("copy_kernel" in row["Kernel_Name"] for row in rows if row not in ours)  # torch's, not a bucket copy
    assert {row["Stream_Id"] for row in ours}.isdisjoint({row["Stream_Id"] for row in gemms})  # DDP's own stream

    end = max(int(row["End_Timestamp"]) for row in rows)
    comm, compute = np.zeros(end, dtype=bool), np.zeros(end, dtype=bool)
    for row in rows:
        cover = comm if "mdx::" in row["Kernel_Name"] else compute
        cover[int(row["Start_Timestamp"]) : int(row["End_Timestamp"])] = True
    ns = 1e-9
    assert r.comm_s == pytest.approx(comm.sum() * ns, abs=1e-12)
    assert r.compute_s == pytest.approx(compute.sum() * ns, abs=1e-12)
    assert r.overlapped_s == pytest.approx((comm & compute).sum() * ns, abs=1e-12)
    assert r.exposed_comm_s == pytest.approx((comm & ~compute).sum() * ns, abs=1e-12)
    assert r.per_kind_s == pytest.approx({"all_reduce": comm.sum() * ns}, abs=1e-12)
    assert r.wall_s == pytest.approx(end * ns, abs=1e-12)
    assert 0 < r.overlapped_s < r.comm_s  # the stream ran part of the path under backward's kernels


def test_package_exports_the_reference_names():
    import minidist

    for name in ("profile_steps", "summarize_collectives", "format_collective_table", "analyze_trace"):
        assert callable(getattr(minidist, name))
    assert P.format_collective_table([]) == "  (no collective events recorded)"
    row = P.CollectiveRow("all_reduce", 4, 0.0, 400.0)
    assert row.avg_us == 100.0 and "all_reduce" in P.format_collective_table([row])
