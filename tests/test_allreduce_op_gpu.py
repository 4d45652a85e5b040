"""Non-SUM all-reduce (mdx_allreduce_op) on the GPU, bit for bit against the oracle.

The reference forwards any ``op`` to ``dist.all_reduce`` / ``dist.reduce_scatter_tensor``
(minidist/comm.py:223-234, 252-265): over a ResidentGroup MAX, MIN and PRODUCT
fold the W replicas in rank order (oracle.gradpath.allreduce_op, pinned
against torch's CPU maximum / minimum / mul).  Inputs carry NaN, +-inf, +-0,
subnormals and values repeated across ranks; gaps between runs keep a
sentinel, so a write outside a run shows up.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.distributed as dist

from conftest import first_mismatch, same_bits
from minidist import ResidentGroup, comm
from minidist import _native as nat
from oracle import gradpath as o
from test_kernels_gpu import DEV, DTYPES, SENTINEL, code, empty_dev, stream, to_dev, to_host, values

pytestmark = pytest.mark.gpu

OPS = {"max": nat.MDX_OP_MAX, "min": nat.MDX_OP_MIN, "product": nat.MDX_OP_PRODUCT}
REDUCE_OPS = {"max": dist.ReduceOp.MAX, "min": dist.ReduceOp.MIN, "product": dist.ReduceOp.PRODUCT}


def _replicas(rng, W, extent, dt, scale=1.0):
    reps = [values(rng, extent, dt, scale=scale) for _ in range(W)]
    zero, neg_zero = o.from_f32(np.array([0.0], np.float32), dt)[0], o.from_f32(np.array([-0.0], np.float32), dt)[0]
    for r in range(W):
        reps[r][: extent // 8] = reps[0][: extent // 8]  # equal across ranks
        k = rng.integers(0, extent, extent // 16)
        reps[r][k] = zero if r % 2 else neg_zero  # ties of -0 and +0 across ranks
    return reps


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("W", [1, 2, 3, 8, 16])
@pytest.mark.parametrize("op", list(OPS))
def test_allreduce_op_matches_oracle(rng, dt, W, op):
    runs = [(3, 1), (17, 4096), (5000, 3), (9000, 2047), (70000, 12345)]  # (offset, numel), increasing
    extent = runs[-1][0] + runs[-1][1] + 9
    reps_host = _replicas(rng, W, extent, dt, scale=2.0 if op == "product" else 1.0)
    reps = [to_dev(h) for h in reps_host]
    out = empty_dev(extent, dt)
    nat.allreduce_op([r.data_ptr() for r in reps], code(dt), OPS[op], [a for a, _ in runs], [n for _, n in runs],
                     out.data_ptr(), stream())
    got = to_host(out)
    want = np.full(extent, SENTINEL[dt], dtype=got.dtype)
    for a, n in runs:
        want[a : a + n] = o.allreduce_op([h[a : a + n] for h in reps_host], dt, op)
    assert same_bits(got, want), first_mismatch(got, want)
    for r in range(W):
        assert same_bits(to_host(reps[r]), reps_host[r]), f"replica {r} was written"


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("W,k", [(4, 0), (4, 3), (8, 5)])
def test_allreduce_op_in_place_on_one_replica(rng, op, W, k):
    n = 300_001
    reps_host = _replicas(rng, W, n, o.F32)
    reps = [to_dev(h) for h in reps_host]
    nat.allreduce_op([r.data_ptr() for r in reps], nat.MDX_F32, OPS[op], [0], [n], reps[k].data_ptr(), stream())
    want = o.allreduce_op(reps_host, o.F32, op)
    got = to_host(reps[k])
    assert same_bits(got, want), first_mismatch(got, want)
    for r in range(W):
        if r != k:
            assert same_bits(to_host(reps[r]), reps_host[r])


def test_allreduce_op_many_runs(rng):
    """130 runs (three dispatches of at most 48 kernel-argument runs) with gaps, bf16 MAX at W = 5."""
    W, dt = 5, o.BF16
    runs, off = [], 0
    for _ in range(130):
        off += int(rng.integers(0, 5))
        n = int(rng.integers(0, 5000))
        runs.append((off, n))
        off += n
    extent = off + 3
    reps_host = _replicas(rng, W, extent, dt)
    reps = [to_dev(h) for h in reps_host]
    out = empty_dev(extent, dt)
    nat.allreduce_op([r.data_ptr() for r in reps], code(dt), nat.MDX_OP_MAX, [a for a, _ in runs],
                     [n for _, n in runs], out.data_ptr(), stream())
    got = to_host(out)
    want = np.full(extent, SENTINEL[dt], dtype=got.dtype)
    for a, n in runs:
        want[a : a + n] = o.allreduce_op([h[a : a + n] for h in reps_host], dt, "max")
    assert same_bits(got, want), first_mismatch(got, want)


def test_allreduce_op_sum_is_allreduce_sum(rng):
    W, n = 6, 40_000
    reps_host = [values(rng, n, o.F32) for _ in range(W)]
    reps = [to_dev(h) for h in reps_host]
    a, b = empty_dev(n, o.F32), empty_dev(n, o.F32)
    nat.allreduce_op([r.data_ptr() for r in reps], nat.MDX_F32, nat.MDX_OP_SUM, [0], [n], a.data_ptr(), stream())
    nat.allreduce_sum([r.data_ptr() for r in reps], nat.MDX_F32, [0], [n], b.data_ptr(), stream())
    assert same_bits(to_host(a), to_host(b)) and same_bits(to_host(a), o.allreduce_sum(reps_host, o.F32))


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_comm_all_reduce_ops_over_a_resident_group(rng, op, dtype):
    """``comm.all_reduce(t, op)`` over a ResidentGroup: a found-inf style flag and a small tensor
    in one symmetric buffer, every replica's copy staged, reduced in place on this rank's row."""
    W, rank = 4, 2
    dt = o.F32 if dtype == torch.float32 else o.BF16
    group = ResidentGroup(W, rank, DEV)
    flag = group.zeros(1, dtype)
    small = group.zeros(1000, dtype)
    hosts = {}
    for name, t in (("flag", flag), ("small", small)):
        reps_host = _replicas(rng, W, t.numel(), dt) if t.numel() > 1 else \
            [o.from_f32(np.array([float(r == 1)], np.float32), dt) for r in range(W)]
        for r, row in enumerate(group.replicas(t)):
            row.copy_(to_dev(reps_host[r]).view(row.shape))
        hosts[name] = reps_host
    with comm.record_comm() as stats:
        comm.all_reduce(flag, op=REDUCE_OPS[op], group=group)
        work = comm.all_reduce(small, op=REDUCE_OPS[op], group=group, async_op=True)
        work.wait()
    assert stats.as_rows()[0][:2] == ("all_reduce", 2)
    for name, t in (("flag", flag), ("small", small)):
        want = o.allreduce_op(hosts[name], dt, op)
        got = to_host(t)
        assert same_bits(got, want), f"{name}: " + first_mismatch(got, want)
        for r, row in enumerate(group.replicas(t)):
            if r != rank:
                assert same_bits(to_host(row), hosts[name][r]), f"{name}: replica {r} was written"


@pytest.mark.parametrize("op", list(OPS))
def test_comm_reduce_scatter_ops_over_a_resident_group(rng, op):
    """``comm.reduce_scatter_tensor(out, in, op)``: this rank's slice of the W replicas, folded."""
    W, rank, S = 8, 5, 777
    group = ResidentGroup(W, rank, DEV)
    inp = group.zeros(S * W, torch.float32)
    reps_host = _replicas(rng, W, S * W, o.F32)
    for r, row in enumerate(group.replicas(inp)):
        row.copy_(to_dev(reps_host[r]))
    out = torch.empty(S, device=DEV)
    comm.reduce_scatter_tensor(out, inp, op=REDUCE_OPS[op], group=group)
    want = o.allreduce_op([h[rank * S : (rank + 1) * S] for h in reps_host], o.F32, op)
    got = to_host(out)
    assert same_bits(got, want), first_mismatch(got, want)


def test_comm_rejects_ops_a_resident_group_does_not_reduce():
    group = ResidentGroup(2, 0, DEV)
    t = group.zeros(4, torch.float32)
    with pytest.raises(NotImplementedError, match="SUM, PRODUCT, MIN and MAX"):
        comm.all_reduce(t, op=dist.ReduceOp.AVG, group=group)


@pytest.mark.parametrize("seed", range(16))
def test_allreduce_op_fuzz(seed):
    """Seeded random cases: W in [1, 16], dtype, op, 1-60 runs of 0-20000 elements at any element
    offset (gaps keep a sentinel), in place on a random replica or into a separate buffer."""
    g = np.random.default_rng(5000 + seed)
    W = int(g.integers(1, 17))
    dt = DTYPES[int(g.integers(0, 3))]
    op = list(OPS)[int(g.integers(0, 3))]
    runs, off = [], int(g.integers(0, 9))
    for _ in range(int(g.integers(1, 61))):
        n = int(g.integers(0, 20001)) if g.random() < 0.8 else int(g.integers(0, 9))
        runs.append((off, n))
        off += n + int(g.integers(0, 9))
    extent = off + 3
    reps_host = _replicas(g, W, extent, dt, scale=1.5 if op == "product" else 1.0)
    reps = [to_dev(h) for h in reps_host]
    in_place = bool(g.integers(0, 2))
    k = int(g.integers(0, W))
    out = reps[k] if in_place else empty_dev(extent, dt)
    print(f"op fuzz seed {seed}: W={W} {dt} {op} runs={len(runs)} in_place={in_place}", flush=True)
    nat.allreduce_op([r.data_ptr() for r in reps], code(dt), OPS[op], [a for a, _ in runs], [n for _, n in runs],
                     out.data_ptr(), stream())
    got = to_host(out)
    want = reps_host[k].copy() if in_place else np.full(extent, SENTINEL[dt], dtype=got.dtype)
    for a, n in runs:
        want[a : a + n] = o.allreduce_op([h[a : a + n] for h in reps_host], dt, op)
    assert same_bits(got, want), first_mismatch(got, want)
    for r in range(W):
        if not (in_place and r == k):
            assert same_bits(to_host(reps[r]), reps_host[r]), f"replica {r} was written"
