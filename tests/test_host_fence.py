"""The IpcGroup's host fence (comm._HostFence) with W processes on the CPU (gloo).

The fence is the barrier between the steps of an IpcGroup collective: every
rank's rows are written before any peer reads them, and read before any rank
writes again.  Checked here without a GPU: the barrier orders the ranks (no
rank leaves barrier k before every rank has entered it), the payloads of
every barrier arrive intact in rank order even when ranks run ahead, a rank
that never arrives makes the others fail with an error instead of hanging,
and nothing is left in /dev/shm.
"""

from __future__ import annotations

import os
import time
from datetime import timedelta

import numpy as np
import pytest
import torch.distributed as dist
import torch.multiprocessing as mp

from minidist.comm import _HostFence


def _segments() -> set[str]:
    try:
        return {n for n in os.listdir("/dev/shm") if n.startswith("mdx_fence_")}
    except FileNotFoundError:
        return set()


def _worker(rank: int, world: int, store: str, out_dir: str, rounds: int) -> None:
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        fence = _HostFence(dist.group.WORLD, world, rank, timeout_s=30)
        seen = np.zeros((rounds, world, 3), dtype=np.int64)
        enter, leave = np.zeros(rounds, dtype=np.int64), np.zeros(rounds, dtype=np.int64)
        for k in range(rounds):
            if (k + rank) % 7 == 0:
                time.sleep(0.002)  # some ranks arrive late, others run ahead
            enter[k] = time.monotonic_ns()  # the host's clock, shared by its processes
            seen[k] = fence.wait([rank, k, 1000 * rank + k])
            leave[k] = time.monotonic_ns()
        t0 = time.perf_counter()
        for _ in range(2000):
            fence.wait()
        us = (time.perf_counter() - t0) / 2000 * 1e6
        fence.close()
        np.savez(os.path.join(out_dir, f"fence_r{rank}.npz"), seen=seen, enter=enter, leave=leave, us=np.array(us))
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("world", [2, 4])
def test_fence_orders_ranks_and_carries_payloads(tmp_path, world):
    before = _segments()
    rounds = 200
    mp.spawn(_worker, args=(world, str(tmp_path / "store"), str(tmp_path), rounds), nprocs=world, join=True)
    res = [np.load(tmp_path / f"fence_r{r}.npz", allow_pickle=False) for r in range(world)]
    want = np.array([[[r, k, 1000 * r + k] for r in range(world)] for k in range(rounds)], dtype=np.int64)
    for r in range(world):
        assert np.array_equal(res[r]["seen"], want), f"rank {r} read another barrier's payloads"
    # No rank leaves barrier k before every rank has entered it.
    enter = np.stack([res[r]["enter"] for r in range(world)], axis=1)
    leave = np.stack([res[r]["leave"] for r in range(world)], axis=1)
    assert (leave.min(axis=1) >= enter.max(axis=1)).all()
    print(f"W={world}: {float(res[0]['us']):.1f} us per host fence", flush=True)
    assert _segments() == before  # rank 0 unlinked the segment once every rank had mapped it


def _absent_worker(rank: int, world: int, store: str, out_dir: str) -> None:
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        fence = _HostFence(dist.group.WORLD, world, rank, timeout_s=2)
        fence.wait()
        error = ""
        if rank == 0:
            try:
                fence.wait()  # rank 1 never comes to this one
            except RuntimeError as exc:
                error = str(exc)
        fence.close()
        with open(os.path.join(out_dir, f"absent_r{rank}.txt"), "w") as fh:
            fh.write(error)
    finally:
        dist.destroy_process_group()


def test_fence_times_out_on_an_absent_rank(tmp_path):
    mp.spawn(_absent_worker, args=(2, str(tmp_path / "store"), str(tmp_path)), nprocs=2, join=True)
    error = (tmp_path / "absent_r0.txt").read_text()
    assert "ranks [1] did not reach host barrier 2" in error
