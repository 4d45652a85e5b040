"""All-reduces over IPC-mapped rows: W processes on the one GPU (comm.IpcGroup).

W processes (2, 3 or 4, all on ``cuda:0``) meet in a gloo group, which carries
only host traffic: the IPC handles of each rank's contribution rows and the
barriers of the protocol.  DDP over an ``IpcGroup`` packs each rank's
gradients into its own row (``mdx_pack``, x 1/W), and after every rank's pack
is done each rank runs the fused rank-ordered reduction + unpack + unscale +
found-inf over the W rows -- its peers' rows read through their IPC mappings.
One-shot: every rank reduces the whole bucket run itself.  Two-shot: every
rank reduces its 1/W share into its (symmetric) bucket, and after a second
barrier unpacks its peers' shares out of their buckets.  The reference hands
each bucket to ``dist.all_reduce`` (minidist/comm.py:223-234, ddp.py:243-274).

Every rank's gradients are checked bit for bit against the oracle's
rank-ordered pipeline over all ranks' seeded gradients, for two steps: the
second with an inf in one rank's gradients, which every rank must flag.
"""

from __future__ import annotations

import os
import time
from datetime import timedelta

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

import tiny_gpt
from conftest import first_mismatch, same_bits
from minidist import DDP, FSDP, DistributedGradScaler, IpcGroup, MixedPrecisionPolicy, comm
from minidist import workloads as wl
from oracle import gradpath as o

pytestmark = pytest.mark.gpu
SCALE = 2.0**16
CAP_MB = 1.0
CFG = dict(n_layer=4, n_embd=256, vocab=1024, ctx=128)  # 52 gradients: one device plan
INF_AT = (1, 3, 17)  # (rank, parameter, element) that overflows in step 1


DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _grads(rank: int, specs, dtype: torch.dtype = torch.float32) -> list[torch.Tensor]:
    g = torch.Generator().manual_seed(1234 + 7919 * rank)
    return [(torch.randn(s.numel, generator=g) * (1e-2 * SCALE)).to(dtype) for s in specs]


def _host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().reshape(-1).cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def _worker(rank: int, world: int, store: str, out_dir: str, dtype_name: str, algorithm: str,
            segment_bytes: int) -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    dtype = DTYPES[dtype_name]
    try:
        group = IpcGroup(dist.group.WORLD, dev, algorithm=algorithm, segment_bytes=segment_bytes)
        specs = wl.gpt_specs(**CFG, dtype=dtype)
        model = wl.SpecModule(specs, dev)
        params = list(model.parameters())
        scaler = DistributedGradScaler(init_scale=SCALE, process_group=group)
        # bf16 parameters: fp32 buckets, with the contributions travelling as bf16 (widening)
        ddp = DDP(model, process_group=group, bucket_cap_mb=CAP_MB, grad_scaler=scaler,
                  reduce_dtype=torch.float32 if dtype != torch.float32 else None)

        class _Opt:
            param_groups = [{"params": params}]

        host = _grads(rank, specs, dtype)
        out = {"buckets": np.array(len(ddp._buckets))}
        for step in range(2):
            if step == 1:
                out["segments"] = np.array(len({b.segment for b in ddp._buckets}))
            for i, (p, g) in enumerate(zip(params, host, strict=True)):
                t = g.clone()
                if step == 1 and (rank, i) == INF_AT[:2]:
                    t[INF_AT[2]] = float("inf")
                p.grad = t.to(dev).view(p.shape)
            t0 = time.perf_counter()
            ddp.finish_gradient_sync()
            found = scaler.unscale_(_Opt())
            out[f"ms_{step}"] = np.array((time.perf_counter() - t0) * 1e3)
            scaler.update()
            out[f"found_{step}"] = np.array(found)
            for i, p in enumerate(params):
                out[f"grad_{step}_{i}"] = _host_bits(p.grad)
        if algorithm == "two_shot":  # the peers read each rank's reduced share out of its buckets
            for b in ddp._buckets:
                group._rows_of(b.buffer)  # raises unless the bucket lies in a symmetric buffer
        if dtype == torch.float32:
            # the reference's own per-bucket sequence over the same group: gather_into_buffer,
            # comm.all_reduce (one-shot SUM of the rows into the bucket), scatter_from_buffer
            for p, g in zip(params, host, strict=True):
                p.grad = g.clone().to(dev).view(p.shape)
            for b in ddp._buckets:
                row = b.gather_into_buffer(1.0 / world)
                comm.all_reduce(row, group=group)
                b.scatter_from_buffer()
            for i, p in enumerate(params):
                out[f"grad_ref_{i}"] = _host_bits(p.grad)
        group.release()
        np.savez(os.path.join(out_dir, f"ipc_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


SEGMENT = 1 << 30  # the default: the model's buckets fit one symmetric buffer per dtype
SMALL_SEGMENT = 4 << 20  # the tiny GPT's 13.8 MB of buckets spread over several buffers


@pytest.mark.parametrize("world,dtype,algorithm,segment_bytes",
                         [(2, "f32", "one_shot", SEGMENT), (3, "f32", "one_shot", SEGMENT),
                          (4, "f32", "one_shot", SEGMENT), (2, "bf16", "one_shot", SEGMENT),
                          (4, "bf16", "one_shot", SEGMENT), (2, "f32", "two_shot", SEGMENT),
                          (3, "f32", "two_shot", SEGMENT), (4, "f32", "two_shot", SEGMENT),
                          (3, "bf16", "two_shot", SEGMENT), (4, "bf16", "two_shot", SEGMENT),
                          (2, "bf16", "one_shot", SMALL_SEGMENT), (3, "f32", "two_shot", SMALL_SEGMENT),
                          (3, "f16", "one_shot", SEGMENT), (4, "f16", "two_shot", SMALL_SEGMENT)])
def test_ipc_all_reduce_bitwise(tmp_path, world, dtype, algorithm, segment_bytes):
    """fp32 gradients into fp32 buckets, or bf16 / fp16 gradients into fp32 buckets with 16-bit rows; in fp32
    also the reference's per-bucket sequence through comm.all_reduce over the group.  Two-shot:
    each rank reduces and unpacks its share of every bucket run, then unpacks its peers' shares
    out of their (symmetric) buckets.  A small ``segment_bytes`` spreads the buckets over several
    symmetric buffers, each launch run then one collective per buffer."""
    store = str(tmp_path / "store")
    print(f"spawning {world} ranks on cuda:0 (IpcGroup {algorithm} all-reduce, {dtype}, "
          f"segments of {segment_bytes} bytes)", flush=True)
    mp.spawn(_worker, args=(world, store, str(tmp_path), dtype, algorithm, segment_bytes), nprocs=world, join=True)
    res = []
    for r in range(world):
        with np.load(tmp_path / f"ipc_r{r}.npz", allow_pickle=False) as d:
            res.append({k: d[k] for k in d.files})
    tdt = DTYPES[dtype]
    odt = {"f32": o.F32, "bf16": o.BF16, "f16": o.F16}[dtype]
    specs = wl.gpt_specs(**CFG, dtype=tdt)
    numels = [s.numel for s in specs]
    n = len(specs)
    assert int(res[0]["buckets"]) > 2
    assert (int(res[0]["segments"]) > 2) == (segment_bytes == SMALL_SEGMENT)
    for step in range(2):
        replica = [[_host_bits(g) for g in _grads(r, specs, tdt)] for r in range(world)]
        if step == 1:
            rr, i, k = INF_AT
            replica[rr][i] = replica[rr][i].copy()
            replica[rr][i][k] = np.uint16(0x7F80) if odt == o.BF16 else np.inf
        for rank in range(world):
            want = o.ddp_pipeline(replica, [odt] * n, numels, CAP_MB, rank, 1.0 / SCALE,
                                  bucket_dtype=o.F32)
            assert bool(res[rank][f"found_{step}"]) == want["found_inf"] == (step == 1)
            for i in range(n):
                got = res[rank][f"grad_{step}_{i}"]
                assert same_bits(got, want["grads"][i]), (
                    f"step {step} rank {rank} param {i}: " + first_mismatch(got, want["grads"][i]))
            if step == 0 and dtype == "f32":
                for i in range(n):  # the reference's sequence: the unscaled average, not unscaled
                    want_ref = o.ddp_pipeline(replica, [odt] * n, numels, CAP_MB, rank, None)["grads"][i]
                    got = res[rank][f"grad_ref_{i}"]
                    assert same_bits(got, want_ref), f"reference sequence rank {rank} param {i}"
    print("step ms per rank:", [[float(res[r][f"ms_{s}"]) for s in range(2)] for r in range(world)], flush=True)


SMALL = (1000, 3000, 3000, 100)  # small symmetric buffers, each an allocation of its own.  Buffer 2 is
# reduced in two views with a gap between them, which keeps each rank's own data; buffer 3 is small
# enough that a two-shot group of three gives one rank an empty share.
GAP = (1000, 2000)


def _small_rows(rank: int, step: int) -> list[np.ndarray]:
    g = np.random.default_rng(77 + 1009 * rank + 31 * step)
    return [(g.standard_normal(n) * 1e3).astype(np.float32) for n in SMALL]


RS_S = 777  # elements of a reduce-scatter output / an all-gather input


def _rs_rows(rank: int, world: int) -> np.ndarray:
    return (np.random.default_rng(991 + rank).standard_normal(RS_S * world) * 1e2).astype(np.float32)


def _in_place_worker(rank: int, world: int, store: str, out_dir: str, algorithm: str) -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        group = IpcGroup(dist.group.WORLD, dev, algorithm=algorithm)
        rows = [group.zeros(n, torch.float32) for n in SMALL]
        out = {"mapped": np.array(len(group._mapped))}
        for step in range(2):
            for row, host in zip(rows, _small_rows(rank, step), strict=True):
                row.copy_(torch.from_numpy(host).to(dev))
            comm.all_reduce(rows[0], group=group)  # in place, one buffer
            comm.all_reduce_coalesced([rows[1][:1500], rows[1][1500:]], group=group)  # two views of the other
            comm.all_reduce_coalesced([rows[2][: GAP[0]], rows[2][GAP[1] :]], group=group)  # views with a gap
            comm.all_reduce(rows[3], group=group)
            for k, row in enumerate(rows):
                out[f"sum_{step}_{k}"] = row.cpu().numpy()
        # comm.reduce_scatter_tensor / all_gather_into_tensor (reference comm.py:237-265) over the rows
        rs_in, ag_in = group.zeros(RS_S * world, torch.float32), group.zeros(RS_S, torch.float32)
        rs_in.copy_(torch.from_numpy(_rs_rows(rank, world)).to(dev))
        ag_in.copy_(torch.from_numpy(_rs_rows(rank, world)[:RS_S]).to(dev))
        rs_out = torch.empty(RS_S, device=dev)
        ag_out = torch.empty(RS_S * world, device=dev)
        comm.reduce_scatter_tensor(rs_out, rs_in, group=group)
        comm.all_gather_into_tensor(ag_out, ag_in, group=group)
        out["rs"], out["ag"] = rs_out.cpu().numpy(), ag_out.cpu().numpy()
        if algorithm == "two_shot":
            # each rank reduces its share of the runs for all the others: ranks handing in
            # different runs are told so, every one of them, before anything is launched
            try:
                comm.all_reduce(rows[0][: 100 + 10 * rank], group=group)
            except RuntimeError as e:
                assert "different runs" in str(e)
            else:
                raise AssertionError("a two-shot all-reduce accepted different runs on different ranks")
        # ranks asking for different symmetric buffers are told so, every one of them, before any
        # peer row is mapped
        try:
            group.zeros(64 + rank, torch.float32)
        except RuntimeError as e:
            assert "different buffers" in str(e)
        else:
            raise AssertionError("IpcGroup.zeros accepted rows of different sizes")
        group.release()
        # a released group maps nothing: every further use is refused, nothing is launched
        for use in (lambda: comm.all_reduce(rows[0], group=group), lambda: group.zeros(16, torch.float32),
                    group.rows_written):
            try:
                use()
            except RuntimeError as e:
                assert "released" in str(e)
            else:
                raise AssertionError("a released IpcGroup accepted a collective")
        np.savez(os.path.join(out_dir, f"inplace_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("world,algorithm", [(2, "one_shot"), (3, "one_shot"), (2, "two_shot"), (3, "two_shot")])
def test_ipc_in_place_all_reduce(tmp_path, world, algorithm):
    """``comm.all_reduce`` in place on rows of an IpcGroup buffer with no reduce target: every rank
    ends with the rank-ordered sum while its peers read its row concurrently, elements between
    reduced views keep each rank's own data, and every row is an allocation of its own, mapped
    once by each peer.  Then ``comm.reduce_scatter_tensor`` and ``comm.all_gather_into_tensor`` over
    symmetric rows."""
    store = str(tmp_path / "store")
    print(f"spawning {world} ranks on cuda:0 (IpcGroup {algorithm} in-place all-reduce)", flush=True)
    mp.spawn(_in_place_worker, args=(world, store, str(tmp_path), algorithm), nprocs=world, join=True)
    for step in range(2):
        hosts = [_small_rows(r, step) for r in range(world)]
        for k in range(len(SMALL)):
            total = hosts[0][k].copy()
            for r in range(1, world):
                total = total + hosts[r][k]  # float32, rank order 0..W-1
            for rank in range(world):
                want = total.copy()
                if k == 2:  # outside the reduced views each rank keeps its own data
                    want[GAP[0] : GAP[1]] = hosts[rank][k][GAP[0] : GAP[1]]
                with np.load(tmp_path / f"inplace_r{rank}.npz", allow_pickle=False) as d:
                    got = d[f"sum_{step}_{k}"]
                    assert int(d["mapped"]) == len(SMALL) * (world - 1)
                assert same_bits(got, want), f"step {step} buffer {k} rank {rank}: " + first_mismatch(got, want)
    inputs = [_rs_rows(r, world) for r in range(world)]
    for rank in range(world):
        with np.load(tmp_path / f"inplace_r{rank}.npz", allow_pickle=False) as d:
            rs, ag = d["rs"], d["ag"]
        want = inputs[0][rank * RS_S : (rank + 1) * RS_S].copy()
        for r in range(1, world):
            want = want + inputs[r][rank * RS_S : (rank + 1) * RS_S]  # float32, rank order
        assert same_bits(rs, want), f"reduce_scatter rank {rank}: " + first_mismatch(rs, want)
        want_ag = np.concatenate([x[:RS_S] for x in inputs])
        assert same_bits(ag, want_ag), f"all_gather rank {rank}: " + first_mismatch(ag, want_ag)


FSDP_DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _fsdp_worker(rank: int, world: int, store: str, out_dir: str, dtype_name: str, unit_batch: int,
                 accumulate: bool = False, segment_bytes: int = SEGMENT, keep_low: bool = False) -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        group = IpcGroup(dist.group.WORLD, dev, segment_bytes=segment_bytes)
        c = tiny_gpt.Config(n_layer=2)
        model = tiny_gpt.GPT(c, seed=rank).to(dev)  # the construction broadcast makes them rank 0's
        params = list(model.parameters())
        index = {id(p): i for i, p in enumerate(params)}
        local: dict[int, torch.Tensor] = {}

        def capture(p):
            local[id(p)] = p.grad.detach().clone()

        for p in params:
            p.register_post_accumulate_grad_hook(capture)
        policy = MixedPrecisionPolicy(param_dtype=FSDP_DTYPES[dtype_name], reduce_dtype=torch.float32,
                                      keep_low_precision_shard=keep_low)
        fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=group, mixed_precision=policy,
                    unit_batch=unit_batch)
        scaler = DistributedGradScaler(init_scale=16.0, process_group=group)
        out = {"units": np.array(len(fsdp._units)), "segments": np.array(len({u.segment for u in fsdp._units}))}
        for u, unit in enumerate(fsdp._units):
            out[f"unit_{u}_params"] = np.array([index[id(p)] for p in unit.params])
        with fsdp.summon_full_params():
            for u, unit in enumerate(fsdp._units):
                out[f"full_{u}"] = _host_bits(unit._full)
        ids, tgt = tiny_gpt.batch(c, 12, seed=6)
        my_ids, my_tgt = ids.chunk(world)[rank].to(dev), tgt.chunk(world)[rank].to(dev)
        if accumulate:
            # two halves under no_sync, then the flush: every unit's share in one multi-unit exchange
            with fsdp.no_sync():
                for h_ids, h_tgt in zip(my_ids.chunk(2), my_tgt.chunk(2), strict=True):
                    _, loss = fsdp(h_ids, h_tgt)
                    (loss / 2).backward()
            fsdp.finish_gradient_sync()
        else:
            _, loss = fsdp(my_ids, my_tgt)
            loss.backward()
        for i, p in enumerate(params):
            out[f"local_{i}"] = _host_bits(local[id(p)])
        for u, unit in enumerate(fsdp._units):
            out[f"shard_grad_{u}"] = _host_bits(unit.flat_shard.grad)
            assert not unit.is_unsharded and all(p.grad is None for p in unit.params)

        class _Opt:
            param_groups = [{"params": list(fsdp.parameters())}]

        if rank == world - 1:  # one rank's shard overflows: every rank must skip
            with torch.no_grad():
                fsdp._units[0].flat_shard.grad[0] = float("inf")
        out["found"] = np.array(scaler.unscale_(_Opt()))
        group.release()
        np.savez(os.path.join(out_dir, f"ipc_fsdp_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


# A tiny-GPT block unit is 12,704 elements (the root 4,672): 64 KB of fp32 rows put every unit in a
# buffer of its own; 40 KB of 16-bit rows put the two blocks apart and the root with the second.
@pytest.mark.parametrize("world,dtype,unit_batch,accumulate,segment_bytes,keep_low",
                         [(2, "f32", 1, False, SEGMENT, False), (3, "bf16", 1, False, SEGMENT, False),
                          (4, "bf16", 2, False, SEGMENT, False), (2, "f16", 3, False, SEGMENT, False),
                          (3, "f32", 1, True, SEGMENT, False), (2, "bf16", 2, True, SEGMENT, False),
                          (3, "bf16", 2, False, 40_000, False), (2, "f32", 1, True, 64_000, False),
                          (3, "bf16", 2, False, SEGMENT, True), (2, "f16", 1, True, SEGMENT, True)])
def test_ipc_fsdp_one_shot_bitwise(tmp_path, world, dtype, unit_batch, accumulate, segment_bytes, keep_low):
    """FSDP over an IpcGroup: each unit's all-gather is its ranks' published shards copied from the
    mapped rows, its reduce-scatter the share kernel over every rank's published full-size gradient
    (the reference's fsdp.py:172-241 with comm.all_gather_into_tensor / reduce_scatter_tensor).
    Gathered parameters, every rank's shard gradient (against the oracle on the ranks' captured
    local gradients) and the found-inf flag exchanged over the host group.  ``accumulate``: two
    half-batch backwards under ``no_sync`` and the flush of every unit at once.  A small
    ``segment_bytes`` spreads the units over several pairs of symmetric buffers.  ``keep_low``: the
    master shards (and their gradients) in the gather dtype."""
    store = str(tmp_path / "store")
    print(f"spawning {world} ranks on cuda:0 (FSDP over an IpcGroup, {dtype}, unit_batch={unit_batch}, "
          f"segments of {segment_bytes} bytes)", flush=True)
    mp.spawn(_fsdp_worker, args=(world, store, str(tmp_path), dtype, unit_batch, accumulate, segment_bytes,
                                 keep_low), nprocs=world, join=True)
    res = []
    for r in range(world):
        with np.load(tmp_path / f"ipc_fsdp_r{r}.npz", allow_pickle=False) as d:
            res.append({k: d[k] for k in d.files})
    c = tiny_gpt.Config(n_layer=2)
    init0 = [p.detach().reshape(-1).numpy().copy() for p in tiny_gpt.GPT(c, seed=0).parameters()]
    pdt = {"f32": o.F32, "bf16": o.BF16, "f16": o.F16}[dtype]
    n_units = int(res[0]["units"])
    assert n_units == c.n_layer + 1
    assert int(res[0]["segments"]) == {SEGMENT: 1, 40_000: 2, 64_000: 3}[segment_bytes]
    for u in range(n_units):
        idx = [int(i) for i in res[0][f"unit_{u}_params"]]
        numels = [init0[i].size for i in idx]
        _, S, P = o.fsdp_layout(numels, world)
        flat = np.zeros(P, np.float32)
        flat[: sum(numels)] = np.concatenate([init0[i] for i in idx])
        gathered = o.fsdp_gather_cast(flat, pdt)
        grads = [[res[r][f"local_{i}"] for i in idx] for r in range(world)]
        for rank in range(world):
            assert same_bits(res[rank][f"full_{u}"], gathered), f"unit {u} rank {rank}: all-gather"
            want = o.fsdp_reduce_scatter_share(grads, pdt, numels, rank, o.F32, pdt if keep_low else o.F32)
            got = res[rank][f"shard_grad_{u}"]
            assert same_bits(got, want), f"unit {u} rank {rank}: " + first_mismatch(got, want)
    assert all(bool(res[r]["found"]) for r in range(world))


BACKWARD_CAP_MB = 0.01  # several bucket runs, launched while backward runs


def _ddp_backward_worker(rank: int, world: int, store: str, out_dir: str, comm_stream: bool = False,
                         algorithm: str = "one_shot") -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        group = IpcGroup(dist.group.WORLD, dev, algorithm=algorithm)
        c = tiny_gpt.Config(n_layer=2)
        model = tiny_gpt.GPT(c, seed=rank).to(dev)  # the construction broadcast makes them rank 0's
        params = list(model.parameters())
        local: dict[int, torch.Tensor] = {}
        state = {"inject": False}

        def capture(p):
            if state["inject"] and rank == 1 and p is params[3]:
                p.grad.view(-1)[5] = float("inf")  # this rank's backward overflowed
            local[id(p)] = p.grad.detach().clone()

        for p in params:
            p.register_post_accumulate_grad_hook(capture)
        scaler = DistributedGradScaler(init_scale=SCALE, process_group=group)
        ddp = DDP(model, process_group=group, bucket_cap_mb=BACKWARD_CAP_MB, grad_scaler=scaler,
                  comm_stream=comm_stream)
        out = {"buckets": np.array(len(ddp._buckets))}

        class _Opt:
            param_groups = [{"params": params}]

        ids, tgt = tiny_gpt.batch(c, 12, seed=5)
        for step in range(2):
            state["inject"] = step == 1
            for p in params:
                p.grad = None
            _, loss = ddp(ids.chunk(world)[rank].to(dev), tgt.chunk(world)[rank].to(dev))
            scaler.scale_loss(loss).backward()
            out[f"found_{step}"] = np.array(scaler.unscale_(_Opt()))
            scaler.update()
            for i, p in enumerate(params):
                out[f"local_{step}_{i}"] = _host_bits(local[id(p)])
                out[f"final_{step}_{i}"] = _host_bits(p.grad)
        group.release()
        np.savez(os.path.join(out_dir, f"ipc_bwd_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("world,comm_stream,algorithm",
                         [(2, False, "one_shot"), (3, False, "one_shot"), (2, True, "one_shot"),
                          (3, False, "two_shot"), (2, True, "two_shot")])
def test_ipc_ddp_during_backward_bitwise(tmp_path, world, comm_stream, algorithm):
    """DDP over an IpcGroup inside a real backward: bucket runs launch from the autograd hooks as
    they fill (pack, fences, the one-shot reduction over the mapped rows), two steps, the second
    with an overflow on one rank that every rank must skip.  Every rank's gradients against the
    oracle's pipeline over all ranks' captured local gradients.  ``comm_stream``: the packs, fences
    and reductions on DDP's dedicated stream."""
    store = str(tmp_path / "store")
    print(f"spawning {world} ranks on cuda:0 (DDP over an {algorithm} IpcGroup, real backward, "
          f"comm_stream={comm_stream})", flush=True)
    mp.spawn(_ddp_backward_worker, args=(world, store, str(tmp_path), comm_stream, algorithm), nprocs=world,
             join=True)
    res = []
    for r in range(world):
        with np.load(tmp_path / f"ipc_bwd_r{r}.npz", allow_pickle=False) as d:
            res.append({k: d[k] for k in d.files})
    assert int(res[0]["buckets"]) > 2
    c = tiny_gpt.Config(n_layer=2)
    numels = [p.numel() for p in tiny_gpt.GPT(c, seed=0).parameters()]
    n = len(numels)
    for step in range(2):
        grads = [[res[r][f"local_{step}_{i}"] for i in range(n)] for r in range(world)]
        for rank in range(world):
            want = o.ddp_pipeline(grads, [o.F32] * n, numels, BACKWARD_CAP_MB, rank, 1.0 / SCALE)
            assert bool(res[rank][f"found_{step}"]) == want["found_inf"] == (step == 1)
            for i in range(n):
                got = res[rank][f"final_{step}_{i}"]
                assert same_bits(got, want["grads"][i]), (
                    f"step {step} rank {rank} param {i}: " + first_mismatch(got, want["grads"][i]))


def _full_size_worker(rank: int, world: int, store: str, out_dir: str) -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=120))
    try:
        groups = {a: IpcGroup(dist.group.WORLD, dev, algorithm=a) for a in IpcGroup.ALGORITHMS}
        specs = wl.gpt_specs(**wl.GPT2_SMALL)
        model = wl.SpecModule(specs, dev)
        params = list(model.parameters())
        gen = torch.Generator(device=dev).manual_seed(4321 + 17 * rank)
        inputs = [torch.randn(p.shape, device=dev, generator=gen) * (1e-3 * SCALE) for p in params]
        if rank == world - 1:
            inputs[7].view(-1)[inputs[7].numel() // 2] = float("inf")  # one rank overflowed: both must flag it
        out = {}
        results = {}
        for name, group in groups.items():
            scaler = DistributedGradScaler(init_scale=SCALE, process_group=group)
            ddp = DDP(model, process_group=group, grad_scaler=scaler, broadcast_parameters=False)

            class _Opt:
                param_groups = [{"params": params}]

            for p, g in zip(params, inputs, strict=True):
                p.grad = g.clone()
            ddp.finish_gradient_sync()
            out[f"found_{name}"] = np.array(scaler.unscale_(_Opt()))
            out[f"buckets_{name}"] = np.array(len(ddp._buckets))
            results[name] = [p.grad.detach().clone() for p in params]
            out[f"bucket_sum_{name}"] = np.array(sum(float(b.buffer.double().nan_to_num(0.0, 0.0, 0.0).sum())
                                                     for b in ddp._buckets))
            del ddp
        one, two = results["one_shot"], results["two_shot"]
        out["equal"] = np.array(all(torch.equal(a.view(torch.int32), b.view(torch.int32))
                                    for a, b in zip(one, two, strict=True)))
        for group in groups.values():
            group.release()
        np.savez(os.path.join(out_dir, f"full_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


def test_ipc_two_shot_equals_one_shot_at_cfg1_size(tmp_path):
    """cfg1's 124M fp32 gradients (148 tensors, 18 buckets in one run of 148 kernel-argument
    runs), two processes: the two-shot all-reduce gives every rank exactly the one-shot's
    gradients (which the oracle pins at small sizes), bit for bit, with an inf in one rank's
    gradient flagged on both."""
    world = 2
    store = str(tmp_path / "store")
    print(f"spawning {world} ranks on cuda:0 (one-shot against two-shot at cfg1 size)", flush=True)
    mp.spawn(_full_size_worker, args=(world, store, str(tmp_path)), nprocs=world, join=True)
    for rank in range(world):
        with np.load(tmp_path / f"full_r{rank}.npz", allow_pickle=False) as d:
            assert int(d["buckets_one_shot"]) == int(d["buckets_two_shot"]) == 18
            assert bool(d["found_one_shot"]) and bool(d["found_two_shot"])
            assert bool(d["equal"]), f"rank {rank}: two-shot gradients differ from one-shot"
            assert float(d["bucket_sum_one_shot"]) == float(d["bucket_sum_two_shot"])


ROW = 1 << 20  # fp32 elements of the row allocated after a large block was cached


def _cached_segment_worker(rank: int, world: int, store: str, out_dir: str) -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        big = torch.empty(3 << 30, dtype=torch.uint8, device=dev)
        del big  # the caching allocator keeps the 3 GiB segment: a small request could be carved from it
        from minidist import _native

        group = IpcGroup(dist.group.WORLD, dev)
        row = group.zeros(ROW, torch.float32)
        h = _native.ipc_export(row.data_ptr())
        row.fill_(float(rank + 1))
        torch.cuda.synchronize()
        dist.barrier()
        seen = []
        for r, addr in enumerate(group.row_addresses(row)):  # every rank's row, through its mapping
            copy = torch.empty(ROW, device=dev)
            _native.pack(_native.spans_array([(addr, copy.data_ptr(), ROW)]), _native.MDX_F32, _native.MDX_F32,
                         1.0, False, torch.cuda.current_stream(dev).cuda_stream)
            torch.cuda.synchronize()
            seen.append(copy.cpu().numpy())
        dist.barrier()
        group.release()
        np.savez(os.path.join(out_dir, f"seg_r{rank}.npz"), offset=np.array(h.offset),
                 alloc=np.array(h.alloc_bytes), seen=np.stack(seen))
    finally:
        dist.destroy_process_group()


def test_ipc_row_is_its_own_allocation(tmp_path):
    """A symmetric row allocated while the caching allocator holds a 3 GiB free segment is still an
    allocation of its own: its IPC export starts at the row (offset 0) and covers the segment the
    allocator sizes for the request alone (20 MiB under 10 MiB, else the request rounded up to
    2 MiB), never split for another tensor -- not the cached segment, which the runtime could not
    map (2 GiB and more) and which would hand every peer unrelated tensors -- and each rank reads
    every peer's row through its mapping."""
    world = 2
    store = str(tmp_path / "store")
    print(f"spawning {world} ranks on cuda:0 (IpcGroup rows after a cached 3 GiB segment)", flush=True)
    mp.spawn(_cached_segment_worker, args=(world, store, str(tmp_path)), nprocs=world, join=True)
    for rank in range(world):
        with np.load(tmp_path / f"seg_r{rank}.npz", allow_pickle=False) as d:
            assert int(d["offset"]) == 0
            assert ROW * 4 <= int(d["alloc"]) <= max(20 << 20, -(-ROW * 4 // (2 << 20)) * (2 << 20))
            for r in range(world):
                assert np.all(d["seen"][r] == float(r + 1)), f"rank {rank} read rank {r}'s row"


OP_N, OP_S = 5000, 611  # all-reduce length; reduce-scatter share per rank


def _op_rows(rank: int, n: int, seed: int) -> np.ndarray:
    g = np.random.default_rng(seed + 131 * rank)
    x = (g.standard_normal(n) * 4).astype(np.float32)
    x[: n // 10] = np.random.default_rng(seed).standard_normal(n // 10).astype(np.float32)  # equal on every rank
    x[g.integers(0, n, n // 50)] = np.float32(-0.0 if rank % 2 else 0.0)
    x[g.integers(0, n, n // 200)] = np.float32(np.nan)
    x[g.integers(0, n, n // 200)] = np.float32(np.inf if rank % 2 else -np.inf)
    return x


def _op_worker(rank: int, world: int, store: str, out_dir: str, algorithm: str) -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        group = IpcGroup(dist.group.WORLD, dev, algorithm=algorithm)
        out = {}
        for k, (name, op) in enumerate((("max", dist.ReduceOp.MAX), ("min", dist.ReduceOp.MIN),
                                        ("product", dist.ReduceOp.PRODUCT))):
            row = group.zeros(OP_N, torch.float32)
            row.copy_(torch.from_numpy(_op_rows(rank, OP_N, 10 + k)).to(dev))
            comm.all_reduce(row, op=op, group=group)  # in place: peers read this row meanwhile
            out[f"ar_{name}"] = row.cpu().numpy()
            inp = group.zeros(OP_S * world, torch.float32)
            inp.copy_(torch.from_numpy(_op_rows(rank, OP_S * world, 20 + k)).to(dev))
            rs = torch.empty(OP_S, device=dev)
            comm.reduce_scatter_tensor(rs, inp, op=op, group=group)
            out[f"rs_{name}"] = rs.cpu().numpy()
        group.release()
        np.savez(os.path.join(out_dir, f"op_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("world,algorithm", [(2, "one_shot"), (3, "two_shot"), (4, "one_shot")])
def test_ipc_non_sum_ops(tmp_path, world, algorithm):
    """``comm.all_reduce`` (in place) and ``comm.reduce_scatter_tensor`` with MAX, MIN and PRODUCT over
    an IpcGroup: one-shot over the mapped rows whatever the group's algorithm, every rank's result
    bit for bit the oracle's rank-ordered fold (NaN, +-inf, +-0 and values equal on every rank)."""
    store = str(tmp_path / "store")
    print(f"spawning {world} ranks on cuda:0 (IpcGroup {algorithm}: MAX / MIN / PRODUCT)", flush=True)
    mp.spawn(_op_worker, args=(world, store, str(tmp_path), algorithm), nprocs=world, join=True)
    for k, name in enumerate(("max", "min", "product")):
        want_ar = o.allreduce_op([_op_rows(r, OP_N, 10 + k) for r in range(world)], o.F32, name)
        rs_in = [_op_rows(r, OP_S * world, 20 + k) for r in range(world)]
        for rank in range(world):
            with np.load(tmp_path / f"op_r{rank}.npz", allow_pickle=False) as d:
                got_ar, got_rs = d[f"ar_{name}"], d[f"rs_{name}"]
            assert same_bits(got_ar, want_ar), f"all_reduce {name} rank {rank}: " + first_mismatch(got_ar, want_ar)
            want_rs = o.allreduce_op([x[rank * OP_S : (rank + 1) * OP_S] for x in rs_in], o.F32, name)
            assert same_bits(got_rs, want_rs), f"reduce_scatter {name} rank {rank}: " + first_mismatch(got_rs, want_rs)
