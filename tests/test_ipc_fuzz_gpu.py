"""Seeded random DDP pipelines and FSDP steps over IPC-mapped rows: W processes on the one GPU
(comm.IpcGroup).

DDP:

Each case draws W in [2, 4], one- or two-shot, the gradient dtype (fp32, bf16
or fp16, the 16-bit ones optionally widened into fp32 buckets), 10-30
parameters of ragged shapes (some empty), a bucket cap from one bucket per
parameter to a single bucket, the symmetric-buffer segment size (so that the
buckets spread over one or several buffers), DDP's communication stream or
not, and the fused scaler or not.  Every rank draws every rank's gradients from
the same seed, with rare special values and, on some ranks, parameters that
received no gradient.  Two steps run (new gradient tensors in the second).
Every rank's gradients and buckets are checked bit for bit against the oracle's
rank-ordered pipeline (``oracle.gradpath.ddp_pipeline``) over all ranks'
gradients, and the found-inf decision against the oracle's.  The reference
hands each bucket to ``dist.all_reduce`` (minidist/comm.py:223-234,
ddp.py:243-274).

FSDP: each case draws W in [2, 4], 1-5 units of random width (frozen biases,
empty parameters) plus the root, the gather dtype, ``unit_batch``,
``reshard_after_forward``, ``keep_low_precision_shard``, one or several
symmetric buffers, and accumulation under ``no_sync`` with the final flush.
Every rank runs its own backward on its own input; every unit's gathered
parameters against the oracle's cast of the initial weights, and every rank's
shard gradient against ``oracle.gradpath.fsdp_reduce_scatter_share`` over all
ranks' captured full-size gradients (the reference's fsdp.py:172-241 over
comm.all_gather_into_tensor / reduce_scatter_tensor).
"""

from __future__ import annotations

import os
from datetime import timedelta

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp
from torch import nn

from conftest import first_mismatch, same_bits
from minidist import DDP, FSDP, DistributedGradScaler, IpcGroup, MixedPrecisionPolicy
from oracle import gradpath as o
from test_fuzz_gpu import _FuzzBlock, _FuzzNet

pytestmark = pytest.mark.gpu
SPECIALS = np.array([np.inf, -np.inf, np.nan, 1e-45, -1e-40, 0.0, -0.0], dtype=np.float32)
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
STEPS = 2


def _case(seed: int) -> dict:
    """The whole case, drawn from ``seed`` alone (the parent and every rank draw the same)."""
    rng = np.random.default_rng(41000 + seed)
    dtype = DTYPES[int(rng.integers(0, 3))]
    widening = dtype != torch.float32 and bool(rng.random() < 0.5)
    gdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(dtype, o.F32)
    W = int(rng.integers(2, 5))
    algorithm = ["one_shot", "two_shot"][int(rng.integers(0, 2))]
    n_params = int(rng.integers(10, 31))
    shapes = []
    for _ in range(n_params):
        u = rng.random()
        shapes.append((0,) if u < 0.1 else (int(rng.integers(1, 5000)),) if u < 0.8
                      else (int(rng.integers(1, 60)), int(rng.integers(1, 50))))
    numels = [int(np.prod(s)) for s in shapes]
    esize = 4 if dtype == torch.float32 or widening else 2
    nbytes = [n * (4 if dtype == torch.float32 else 2) for n in numels]
    total_mb = sum(nbytes) / 2**20
    cap = float(rng.choice([1e-6, total_mb / 5, total_mb / 2, 1e6]))
    # segments: the default, or small enough that the buckets spread over several buffers
    largest = max(sum(numels[i] for i in idxs) for idxs in o.build_buckets(nbytes, cap))
    small = max(256, (largest * esize + 255) // 256 * 256, int(rng.integers(1, 5)) * 16384)
    segment_bytes = [1 << 30, small][int(rng.integers(0, 2))]
    use_scaler = bool(rng.random() < 0.6)
    scale = 2.0 ** int(rng.integers(0, 14 if dtype != torch.float16 else 10)) if use_scaler else 1.0
    comm_stream = bool(rng.random() < 0.4)
    grads = []  # [step][rank][param]
    for _ in range(STEPS):
        per_rank = []
        for _ in range(W):
            row = []
            for n in numels:
                g = (rng.standard_normal(n) * 1e-3 * scale).astype(np.float32)
                if n and rng.random() < 0.04:
                    g[int(rng.integers(0, n))] = SPECIALS[int(rng.integers(0, len(SPECIALS)))]
                row.append(o.from_f32(g, gdt))
            for i in rng.integers(0, n_params, int(rng.integers(0, 3))):  # never received on this rank
                row[int(i)] = None
            per_rank.append(row)
        grads.append(per_rank)
    return dict(dtype=dtype, widening=widening, gdt=gdt, W=W, algorithm=algorithm, shapes=shapes, numels=numels,
                cap=cap, segment_bytes=segment_bytes, use_scaler=use_scaler, scale=scale, comm_stream=comm_stream,
                grads=grads)


def _describe(seed: int, c: dict) -> str:
    return (f"ipc fuzz seed {seed}: W={c['W']} {c['algorithm']} {c['dtype']} widening={c['widening']} "
            f"params={len(c['shapes'])} cap={c['cap']:.3g} MB segment={c['segment_bytes']} "
            f"comm_stream={c['comm_stream']} scale={c['scale']:g}")


class _Flat(nn.Module):
    def __init__(self, shapes, dtype, dev):
        super().__init__()
        self.ps = nn.ParameterList([nn.Parameter(torch.zeros(s, dtype=dtype, device=dev)) for s in shapes])


def _to_dev(a: np.ndarray, shape, dev) -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(dev).view(shape)
    return torch.from_numpy(a.copy()).to(dev).view(shape)


def _host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().reshape(-1).cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def _worker(rank: int, world: int, store: str, out_dir: str, seed: int) -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        c = _case(seed)
        group = IpcGroup(dist.group.WORLD, dev, algorithm=c["algorithm"], segment_bytes=c["segment_bytes"])
        model = _Flat(c["shapes"], c["dtype"], dev)
        params = list(model.parameters())
        scaler = DistributedGradScaler(init_scale=c["scale"], process_group=group) if c["use_scaler"] else None
        ddp = DDP(model, process_group=group, bucket_cap_mb=c["cap"], grad_scaler=scaler,
                  reduce_dtype=torch.float32 if c["widening"] else None, comm_stream=c["comm_stream"])

        class _Opt:
            param_groups = [{"params": params}]

        out = {"buckets": np.array(len(ddp._buckets)), "segments": np.array(len({b.segment for b in ddp._buckets}))}
        for step in range(STEPS):
            for p, g in zip(params, c["grads"][step][rank], strict=True):
                p.grad = None if g is None else _to_dev(g, p.shape, dev)
            ddp.finish_gradient_sync()
            if scaler is not None:
                out[f"found_{step}"] = np.array(scaler.unscale_(_Opt()))
                scaler.update()
                out[f"scale_after_{step}"] = np.array(scaler.scale)
            torch.cuda.synchronize()
            for i, p in enumerate(params):
                out[f"grad_{step}_{i}"] = _host_bits(p.grad)
            for b, bucket in enumerate(ddp._buckets):
                out[f"bucket_{step}_{b}"] = _host_bits(bucket.buffer[: bucket.numel])
        group.release()
        np.savez(os.path.join(out_dir, f"fuzz_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("seed", range(12))
def test_random_ipc_pipeline_matches_oracle(tmp_path, seed):
    c = _case(seed)
    case = _describe(seed, c)
    print(case, flush=True)
    W = c["W"]
    mp.spawn(_worker, args=(W, str(tmp_path / "store"), str(tmp_path), seed), nprocs=W, join=True)
    res = []
    for r in range(W):
        with np.load(tmp_path / f"fuzz_r{r}.npz", allow_pickle=False) as d:
            res.append({k: d[k] for k in d.files})
    n = len(c["numels"])
    print(f"  {int(res[0]['buckets'])} buckets in {int(res[0]['segments'])} symmetric buffer(s)", flush=True)
    scaler = o.ScalerState(scale=c["scale"])  # a step that found an inf halves the next step's scale
    for step in range(STEPS):
        for rank in range(W):
            want = o.ddp_pipeline(c["grads"][step], [c["gdt"]] * n, c["numels"], c["cap"], rank,
                                  1.0 / scaler.scale if c["use_scaler"] else None,
                                  bucket_dtype=o.F32 if c["widening"] else None)
            assert int(res[rank]["buckets"]) == len(want["layout"]), case
            if c["use_scaler"]:
                assert bool(res[rank][f"found_{step}"]) == want["found_inf"], f"{case} step {step} rank {rank}"
            for i in range(n):
                got = res[rank][f"grad_{step}_{i}"]
                assert same_bits(got, want["grads"][i]), (
                    f"{case} step {step} rank {rank} param {i}: " + first_mismatch(got, want["grads"][i]))
            for b, red in enumerate(want["reduced"]):
                got = res[rank][f"bucket_{step}_{b}"]
                assert same_bits(got, red), f"{case} step {step} rank {rank} bucket {b}: " + first_mismatch(got, red)
        if c["use_scaler"]:
            scaler.update(want["found_inf"])
            assert all(float(res[r][f"scale_after_{step}"]) == scaler.scale for r in range(W)), case


def _fsdp_case(seed: int) -> dict:
    rng = np.random.default_rng(43000 + seed)
    W = int(rng.integers(2, 5))
    h = int(rng.integers(3, 41))
    blocks = [(bool(rng.random() < 0.3), bool(rng.random() < 0.3)) for _ in range(int(rng.integers(1, 6)))]
    param_dtype = DTYPES[int(rng.integers(0, 3))]
    # every unit's full-size rows within the segment: blocks h*h + h (+3), the root the head's h + 1
    largest = max([h * h + h + (0 if empty else 3) for _, empty in blocks] + [h + 1])
    padded = -(-largest // W) * W
    segment_bytes = [1 << 30, max(256, (padded * 4 + 255) // 256 * 256)][int(rng.integers(0, 2))]
    return dict(W=W, h=h, blocks=blocks, param_dtype=param_dtype, unit_batch=int(rng.integers(1, 4)),
                reshard=bool(rng.random() < 0.7), keep_low=bool(rng.random() < 0.3),
                accumulate=bool(rng.random() < 0.4), segment_bytes=segment_bytes)


def _fsdp_model(seed: int, c: dict, dev) -> nn.Module:
    blocks = [_FuzzBlock(c["h"], 1000 * seed + k, frozen, empty) for k, (frozen, empty) in enumerate(c["blocks"])]
    return _FuzzNet(blocks, c["h"]).to(dev)


def _fsdp_worker(rank: int, world: int, store: str, out_dir: str, seed: int) -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        c = _fsdp_case(seed)
        group = IpcGroup(dist.group.WORLD, dev, segment_bytes=c["segment_bytes"])
        model = _fsdp_model(seed, c, dev)
        init = {id(p): p.detach().float().reshape(-1).cpu().numpy().copy() for p in model.parameters()}
        captured: dict[int, torch.Tensor] = {}
        for p in model.parameters():
            if p.requires_grad:
                p.register_post_accumulate_grad_hook(lambda q: captured.__setitem__(id(q), q.grad.detach().clone()))
        policy = MixedPrecisionPolicy(param_dtype=c["param_dtype"], reduce_dtype=torch.float32,
                                      keep_low_precision_shard=c["keep_low"])
        fsdp = FSDP(model, unit_types=(_FuzzBlock,), process_group=group, mixed_precision=policy,
                    unit_batch=c["unit_batch"], reshard_after_forward=c["reshard"])
        out = {"units": np.array(len(fsdp._units)), "segments": np.array(len({u.segment for u in fsdp._units}))}
        with fsdp.summon_full_params():
            for u, unit in enumerate(fsdp._units):
                out[f"full_{u}"] = _host_bits(unit._full)
        x = torch.randn(6, c["h"], generator=torch.Generator().manual_seed(100 * seed + rank)).to(dev)
        if c["accumulate"]:
            with fsdp.no_sync():
                for half in x.chunk(2):
                    (fsdp(half) / 2).backward()
        else:
            fsdp(x).backward()
        fsdp.finish_gradient_sync()
        torch.cuda.synchronize()
        for u, unit in enumerate(fsdp._units):
            out[f"numels_{u}"] = np.array(unit.numels, dtype=np.int64)
            out[f"init_{u}"] = (np.concatenate([init[id(p)] for p in unit.params]) if unit.params
                                else np.zeros(0, np.float32))
            for k, p in enumerate(unit.params):
                if id(p) in captured:
                    out[f"local_{u}_{k}"] = _host_bits(captured[id(p)])
            out[f"shard_grad_{u}"] = _host_bits(unit.flat_shard.grad)
            out[f"sharded_{u}"] = np.array(not unit.is_unsharded and all(p.grad is None for p in unit.params))
        group.release()
        np.savez(os.path.join(out_dir, f"fsdp_fuzz_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("seed", range(8))
def test_random_ipc_fsdp_matches_oracle(tmp_path, seed):
    c = _fsdp_case(seed)
    W = c["W"]
    pdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(c["param_dtype"], o.F32)
    case = (f"ipc fsdp fuzz seed {seed}: W={W} h={c['h']} blocks={len(c['blocks'])} {c['param_dtype']} "
            f"unit_batch={c['unit_batch']} reshard={c['reshard']} keep_low={c['keep_low']} "
            f"accumulate={c['accumulate']} segment={c['segment_bytes']}")
    print(case, flush=True)
    mp.spawn(_fsdp_worker, args=(W, str(tmp_path / "store"), str(tmp_path), seed), nprocs=W, join=True)
    res = []
    for r in range(W):
        with np.load(tmp_path / f"fsdp_fuzz_r{r}.npz", allow_pickle=False) as d:
            res.append({k: d[k] for k in d.files})
    n_units = int(res[0]["units"])
    assert n_units == len(c["blocks"]) + 1, case
    print(f"  {n_units} units in {int(res[0]['segments'])} pair(s) of symmetric buffers", flush=True)
    for u in range(n_units):
        numels = [int(n) for n in res[0][f"numels_{u}"]]
        _, _, P = o.fsdp_layout(numels, W)
        flat = np.zeros(P, np.float32)
        flat[: sum(numels)] = res[0][f"init_{u}"]
        gathered = o.fsdp_gather_cast(flat, pdt)
        grads = [[res[r][f"local_{u}_{k}"] if f"local_{u}_{k}" in res[r] else o.zeros(n, pdt)
                  for k, n in enumerate(numels)] for r in range(W)]
        for rank in range(W):
            assert bool(res[rank][f"sharded_{u}"]), f"{case}: unit {u} rank {rank} still gathered after backward"
            assert same_bits(res[rank][f"full_{u}"], gathered), f"{case}: unit {u} rank {rank} all-gather"
            want = o.fsdp_reduce_scatter_share(grads, pdt, numels, rank, o.F32, pdt if c["keep_low"] else o.F32)
            got = res[rank][f"shard_grad_{u}"]
            assert same_bits(got, want), f"{case}: unit {u} rank {rank} shard grad: " + first_mismatch(got, want)


REDUCE_OPS = {"sum": dist.ReduceOp.SUM, "max": dist.ReduceOp.MAX, "min": dist.ReduceOp.MIN,
              "product": dist.ReduceOp.PRODUCT}
ODT = {torch.float32: o.F32, torch.bfloat16: o.BF16, torch.float16: o.F16}


def _collectives_case(seed: int) -> dict:
    """Symmetric buffers, every rank's starting rows and a sequence of in-place collectives on views."""
    rng = np.random.default_rng(47000 + seed)
    W = int(rng.integers(2, 5))
    bufs = [(int(rng.integers(1, 5000)), DTYPES[int(rng.integers(0, 3))]) for _ in range(int(rng.integers(1, 4)))]
    rows = []  # [rank][buffer] in the oracle's representation
    for _ in range(W):
        per = []
        for n, dt in bufs:
            v = (rng.standard_normal(n) * (0.01 if dt == torch.float16 else 1.0)).astype(np.float32)
            v[rng.random(n) < 0.05] = 0.0
            v[rng.random(n) < 0.05] = -0.0
            per.append(o.from_f32(v, ODT[dt]))
        rows.append(per)
    ops = []
    for _ in range(int(rng.integers(3, 9))):
        b = int(rng.integers(0, len(bufs)))
        n = bufs[b][0]
        if rng.random() < 0.3 and n >= 4:  # several views of one buffer in one coalesced SUM
            cuts = sorted(int(x) for x in rng.choice(np.arange(1, n), size=min(n - 1, int(rng.integers(2, 5))),
                                                      replace=False))
            spans = [(a, c) for a, c in zip([0, *cuts], [*cuts, n], strict=True)][:: int(rng.integers(1, 3))]
            ops.append(("coalesced", b, spans, "sum", bool(rng.random() < 0.5)))
        else:
            a = int(rng.integers(0, n))
            c = int(rng.integers(a + 1, n + 1))
            ops.append(("single", b, [(a, c)], list(REDUCE_OPS)[int(rng.integers(0, 4))], bool(rng.random() < 0.5)))
    return dict(W=W, algorithm=["one_shot", "two_shot"][seed % 2], bufs=bufs, rows=rows, ops=ops)


def _collectives_worker(rank: int, world: int, store: str, out_dir: str, seed: int) -> None:
    from minidist import comm

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        c = _collectives_case(seed)
        group = IpcGroup(dist.group.WORLD, dev, algorithm=c["algorithm"])
        rows = [group.zeros(n, dt) for n, dt in c["bufs"]]
        for row, host in zip(rows, c["rows"][rank], strict=True):
            row.copy_(_to_dev(host, row.shape, dev))
        for kind, b, spans, op, async_op in c["ops"]:
            views = [rows[b][a:e] for a, e in spans]
            if kind == "coalesced":
                work = comm.all_reduce_coalesced(views, group=group, async_op=async_op)
            else:
                work = comm.all_reduce(views[0], op=REDUCE_OPS[op], group=group, async_op=async_op)
            if async_op and work is not None:
                work.wait()
        torch.cuda.synchronize()
        np.savez(os.path.join(out_dir, f"coll_r{rank}.npz"), **{f"buf_{b}": _host_bits(r) for b, r in enumerate(rows)})
        group.release()
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("seed", range(8))
def test_random_ipc_in_place_collectives(tmp_path, seed):
    """Seeded random sequences of in-place ``comm.all_reduce`` (SUM, MAX, MIN, PRODUCT) and
    ``comm.all_reduce_coalesced`` (several views of one buffer) on views of 1-3 symmetric fp32 / bf16
    / fp16 buffers of an IpcGroup with no reduce target, one- or two-shot, synchronous or async:
    every rank's rows after the sequence against the oracle replaying it (each view replaced, on
    every rank, by the rank-ordered fold of all ranks' values; everything else kept)."""
    c = _collectives_case(seed)
    W = c["W"]
    print(f"ipc collectives seed {seed}: W={W} {c['algorithm']} buffers={[(n, str(d)) for n, d in c['bufs']]} "
          f"ops={[(k, b, len(s), op) for k, b, s, op, _ in c['ops']]}", flush=True)
    mp.spawn(_collectives_worker, args=(W, str(tmp_path / "store"), str(tmp_path), seed), nprocs=W, join=True)
    want = [[np.array(x, copy=True) for x in per] for per in c["rows"]]
    for kind, b, spans, op, _ in c["ops"]:
        dt = ODT[c["bufs"][b][1]]
        for a, e in spans:
            parts = [want[r][b][a:e] for r in range(W)]
            red = o.allreduce_sum(parts, dt) if op == "sum" else o.allreduce_op(parts, dt, op)
            for r in range(W):
                want[r][b][a:e] = red
    for r in range(W):
        with np.load(tmp_path / f"coll_r{r}.npz", allow_pickle=False) as d:
            for b in range(len(c["bufs"])):
                got = d[f"buf_{b}"]
                assert same_bits(got, want[r][b]), f"seed {seed} rank {r} buffer {b}: " + first_mismatch(got, want[r][b])
