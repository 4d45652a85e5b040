"""DDP and FSDP over a real torch.distributed process group: two processes on the one GPU.

Both ranks run on ``cuda:0`` and meet in a gloo group (FileStore rendezvous).
gloo moves host memory, so minidist stages every device tensor it hands to a
gloo collective through the host (``comm.dist_*``); everything else is the
product path as it runs over RCCL:

* DDP: the construction-time broadcast from rank 0, the gradient hooks, pack
  (kernel) -> ``comm.all_reduce`` -> ``Work.wait`` -> unpack + fused unscale and
  found-inf (kernel), and the scaler's MAX exchange of the flag
  (minidist/amp.py:216-217), over two steps, the second with an overflow on
  rank 1 only.
* FSDP: the broadcast, the cast of the master shard into this rank's slot and
  the in-place all-gather, and pack (kernel) -> ``reduce_scatter_tensor`` ->
  shard epilogue (kernel).

With W = 2 the backend's sum is a + b, which IEEE makes independent of order,
so each rank's results are checked bit for bit against the oracle fed with
both ranks' local gradients.  Those are captured by hooks registered before
the wrapper's own, which therefore run first.
"""

from __future__ import annotations

import os
from contextlib import nullcontext
from datetime import timedelta

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

import tiny_gpt
from conftest import first_mismatch, same_bits
from minidist import DDP, FSDP, DistributedGradScaler, MixedPrecisionPolicy, comm
from oracle import gradpath as o

pytestmark = pytest.mark.gpu
W = 2
SCALE = 2.0**10
CAP_MB = 0.01
DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().reshape(-1).cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy().copy()


def _worker(rank: int, kind: str, store: str, out_dir: str) -> None:
    torch.cuda.set_device(0)
    # a collective that one rank never joins fails after a minute instead of hanging
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=W,
                            timeout=timedelta(seconds=60))
    try:
        if kind.startswith("ddp"):
            _ddp_rank(rank, out_dir, comm_stream=kind == "ddp-stream")
        elif kind == "fsdp-vs-ddp":
            _fsdp_vs_ddp_rank(rank, out_dir)
        else:
            _fsdp_rank(rank, DTYPES[kind.split("-")[1]], out_dir, unit_batch=2 if kind.endswith("-ub2") else 1)
    finally:
        dist.destroy_process_group()


def _ddp_rank(rank: int, out_dir: str, comm_stream: bool) -> None:
    dev = torch.device("cuda", 0)
    c = tiny_gpt.Config(n_layer=2)
    model = tiny_gpt.GPT(c, seed=rank).to(dev)  # different on each rank until DDP broadcasts rank 0's
    params = list(model.parameters())
    local: dict[int, torch.Tensor] = {}
    state = {"inject": False}

    def capture(p):
        if state["inject"] and rank == 1 and p is params[3]:
            p.grad.view(-1)[5] = float("inf")  # this rank's backward overflowed
        local[id(p)] = p.grad.detach().clone()

    for p in params:
        p.register_post_accumulate_grad_hook(capture)
    scaler = DistributedGradScaler(init_scale=SCALE)
    ddp = DDP(model, bucket_cap_mb=CAP_MB, grad_scaler=scaler, comm_stream=comm_stream)
    out = {f"init_{i}": _bits(p) for i, p in enumerate(params)}

    class _Opt:
        param_groups = [{"params": params}]

    ids, tgt = tiny_gpt.batch(c, 8, seed=5)
    for step in range(2):
        state["inject"] = step == 1
        for p in params:
            p.grad = None
        with comm.record_comm() if step == 0 else nullcontext() as stats:
            _, loss = ddp(ids.chunk(W)[rank].to(dev), tgt.chunk(W)[rank].to(dev))
            scaler.scale_loss(loss).backward()
            out[f"found_{step}"] = np.array(scaler.unscale_(_Opt()))
        if step == 0:
            _save_rows(out, stats)
        scaler.update()
        for i, p in enumerate(params):
            out[f"local_{step}_{i}"] = _bits(local[id(p)])
            out[f"final_{step}_{i}"] = _bits(p.grad)
    out["scale_after"] = np.array(scaler.scale)
    np.savez(os.path.join(out_dir, f"ddp_r{rank}.npz"), **out)


def _fsdp_rank(rank: int, param_dtype: torch.dtype, out_dir: str, unit_batch: int = 1) -> None:
    dev = torch.device("cuda", 0)
    c = tiny_gpt.Config(n_layer=2)
    model = tiny_gpt.GPT(c, seed=rank).to(dev)
    params = list(model.parameters())
    index = {id(p): i for i, p in enumerate(params)}
    local: dict[int, torch.Tensor] = {}

    def capture(p):
        local[id(p)] = p.grad.detach().clone()

    for p in params:
        p.register_post_accumulate_grad_hook(capture)
    policy = MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32)
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), mixed_precision=policy, unit_batch=unit_batch)
    out = {}
    for u, unit in enumerate(fsdp._units):
        out[f"unit_{u}_params"] = np.array([index[id(p)] for p in unit.params])
        out[f"master_{u}"] = _bits(unit.flat_shard)
    with fsdp.summon_full_params():
        for u, unit in enumerate(fsdp._units):
            out[f"full_{u}"] = _bits(unit._full)
    ids, tgt = tiny_gpt.batch(c, 8, seed=6)
    with comm.record_comm() as stats:
        _, loss = fsdp(ids.chunk(W)[rank].to(dev), tgt.chunk(W)[rank].to(dev))
        loss.backward()
    _save_rows(out, stats)
    for i, p in enumerate(params):
        out[f"local_{i}"] = _bits(local[id(p)])
    for u, unit in enumerate(fsdp._units):
        out[f"shard_grad_{u}"] = _bits(unit.flat_shard.grad)
    out["units"] = np.array(len(fsdp._units))
    np.savez(os.path.join(out_dir, f"fsdp_r{rank}.npz"), **out)


def _save_rows(out: dict, stats: comm.CommStats) -> None:
    rows = stats.as_rows()
    out["comm_names"] = np.array([r[0] for r in rows])
    out["comm_rows"] = np.array([r[1:] for r in rows], dtype=np.int64).reshape(len(rows), 3)


def _recorded(res: dict) -> dict[str, tuple[int, int, int]]:
    return {str(n): tuple(int(v) for v in row) for n, row in zip(res["comm_names"], res["comm_rows"], strict=True)}


def _train(model, rank: int, steps: int = 4, lr: float = 1e-2):
    """SGD on this rank's chunk of seeded batches (the reference's tests/test_fsdp.py:50-62 loop)."""
    c = tiny_gpt.Config(n_layer=2)
    dev = torch.device("cuda", 0)
    opt = torch.optim.SGD(model.parameters(), lr=lr)
    losses = []
    for step in range(steps):
        ids, tgt = tiny_gpt.batch(c, 8, seed=100 + step)
        opt.zero_grad(set_to_none=True)
        _, loss = model(ids.chunk(W)[rank].to(dev), tgt.chunk(W)[rank].to(dev))
        loss.backward()
        opt.step()
        losses.append(loss.item())
    return losses


def _fsdp_vs_ddp_rank(rank: int, out_dir: str) -> None:
    """The reference's tests/test_fsdp.py:65-130 over a real group: DDP and FSDP (resharding after
    forward, and not) from the same initial weights, their gradients after one backward and their
    weights after four SGD steps."""
    dev = torch.device("cuda", 0)
    c = tiny_gpt.Config(n_layer=2)
    ids, tgt = tiny_gpt.batch(c, 8, seed=99)
    out = {}
    ddp = DDP(tiny_gpt.GPT(c, seed=0).to(dev))
    _, loss = ddp(ids.chunk(W)[rank].to(dev), tgt.chunk(W)[rank].to(dev))
    loss.backward()
    names = [n for n, _ in ddp.module.named_parameters()]
    for i, p in enumerate(ddp.module.parameters()):
        out[f"ddp_grad_{i}"] = _bits(p.grad)
    out["ddp_losses"] = np.array(_train(ddp, rank))
    for i, p in enumerate(ddp.module.parameters()):
        out[f"ddp_weight_{i}"] = _bits(p)
    for tag, reshard in (("fsdp", True), ("fsdp_keep", False)):
        model = tiny_gpt.GPT(c, seed=0).to(dev)
        index = {id(p): i for i, p in enumerate(model.parameters())}
        fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), reshard_after_forward=reshard)
        _, loss = fsdp(ids.chunk(W)[rank].to(dev), tgt.chunk(W)[rank].to(dev))
        if not reshard:  # the blocks stay gathered between forward and backward
            out[f"{tag}_blocks_gathered"] = np.array(all(u.is_unsharded for u in fsdp._units[:-1]))
        loss.backward()
        for u, unit in enumerate(fsdp._units):
            out[f"{tag}_unit_{u}_params"] = np.array([index[id(p)] for p in unit.params])
            out[f"{tag}_shard_grad_{u}"] = _bits(unit.flat_shard.grad)
        out[f"{tag}_losses"] = np.array(_train(fsdp, rank))
        with fsdp.summon_full_params():
            for i, p in enumerate(model.parameters()):
                out[f"{tag}_weight_{i}"] = _bits(p)
        out[f"{tag}_units"] = np.array(len(fsdp._units))
    out["n_params"] = np.array(len(names))
    np.savez(os.path.join(out_dir, f"fsdp_r{rank}.npz"), **out)


def _run(kind: str, tmp_path) -> list[dict]:
    store = str(tmp_path / "store")
    print(f"spawning 2 ranks on cuda:0 ({kind})", flush=True)
    mp.spawn(_worker, args=(kind, store, str(tmp_path)), nprocs=W, join=True)
    prefix = "ddp" if kind.startswith("ddp") else "fsdp"
    res = []
    for r in range(W):
        with np.load(tmp_path / f"{prefix}_r{r}.npz", allow_pickle=False) as d:
            res.append({k: d[k] for k in d.files})
    return res


def _rank0_init(c: tiny_gpt.Config) -> list[np.ndarray]:
    return [p.detach().reshape(-1).numpy().copy() for p in tiny_gpt.GPT(c, seed=0).parameters()]


@pytest.mark.parametrize("comm_stream", [False, True])
def test_ddp_two_processes_bitwise(tmp_path, comm_stream):
    res = _run("ddp-stream" if comm_stream else "ddp", tmp_path)
    c = tiny_gpt.Config(n_layer=2)
    init0 = _rank0_init(c)
    n = len(init0)
    for r in range(W):  # the broadcast gave every rank rank 0's parameters
        for i in range(n):
            assert np.array_equal(res[r][f"init_{i}"], init0[i]), f"rank {r} param {i}"
    numels = [a.size for a in init0]
    for step in range(2):
        grads = [[res[r][f"local_{step}_{i}"] for i in range(n)] for r in range(W)]
        for rank in range(W):
            want = o.ddp_pipeline(grads, [o.F32] * n, numels, CAP_MB, rank, 1.0 / SCALE)
            for i in range(n):
                got = res[rank][f"final_{step}_{i}"]
                assert same_bits(got, want["grads"][i]), f"step {step} rank {rank} param {i}: " + first_mismatch(
                    got, want["grads"][i])
            # the MAX exchange makes the decision unanimous: only rank 1 overflowed in step 1
            assert bool(res[rank][f"found_{step}"]) == want["found_inf"] == (step == 1)
    assert all(float(res[r]["scale_after"]) == SCALE / 2 for r in range(W))
    # what step 0 recorded (comm.py:232-233): one all-reduce per bucket of the oracle's partition; the
    # scaler's flag exchange goes straight to the backend, unrecorded, as in the reference (amp.py:216-217)
    layout = o.build_buckets([k * 4 for k in numels], CAP_MB)
    payloads = [sum(numels[i] * 4 for i in b) for b in layout]
    want = {"all_reduce": (len(layout), sum(payloads), sum(int(2 * (W - 1) / W * b) for b in payloads))}
    assert all(_recorded(res[r]) == want for r in range(W))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16", "bf16-ub2"])
def test_fsdp_two_processes_bitwise(tmp_path, dtype):
    """bf16-ub2: ``unit_batch=2``, the two blocks gathered together and their reduce-scatters held
    until both are ready (each still its own collective over the real group)."""
    res = _run(f"fsdp-{dtype}", tmp_path)
    dtype = dtype.split("-")[0]
    c = tiny_gpt.Config(n_layer=2)
    init0 = _rank0_init(c)
    pdt = {"f32": o.F32, "bf16": o.BF16, "f16": o.F16}[dtype]
    n_units = int(res[0]["units"])
    assert n_units == c.n_layer + 1
    for u in range(n_units):
        idx = [int(i) for i in res[0][f"unit_{u}_params"]]
        numels = [init0[i].size for i in idx]
        _, S, P = o.fsdp_layout(numels, W)
        flat = np.zeros(P, np.float32)
        flat[: sum(numels)] = np.concatenate([init0[i] for i in idx])
        grads = [[res[r][f"local_{i}"] for i in idx] for r in range(W)]
        gathered = o.fsdp_gather_cast(flat, pdt)
        for rank in range(W):
            assert np.array_equal(res[rank][f"master_{u}"], flat[rank * S : (rank + 1) * S])
            assert same_bits(res[rank][f"full_{u}"], gathered), f"unit {u} rank {rank}: all-gather"
            want = o.fsdp_reduce_scatter_share(grads, pdt, numels, rank, o.F32, o.F32)
            got = res[rank][f"shard_grad_{u}"]
            assert same_bits(got, want), f"unit {u} rank {rank}: " + first_mismatch(got, want)
    # what the step recorded (comm.py:247-248, 263-264): every block unit gathered for its forward and
    # its backward, the root unit (the last) once; one reduce-scatter of the padded fp32 buffer per unit
    padded = []
    for u in range(n_units):
        total = sum(init0[int(i)].size for i in res[0][f"unit_{u}_params"])
        padded.append(-(-total // W) * W)
    gathers = [p for p in padded[:-1] for _ in range(2)] + [padded[-1]]
    gb = 4 if pdt == o.F32 else 2
    want = {"all_gather": (len(gathers), sum(p * gb for p in gathers), sum(int((W - 1) / W * p * gb) for p in gathers)),
            "reduce_scatter": (n_units, sum(p * 4 for p in padded), sum(int((W - 1) / W * p * 4) for p in padded))}
    assert all(_recorded(res[r]) == want for r in range(W))


def _close(got: np.ndarray, want: np.ndarray, tol: float) -> float:
    """Relative error as the reference's assert_close measures it (tests/common.py:78-88)."""
    err = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max(initial=0.0))
    return err / max(float(np.abs(want).max(initial=0.0)), 1.0)


def test_fsdp_matches_ddp_two_processes(tmp_path):
    """Reference tests/test_fsdp.py:65-130 and :260: FSDP's reassembled gradient equals DDP's
    (tolerance 1e-6), the weights agree after four SGD steps (1e-5) and the losses step by step
    (1e-5), whether or not the blocks are resharded after forward."""
    res = _run("fsdp-vs-ddp", tmp_path)
    n = int(res[0]["n_params"])
    for tag in ("fsdp", "fsdp_keep"):
        n_units = int(res[0][f"{tag}_units"])
        full = {}
        for u in range(n_units):
            idx = [int(i) for i in res[0][f"{tag}_unit_{u}_params"]]
            sizes = [res[0][f"ddp_grad_{i}"].size for i in idx]
            flat = np.concatenate([res[r][f"{tag}_shard_grad_{u}"] for r in range(W)])
            off = 0
            for i, k in zip(idx, sizes, strict=True):
                full[i] = flat[off : off + k]
                off += k
        for rank in range(W):
            for i in range(n):
                assert _close(full[i], res[rank][f"ddp_grad_{i}"], 1e-6) <= 1e-6, f"{tag} grad {i}"
                assert _close(res[rank][f"{tag}_weight_{i}"], res[rank][f"ddp_weight_{i}"], 1e-5) <= 1e-5, (
                    f"{tag} rank {rank} weight {i}")
            assert np.abs(res[rank][f"{tag}_losses"] - res[rank]["ddp_losses"]).max() < 1e-5
        if tag == "fsdp_keep":
            assert all(bool(res[r]["fsdp_keep_blocks_gathered"]) for r in range(W))



def _random_ddp_case(seed: int) -> dict:
    rng = np.random.default_rng(37000 + seed)
    dtype = [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]
    return dict(dtype=dtype, model_seed=int(rng.integers(0, 1 << 30)), cap=float(rng.choice([1e-6, 1e-3, 4e-3, 1e6])),
                overlap=bool(rng.random() < 0.75), comm_stream=bool(rng.random() < 0.4),
                use_scaler=bool(rng.random() < 0.7), scale=2.0 ** int(rng.integers(0, 12)),
                zero=["none", "zero", "keep"][int(rng.integers(0, 3))], steps=int(rng.integers(2, 4)),
                inject=[bool(rng.random() < 0.3) for _ in range(4)])


def _random_ddp_worker(rank: int, seed: int, store: str, out_dir: str) -> None:
    """One rank of a random DDP case over the default gloo group (see test_random_ddp_two_processes)."""
    from test_fuzz_gpu import _HookNet

    torch.cuda.set_device(0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=W,
                            timeout=timedelta(seconds=60))
    try:
        c = _random_ddp_case(seed)
        dev = torch.device("cuda", 0)
        model = _HookNet(np.random.default_rng(c["model_seed"]), c["dtype"])  # one architecture on every rank
        params = [p for p in model.parameters() if p.requires_grad]
        local: dict[int, torch.Tensor] = {}
        for p in params:
            p.register_post_accumulate_grad_hook(lambda q: local.__setitem__(id(q), q.grad.detach().clone()))
        scaler = DistributedGradScaler(init_scale=c["scale"]) if c["use_scaler"] else None
        ddp = DDP(model, bucket_cap_mb=c["cap"], overlap_with_backward=c["overlap"], grad_scaler=scaler,
                  reduce_dtype=torch.float32 if c["dtype"] != torch.float32 else None, comm_stream=c["comm_stream"])

        class _Opt:
            param_groups = [{"params": params}]

        out = {"h": np.array(model.h), "buckets": np.array(len(ddp._buckets))}
        for step in range(c["steps"]):
            local.clear()
            before = [None if p.grad is None else _bits(p.grad) for p in params]
            x = torch.randn(5, model.h, generator=torch.Generator().manual_seed(100 * step + rank)).to(dev, c["dtype"])
            loss = ddp(x) * (scaler.scale if scaler is not None else 1.0)
            if c["inject"][step] and rank == 1:
                loss = loss * float("inf")  # this rank's backward overflows
            loss.backward()
            if scaler is not None:
                out[f"found_{step}"] = np.array(scaler.unscale_(_Opt()))
                out[f"scale_{step}"] = np.array(scaler.scale)
                scaler.update()
            torch.cuda.synchronize()
            for i, p in enumerate(params):
                own = _bits(local[id(p)]) if id(p) in local else before[i]
                out[f"local_{step}_{i}"] = own if own is not None else np.zeros(0, np.float32)
                out[f"has_{step}_{i}"] = np.array(own is not None)
                out[f"final_{step}_{i}"] = _bits(p.grad)
            if c["zero"] == "none":
                for p in params:
                    p.grad = None
            elif c["zero"] == "zero":
                for p in params:
                    p.grad.zero_()
        np.savez(os.path.join(out_dir, f"rand_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("seed", range(6))
def test_random_ddp_two_processes(tmp_path, seed):
    """Seeded random DDP cases over a real two-process gloo group: random layer widths run in a random
    order (a layer used twice, a frozen layer, a parameter forward never touches), fp32 or bf16
    gradients into fp32 buckets, bucket caps from one bucket per parameter to one, launched from the
    hooks or at the end, on ``comm_stream`` or not, the fused scaler with an overflow on one rank in
    some steps, ``zero_grad`` to None, to zero or not at all.  Each rank's gradients and found-inf
    decision every step against the oracle over both ranks' local gradients (W = 2: the backend's
    a + b is order-free, so bit for bit)."""
    c = _random_ddp_case(seed)
    print(f"seed {seed}: {c}", flush=True)
    mp.spawn(_random_ddp_worker, args=(seed, str(tmp_path / "store"), str(tmp_path)), nprocs=W, join=True)
    res = []
    for r in range(W):
        with np.load(tmp_path / f"rand_r{r}.npz", allow_pickle=False) as d:
            res.append({k: d[k] for k in d.files})
    n = sum(1 for k in res[0] if k.startswith("final_0_"))
    gdt = o.BF16 if c["dtype"] == torch.bfloat16 else o.F32
    for step in range(c["steps"]):
        grads = [[res[r][f"local_{step}_{i}"] if bool(res[r][f"has_{step}_{i}"]) else None for i in range(n)]
                 for r in range(W)]
        numels = [res[0][f"final_{step}_{i}"].size for i in range(n)]
        for rank in range(W):
            inv = 1.0 / float(res[rank][f"scale_{step}"]) if c["use_scaler"] else None
            want = o.ddp_pipeline(grads, [gdt] * n, numels, c["cap"], rank, inv,
                                  bucket_dtype=o.F32 if gdt == o.BF16 else None)
            where = f"seed {seed} step {step} rank {rank}"
            if c["use_scaler"]:
                assert bool(res[rank][f"found_{step}"]) == want["found_inf"], where
                assert want["found_inf"] or not c["inject"][step], where  # rank 1's overflow reaches both
            for i in range(n):
                got = res[rank][f"final_{step}_{i}"]
                assert same_bits(got, want["grads"][i]), f"{where} param {i}: " + first_mismatch(got, want["grads"][i])


def _random_fsdp_case(seed: int) -> dict:
    rng = np.random.default_rng(39000 + seed)
    h = int(rng.integers(3, 41))
    blocks = [(bool(rng.random() < 0.3), bool(rng.random() < 0.3)) for _ in range(int(rng.integers(1, 6)))]
    return dict(h=h, blocks=blocks, param_dtype=[torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))],
                unit_batch=int(rng.integers(1, 4)), reshard=bool(rng.random() < 0.7), keep_low=bool(rng.random() < 0.3),
                accumulate=bool(rng.random() < 0.4), comm_streams=bool(rng.random() < 0.3))


def _random_fsdp_worker(rank: int, seed: int, store: str, out_dir: str) -> None:
    """One rank of a random FSDP case over the default gloo group (see test_random_fsdp_two_processes)."""
    from test_fuzz_gpu import _FuzzBlock, _FuzzNet

    torch.cuda.set_device(0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=W,
                            timeout=timedelta(seconds=60))
    try:
        c = _random_fsdp_case(seed)
        dev = torch.device("cuda", 0)
        blocks = [_FuzzBlock(c["h"], 1000 * seed + k, frozen, empty) for k, (frozen, empty) in enumerate(c["blocks"])]
        model = _FuzzNet(blocks, c["h"]).to(dev)
        init = {id(p): p.detach().float().reshape(-1).cpu().numpy().copy() for p in model.parameters()}
        local: dict[int, torch.Tensor] = {}
        for p in model.parameters():
            if p.requires_grad:
                p.register_post_accumulate_grad_hook(lambda q: local.__setitem__(id(q), q.grad.detach().clone()))
        policy = MixedPrecisionPolicy(param_dtype=c["param_dtype"], reduce_dtype=torch.float32,
                                      keep_low_precision_shard=c["keep_low"])
        fsdp = FSDP(model, unit_types=(_FuzzBlock,), mixed_precision=policy, unit_batch=c["unit_batch"],
                    reshard_after_forward=c["reshard"], comm_streams=c["comm_streams"])
        out = {"units": np.array(len(fsdp._units))}
        with fsdp.summon_full_params():
            for u, unit in enumerate(fsdp._units):
                out[f"full_{u}"] = _bits(unit._full)
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
                if id(p) in local:
                    out[f"local_{u}_{k}"] = _bits(local[id(p)])
            out[f"shard_grad_{u}"] = _bits(unit.flat_shard.grad)
            out[f"sharded_{u}"] = np.array(not unit.is_unsharded and all(p.grad is None for p in unit.params))
        np.savez(os.path.join(out_dir, f"frand_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("seed", range(6))
def test_random_fsdp_two_processes(tmp_path, seed):
    """Seeded random FSDP cases over a real two-process gloo group: 1-5 units of random width (frozen
    biases, empty parameters) and the root, the gather dtype, ``unit_batch``, ``reshard_after_forward``,
    ``keep_low_precision_shard``, side streams, accumulation under ``no_sync`` and the flush.  Every
    unit's gathered parameters against the oracle's cast of rank 0's weights, every rank's shard
    gradient against the oracle over both ranks' captured gradients (W = 2: order-free), every unit
    sharded after backward."""
    c = _random_fsdp_case(seed)
    print(f"seed {seed}: {c}", flush=True)
    mp.spawn(_random_fsdp_worker, args=(seed, str(tmp_path / "store"), str(tmp_path)), nprocs=W, join=True)
    res = []
    for r in range(W):
        with np.load(tmp_path / f"frand_r{r}.npz", allow_pickle=False) as d:
            res.append({k: d[k] for k in d.files})
    pdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(c["param_dtype"], o.F32)
    assert int(res[0]["units"]) == len(c["blocks"]) + 1
    for u in range(int(res[0]["units"])):
        numels = [int(n) for n in res[0][f"numels_{u}"]]
        _, _, P = o.fsdp_layout(numels, W)
        flat = np.zeros(P, np.float32)
        flat[: sum(numels)] = res[0][f"init_{u}"]
        gathered = o.fsdp_gather_cast(flat, pdt)
        grads = [[res[r][f"local_{u}_{k}"] if f"local_{u}_{k}" in res[r] else o.zeros(n, pdt)
                  for k, n in enumerate(numels)] for r in range(W)]
        for rank in range(W):
            where = f"seed {seed} unit {u} rank {rank}"
            assert bool(res[rank][f"sharded_{u}"]), f"{where}: still gathered after backward"
            assert same_bits(res[rank][f"full_{u}"], gathered), f"{where}: all-gather"
            want = o.fsdp_reduce_scatter_share(grads, pdt, numels, rank, o.F32, pdt if c["keep_low"] else o.F32)
            got = res[rank][f"shard_grad_{u}"]
            assert same_bits(got, want), f"{where}: shard grad: " + first_mismatch(got, want)
