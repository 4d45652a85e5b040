"""DDP and FSDP over a real process group's code path, on one GPU.

With a torch.distributed process group (RCCL on a multi-GPU node) the path
is: pack + 1/W into the bucket (gfx950 kernel), ``comm.all_reduce`` ->
``dist.all_reduce`` on the bucket, ``Work.wait()``, then unpack + fused
unscale / found-inf (gfx950 kernel); FSDP packs + divides into a flat
``reduce_dtype`` buffer, calls ``dist.reduce_scatter_tensor`` and finishes
the shard with the share kernel; ``unshard`` casts into this rank's slot and
calls ``dist.all_gather_into_tensor``.

Only one GPU exists here, so the three torch.distributed collectives (and
the world size / rank queries) are replaced by a test double that performs
each collective's arithmetic with plain torch ops on peer contributions
staged in HBM: ``acc = c_0; acc = acc + c_r`` for r = 1..W-1 (rank order),
slices for the reduce-scatter, copies for the all-gather.  Everything else is
the product's own code, and the results are compared bit for bit with the
oracle (tests/test_oracle.py pins it).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.distributed as dist
from torch import nn

from conftest import first_mismatch, same_bits
from minidist import DDP, FSDP, DistributedGradScaler, MixedPrecisionPolicy, comm
from oracle import gradpath as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().reshape(-1)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().astype(np.uint16)
    return t.numpy().copy()


def dev_from(a: np.ndarray) -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(a.copy()).to(DEV)


class FakeGroup:
    """Stands for a torch.distributed ProcessGroup of ``world`` ranks; this process is ``rank``."""

    def __init__(self, world: int, rank: int):
        self.world, self.rank = world, rank
        self.peers: dict[int, list[torch.Tensor | None]] = {}  # data_ptr of own tensor -> W contributions
        self.gather_rows: list[torch.Tensor | None] | None = None  # the peers' shards for all_gather
        self.calls: list[str] = []

    def contributions(self, own: torch.Tensor) -> list[torch.Tensor]:
        rows = self.peers[own.data_ptr()]
        return [own if r == self.rank else rows[r] for r in range(self.world)]


@pytest.fixture
def fake_dist(monkeypatch):
    """Install the collective double; yields a factory of FakeGroups."""
    groups: list[FakeGroup] = []

    def group_of(group) -> FakeGroup:
        if group is None:  # the default group: the one the test built
            return groups[-1]
        assert isinstance(group, FakeGroup), "every collective must go to the DDP / FSDP group"
        return group

    def all_reduce(tensor, op=dist.ReduceOp.SUM, group=None, async_op=False):
        g = group_of(group)
        if op == dist.ReduceOp.MAX:  # the scaler's found-inf flag: peers report 0
            g.calls.append("all_reduce_max")
            return _Work() if async_op else None
        g.calls.append("all_reduce")
        assert op == dist.ReduceOp.SUM
        parts = [t.clone() for t in g.contributions(tensor)]
        acc = parts[0]
        for r in range(1, g.world):
            acc = acc + parts[r]
        tensor.copy_(acc)
        return _Work() if async_op else None

    def reduce_scatter_tensor(output, input_, op=dist.ReduceOp.SUM, group=None, async_op=False):
        g = group_of(group)
        g.calls.append("reduce_scatter")
        S = output.numel()
        parts = [c[g.rank * S : (g.rank + 1) * S] for c in g.contributions(input_)]
        acc = parts[0].clone()
        for r in range(1, g.world):
            acc = acc + parts[r]
        output.copy_(acc)
        return _Work() if async_op else None

    def all_gather_into_tensor(output, input_, group=None, async_op=False):
        g = group_of(group)
        g.calls.append("all_gather")
        S = input_.numel()
        for r in range(g.world):
            output[r * S : (r + 1) * S].copy_(input_ if r == g.rank else g.gather_rows[r])
        return _Work() if async_op else None

    monkeypatch.setattr(comm, "is_distributed", lambda: True)
    monkeypatch.setattr(dist, "get_world_size", lambda group=None: group_of(group).world)
    monkeypatch.setattr(dist, "get_rank", lambda group=None: group_of(group).rank)
    monkeypatch.setattr(dist, "get_backend", lambda group=None: "nccl")  # device tensors go straight in
    monkeypatch.setattr(dist, "all_reduce", all_reduce)
    monkeypatch.setattr(dist, "reduce_scatter_tensor", reduce_scatter_tensor)
    monkeypatch.setattr(dist, "all_gather_into_tensor", all_gather_into_tensor)

    def make(world: int, rank: int) -> FakeGroup:
        groups.append(FakeGroup(world, rank))
        return groups[-1]

    yield make


class _Work:
    def wait(self, timeout=None):
        return True


class Flat(nn.Module):
    def __init__(self, shapes, dtype=torch.float32):
        super().__init__()
        self.ps = nn.ParameterList([nn.Parameter(torch.zeros(s, dtype=dtype, device=DEV)) for s in shapes])


def odt(dtype: torch.dtype) -> str:
    return {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(dtype, o.F32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("W,rank,cap", [(2, 1, 25.0), (4, 2, 0.01), (8, 5, 1e-6), (3, 0, 0.004)])
@pytest.mark.parametrize("inject", [False, True])
def test_ddp_real_group_path(fake_dist, rng, dtype, W, rank, cap, inject):
    """pack (kernel) -> dist.all_reduce per bucket -> wait -> unpack + fused unscale (kernel)."""
    group = fake_dist(W, rank)
    shapes = [(int(rng.integers(1, 200)),) if i % 2 else (int(rng.integers(1, 30)), 17) for i in range(23)]
    numels = [int(np.prod(s)) for s in shapes]
    scale = 2.0**12
    model = Flat(shapes, dtype)
    scaler = DistributedGradScaler(init_scale=scale)
    ddp = DDP(model, process_group=group, bucket_cap_mb=cap, broadcast_parameters=False, grad_scaler=scaler)
    assert ddp.world_size == W and not ddp._resident
    grads = [[o.from_f32((rng.standard_normal(n) * 1e-3 * scale).astype(np.float32), odt(dtype)) for n in numels]
             for _ in range(W)]
    if inject:
        r_inf = (rank + 1) % W
        grads[r_inf][3] = grads[r_inf][3].copy()
        grads[r_inf][3][0] = {torch.float32: np.float32(np.inf), torch.bfloat16: np.uint16(0x7F80),
                              torch.float16: np.float16(np.inf)}[dtype]
    ddp.allocate_buckets()
    index = {id(p): i for i, p in enumerate(model.parameters())}
    for bucket in ddp._buckets:
        idxs = [index[id(p)] for p in bucket.params]
        rows = [None] * W
        for r in range(W):
            if r != rank:
                packed = o.pack([grads[r][i] for i in idxs], [odt(dtype)] * len(idxs),
                                [numels[i] for i in idxs], odt(bucket.dtype), 1.0 / W)
                rows[r] = dev_from(packed)
        group.peers[bucket.buffer.data_ptr()] = rows
    for p, g in zip(model.parameters(), grads[rank], strict=True):
        p.grad = dev_from(g).view(p.shape)
    ddp.finish_gradient_sync()

    class _Opt:
        param_groups = [{"params": list(model.parameters())}]

    found = scaler.unscale_(_Opt())
    want = o.ddp_pipeline(grads, [odt(dtype)] * len(shapes), numels, cap, rank, 1.0 / scale)
    assert group.calls.count("all_reduce") == len(ddp._buckets)
    assert group.calls.count("all_reduce_max") == 1  # the scaler's flag exchange (amp.py:216-217)
    assert found == want["found_inf"] == inject
    for i, p in enumerate(model.parameters()):
        got = host_bits(p.grad)
        assert same_bits(got, want["grads"][i]), f"param {i}: {first_mismatch(got, want['grads'][i])}"


class _Block(nn.Module):
    def __init__(self, shapes):
        super().__init__()
        self.ps = nn.ParameterList([nn.Parameter(torch.randn(s, device=DEV) * 0.02) for s in shapes])


class _Net(nn.Module):
    def __init__(self, n_blocks, shapes):
        super().__init__()
        torch.manual_seed(5)
        self.blocks = nn.ModuleList([_Block(shapes) for _ in range(n_blocks)])


@pytest.mark.parametrize("W,rank", [(2, 0), (4, 3), (8, 5)])
def test_fsdp_real_group_path(fake_dist, rng, W, rank):
    """unshard: cast into own slot (kernel) + dist.all_gather_into_tensor; reduce_scatter_grads:
    pack + divide (kernel) -> dist.reduce_scatter_tensor -> shard epilogue (kernel), set then accumulate."""
    group = fake_dist(W, rank)
    shapes = [(7,), (12, 5), (33,), (3, 3)]
    policy = MixedPrecisionPolicy(param_dtype=torch.bfloat16, reduce_dtype=torch.float32)
    net = _Net(2, shapes)
    init = [p.detach().clone() for p in net.parameters()]
    fsdp = FSDP(net, unit_types=(_Block,), process_group=group, mixed_precision=policy,
                broadcast_parameters=False, device=DEV)
    assert len(fsdp._units) == 2
    unit = fsdp._units[1]
    numels = unit.numels
    _, S, P = o.fsdp_layout(numels, W)
    assert (unit.shard_numel, unit.padded_numel) == (S, P)

    # unshard: this rank's master shard cast to bf16 in its slot, the peers' shards gathered
    flat = np.zeros(P, dtype=np.float32)
    flat[: sum(numels)] = np.concatenate([host_bits(t) for t in init[len(shapes):]])
    peer_shards = [o.fsdp_gather_cast(flat[r * S : (r + 1) * S], o.BF16) for r in range(W)]
    group.gather_rows = [dev_from(s) if r != rank else None for r, s in enumerate(peer_shards)]
    unit.unshard()
    assert "all_gather" in group.calls
    assert same_bits(host_bits(unit._full), np.concatenate(peer_shards))

    # reduce_scatter_grads, twice: the second call accumulates into flat_shard.grad
    existing = None
    for _ in range(2):
        grads = [[o.from_f32((rng.standard_normal(n) * 1e-3).astype(np.float32), o.BF16) for n in numels]
                 for _ in range(W)]
        bufs = [o.div_scalar(o.fsdp_flatten(g, o.BF16, numels, P, o.F32), o.F32, W) for g in grads]
        captured = {}
        real_rs = dist.reduce_scatter_tensor

        def rs_capture(output, input_, *a, _real=real_rs, **k):
            captured["own_buf"] = host_bits(input_)
            group.peers[input_.data_ptr()] = [dev_from(b) if r != rank else None for r, b in enumerate(bufs)]
            return _real(output, input_, *a, **k)

        dist.reduce_scatter_tensor = rs_capture
        try:
            for p, g in zip(unit.params, grads[rank], strict=True):
                p.grad = dev_from(g).view(p.shape)
            unit.reduce_scatter_grads()
        finally:
            dist.reduce_scatter_tensor = real_rs
        # this rank's flattened, divided buffer is exactly what the reference would send
        assert same_bits(captured["own_buf"], bufs[rank])
        want = o.fsdp_reduce_scatter_share(grads, o.BF16, numels, rank, existing=existing)
        got = host_bits(unit.flat_shard.grad)
        assert same_bits(got, want), first_mismatch(got, want)
        assert all(p.grad is None for p in unit.params)
        existing = want
