"""Seeded random DDP pipelines on the GPU, bit for bit against the oracle.

Each case draws its own configuration: gradient dtype (fp32, bf16 or fp16,
and for the 16-bit ones optionally fp32 buckets, the widening path), W in [2, 16], the rank,
20-40 parameters of ragged shapes, a bucket cap between one bucket per
parameter and a single bucket, gradients that are views at odd element
offsets of a larger buffer (so that no pointer need be 16-byte aligned),
parameters without a gradient, special values (+-inf, NaN, subnormals) in
some peers' gradients, and with or without the fused scaler.  The whole
pipeline runs through the Python API (DistributedDataParallel over a
ResidentGroup, DistributedGradScaler) and is compared with
oracle.ddp_pipeline: every gradient, every bucket, the found-inf decision.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from conftest import first_mismatch, same_bits
from minidist import DDP, DistributedGradScaler, ResidentGroup
from oracle import gradpath as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
SPECIALS = np.array([np.inf, -np.inf, np.nan, 1e-45, -1e-40, 0.0, -0.0], dtype=np.float32)


def host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().reshape(-1)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().astype(np.uint16)
    return t.numpy().copy()


def dev_view(a: np.ndarray, shape, offset: int) -> torch.Tensor:
    """``a`` on the GPU as a view ``offset`` elements into a larger buffer."""
    n = a.size
    if a.dtype == np.uint16:
        buf = torch.zeros(n + offset + 8, dtype=torch.int16, device=DEV)
        buf[offset : offset + n].copy_(torch.from_numpy(a.view(np.int16).copy()))
        return buf.view(torch.bfloat16)[offset : offset + n].view(shape)
    buf = torch.zeros(n + offset + 8, dtype=torch.float16 if a.dtype == np.float16 else torch.float32, device=DEV)
    buf[offset : offset + n].copy_(torch.from_numpy(a.copy()))
    return buf[offset : offset + n].view(shape)


def dev_from(a: np.ndarray) -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(a.copy()).to(DEV)


class Flat(nn.Module):
    def __init__(self, shapes, dtype):
        super().__init__()
        self.ps = nn.ParameterList([nn.Parameter(torch.zeros(s, dtype=dtype, device=DEV)) for s in shapes])


@pytest.mark.parametrize("seed", range(24))
def test_random_pipeline_matches_oracle(seed):
    _pipeline_case(seed, np.random.default_rng(9000 + seed))


@pytest.mark.parametrize("seed", range(8))
def test_random_pipeline_with_empty_parameters(seed):
    """The same draws with about a fifth of the parameters replaced by empty ones (so some
    buckets hold no elements at one bucket per parameter)."""
    _pipeline_case(seed, np.random.default_rng(19000 + seed), empty_rate=0.2)


def _pipeline_case(seed: int, rng, empty_rate: float = 0.0) -> None:
    dtype = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
    widening = dtype != torch.float32 and rng.random() < 0.5
    gdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(dtype, o.F32)
    W = int(rng.integers(2, 17))
    rank = int(rng.integers(0, W))
    n_params = int(rng.integers(20, 41))
    shapes = [(int(rng.integers(1, 3000)),) if rng.random() < 0.7 else (int(rng.integers(1, 60)), int(rng.integers(1, 40)))
              for _ in range(n_params)]
    if empty_rate:
        shapes = [(0,) if rng.random() < empty_rate else s for s in shapes]
    numels = [int(np.prod(s)) for s in shapes]
    total_mb = sum(numels) * (4 if dtype == torch.float32 else 2) / 2**20
    cap = float(rng.choice([1e-6, total_mb / 7, total_mb / 3, 1e6]))
    use_scaler = rng.random() < 0.6
    scale = 2.0 ** int(rng.integers(0, 14 if dtype != torch.float16 else 10)) if use_scaler else 1.0

    grads = []
    for r in range(W):
        row = []
        for n in numels:
            g = (rng.standard_normal(n) * 1e-3 * scale).astype(np.float32)
            if n and rng.random() < 0.05:  # a rare special value in this gradient
                g[int(rng.integers(0, n))] = SPECIALS[int(rng.integers(0, len(SPECIALS)))]
            row.append(o.from_f32(g, gdt))
        grads.append(row)
    for i in rng.integers(0, n_params, int(rng.integers(0, 3))):  # gradients this rank never received
        grads[rank][int(i)] = None

    model = Flat(shapes, dtype)
    scaler = DistributedGradScaler(init_scale=scale) if use_scaler else None
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, grad_scaler=scaler,
              reduce_dtype=torch.float32 if widening else None)
    params = list(model.parameters())
    index = {id(p): i for i, p in enumerate(params)}
    for b, bucket in enumerate(ddp._buckets):
        idxs = [index[id(p)] for p in bucket.params]
        rows = ddp.bucket_replicas(b)
        wire_dtype, prescaled = ddp.bucket_wire_format(b)
        wdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(wire_dtype, o.F32)
        for r in range(W):
            if r != rank:
                packed = o.pack([grads[r][i] for i in idxs], [gdt] * len(idxs), [numels[i] for i in idxs], wdt,
                                1.0 / W if prescaled else 1.0)
                rows[r].copy_(dev_from(packed))
    for p, g in zip(params, grads[rank], strict=True):
        p.grad = None if g is None else dev_view(g, p.shape, int(rng.integers(0, 9)))
    ddp.finish_gradient_sync()
    found = None
    if scaler is not None:

        class _Opt:
            param_groups = [{"params": params}]

        found = scaler.unscale_(_Opt())

    want = o.ddp_pipeline(grads, [gdt] * n_params, numels, cap, rank, 1.0 / scale if use_scaler else None,
                          bucket_dtype=o.F32 if widening else None)
    case = f"seed {seed}: {dtype} widening={widening} W={W} rank={rank} cap={cap:.3g} scale={scale:g}"
    for i, p in enumerate(params):
        got = host_bits(p.grad)
        assert same_bits(got, want["grads"][i]), f"{case} param {i}: {first_mismatch(got, want['grads'][i])}"
    for b, bucket in enumerate(ddp._buckets):
        assert same_bits(host_bits(bucket.buffer), want["reduced"][b]), f"{case} bucket {b}"
    if scaler is not None:
        assert found == want["found_inf"], case


@pytest.mark.parametrize("seed", range(12))
def test_random_pipeline_launch_modes_over_steps(seed):
    """Seeded random pipelines run for four steps in one launch mode -- eager, on DDP's
    communication stream, or replayed from captured HIP graphs -- with or without the bucket
    average kept, and each step hands over its gradients one of three ways: new tensors (at odd
    offsets of larger buffers), the same tensors overwritten in place (a graph then replays), or
    new tensors with some parameters left without a gradient.  An overflow backs the scale off
    for the next step, as the reference's scaler does.  Every step's gradients, buckets and
    found-inf decision against the oracle."""
    rng = np.random.default_rng(23000 + seed)
    dtype = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
    widening = dtype != torch.float32 and bool(rng.random() < 0.5)
    gdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(dtype, o.F32)
    W = int(rng.integers(2, 17))
    rank = int(rng.integers(0, W))
    n_params = int(rng.integers(10, 31))
    shapes = [(0,) if rng.random() < 0.1 else (int(rng.integers(1, 3000)),) for _ in range(n_params)]
    numels = [int(np.prod(s)) for s in shapes]
    total_mb = sum(numels) * (4 if dtype == torch.float32 else 2) / 2**20
    cap = float(rng.choice([1e-6, total_mb / 5, total_mb / 2, 1e6]))
    mode = ["eager", "comm_stream", "graphs"][int(rng.integers(0, 3))]
    keep = bool(rng.random() < 0.5)
    use_scaler = bool(rng.random() < 0.7)
    scale = 2.0 ** int(rng.integers(0, 14 if dtype != torch.float16 else 10)) if use_scaler else 1.0
    case = (f"seed {seed}: {dtype} widening={widening} W={W} rank={rank} cap={cap:.3g} {mode} "
            f"keep_bucket_average={keep} scale={scale:g}")
    print(case, flush=True)

    model = Flat(shapes, dtype)
    scaler = DistributedGradScaler(init_scale=scale) if use_scaler else None
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, grad_scaler=scaler,
              reduce_dtype=torch.float32 if widening else None, comm_stream=mode == "comm_stream",
              capture_graphs=mode == "graphs", keep_bucket_average=keep)
    params = list(model.parameters())
    index = {id(p): i for i, p in enumerate(params)}

    class _Opt:
        param_groups = [{"params": params}]

    state = o.ScalerState(scale=scale)
    for step in range(4):
        how = "new" if step == 0 else ["new", "in_place", "missing"][int(rng.integers(0, 3))]
        grads = []
        for r in range(W):
            row = []
            for n in numels:
                g = (rng.standard_normal(n) * 1e-3 * scale).astype(np.float32)
                if n and rng.random() < 0.03:
                    g[int(rng.integers(0, n))] = SPECIALS[int(rng.integers(0, len(SPECIALS)))]
                row.append(o.from_f32(g, gdt))
            grads.append(row)
        if how == "missing":
            for i in rng.integers(0, n_params, int(rng.integers(1, 4))):
                grads[rank][int(i)] = None
        for b, bucket in enumerate(ddp._buckets):
            idxs = [index[id(p)] for p in bucket.params]
            rows = ddp.bucket_replicas(b)
            wire_dtype, prescaled = ddp.bucket_wire_format(b)
            wdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(wire_dtype, o.F32)
            for r in range(W):
                if r != rank:
                    packed = o.pack([grads[r][i] for i in idxs], [gdt] * len(idxs), [numels[i] for i in idxs],
                                    wdt, 1.0 / W if prescaled else 1.0)
                    rows[r].copy_(dev_from(packed))
        for p, g in zip(params, grads[rank], strict=True):
            if g is None:
                p.grad = None
            elif how == "in_place" and p.grad is not None:
                p.grad.copy_(dev_from(g).view(p.shape))
            else:
                p.grad = dev_view(g, p.shape, int(rng.integers(0, 9)))
        ddp.finish_gradient_sync()
        found = scaler.unscale_(_Opt()) if scaler is not None else None
        want = o.ddp_pipeline(grads, [gdt] * n_params, numels, cap, rank, 1.0 / state.scale if use_scaler else None,
                              bucket_dtype=o.F32 if widening else None)
        where = f"{case} step {step} ({how})"
        for i, p in enumerate(params):
            got = host_bits(p.grad)
            assert same_bits(got, want["grads"][i]), f"{where} param {i}: {first_mismatch(got, want['grads'][i])}"
        if keep:
            for b, bucket in enumerate(ddp._buckets):
                assert same_bits(host_bits(bucket.buffer), want["reduced"][b]), f"{where} bucket {b}"
        if scaler is not None:
            assert found == want["found_inf"], where
            scaler.update()
            state.update(want["found_inf"])
            assert scaler.scale == state.scale, where


class _HookNet(nn.Module):
    """Linear layers of random widths, used by forward in a random order; optionally one layer
    used twice (its weight and bias are each one parameter fed from two places), one frozen
    layer, and one parameter that forward never touches (its gradient stays None)."""

    def __init__(self, rng, dtype):
        super().__init__()
        n = int(rng.integers(2, 7))
        self.h = int(rng.integers(4, 33))
        self.layers = nn.ModuleList([nn.Linear(self.h, self.h) for _ in range(n)])
        self.unused = nn.Parameter(torch.zeros(int(rng.integers(1, 50))))
        self.order = [int(i) for i in rng.permutation(n)]
        if rng.random() < 0.4:
            self.order.append(self.order[0])  # one layer twice
        self.frozen = int(rng.integers(0, n)) if rng.random() < 0.3 else None
        g = torch.Generator().manual_seed(int(rng.integers(0, 1 << 30)))
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g) * 0.3)
        if self.frozen is not None:
            self.layers[self.frozen].requires_grad_(False)
        self.to(device=DEV, dtype=dtype)

    def forward(self, x):
        for i in self.order:
            x = torch.tanh(self.layers[i](x))
        return x.float().square().mean()


@pytest.mark.parametrize("seed", range(12))
def test_random_backward_pipelines(seed):
    """Seeded random models through a real backward, DDP's bucket runs launched from the autograd
    hooks as buckets fill (or all at the end without ``overlap_with_backward``), eagerly, on
    ``comm_stream`` or from captured graphs, over two or three steps with ``zero_grad`` to None,
    to zero, or not at all (backward then accumulates onto the previous step's averages).  Every
    step's gradients -- unused parameter included -- and found-inf decision against the oracle
    over this rank's captured local gradients and the staged peers'."""
    rng = np.random.default_rng(27000 + seed)
    dtype = [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]
    widening = dtype == torch.bfloat16 and bool(rng.random() < 0.5)
    gdt = o.BF16 if dtype == torch.bfloat16 else o.F32
    model = _HookNet(rng, dtype)
    W = int(rng.integers(2, 9))
    rank = int(rng.integers(0, W))
    params = [p for p in model.parameters() if p.requires_grad]
    numels = [p.numel() for p in params]
    total_mb = sum(numels) * (4 if dtype == torch.float32 else 2) / 2**20
    cap = float(rng.choice([1e-6, total_mb / 4, total_mb / 2, 1e6]))
    overlap = bool(rng.random() < 0.75)
    mode = ["eager", "comm_stream", "graphs"][int(rng.integers(0, 3))]
    use_scaler = bool(rng.random() < 0.6)
    scale = 2.0 ** int(rng.integers(0, 12)) if use_scaler else 1.0
    zero = ["none", "zero", "keep"][int(rng.integers(0, 3))]
    steps = int(rng.integers(2, 4))
    case = (f"seed {seed}: {dtype} widening={widening} W={W} rank={rank} layers={len(model.layers)} "
            f"order={model.order} frozen={model.frozen} cap={cap:.3g} overlap={overlap} {mode} "
            f"scale={scale:g} zero_grad={zero} steps={steps}")
    print(case, flush=True)

    captured: dict[int, torch.Tensor] = {}
    for p in params:  # registered before DDP's hooks, so they see the local gradient
        p.register_post_accumulate_grad_hook(lambda q: captured.__setitem__(id(q), q.grad.detach().clone()))
    scaler = DistributedGradScaler(init_scale=scale) if use_scaler else None
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, overlap_with_backward=overlap,
              grad_scaler=scaler, reduce_dtype=torch.float32 if widening else None,
              comm_stream=mode == "comm_stream", capture_graphs=mode == "graphs")
    index = {id(p): i for i, p in enumerate(params)}

    class _Opt:
        param_groups = [{"params": params}]

    state = o.ScalerState(scale=scale)
    for step in range(steps):
        peers = []
        for _ in range(W):
            row = []
            for n in numels:
                g = (rng.standard_normal(n) * 1e-2 * state.scale).astype(np.float32)
                if rng.random() < 0.02:
                    g[int(rng.integers(0, n))] = SPECIALS[int(rng.integers(0, 3))]  # +-inf or NaN
                row.append(o.from_f32(g, gdt))
            peers.append(row)
        for b, bucket in enumerate(ddp._buckets):
            idxs = [index[id(p)] for p in bucket.params]
            rows = ddp.bucket_replicas(b)
            wire_dtype, prescaled = ddp.bucket_wire_format(b)
            wdt = {torch.bfloat16: o.BF16}.get(wire_dtype, o.F32)
            for r in range(W):
                if r != rank:
                    packed = o.pack([peers[r][i] for i in idxs], [gdt] * len(idxs), [numels[i] for i in idxs], wdt,
                                    1.0 / W if prescaled else 1.0)
                    rows[r].copy_(dev_from(packed))
        captured.clear()
        # what a parameter backward does not reach contributes: its gradient as it stands (None, the
        # zeros zero_grad left, or the previous step's average)
        before = [None if p.grad is None else host_bits(p.grad) for p in params]
        x = torch.randn(5, model.h, generator=torch.Generator().manual_seed(1000 * seed + step)).to(DEV, dtype)
        loss = ddp(x) * state.scale
        loss.backward()
        found = scaler.unscale_(_Opt()) if scaler is not None else None
        own = [host_bits(captured[id(p)]) if id(p) in captured else before[i] for i, p in enumerate(params)]
        assert id(model.unused) not in captured
        grads = [own if r == rank else peers[r] for r in range(W)]
        want = o.ddp_pipeline(grads, [gdt] * len(params), numels, cap, rank, 1.0 / state.scale if use_scaler else None,
                              bucket_dtype=o.F32 if widening else None)
        where = f"{case} step {step}"
        for i, p in enumerate(params):
            got = host_bits(p.grad)
            assert same_bits(got, want["grads"][i]), f"{where} param {i}: {first_mismatch(got, want['grads'][i])}"
        if scaler is not None:
            assert found == want["found_inf"], where
            scaler.update()
            state.update(want["found_inf"])
        if zero == "none":
            for p in params:
                p.grad = None
        elif zero == "zero":
            for p in params:
                p.grad.zero_()


class _FuzzBlock(nn.Module):
    """A random FSDP unit: a square Linear (its bias frozen in some), and an extra parameter that
    is empty in some."""

    def __init__(self, h: int, seed: int, frozen_bias: bool, empty_extra: bool):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.lin = nn.Linear(h, h)
        self.extra = nn.Parameter(torch.zeros(0 if empty_extra else 3))
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g) * 0.5)
        self.lin.bias.requires_grad_(not frozen_bias)

    def forward(self, x):
        x = x.to(self.lin.weight.dtype)
        return torch.tanh(self.lin(x)) + self.extra.sum()


class _FuzzNet(nn.Module):
    def __init__(self, blocks: list[_FuzzBlock], h: int):
        super().__init__()
        self.blocks = nn.ModuleList(blocks)
        self.head = nn.Linear(h, 1)

    def forward(self, x):
        for b in self.blocks:
            x = b(x)
        return self.head(x.to(self.head.weight.dtype)).float().square().mean()


@pytest.mark.parametrize("seed", range(16))
def test_random_fsdp_matches_oracle(seed):
    """Seeded random FSDP configurations through the Python API: W, rank, 1-5 units of random
    width (frozen biases, empty parameters), the gather dtype, ``unit_batch``,
    ``reshard_after_forward`` and accumulation under ``no_sync`` with the final flush.  The peers'
    full-size gradients are staged at random; every unit's shard gradient bit for bit against
    oracle.fsdp_reduce_scatter_share on them and the gradients this rank's backward produced."""
    from minidist import FSDP, MixedPrecisionPolicy

    rng = np.random.default_rng(29000 + seed)
    W = int(rng.integers(2, 9))
    rank = int(rng.integers(0, W))
    h = int(rng.integers(3, 41))
    n_blocks = int(rng.integers(1, 6))
    param_dtype = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
    unit_batch = int(rng.integers(1, 4))
    reshard = bool(rng.random() < 0.7)
    accumulate = bool(rng.random() < 0.4)
    blocks = [_FuzzBlock(h, 1000 * seed + k, bool(rng.random() < 0.3), bool(rng.random() < 0.3))
              for k in range(n_blocks)]
    model = _FuzzNet(blocks, h).to(DEV)
    captured: dict[int, torch.Tensor] = {}
    for p in model.parameters():
        if p.requires_grad:
            p.register_post_accumulate_grad_hook(lambda q: captured.__setitem__(id(q), q.grad.detach().clone()))
    policy = MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32)
    fsdp = FSDP(model, unit_types=(_FuzzBlock,), process_group=ResidentGroup(W, rank, DEV), mixed_precision=policy,
                unit_batch=unit_batch, reshard_after_forward=reshard)
    gdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(param_dtype, o.F32)
    peer = {}  # (unit index, rank) -> per-parameter gradients in the gather dtype
    for u, unit in enumerate(fsdp._units):
        rows = unit.peer_grad_contributions()
        for r in range(W):
            if r == rank:
                continue
            per = [o.from_f32((rng.standard_normal(n) * 0.1).astype(np.float32), gdt) for n in unit.numels]
            peer[u, r] = per
            flat = np.concatenate([x.reshape(-1) for x in per]) if per else np.zeros(0, np.float32)
            if flat.size:
                rows[r, : flat.size].copy_(dev_from(flat))
    x = torch.randn(6, h, generator=torch.Generator().manual_seed(seed)).to(DEV)
    if accumulate:
        with fsdp.no_sync():
            for half in x.chunk(2):
                (fsdp(half) / 2).backward()
        fsdp.finish_gradient_sync()
    else:
        fsdp(x).backward()
        fsdp.finish_gradient_sync()
    case = f"seed {seed}: W={W} rank={rank} h={h} units={len(fsdp._units)} {param_dtype} ub={unit_batch} " \
           f"reshard={reshard} accumulate={accumulate}"
    for u, unit in enumerate(fsdp._units):
        assert all(p.grad is None for p in unit.params), case
        own = [host_bits(captured[id(p)]) if id(p) in captured else o.zeros(n, gdt)
               for p, n in zip(unit.params, unit.numels, strict=True)]
        grads = [own if r == rank else peer[u, r] for r in range(W)]
        want = o.fsdp_reduce_scatter_share(grads, gdt, unit.numels, rank, o.F32, o.F32)
        got = host_bits(unit.flat_shard.grad)
        assert same_bits(got, want), f"{case} unit {unit.name}: " + first_mismatch(got, want)
