"""The benchmark configurations at their real shapes, through the Python API, on the GPU.

cfg0 (tiny GPT, W=4) is small enough for the oracle on every element.  The
large configurations use three checks that do not depend on size:

* every element against a torch-on-GPU replay of the reference's op chain
  (``copy_``, ``mul_(1/W)``, rank-ordered ``add_``, ``copy_`` into the grad,
  ``mul_(inv_scale)``) on the same inputs -- the peers' rows, which the step
  does not write, and this rank's gradients as they were before it -- a
  second, independent implementation of the same IEEE arithmetic;
* a seeded sample of elements of every bucket against the numpy oracle;
* the configuration's own property: identical results across bucket caps
  (cfg2), found-inf and the skipped step when one +inf is injected (cfg1),
  shard offsets of two ranks (cfg3).

Inputs follow the configurations' recipes (seeded ``randn`` times the stated
scales); the large ones are generated on the GPU.

The last section takes the path to its size limits with the same checks: a
bucket and an FSDP unit whose element offsets pass 2^31 (4-16 GB buffers).
"""

from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

from conftest import first_mismatch, same_bits
from minidist import DDP, FSDP, DistributedGradScaler, MixedPrecisionPolicy, ResidentGroup
from minidist import workloads as wl
from oracle import gradpath as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _release_memory():
    yield
    torch.cuda.synchronize()
    # A wrapper and its module reference each other through the gradient hooks, so the
    # multi-GB buffers of these configurations are freed by the cycle collector, not by
    # reference counting.
    gc.collect()
    torch.cuda.empty_cache()


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().reshape(-1).cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy().copy()


def odt(dtype: torch.dtype) -> str:
    return o.BF16 if dtype == torch.bfloat16 else o.F32


def same_gpu(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bitwise equality of two device tensors of one dtype (NaNs excepted, none are generated)."""
    ia = a.reshape(-1).view(torch.int32 if a.dtype == torch.float32 else torch.int16)
    ib = b.reshape(-1).view(torch.int32 if b.dtype == torch.float32 else torch.int16)
    return bool(torch.equal(ia, ib))


class _Opt:
    def __init__(self, params):
        self.param_groups = [{"params": list(params)}]


def _bucket_map(ddp: DDP):
    """param id -> (bucket index, element offset in the bucket)."""
    out = {}
    for b, bucket in enumerate(ddp._buckets):
        for p, off in zip(bucket.params, bucket.offsets, strict=True):
            out[id(p)] = (b, off)
    return out


def _stage_gpu(ddp: DDP, W: int, rank: int, gen: torch.Generator, scale: float) -> None:
    """Own grads and every peer's contribution row, seeded randn * scale, in the wire format."""
    for p in ddp.module.parameters():
        p.grad = (torch.randn(p.shape, device=DEV, generator=gen, dtype=torch.float32) * scale).to(p.dtype)
    for b in range(len(ddp._buckets)):
        rows = ddp.bucket_replicas(b)
        wire_dtype, prescaled = ddp.bucket_wire_format(b)
        for r in range(W):
            if r == rank:
                continue
            x = torch.randn(rows[r].shape, device=DEV, generator=gen, dtype=torch.float32) * scale
            if prescaled:  # what the peer's pack wrote: its gradients x 1/W in the bucket dtype
                x = x.to(wire_dtype).to(torch.float32).mul_(1.0 / W)
            rows[r].copy_(x.to(wire_dtype))


def _snapshot(ddp: DDP) -> dict[int, torch.Tensor]:
    """This rank's gradients before the step (the step overwrites them)."""
    return {id(p): p.grad.detach().clone() for p in ddp.module.parameters()}


def _check_chain(ddp: DDP, W: int, rank: int, inv_scale: float, own_grads) -> None:
    """After the step: every bucket and gradient vs the reference's op chain replayed with torch.

    The peers' rows are inputs the step does not write; this rank's contribution
    is rebuilt from the gradients it had before the step."""
    for b, bucket in enumerate(ddp._buckets):
        rows = ddp.bucket_replicas(b)
        wire_dtype, prescaled = ddp.bucket_wire_format(b)
        own = torch.zeros(bucket.numel, dtype=bucket.dtype, device=DEV)  # ddp.py:83-84
        for p, off in zip(bucket.params, bucket.offsets, strict=True):
            own[off : off + p.numel()].copy_(own_grads[id(p)].reshape(-1))  # ddp.py:90
        acc = None
        for r in range(W):
            if r == rank:
                x = own.mul_(1.0 / W)  # ddp.py:91
            elif prescaled:
                x = rows[r].to(bucket.dtype)
            else:  # raw bf16 gradients: what the peer's pack into an fp32 bucket makes of them
                x = rows[r].to(bucket.dtype).mul_(1.0 / W)
            acc = x.clone() if acc is None else acc.add_(x)  # rank-ordered SUM
        assert same_gpu(bucket.buffer, acc), f"bucket {b}"
        for p, off in zip(bucket.params, bucket.offsets, strict=True):
            g = torch.empty_like(p.grad).copy_(acc[off : off + p.numel()].view(p.shape))  # ddp.py:100-101
            if inv_scale != 1.0:
                g.mul_(inv_scale)  # amp.py:212
            assert same_gpu(p.grad, g), f"bucket {b}, parameter {tuple(p.shape)}"


def _sample_before(ddp: DDP, rng, per_param: int = 64):
    """Sampled own-gradient values (host) keyed by param id, taken before the step."""
    out = {}
    for p in ddp.module.parameters():
        n = p.numel()
        idx = np.unique(np.concatenate([np.arange(min(n, 4)), np.arange(max(0, n - 4), n),
                                        rng.integers(0, n, min(n, per_param))]))
        ti = torch.from_numpy(idx).to(DEV)
        out[id(p)] = (idx, bits(p.grad.reshape(-1)[ti]))
    return out


def _oracle_sample(ddp: DDP, W: int, rank: int, inv_scale: float, before) -> None:
    """Every sampled element vs the oracle's pack / SUM / unpack / unscale on that element."""
    where = _bucket_map(ddp)
    for p in ddp.module.parameters():
        idx, own_vals = before[id(p)]
        b, off = where[id(p)]
        bucket = ddp._buckets[b]
        rows = ddp.bucket_replicas(b)
        wire_dtype, prescaled = ddp.bucket_wire_format(b)
        bdt, wdt, gdt = odt(bucket.dtype), odt(wire_dtype), odt(p.grad.dtype)
        ti = torch.from_numpy(idx + off).to(DEV)
        xs = []
        for r in range(W):
            if r == rank:
                x = o.convert(own_vals, gdt, bdt)
                xs.append(o.mul_scalar(x, bdt, 1.0 / W))
            else:
                x = bits(rows[r][ti])
                xs.append(x if prescaled else o.mul_scalar(o.convert(x, wdt, bdt), bdt, 1.0 / W))
        acc = o.allreduce_sum(xs, bdt)
        want = o.convert(acc, bdt, gdt)
        if inv_scale != 1.0:
            want = o.mul_scalar(want, gdt, inv_scale)
        got = bits(p.grad.reshape(-1)[torch.from_numpy(idx).to(DEV)])
        assert same_bits(got, want), f"{tuple(p.shape)}: " + first_mismatch(got, want)
        assert same_bits(bits(bucket.buffer[ti]), acc)


# ---------------------------------------------------------------------------
# cfg0: tiny GPT, W = 4, fp32 grads randn * 1e-2 * 2^16, 25 MB cap -- every element vs the oracle
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("rank", [0, 3])
def test_cfg0_tiny_gpt_every_element_vs_oracle(rank):
    specs = wl.gpt_specs(**wl.TINY_GPT)
    W, S = 4, 2.0**16
    model = wl.SpecModule(specs, DEV)
    scaler = DistributedGradScaler(init_scale=S)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=25.0, grad_scaler=scaler)
    assert len(ddp._buckets) == 1
    # Seeds per replica as the configuration states: Generator(1234 + 7919 r), tensors in parameter order.
    grads = []
    for r in range(W):
        g = torch.Generator().manual_seed(1234 + 7919 * r)
        grads.append([(torch.randn(s.shape, generator=g) * 1e-2 * S).reshape(-1).numpy() for s in specs])
    numels = [s.numel for s in specs]
    rows = ddp.bucket_replicas(0)
    for r in range(W):
        if r != rank:
            packed = o.pack([grads[r][i] for i in reversed(range(len(specs)))], [o.F32] * len(specs),
                            list(reversed(numels)), o.F32, 1.0 / W)
            rows[r].copy_(torch.from_numpy(packed).to(DEV))
    for p, g in zip(model.parameters(), grads[rank], strict=True):
        p.grad = torch.from_numpy(g).to(DEV).view(p.shape)
    ddp.finish_gradient_sync()
    found = scaler.unscale_(_Opt(model.parameters()))
    want = o.ddp_pipeline(grads, [o.F32] * len(specs), numels, 25.0, rank, 1.0 / S)
    assert want["layout"] == [list(reversed(range(len(specs))))]
    for i, p in enumerate(model.parameters()):
        got = bits(p.grad)
        assert same_bits(got, want["grads"][i]), f"param {i}: " + first_mismatch(got, want["grads"][i])
    assert same_bits(bits(ddp._buckets[0].buffer), want["reduced"][0])
    assert found is False and want["found_inf"] is False


# ---------------------------------------------------------------------------
# cfg1: GPT-2-124M, W = 8, fp32 grads randn * 1e-3 * 2^16, 25 MB buckets; + the +inf variant
# ---------------------------------------------------------------------------


def _cfg1(rank: int, seed: int, **ddp_options):
    specs = wl.gpt_specs(**wl.GPT2_SMALL)
    W, S = 8, 2.0**16
    model = wl.SpecModule(specs, DEV)
    scaler = DistributedGradScaler(init_scale=S)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=25.0, grad_scaler=scaler,
              **ddp_options)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    _stage_gpu(ddp, W, rank, gen, 1e-3 * S)
    return model, scaler, ddp, W, S


@pytest.mark.parametrize("rank,options", [(0, {}), (6, {}), (3, {"comm_stream": True}), (5, {"capture_graphs": True})])
def test_cfg1_gpt2_small_full_size(rank, options):
    """Full size, the default launch path and, on other ranks, the dedicated communication
    stream and the graph-captured launch."""
    model, scaler, ddp, W, S = _cfg1(rank, 1234 + rank, **options)
    assert len(ddp._buckets) == 18 and sum(p.numel() for p in model.parameters()) == 124_439_808
    rng = np.random.default_rng(rank)
    before = _sample_before(ddp, rng)
    own = _snapshot(ddp)
    ddp.finish_gradient_sync()
    found = scaler.unscale_(_Opt(model.parameters()))
    assert found is False
    _check_chain(ddp, W, rank, 1.0 / S, own)
    _oracle_sample(ddp, W, rank, 1.0 / S, before)


def test_cfg1_inf_injection_skips_the_step():
    """One +inf at a seeded (replica, flat index) -> found-inf, a skipped step, scale halves."""
    rank = 0
    model, scaler, ddp, W, S = _cfg1(rank, 99)
    params = list(model.parameters())
    N = sum(p.numel() for p in params)
    pick = torch.Generator().manual_seed(4242)
    replica = int(torch.randint(0, W, (1,), generator=pick))
    flat = int(torch.randint(0, N, (1,), generator=pick))
    # locate the flat index (parameter order) and plant the +inf in that replica's contribution
    off = 0
    for p in params:
        if flat < off + p.numel():
            j = flat - off
            break
        off += p.numel()
    b, boff = _bucket_map(ddp)[id(p)]
    if replica == rank:
        p.grad.view(-1)[j] = float("inf")
    else:
        ddp.bucket_replicas(b)[replica][boff + j] = float("inf")
    own = _snapshot(ddp)
    ddp.finish_gradient_sync()

    class Opt(_Opt):
        stepped = False

        def step(self):
            Opt.stepped = True

    opt = Opt(params)
    applied = scaler.step(opt)
    scaler.update()
    assert applied is False and not Opt.stepped
    assert scaler.scale == S / 2 and scaler.num_skipped == 1
    assert torch.isinf(p.grad.view(-1)[j])
    _check_chain(ddp, W, rank, 1.0 / S, own)


# ---------------------------------------------------------------------------
# cfg2: GPT-2-medium, W = 4, fp32 randn * 1e-3; caps 1 byte / 25 MB / one giant bucket agree exactly
# ---------------------------------------------------------------------------


def test_cfg2_gpt2_medium_bucket_caps_identical():
    specs = wl.gpt_specs(**wl.GPT2_MEDIUM)
    W, rank = 4, 1
    assert wl.total_numel(specs) == 354_823_168
    gen = torch.Generator(device=DEV).manual_seed(2024)
    own = [torch.randn(s.shape, device=DEV, generator=gen) * 1e-3 for s in specs]
    peers = [[torch.randn(s.shape, device=DEV, generator=gen) * 1e-3 for s in specs] for _ in range(W - 1)]
    results, counts = [], []
    for cap in (1.0 / 2**20, 25.0, 1e6):  # 1 byte, 25 MB, one bucket
        model = wl.SpecModule(specs, DEV)
        ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap)
        counts.append(len(ddp._buckets))
        params = list(model.parameters())
        index = {id(p): i for i, p in enumerate(params)}
        for b, bucket in enumerate(ddp._buckets):
            rows = ddp.bucket_replicas(b)
            peer_rows = [rows[r] for r in range(W) if r != rank]
            for row, grads in zip(peer_rows, peers, strict=True):
                for p, off in zip(bucket.params, bucket.offsets, strict=True):
                    # the peer's pack: copy_ then mul_(1/W)
                    row[off : off + p.numel()].copy_(grads[index[id(p)]].reshape(-1)).mul_(1.0 / W)
        for p, g in zip(params, own, strict=True):
            p.grad = g.clone()
        if cap == 25.0:
            rng = np.random.default_rng(7)
            before = _sample_before(ddp, rng, per_param=16)
        ddp.finish_gradient_sync()
        if cap == 25.0:
            _oracle_sample(ddp, W, rank, 1.0, before)
        results.append(torch.cat([p.grad.reshape(-1) for p in params]))
        del ddp, model, params
        torch.cuda.empty_cache()
    assert counts == [292, 74, 1]
    assert same_gpu(results[0], results[1]) and same_gpu(results[1], results[2])


# ---------------------------------------------------------------------------
# cfg3: FSDP unit of one GPT-2-XL block (S = 3,842,600 at W = 8): bf16 gather cast, RS share
# ---------------------------------------------------------------------------


class _Block(torch.nn.Module):
    def __init__(self, specs):
        super().__init__()
        self.ps = torch.nn.ParameterList([torch.nn.Parameter(torch.empty(s.shape, device=DEV)) for s in specs])


class _XLUnit(torch.nn.Module):
    def __init__(self, specs, seed):
        super().__init__()
        self.block = _Block(specs)
        g = torch.Generator(device=DEV).manual_seed(seed)
        with torch.no_grad():
            for p in self.block.parameters():
                p.copy_(torch.randn(p.shape, device=DEV, generator=g) * 0.02)


@pytest.mark.parametrize("rank", [0, 5])
def test_cfg3_fsdp_gpt2_xl_block_unit(rank):
    specs = wl.gpt_block_specs(0, wl.GPT2_XL["n_embd"])
    W = 8
    m = _XLUnit(specs, seed=77)
    master_full = torch.cat([p.detach().reshape(-1) for p in m.block.parameters()])
    policy = MixedPrecisionPolicy(param_dtype=torch.bfloat16, reduce_dtype=torch.float32)
    f = FSDP(m, unit_types=(_Block,), process_group=ResidentGroup(W, rank, DEV), mixed_precision=policy)
    unit = f._units[0]
    S, P = unit.shard_numel, unit.padded_numel
    assert (unit.total_numel, S, P) == (30_740_800, 3_842_600, 30_740_800)
    # gather cast: this rank's slot of the gather buffer == RNE bf16 of the fp32 master shard
    unit.unshard()
    shard_f32 = bits(master_full[rank * S : (rank + 1) * S])
    assert same_bits(bits(unit.flat_shard), shard_f32)
    want_cast = o.fsdp_gather_cast(shard_f32, o.BF16)
    got_cast = bits(unit._full[rank * S : (rank + 1) * S])
    assert same_bits(got_cast, want_cast), first_mismatch(got_cast, want_cast)
    # reduce-scatter share: 8 full-size bf16 contributions randn * 1e-3 summed in fp32 into the shard
    gen = torch.Generator(device=DEV).manual_seed(100 + rank)
    peers = unit.peer_grad_contributions()
    for r in range(W):
        if r != rank:
            peers[r].copy_((torch.randn(P, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16))
    own_full = (torch.randn(P, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
    off = 0
    for p in unit.params:
        p.grad = own_full[off : off + p.numel()].view(p.shape).clone()
        off += p.numel()
    unit.reduce_scatter_grads()
    lo = rank * S
    slices = [bits(own_full[lo : lo + S]) if r == rank else bits(peers[r, lo : lo + S]) for r in range(W)]
    # fsdp.py:218-233 on this rank's slice: widen, div_(W), rank-ordered SUM, to(fp32)
    parts = [o.div_scalar(o.convert(x, o.BF16, o.F32), o.F32, W) for x in slices]
    want = o.allreduce_sum(parts, o.F32)
    got = bits(unit.flat_shard.grad)
    assert same_bits(got, want), first_mismatch(got, want)
    assert all(p.grad is None for p in unit.params)
    # a second backward accumulates into the shard gradient (fsdp.py:234-237)
    off = 0
    for p in unit.params:
        p.grad = own_full[off : off + p.numel()].view(p.shape).clone()
        off += p.numel()
    unit.reduce_scatter_grads()
    got2 = bits(unit.flat_shard.grad)
    want2 = o.add(want, want, o.F32)
    assert same_bits(got2, want2), first_mismatch(got2, want2)


class _XLStack(torch.nn.Module):
    def __init__(self, specs, n_blocks, seed):
        super().__init__()
        self.blocks = torch.nn.ModuleList([_Block(specs) for _ in range(n_blocks)])
        g = torch.Generator(device=DEV).manual_seed(seed)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, device=DEV, generator=g) * 0.02)


def test_cfg3_all_48_units_batched_full_size():
    """cfg3 as the bench issues it: the 48 units' gather casts in one dispatch and their reduce-scatter
    shares in one multi-unit dispatch (144 pieces, a device plan), at full size (23.6 GB of peer
    contributions).  Every unit's slot against the oracle's RNE cast, every unit's shard gradient
    against the per-unit reduce_scatter_grads of the same inputs, and three units' against the oracle."""
    specs = wl.gpt_block_specs(0, wl.GPT2_XL["n_embd"])
    W, rank, n = 8, 5, wl.GPT2_XL["n_layer"]
    m = _XLStack(specs, n, seed=78)
    masters = [torch.cat([p.detach().reshape(-1) for p in b.parameters()]) for b in m.blocks]
    policy = MixedPrecisionPolicy(param_dtype=torch.bfloat16, reduce_dtype=torch.float32)
    f = FSDP(m, unit_types=(_Block,), process_group=ResidentGroup(W, rank, DEV), mixed_precision=policy,
             reshard_after_forward=False)
    units = f._units
    assert len(units) == n
    S, P = units[0].shard_numel, units[0].padded_numel
    for u in units:
        u.unshard()
    f._cast_own_slots(units)
    for k, u in enumerate(units):
        want = o.fsdp_gather_cast(bits(masters[k][rank * S : (rank + 1) * S]), o.BF16)
        got = bits(u._full[rank * S : (rank + 1) * S])
        assert same_bits(got, want), f"unit {k}: " + first_mismatch(got, want)
    gen = torch.Generator(device=DEV).manual_seed(200)
    own = []
    for u in units:
        peers = u.peer_grad_contributions()
        for r in range(W):
            if r != rank:
                peers[r].copy_((torch.randn(P, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16))
        own.append((torch.randn(P, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16))

    def give(u, k):
        off = 0
        for p in u.params:
            p.grad = own[k][off : off + p.numel()].view(p.shape).clone()
            off += p.numel()

    for k, u in enumerate(units):
        give(u, k)
    f.finish_gradient_sync()  # every unit holds gradients: one multi-unit share
    batched = [u.flat_shard.grad.clone() for u in units]
    assert all(p.grad is None for u in units for p in u.params)
    for k, u in enumerate(units):
        u.flat_shard.grad = None
        give(u, k)
        u.reduce_scatter_grads()
        assert torch.equal(batched[k].view(torch.int32), u.flat_shard.grad.view(torch.int32)), f"unit {k}"
    lo = rank * S
    for k in (0, 23, 47):
        peers = units[k].peer_grad_contributions()
        slices = [bits(own[k][lo : lo + S]) if r == rank else bits(peers[r, lo : lo + S]) for r in range(W)]
        want = o.allreduce_sum([o.div_scalar(o.convert(x, o.BF16, o.F32), o.F32, W) for x in slices], o.F32)
        got = bits(batched[k])
        assert same_bits(got, want), f"unit {k}: " + first_mismatch(got, want)


# ---------------------------------------------------------------------------
# cfg4: Llama-7B bf16 grads randn * 1e-3 * 2^12, W = 8 (~108 GB of contributions), fp32 buckets
# ---------------------------------------------------------------------------


def test_cfg4_llama7b_bf16_widening_full_size():
    specs = wl.llama_specs(**wl.LLAMA_7B)
    W, rank, S = 8, 3, 2.0**12
    model = wl.SpecModule(specs, DEV)
    scaler = DistributedGradScaler(init_scale=S)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=25.0, grad_scaler=scaler,
              reduce_dtype=torch.float32)
    assert len(ddp._buckets) == 291 and all(b.widening for b in ddp._buckets)
    gen = torch.Generator(device=DEV).manual_seed(4096)
    _stage_gpu(ddp, W, rank, gen, 1e-3 * S)
    # every bucket (one parameter each here): its first and last 4 elements plus 32 seeded ones
    before = _sample_before(ddp, np.random.default_rng(11), per_param=32)
    own = _snapshot(ddp)
    ddp.finish_gradient_sync()
    found = scaler.unscale_(_Opt(model.parameters()))
    assert found is False
    _oracle_sample(ddp, W, rank, 1.0 / S, before)
    _check_chain(ddp, W, rank, 1.0 / S, own)


# ---------------------------------------------------------------------------
# Maximum sizes: element offsets past 2^31 in a bucket and in an FSDP unit
# ---------------------------------------------------------------------------


class _BigAndSmall(torch.nn.Module):
    """Registered small first, so the reverse-order bucket holds the big gradient at offset 0
    and the small one at offset n_big (past 2^31)."""

    def __init__(self, n_big: int, n_small: int, dtype: torch.dtype):
        super().__init__()
        self.small = torch.nn.Parameter(torch.zeros(n_small, dtype=dtype, device=DEV))
        self.big = torch.nn.Parameter(torch.zeros(n_big, dtype=dtype, device=DEV))


@pytest.mark.parametrize("widening", [False, True])
def test_bucket_offsets_beyond_2_31_elements(widening):
    """One bucket of 2^31 + 4104 elements (bf16 grads; bf16 or fp32 bucket), W = 2, fused unscale.
    The big gradient is cut into runs on the host; the small one starts 2^31 + 5 elements in."""
    n_big, n_small = 2**31 + 5, 4099
    W, rank, S = 2, 1, 2.0**10
    model = _BigAndSmall(n_big, n_small, torch.bfloat16)
    scaler = DistributedGradScaler(init_scale=S)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=1e6, grad_scaler=scaler,
              reduce_dtype=torch.float32 if widening else None)
    assert len(ddp._buckets) == 1 and ddp._buckets[0].widening == widening
    where = _bucket_map(ddp)
    assert where[id(model.big)] == (0, 0) and where[id(model.small)] == (0, n_big)
    gen = torch.Generator(device=DEV).manual_seed(31)
    _stage_gpu(ddp, W, rank, gen, 1e-3 * S)
    before = _sample_before(ddp, np.random.default_rng(12), per_param=256)
    # and the big gradient's elements on either side of 2^31
    idx, _ = before[id(model.big)]
    idx = np.unique(np.concatenate([idx, np.arange(2**31 - 3, 2**31 + 3)]))
    before[id(model.big)] = (idx, bits(model.big.grad[torch.from_numpy(idx).to(DEV)]))
    own = _snapshot(ddp)
    ddp.finish_gradient_sync()
    assert scaler.unscale_(_Opt(model.parameters())) is False
    _oracle_sample(ddp, W, rank, 1.0 / S, before)
    _check_chain(ddp, W, rank, 1.0 / S, own)


class _Shape:
    def __init__(self, n: int):
        self.shape = (n,)


class _BigUnitRoot(torch.nn.Module):
    def __init__(self, numels, seed):
        super().__init__()
        self.block = _Block([_Shape(n) for n in numels])
        g = torch.Generator(device=DEV).manual_seed(seed)
        with torch.no_grad():
            for p in self.block.parameters():
                p.copy_(torch.randn(p.shape, device=DEV, generator=g) * 0.02)


@pytest.mark.parametrize("rank", [6, 7])
def test_fsdp_shard_offsets_beyond_2_31_elements(rank):
    """One FSDP unit of 2,550,150,955 elements at W = 8 (S = 318,768,870): rank 6's shard crosses
    element 2^31 and the big parameter's end, rank 7's starts past 2^31 and ends in the padding.
    Gather cast and reduce-scatter share vs the torch op chain on every element and the oracle on a
    sample."""
    numels = [2**31 + 1001, 3 * 2**27 + 12345, 777]
    W = 8
    m = _BigUnitRoot(numels, seed=7)
    master_full = torch.cat([p.detach().reshape(-1) for p in m.block.parameters()])
    policy = MixedPrecisionPolicy(param_dtype=torch.bfloat16, reduce_dtype=torch.float32)
    f = FSDP(m, unit_types=(_Block,), process_group=ResidentGroup(W, rank, DEV), mixed_precision=policy)
    unit = f._units[0]
    T = sum(numels)
    S, P = unit.shard_numel, unit.padded_numel
    assert (unit.total_numel, S, P) == (T, -(-T // W), W * -(-T // W))
    lo = rank * S
    assert (lo < 2**31 < lo + S) if rank == 6 else (lo > 2**31 and lo + S > T)
    rng = np.random.default_rng(rank)
    sample = np.unique(np.concatenate([np.arange(4), np.arange(S - 4, S), rng.integers(0, S, 4096),
                                       np.arange(-3, 3) + (2**31 - lo), np.arange(-3, 3) + (numels[0] - lo),
                                       np.arange(-3, 3) + (T - lo)]))
    sample = sample[(sample >= 0) & (sample < S)]
    ts = torch.from_numpy(sample).to(DEV)

    # gather cast: this rank's slot == RNE bf16 of the fp32 master shard
    want_shard = torch.zeros(S, device=DEV)
    n_real = max(0, min(S, T - lo))
    want_shard[:n_real].copy_(master_full[lo : lo + n_real])
    del master_full
    assert same_gpu(unit.flat_shard, want_shard)
    unit.unshard()
    slot = unit._full[lo : lo + S]
    assert same_gpu(slot, want_shard.to(torch.bfloat16))
    got_cast = bits(slot[ts])
    want_cast = o.fsdp_gather_cast(bits(want_shard[ts]), o.BF16)
    assert same_bits(got_cast, want_cast), first_mismatch(got_cast, want_cast)
    del want_shard

    # reduce-scatter share: 8 full-size bf16 contributions summed in fp32 into the shard
    gen = torch.Generator(device=DEV).manual_seed(200 + rank)
    peers = unit.peer_grad_contributions()
    for r in range(W):
        if r != rank:
            peers[r].copy_((torch.randn(P, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16))
    own_full = torch.zeros(P, dtype=torch.bfloat16, device=DEV)
    own_full[:T].copy_((torch.randn(T, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16))
    off = 0
    for p in unit.params:
        p.grad = own_full[off : off + p.numel()].view(p.shape).clone()
        off += p.numel()
    unit.reduce_scatter_grads()
    slices = [own_full[lo : lo + S] if r == rank else peers[r, lo : lo + S] for r in range(W)]
    acc = None
    for x in slices:  # fsdp.py:218-233 on this rank's slice: widen, div_(W), rank-ordered SUM
        part = x.to(torch.float32).div_(W)
        acc = part if acc is None else acc.add_(part)
    got = unit.flat_shard.grad
    assert same_gpu(got, acc)
    parts = [o.div_scalar(o.convert(bits(x[ts]), o.BF16, o.F32), o.F32, W) for x in slices]
    want = o.allreduce_sum(parts, o.F32)
    assert same_bits(bits(got[ts]), want), first_mismatch(bits(got[ts]), want)
    assert all(p.grad is None for p in unit.params)
