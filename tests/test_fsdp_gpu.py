"""FSDP through the Python API on the GPU (reference tests/test_fsdp.py on one GPU).

Rank ``rank`` of a W-way ResidentGroup runs the real FSDP hooks; the peers'
full-size gradients (what their reduce-scatter would contribute) are staged in
each unit's resident rows.  The sharded gradient is compared bit for bit with
oracle.fsdp_reduce_scatter_share on the gradients this rank actually produced
(captured by a hook that runs before FSDP's), and within the reference's
tolerance with the full-batch gradient.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import tiny_gpt
from conftest import first_mismatch, same_bits
from minidist import FSDP, MixedPrecisionPolicy, ResidentGroup
from oracle import gradpath as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().reshape(-1)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().astype(np.uint16)
    return t.numpy().copy()


def _replica_grads(c, W, ids, tgt, dtype=torch.float32):
    out = []
    for r in range(W):
        m = tiny_gpt.GPT(c).to(DEV).to(dtype)
        _, l = m(ids.chunk(W)[r].to(DEV), tgt.chunk(W)[r].to(DEV))
        l.backward()
        out.append({n: p.grad.detach().clone() for n, p in m.named_parameters()})
    return out


def _stage(fsdp, names_by_id, replica, rank, W):
    for unit in fsdp._units:
        rows = unit.peer_grad_contributions()
        for r in range(W):
            if r != rank:
                off = 0
                for p, n in zip(unit.params, unit.numels, strict=True):
                    rows[r, off : off + n].copy_(replica[r][names_by_id[id(p)]].reshape(-1).to(rows.dtype))
                    off += n


def _capture(store):
    def hook(p):
        store[id(p)] = p.grad.detach().clone()

    return hook


@pytest.mark.parametrize("W", [2, 4, 3])
@pytest.mark.parametrize("param_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("comm_streams", [False, True])
@pytest.mark.parametrize("unit_batch", [1, 2, 8])
def test_shard_grads_match_oracle_and_full_batch(W, param_dtype, comm_streams, unit_batch):
    """With ``comm_streams`` the gathers and reduce-scatters run on side streams, and with
    ``unit_batch`` they go out for several units at once (2: the 4 units in pairs; 8: every unit's
    reduce-scatter held to the end of backward): the same bits."""
    _check_shard_grads(W, param_dtype, comm_streams, unit_batch, reshard_after_forward=True)


@pytest.mark.parametrize("W,param_dtype,comm_streams,unit_batch",
                         [(2, torch.float32, False, 1), (4, torch.bfloat16, False, 2), (3, torch.float32, True, 3),
                          (4, torch.float16, True, 8)])
def test_shard_grads_without_reshard_after_forward(W, param_dtype, comm_streams, unit_batch):
    """``reshard_after_forward=False``: the units stay gathered from forward to backward (no backward
    gathers), and are freed after their reduce-scatter as with the default: the same bits."""
    _check_shard_grads(W, param_dtype, comm_streams, unit_batch, reshard_after_forward=False)


def _check_shard_grads(W, param_dtype, comm_streams, unit_batch, reshard_after_forward):
    c = tiny_gpt.Config(n_layer=3)
    ids, tgt = tiny_gpt.batch(c, 12 if W == 3 else 8, seed=1234)
    rank = W - 1
    model = tiny_gpt.GPT(c).to(DEV)
    names_by_id = {id(p): n for n, p in model.named_parameters()}
    captured: dict[int, torch.Tensor] = {}
    for p in model.parameters():
        p.register_post_accumulate_grad_hook(_capture(captured))
    policy = MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32)
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, rank, DEV), mixed_precision=policy,
                comm_streams=comm_streams, unit_batch=unit_batch, reshard_after_forward=reshard_after_forward)
    # peers' gradients are computed by replicas whose parameters are the gathered (param_dtype) values
    replica = []
    for r in range(W):
        m = tiny_gpt.GPT(c).to(DEV)
        with torch.no_grad():
            for p in m.parameters():
                p.copy_(p.to(param_dtype).float())
        m = m.to(param_dtype)
        _, l = m(ids.chunk(W)[r].to(DEV), tgt.chunk(W)[r].to(DEV))
        l.backward()
        replica.append({n: p.grad.detach().clone() for n, p in m.named_parameters()})
    _stage(fsdp, names_by_id, replica, rank, W)
    _, loss = fsdp(ids.chunk(W)[rank].to(DEV), tgt.chunk(W)[rank].to(DEV))
    loss.backward()

    gdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(param_dtype, o.F32)
    for unit in fsdp._units:
        assert not unit.is_unsharded and unit._full.untyped_storage().nbytes() == 0
        assert all(p.grad is None for p in unit.params)
        grads = []
        for r in range(W):
            if r == rank:
                grads.append([host_bits(captured[id(p)]) for p in unit.params])
            else:
                grads.append([host_bits(replica[r][names_by_id[id(p)]]) for p in unit.params])
        want = o.fsdp_reduce_scatter_share(grads, gdt, unit.numels, rank, o.F32, o.F32)
        got = host_bits(unit.flat_shard.grad)
        assert same_bits(got, want), f"unit {unit.name}: " + first_mismatch(got, want)

    if param_dtype == torch.float32:
        # full-batch gradient, this rank's shard of it (reference tolerance 1e-6 relative)
        full = tiny_gpt.GPT(c).to(DEV)
        _, lf = full(ids.to(DEV), tgt.to(DEV))
        lf.backward()
        fg = {n: p.grad for n, p in full.named_parameters()}
        for unit in fsdp._units:
            flat = torch.cat([fg[names_by_id[id(p)]].reshape(-1) for p in unit.params])
            flat = torch.cat([flat, flat.new_zeros(unit.padded_numel - unit.total_numel)])
            S = unit.shard_numel
            ref = flat[rank * S : (rank + 1) * S]
            rel = (unit.flat_shard.grad - ref).abs().max().item() / max(ref.abs().max().item(), 1.0)
            assert rel <= 1e-6


@pytest.mark.parametrize("comm_streams", [False, True])
def test_unshard_casts_into_own_slot_and_gathers_peers(comm_streams):
    c = tiny_gpt.Config()
    W, rank = 4, 2
    model = tiny_gpt.GPT(c).to(DEV)
    init = {n: p.detach().clone() for n, p in model.named_parameters()}
    fsdp = FSDP(
        model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, rank, DEV),
        mixed_precision=MixedPrecisionPolicy(param_dtype=torch.bfloat16), comm_streams=comm_streams,
    )
    with fsdp.summon_full_params():
        for n, p in model.named_parameters():
            want = o.bf16_from_f32(init[n].cpu().numpy().reshape(-1))
            assert np.array_equal(host_bits(p), want), n
    for u in fsdp._units:
        assert u.flat_shard.dtype == torch.float32
        assert not u.is_unsharded


@pytest.mark.parametrize("param_dtype", [torch.float32, torch.bfloat16])
def test_unit_and_memory_summaries(param_dtype):
    """unit_summary() and memory_summary() (fsdp.py:472-492) from their definitions: per unit
    (name, full elements, shard elements); per rank, MiB of the shards and of the replicated model,
    four shard-dtype copies (parameters, gradients, Adam's two moments) sharded or whole, and the
    largest unit gathered in param_dtype."""
    c = tiny_gpt.Config(n_layer=3)
    W = 4
    model = tiny_gpt.GPT(c).to(DEV)
    sizes = {n: p.numel() for n, p in model.named_parameters()}
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, 1, DEV),
                mixed_precision=MixedPrecisionPolicy(param_dtype=param_dtype))
    rows = fsdp.unit_summary()
    assert [r[0] for r in rows] == ["blocks.0", "blocks.1", "blocks.2", "<root>"]
    block = sum(v for n, v in sizes.items() if n.startswith("blocks.0."))
    root = sum(v for n, v in sizes.items() if not n.startswith("blocks."))
    assert [r[1] for r in rows] == [block, block, block, root]
    assert [r[2] for r in rows] == [-(-n // W) for n in (block, block, block, root)]
    total, shard = sum(r[1] for r in rows), sum(r[2] for r in rows)
    mib, gather = 2.0**20, torch.empty((), dtype=param_dtype).element_size()
    assert fsdp.memory_summary() == {
        "params_total_M": total / 1e6,
        "shard_params_MB": shard * 4 / mib,
        "replicated_params_MB": total * 4 / mib,
        "fsdp_state_MB": shard * 4 * 4 / mib,
        "ddp_state_MB": total * 4 * 4 / mib,
        "transient_gather_MB": max(block, root) * gather / mib,
        "num_units": 4,
    }


class _HollowBlock(torch.nn.Module):
    """A unit whose parameters include empty ones: a Linear with no input features (weight
    [8, 0]) and a parameter with no elements (its gradient is empty too)."""

    def __init__(self, seed: int):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.a = torch.nn.Linear(8, 8)
        self.hollow = torch.nn.Linear(0, 8)
        self.nothing = torch.nn.Parameter(torch.zeros(0))
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g))

    def forward(self, x):
        return torch.tanh(self.a(x) + self.hollow(x[..., :0]) + self.nothing.sum())


class _HollowNet(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.blocks = torch.nn.ModuleList([_HollowBlock(s) for s in range(3)])
        self.empty_root = torch.nn.Parameter(torch.zeros(0, 3))

    def forward(self, x):
        for b in self.blocks:
            x = b(x)
        return x.square().mean()


@pytest.mark.parametrize("W,rank,unit_batch", [(2, 0, 1), (3, 2, 2)])
def test_zero_element_parameters(W, rank, unit_batch):
    """Units holding parameters with no elements, and a root unit whose only parameter is empty and
    unused (it never completes, as in the reference, and ``finish_gradient_sync`` finds no gradient
    to flush): every shard gradient bit for bit against the oracle on the gradients this rank
    produced (peers contribute zeros)."""
    model = _HollowNet().to(DEV)
    captured: dict[int, torch.Tensor] = {}
    for p in model.parameters():
        p.register_post_accumulate_grad_hook(_capture(captured))
    fsdp = FSDP(model, unit_types=(_HollowBlock,), process_group=ResidentGroup(W, rank, DEV), unit_batch=unit_batch)
    assert len(fsdp._units) == 4 and any(0 in u.numels for u in fsdp._units)
    x = torch.randn(5, 8, generator=torch.Generator().manual_seed(3)).to(DEV)
    fsdp(x).backward()
    fsdp.finish_gradient_sync()
    for unit in fsdp._units:
        assert all(p.grad is None for p in unit.params)
        own = [host_bits(captured[id(p)]) if id(p) in captured else np.zeros(n, np.float32)
               for p, n in zip(unit.params, unit.numels, strict=True)]
        grads = [own if r == rank else [np.zeros(n, np.float32) for n in unit.numels] for r in range(W)]
        want = o.fsdp_reduce_scatter_share(grads, o.F32, unit.numels, rank, o.F32, o.F32)
        got = host_bits(unit.flat_shard.grad) if unit.flat_shard.grad is not None else np.zeros(0, np.float32)
        assert same_bits(got, want), f"unit {unit.name}: " + first_mismatch(got, want)


@pytest.mark.parametrize("W,rank,unit_batch", [(2, 1, 1), (4, 0, 3)])
def test_frozen_parameters(W, rank, unit_batch):
    """Parameters that do not require gradients stay in their unit's flat shard (the reference
    flattens every parameter) but get no hook: a unit completes when its trainable gradients
    have arrived, and the frozen ones contribute zeros.  Shard gradients bit for bit against the
    oracle on the gradients this rank produced (peers contribute zeros)."""
    c = tiny_gpt.Config(n_layer=2)
    model = tiny_gpt.GPT(c).to(DEV)
    frozen = [p for n, p in model.named_parameters() if n.endswith(("ln1.weight", "proj.bias"))]
    assert frozen
    for p in frozen:
        p.requires_grad_(False)
    captured: dict[int, torch.Tensor] = {}
    for p in model.parameters():
        if p.requires_grad:
            p.register_post_accumulate_grad_hook(_capture(captured))
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, rank, DEV), unit_batch=unit_batch)
    ids, tgt = tiny_gpt.batch(c, 8, seed=11)
    _, loss = fsdp(ids.to(DEV), tgt.to(DEV))
    loss.backward()
    for unit in fsdp._units:
        assert not unit.is_unsharded and all(p.grad is None for p in unit.params)
        own = [host_bits(captured[id(p)]) if p.requires_grad else np.zeros(n, np.float32)
               for p, n in zip(unit.params, unit.numels, strict=True)]
        grads = [own if r == rank else [np.zeros(n, np.float32) for n in unit.numels] for r in range(W)]
        want = o.fsdp_reduce_scatter_share(grads, o.F32, unit.numels, rank, o.F32, o.F32)
        got = host_bits(unit.flat_shard.grad)
        assert same_bits(got, want), f"unit {unit.name}: " + first_mismatch(got, want)


class _MixedBlock(torch.nn.Module):
    """A unit whose parameters come in two dtypes: a bf16 scale -- the module's own parameter, so
    ``parameters()`` yields it before its child's -- and the child's fp32 weights."""

    def __init__(self, seed: int):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.lin = torch.nn.Linear(6, 6)
        self.scale = torch.nn.Parameter(torch.randn(6, generator=g).to(torch.bfloat16))
        with torch.no_grad():
            self.lin.weight.copy_(torch.randn(6, 6, generator=g))
            self.lin.bias.copy_(torch.randn(6, generator=g))

    def forward(self, x):
        return self.lin(x) * self.scale.float()


@pytest.mark.parametrize("param_dtype", [torch.float32, torch.bfloat16])
def test_units_of_mixed_dtypes_flatten_as_copy_converts(param_dtype):
    """The flat parameter takes the unit's first parameter's dtype and every parameter is converted
    into it as the reference's ``copy_`` converts it (fsdp.py:144-148) -- here the fp32 weights
    are rounded to bf16, the first parameter's dtype: gathered, each parameter holds its value
    taken through that dtype and then ``param_dtype``, bit for bit."""
    net = torch.nn.Sequential(_MixedBlock(1), _MixedBlock(2)).to(DEV)
    originals = [p.detach().clone() for p in net.parameters()]
    assert [p.dtype for p in net[0].parameters()] == [torch.bfloat16, torch.float32, torch.float32]
    policy = MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32)
    fsdp = FSDP(net, unit_types=(_MixedBlock,), process_group=ResidentGroup(2, 1, DEV), mixed_precision=policy)
    assert all(u.flat_shard.dtype == torch.bfloat16 for u in fsdp._units)
    with fsdp.summon_full_params():
        for p, want in zip(net.parameters(), originals, strict=True):
            expect = want.to(torch.bfloat16).to(param_dtype)
            assert p.dtype == param_dtype and torch.equal(p.detach(), expect)


@pytest.mark.parametrize("param_dtype", [torch.float32, torch.bfloat16])
def test_single_process_without_a_group(param_dtype):
    """FSDP with no process group (world 1, the reference trainer run as one process): every unit
    holds the whole flat parameter as its shard, and its reduce-scatter is the world-1 path of
    fsdp.py:230-231 -- the flattened gradients, unscaled by nothing, set as the shard gradient --
    bit for bit against the oracle on the gradients backward produced."""
    c = tiny_gpt.Config(n_layer=2)
    model = tiny_gpt.GPT(c).to(DEV)
    captured: dict[int, torch.Tensor] = {}
    for p in model.parameters():
        p.register_post_accumulate_grad_hook(_capture(captured))
    policy = MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32)
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), mixed_precision=policy, device=DEV)
    assert fsdp.world_size == 1 and all(u.shard_numel == u.total_numel for u in fsdp._units)
    ids, tgt = tiny_gpt.batch(c, 4, seed=21)
    _, loss = fsdp(ids.to(DEV), tgt.to(DEV))
    loss.backward()
    gdt = {torch.bfloat16: o.BF16}.get(param_dtype, o.F32)
    for unit in fsdp._units:
        assert all(p.grad is None for p in unit.params)
        want = o.fsdp_reduce_scatter_share([[host_bits(captured[id(p)]) for p in unit.params]], gdt, unit.numels,
                                           0, o.F32, o.F32)
        got = host_bits(unit.flat_shard.grad)
        assert same_bits(got, want), f"unit {unit.name}: " + first_mismatch(got, want)


@pytest.mark.parametrize("unit_batch", [1, 4])
def test_root_unit_only(unit_batch):
    """No unit types: the whole model is the root unit (fsdp.py:343-354), gathered before forward,
    reduced when its last gradient arrives.  Its shard gradient bit for bit against the oracle on
    this rank's gradients (peers contribute zeros)."""
    c = tiny_gpt.Config(n_layer=2)
    model = tiny_gpt.GPT(c).to(DEV)
    captured: dict[int, torch.Tensor] = {}
    for p in model.parameters():
        p.register_post_accumulate_grad_hook(_capture(captured))
    W, rank = 4, 2
    fsdp = FSDP(model, process_group=ResidentGroup(W, rank, DEV), unit_batch=unit_batch)
    assert [u.name for u in fsdp._units] == ["<root>"]
    ids, tgt = tiny_gpt.batch(c, 4, seed=8)
    _, loss = fsdp(ids.to(DEV), tgt.to(DEV))
    loss.backward()
    unit = fsdp._units[0]
    assert not unit.is_unsharded and all(p.grad is None for p in unit.params)
    own = [host_bits(captured[id(p)]) for p in unit.params]
    grads = [own if r == rank else [np.zeros(n, np.float32) for n in unit.numels] for r in range(W)]
    want = o.fsdp_reduce_scatter_share(grads, o.F32, unit.numels, rank, o.F32, o.F32)
    got = host_bits(unit.flat_shard.grad)
    assert same_bits(got, want), first_mismatch(got, want)


def test_sharding_is_real_and_unit_count():
    c = tiny_gpt.Config(n_layer=3)
    for W in (2, 4):
        model = tiny_gpt.GPT(c).to(DEV)
        full = sum(p.numel() for p in model.parameters())
        fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, 0, DEV))
        local = sum(p.numel() for p in fsdp.parameters())
        assert local <= full / W * 1.25
        s = fsdp.memory_summary()
        assert s["num_units"] == c.n_layer + 1
        assert s["fsdp_state_MB"] < s["ddp_state_MB"]
        # what an optimizer sees: the flat shards only, named as the reference names them
        n = c.n_layer + 1
        assert [name for name, _ in fsdp.named_parameters()] == [f"_flat_shard_{i}" for i in range(n)]
        assert [name for name, _ in fsdp.named_parameters(prefix="m")] == [f"m._flat_shard_{i}" for i in range(n)]
        assert [p is u.flat_shard for p, u in zip(fsdp.parameters(), fsdp._units, strict=True)] == [True] * n
        assert [k for k in fsdp.state_dict() if k.startswith("_shards.")] == [f"_shards.{i}" for i in range(n)]


@pytest.mark.parametrize("comm_streams,unit_batch", [(False, 1), (True, 1), (False, 3), (True, 3)])
def test_no_sync_accumulates_then_flushes(comm_streams, unit_batch):
    """Reference tests/test_fsdp.py:214-238 on one GPU (world emulated, peers zero)."""
    c = tiny_gpt.Config()
    W, rank = 2, 1
    ids, tgt = tiny_gpt.batch(c, 8)
    my_ids, my_tgt = ids.chunk(W)[rank].to(DEV), tgt.chunk(W)[rank].to(DEV)

    single = FSDP(tiny_gpt.GPT(c).to(DEV), unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, rank, DEV),
                  comm_streams=comm_streams, unit_batch=unit_batch)
    _, loss = single(my_ids, my_tgt)
    loss.backward()
    expected = [p.grad.clone() for p in single.parameters()]

    accum = FSDP(tiny_gpt.GPT(c).to(DEV), unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, rank, DEV),
                 comm_streams=comm_streams, unit_batch=unit_batch)
    with accum.no_sync():
        for h_ids, h_tgt in zip(my_ids.chunk(2), my_tgt.chunk(2), strict=True):
            _, l = accum(h_ids, h_tgt)
            (l / 2).backward()
    accum.finish_gradient_sync()
    for got, want in zip(accum.parameters(), expected, strict=True):
        rel = (got.grad - want).abs().max().item() / max(want.abs().max().item(), 1.0)
        assert rel <= 2e-5


def test_non_contiguous_gradient_is_rejected():
    """The shard kernels read each full-size gradient as one flat span: a strided gradient is refused
    with an error before anything is launched, and the unit's gradients are left as they were."""
    c = tiny_gpt.Config(n_layer=1)
    fsdp = FSDP(tiny_gpt.GPT(c).to(DEV), unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(2, 0, DEV))
    unit = next(u for u in fsdp._units if any(p.dim() == 2 for p in u.params))
    unit.unshard()
    for p in unit.params:
        if p.dim() == 2:
            p.grad = torch.zeros(p.shape[::-1], dtype=p.dtype, device=DEV).t()  # right shape, transposed strides
            assert not p.grad.is_contiguous()
        else:
            p.grad = torch.zeros_like(p)
    with pytest.raises(RuntimeError, match="not contiguous"):
        unit.reduce_scatter_grads()
    assert all(p.grad is not None for p in unit.params)
    assert unit.flat_shard.grad is None


def test_second_backward_accumulates_into_shard_grad():
    c = tiny_gpt.Config()
    W, rank = 2, 0
    ids, tgt = tiny_gpt.batch(c, 4)
    fsdp = FSDP(tiny_gpt.GPT(c).to(DEV), unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, rank, DEV))
    _, l = fsdp(ids.to(DEV), tgt.to(DEV))
    l.backward()
    first = [p.grad.clone() for p in fsdp.parameters()]
    _, l = fsdp(ids.to(DEV), tgt.to(DEV))
    l.backward()
    for p, f in zip(fsdp.parameters(), first, strict=True):
        # the same batch twice: the shard gradient doubles (bitwise accumulation
        # is covered by the kernel tests; backward kernels need not be deterministic)
        rel = (p.grad - 2 * f).abs().max().item() / max((2 * f).abs().max().item(), 1.0)
        assert rel <= 1e-6


def _sgd_run(W, rank, param_dtype, steps=4, lr=0.1, comm_streams=False, unit_batch=1):
    """FSDP on rank ``rank`` of a ResidentGroup next to a full-batch reference, both SGD.

    Every step the emulated peers get what they would hold: their shard of the
    current weights (as gathered, in ``param_dtype``) and the local gradients of a
    replica holding those weights on their chunk of the batch."""
    c = tiny_gpt.Config(n_layer=2)
    ids, tgt = tiny_gpt.batch(c, 8, seed=99)
    ref = tiny_gpt.GPT(c).to(DEV)
    model = tiny_gpt.GPT(c).to(DEV)
    names_by_id = {id(p): n for n, p in model.named_parameters()}
    policy = MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32)
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, rank, DEV), mixed_precision=policy,
                comm_streams=comm_streams, unit_batch=unit_batch)
    opt = torch.optim.SGD(fsdp.parameters(), lr=lr)
    opt_ref = torch.optim.SGD(ref.parameters(), lr=lr)
    out = []
    for _ in range(steps):
        cur = {n: p.detach().clone() for n, p in ref.named_parameters()}
        for unit in fsdp._units:
            flat = torch.cat([cur[names_by_id[id(p)]].reshape(-1) for p in unit.params])
            flat = torch.cat([flat, flat.new_zeros(unit.padded_numel - unit.total_numel)])
            S, shards = unit.shard_numel, unit.peer_param_shards()
            for r in range(W):
                if r != rank:
                    shards[r].copy_(flat[r * S : (r + 1) * S].to(shards.dtype))
        replica = []
        for r in range(W):
            if r == rank:
                replica.append({})
                continue
            m = tiny_gpt.GPT(c).to(DEV)
            with torch.no_grad():
                for n, p in m.named_parameters():
                    p.copy_(cur[n].to(param_dtype).float())
            m = m.to(param_dtype)
            _, l_r = m(ids.chunk(W)[r].to(DEV), tgt.chunk(W)[r].to(DEV))
            l_r.backward()
            replica.append({n: p.grad.detach().clone() for n, p in m.named_parameters()})
        _stage(fsdp, names_by_id, replica, rank, W)
        _, loss = fsdp(ids.chunk(W)[rank].to(DEV), tgt.chunk(W)[rank].to(DEV))
        loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
        _, lref = ref(ids.to(DEV), tgt.to(DEV))
        lref.backward()
        opt_ref.step()
        opt_ref.zero_grad(set_to_none=True)
        out.append((loss.item(), lref.item()))
    return fsdp, ref, names_by_id, out


@pytest.mark.parametrize("W,rank,comm_streams,unit_batch",
                         [(2, 1, False, 1), (4, 2, False, 1), (4, 2, True, 1), (4, 2, False, 2), (4, 1, True, 3)])
def test_sgd_steps_track_full_batch(W, rank, comm_streams, unit_batch):
    """Reference tests/test_fsdp.py:92-127: after 4 SGD steps this rank's shard equals its slice of
    the full-batch model's weights (the reference compares with DDP; both equal the full batch).
    With ``comm_streams`` the optimizer must see the side streams' shard gradients, and with
    ``unit_batch`` the reduce-scatters held to the end of backward."""
    fsdp, ref, names_by_id, _ = _sgd_run(W, rank, torch.float32, comm_streams=comm_streams, unit_batch=unit_batch)
    final = {n: p.detach() for n, p in ref.named_parameters()}
    for unit in fsdp._units:
        flat = torch.cat([final[names_by_id[id(p)]].reshape(-1) for p in unit.params])
        flat = torch.cat([flat, flat.new_zeros(unit.padded_numel - unit.total_numel)])
        S = unit.shard_numel
        want = flat[rank * S : (rank + 1) * S]
        rel = (unit.flat_shard.detach() - want).abs().max().item() / max(want.abs().max().item(), 1.0)
        assert rel <= 1e-5, f"unit {unit.name}: {rel:.3e}"


class _OrderBlock(torch.nn.Module):
    def __init__(self, gen: torch.Generator):
        super().__init__()
        self.lin = torch.nn.Linear(8, 8)
        with torch.no_grad():
            self.lin.weight.copy_(torch.randn(8, 8, generator=gen) * 0.5)
            self.lin.bias.copy_(torch.randn(8, generator=gen) * 0.1)

    def forward(self, x):
        return torch.tanh(self.lin(x))


class _OutOfOrderNet(torch.nn.Module):
    """Blocks registered 0..n-1 but run in ``order`` (which may leave some out): the unit chain a
    batched gather walks (registration order) is not the order the units run in."""

    def __init__(self, order: list[int], seed: int = 17, n_blocks: int | None = None):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.order = list(order)
        self.inp = torch.nn.Linear(4, 8)
        self.blocks = torch.nn.ModuleList([_OrderBlock(g) for _ in range(n_blocks or len(order))])
        self.head = torch.nn.Linear(8, 1)
        with torch.no_grad():
            for p in (*self.inp.parameters(), *self.head.parameters()):
                p.copy_(torch.randn(p.shape, generator=g) * 0.5)

    def forward(self, x):
        x = torch.tanh(self.inp(x))
        for i in self.order:
            x = self.blocks[i](x)
        return self.head(x).square().mean()


@pytest.mark.parametrize("order", [[3, 2, 1, 0], [0, 2, 1, 3], [1, 3, 0, 2]])
@pytest.mark.parametrize("unit_batch", [2, 3])
def test_units_run_out_of_registration_order(order, unit_batch):
    """A batched backward gather walks the units in registration order; when the model runs
    them in another order it must not bring back a unit whose backward has already finished
    (it would stay gathered past the optimizer step and the next forward would use pre-update
    weights).  Every unit is sharded after each backward (the reference's invariant,
    fsdp.py:199-213), and after 3 SGD steps this rank's shards equal its slice of the
    full-batch model's weights."""
    _train_out_of_order(order, len(order), unit_batch)


@pytest.mark.parametrize("order,n_blocks", [([0, 1, 3], 4), ([2, 0], 4), ([3, 1], 5)])
@pytest.mark.parametrize("unit_batch", [2, 3])
def test_units_skipped_in_forward(order, n_blocks, unit_batch):
    """A batched forward gather brings the next units in registration order along; one the model
    then skips never runs, so no hook reshards it: it is freed when the engine finishes the
    backward, and every unit is sharded after each backward (the reference never gathers a
    skipped unit).  The skipped units get no gradient and keep their weights; the SGD
    trajectory still matches the full batch."""
    _train_out_of_order(order, n_blocks, unit_batch)


@pytest.mark.parametrize("seed", range(12))
def test_random_unit_orders_track_full_batch(seed):
    """Seeded random cases of the two tests above: 2-6 registered blocks run as a random
    permutation of a random subset, W in [2, 4], any rank, ``unit_batch`` 1-4, side streams or
    not, ``reshard_after_forward`` or not; 3 SGD steps, every unit sharded after each backward
    and the final shards on this rank's slice of the full-batch model's weights."""
    rng = np.random.default_rng(31000 + seed)
    n_blocks = int(rng.integers(2, 7))
    order = [int(i) for i in rng.permutation(n_blocks)[: int(rng.integers(1, n_blocks + 1))]]
    W = int(rng.integers(2, 5))
    rank = int(rng.integers(0, W))
    unit_batch = int(rng.integers(1, 5))
    comm_streams, reshard = bool(rng.random() < 0.3), bool(rng.random() < 0.7)
    print(f"seed {seed}: {n_blocks} blocks run as {order}, W={W} rank={rank} unit_batch={unit_batch} "
          f"comm_streams={comm_streams} reshard_after_forward={reshard}", flush=True)
    _train_out_of_order(order, n_blocks, unit_batch, W=W, rank=rank, comm_streams=comm_streams, reshard=reshard,
                        seed=100 + seed)


def _train_out_of_order(order, n_blocks, unit_batch, W=2, rank=1, comm_streams=False, reshard=True, seed=17):
    steps, lr = 3, 0.2
    x = torch.randn(12, 4, generator=torch.Generator().manual_seed(23)).to(DEV)  # W equal chunks for W = 2, 3, 4
    ref = _OutOfOrderNet(order, seed=seed, n_blocks=n_blocks).to(DEV)
    model = _OutOfOrderNet(order, seed=seed, n_blocks=n_blocks).to(DEV)
    names_by_id = {id(p): n for n, p in model.named_parameters()}
    fsdp = FSDP(model, unit_types=(_OrderBlock,), process_group=ResidentGroup(W, rank, DEV), unit_batch=unit_batch,
                comm_streams=comm_streams, reshard_after_forward=reshard)
    opt = torch.optim.SGD(fsdp.parameters(), lr=lr)
    opt_ref = torch.optim.SGD(ref.parameters(), lr=lr)
    for _ in range(steps):
        cur = {n: p.detach().clone() for n, p in ref.named_parameters()}
        for unit in fsdp._units:
            flat = torch.cat([cur[names_by_id[id(p)]].reshape(-1) for p in unit.params])
            flat = torch.cat([flat, flat.new_zeros(unit.padded_numel - unit.total_numel)])
            S, shards = unit.shard_numel, unit.peer_param_shards()
            for r in range(W):
                if r != rank:
                    shards[r].copy_(flat[r * S : (r + 1) * S])
        replica = [{} for _ in range(W)]
        for r in range(W):  # the peers' backward on their own chunks, from the same weights
            if r == rank:
                continue
            peer = _OutOfOrderNet(order, seed=seed, n_blocks=n_blocks).to(DEV)
            with torch.no_grad():
                for n, p in peer.named_parameters():
                    p.copy_(cur[n])
            peer(x.chunk(W)[r]).backward()
            replica[r] = {n: p.grad.detach().clone() if p.grad is not None else torch.zeros_like(p)
                          for n, p in peer.named_parameters()}
        _stage(fsdp, names_by_id, replica, rank, W)
        fsdp(x.chunk(W)[rank]).backward()
        assert not any(u.is_unsharded for u in fsdp._units), "a unit is still gathered after backward"
        opt.step()
        opt.zero_grad(set_to_none=True)
        ref(x).backward()
        opt_ref.step()
        opt_ref.zero_grad(set_to_none=True)
    final = {n: p.detach() for n, p in ref.named_parameters()}
    for unit in fsdp._units:
        flat = torch.cat([final[names_by_id[id(p)]].reshape(-1) for p in unit.params])
        flat = torch.cat([flat, flat.new_zeros(unit.padded_numel - unit.total_numel)])
        S = unit.shard_numel
        want = flat[rank * S : (rank + 1) * S]
        rel = (unit.flat_shard.detach() - want).abs().max().item() / max(want.abs().max().item(), 1.0)
        assert rel <= 1e-5, f"unit {unit.name}: {rel:.3e}"


@pytest.mark.parametrize("param_dtype", [torch.bfloat16, torch.float16])
def test_low_precision_params_track_fp32_training(param_dtype):
    """Reference tests/test_fsdp.py:189-211: bf16 gathered parameters with fp32 reduction keep the
    loss within 0.05 of fp32 training, and the master shard stays fp32; likewise fp16, the
    reference trainer's --fsdp-param-dtype fp16."""
    fsdp, _, _, low = _sgd_run(2, 0, param_dtype)
    _, _, _, fp32 = _sgd_run(2, 0, torch.float32)
    for (mine, _), (want, _) in zip(low, fp32, strict=True):  # this rank's loss on its chunk, both runs
        assert abs(mine - want) <= 0.05
    assert all(u.flat_shard.dtype == torch.float32 for u in fsdp._units)


@pytest.mark.parametrize("param_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("W,rank", [(2, 1), (4, 3)])
def test_keep_low_precision_shard(param_dtype, W, rank):
    """MixedPrecisionPolicy(keep_low_precision_shard=True) (fsdp.py:138-140): the master shard is
    kept in param_dtype, unshard gathers it without a cast, and reduce_scatter_grads rounds the
    fp32 reduction to param_dtype (fsdp.py:233) and accumulates in it (fsdp.py:237)."""
    odt = o.BF16 if param_dtype == torch.bfloat16 else o.F16
    c = tiny_gpt.Config(n_layer=2)
    model = tiny_gpt.GPT(c).to(DEV)
    init = {n: p.detach().clone() for n, p in model.named_parameters()}
    names = {id(p): n for n, p in model.named_parameters()}
    policy = MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32, keep_low_precision_shard=True)
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, rank, DEV), mixed_precision=policy)
    rng = np.random.default_rng(21 + W)
    for unit in fsdp._units:
        assert unit.flat_shard.dtype == param_dtype
        S, P = unit.shard_numel, unit.padded_numel
        flat = np.zeros(P, np.float32)
        flat[: unit.total_numel] = np.concatenate([init[names[id(p)]].cpu().numpy().reshape(-1) for p in unit.params])
        want_shard = o.from_f32(flat[rank * S : (rank + 1) * S], odt)
        assert same_bits(host_bits(unit.flat_shard), want_shard)
        unit.unshard()
        assert same_bits(host_bits(unit._full[rank * S : (rank + 1) * S]), want_shard)
        existing = None
        for _ in range(2):  # set, then accumulate in param_dtype
            grads = [[o.from_f32((rng.standard_normal(n) * 1e-3).astype(np.float32), odt) for n in unit.numels]
                     for _ in range(W)]
            peers = unit.peer_grad_contributions()
            for r in range(W):
                if r != rank:
                    peers[r].copy_(torch.from_numpy(o.fsdp_flatten(grads[r], odt, unit.numels, P, odt).view(
                        np.int16 if odt == o.BF16 else np.float16).copy()).to(DEV).view(param_dtype))
            for p, g in zip(unit.params, grads[rank], strict=True):
                t = torch.from_numpy(g.view(np.int16) if odt == o.BF16 else g.copy())
                p.grad = t.to(DEV).view(param_dtype).view(p.shape)
            unit.reduce_scatter_grads()
            want = o.fsdp_reduce_scatter_share(grads, odt, unit.numels, rank, o.F32, odt, existing=existing)
            got = host_bits(unit.flat_shard.grad)
            assert unit.flat_shard.grad.dtype == param_dtype
            assert same_bits(got, want), f"unit {unit.name}: " + first_mismatch(got, want)
            existing = want
        unit.reshard()


def test_dropped_fsdp_frees_its_buffers():
    """The gradient hooks hold the wrapper and its units weakly: dropping the wrapper and the
    module frees the shards, the gather buffers and the resident peer buffers."""
    import gc
    import weakref

    c = tiny_gpt.Config(n_layer=2, n_embd=256)
    torch.cuda.synchronize()
    gc.collect()
    base = torch.cuda.memory_allocated(DEV)
    model = tiny_gpt.GPT(c).to(DEV)
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(4, 1, DEV),
                mixed_precision=MixedPrecisionPolicy(param_dtype=torch.bfloat16))
    ids, tgt = tiny_gpt.batch(c, 4, seed=3)
    logits, loss = fsdp(ids.to(DEV), tgt.to(DEV))
    loss.backward()
    refs = [weakref.ref(fsdp), weakref.ref(fsdp._units[0]), weakref.ref(fsdp._units[0].flat_shard)]
    assert torch.cuda.memory_allocated(DEV) > base
    # (an output kept alive would hold its autograd graph, and the graph the module hooks)
    del fsdp, model, loss, logits
    gc.collect()
    assert all(r() is None for r in refs)
    assert torch.cuda.memory_allocated(DEV) == base



class _Blk(torch.nn.Module):
    def __init__(self, k: int, gen: torch.Generator):
        super().__init__()
        self.w = torch.nn.Parameter(torch.randn(17 + k % 7, 9, generator=gen) * 0.02)
        self.b = torch.nn.Parameter(torch.randn(5 + k % 3, generator=gen) * 0.02)


class _Stack(torch.nn.Module):
    def __init__(self, n: int, seed: int = 5):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        self.blocks = torch.nn.ModuleList([_Blk(k, gen) for k in range(n)])


def _grad_bits(rng, n, dt):
    return o.from_f32((rng.standard_normal(n) * 1e-3).astype(np.float32), dt)


def _dev_from_bits(bits, dtype):
    if dtype == torch.bfloat16:
        return torch.from_numpy(bits.view(np.int16).copy()).to(DEV).view(torch.bfloat16)
    return torch.from_numpy(bits.copy()).to(DEV)


@pytest.mark.parametrize("param_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n_blocks", [3, 60])
@pytest.mark.parametrize("comm_streams", [False, True])
def test_flush_of_many_units_matches_per_unit_and_oracle(param_dtype, n_blocks, comm_streams):
    """finish_gradient_sync with gradients on every unit sends all units' shares out together (one
    multi-unit dispatch; a device plan beyond 48 pieces).  Every shard gradient equals the per-unit
    reduce_scatter_grads result and the oracle bit for bit; a second flush accumulates into them."""
    W, rank = 4, 2
    dt = o.BF16 if param_dtype == torch.bfloat16 else o.F32
    policy = MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32)
    wraps = [FSDP(_Stack(n_blocks).to(DEV), unit_types=(_Blk,), process_group=ResidentGroup(W, rank, DEV),
                  mixed_precision=policy, comm_streams=comm_streams and i == 0) for i in range(2)]
    batched, per_unit = wraps
    assert len(batched._units) == n_blocks
    rng = np.random.default_rng(77 + n_blocks)
    existing = [None] * n_blocks
    for flush in range(2):
        for u, (ua, ub) in enumerate(zip(batched._units, per_unit._units, strict=True)):
            grads = [[_grad_bits(rng, n, dt) for n in ua.numels] for _ in range(W)]
            for fs in (ua, ub):
                peers = fs.peer_grad_contributions()
                for r in range(W):
                    if r != rank:
                        peers[r].copy_(_dev_from_bits(o.fsdp_flatten(grads[r], dt, fs.numels, fs.padded_numel, dt),
                                                      param_dtype))
                for p, g in zip(fs.params, grads[rank], strict=True):
                    p.grad = _dev_from_bits(g, param_dtype).view(p.shape)
            existing[u] = o.fsdp_reduce_scatter_share(grads, dt, ua.numels, rank, o.F32, o.F32, existing=existing[u])
        batched.finish_gradient_sync()
        for ub in per_unit._units:
            ub.reduce_scatter_grads()
        for u, (ua, ub) in enumerate(zip(batched._units, per_unit._units, strict=True)):
            got, ref = host_bits(ua.flat_shard.grad), host_bits(ub.flat_shard.grad)
            assert same_bits(got, ref), f"flush {flush} unit {u}: " + first_mismatch(got, ref)
            assert same_bits(got, existing[u]), f"flush {flush} unit {u}: " + first_mismatch(got, existing[u])
            assert all(p.grad is None for p in ua.params)


@pytest.mark.parametrize("comm_streams", [False, True])
def test_summon_of_many_units_gathers_every_parameter(comm_streams):
    """summon_full_params over 60 units: the casts and the peers' gather copies go out batched (device
    plans beyond 48 spans); every gathered parameter is the bf16 cast of its initial value, and the
    units are freed again afterwards."""
    W, rank = 4, 1
    model = _Stack(60).to(DEV)
    init = {n: p.detach().clone() for n, p in model.named_parameters()}
    fsdp = FSDP(model, unit_types=(_Blk,), process_group=ResidentGroup(W, rank, DEV),
                mixed_precision=MixedPrecisionPolicy(param_dtype=torch.bfloat16), comm_streams=comm_streams)
    with fsdp.summon_full_params():
        for n, p in model.named_parameters():
            want = o.bf16_from_f32(init[n].cpu().numpy().reshape(-1))
            assert np.array_equal(host_bits(p), want), n
    assert not any(u.is_unsharded for u in fsdp._units)
