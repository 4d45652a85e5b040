"""DDP and the grad scaler through the Python API, on the GPU, vs the oracle.

W data-parallel replicas are emulated on one GPU with a ResidentGroup: the
peers' packed, pre-scaled bucket contributions (what would arrive over the
wire) are staged with the oracle's pack, this rank's gradients go through the
real DDP hooks / finish_gradient_sync, and the results are compared bit for
bit with oracle.ddp_pipeline, and within the reference's 2e-5 tolerance with
the single-process full-batch gradient (reference tests/test_ddp.py:32-146).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

import tiny_gpt
from conftest import first_mismatch, same_bits
from minidist import DDP, DistributedGradScaler, ResidentGroup
from oracle import gradpath as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().reshape(-1)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().astype(np.uint16)
    return t.numpy().copy()


def dev_from(a: np.ndarray, shape) -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(DEV).view(shape)
    return torch.from_numpy(a.copy()).to(DEV).view(shape)


def odt(dtype: torch.dtype) -> str:
    return {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(dtype, o.F32)


class Flat(nn.Module):
    """Parameters of given shapes, registered in order (no forward needed)."""

    def __init__(self, shapes, dtype=torch.float32):
        super().__init__()
        self.ps = nn.ParameterList([nn.Parameter(torch.zeros(s, dtype=dtype, device=DEV)) for s in shapes])


def stage_peers(ddp: DDP, replica_grads, dtypes, rank: int, W: int) -> None:
    """Write every peer's contribution into its resident row, in the bucket's wire format:
    its packed, 1/W-scaled bucket, or for a widening bucket its raw gradients."""
    params = [p for p in ddp.module.parameters() if p.requires_grad]
    index = {id(p): i for i, p in enumerate(params)}
    for b, bucket in enumerate(ddp._buckets):
        idxs = [index[id(p)] for p in bucket.params]
        rows = ddp.bucket_replicas(b)
        wire_dtype, prescaled = ddp.bucket_wire_format(b)
        for r in range(W):
            if r == rank:
                continue
            packed = o.pack([replica_grads[r][i] for i in idxs], [dtypes[i] for i in idxs],
                            [params[i].numel() for i in idxs], odt(wire_dtype), 1.0 / W if prescaled else 1.0)
            rows[r].copy_(dev_from(packed, rows[r].shape))


def synthetic_grads(rng, shapes, W, dtype, scale, none_at=()):
    out = []
    for r in range(W):
        row = []
        for i, s in enumerate(shapes):
            n = int(np.prod(s))
            g = (rng.standard_normal(n) * 1e-3 * scale).astype(np.float32)
            row.append(o.from_f32(g, odt(dtype)))
        out.append(row)
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("W,rank", [(2, 1), (4, 0), (8, 5), (3, 2)])
@pytest.mark.parametrize("cap", [1e-6, 0.01, 25.0, 1e6])
def test_finish_gradient_sync_bitwise(rng, dtype, W, rank, cap):
    shapes = [(33,), (64, 8), (5,), (130,), (1,), (7, 9), (256, 4), (3,)]
    model = Flat(shapes, dtype)
    grp = ResidentGroup(W, rank, DEV)
    ddp = DDP(model, process_group=grp, bucket_cap_mb=cap)
    grads = synthetic_grads(rng, shapes, W, dtype, 2.0**10)
    grads[rank][2] = None  # a parameter that received no gradient on this rank
    dts = [odt(dtype)] * len(shapes)
    stage_peers(ddp, grads, dts, rank, W)
    for p, g in zip(model.parameters(), grads[rank], strict=True):
        p.grad = None if g is None else dev_from(g, p.shape)
    ddp.finish_gradient_sync()
    want = o.ddp_pipeline(grads, dts, [int(np.prod(s)) for s in shapes], cap, rank, None)
    for i, p in enumerate(model.parameters()):
        got = host_bits(p.grad)
        assert same_bits(got, want["grads"][i]), f"param {i}: " + first_mismatch(got, want["grads"][i])
    for b, bucket in enumerate(ddp._buckets):
        assert same_bits(host_bits(bucket.buffer), want["reduced"][b])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cap", [1e-6, 25.0])
def test_zero_element_parameters(rng, dtype, cap):
    """Parameters with no elements (a shape with a 0) anywhere in the order, as the reference's
    ``copy_`` of an empty gradient allows: with one bucket per parameter some buckets are empty.
    Every gradient and bucket bit for bit against the oracle, two steps."""
    shapes = [(0,), (33,), (0, 4), (5, 7), (0,), (1,), (64,), (0, 0)]
    W, rank = 4, 1
    model = Flat(shapes, dtype)
    grp = ResidentGroup(W, rank, DEV)
    scaler = DistributedGradScaler(init_scale=2.0**8)
    ddp = DDP(model, process_group=grp, bucket_cap_mb=cap, grad_scaler=scaler)
    assert any(b.numel == 0 for b in ddp._buckets) == (cap < 1)
    dts = [odt(dtype)] * len(shapes)
    numels = [int(np.prod(s)) for s in shapes]

    class _Opt:
        param_groups = [{"params": list(model.parameters())}]

    for step in range(2):
        grads = synthetic_grads(rng, shapes, W, dtype, 2.0**8)
        stage_peers(ddp, grads, dts, rank, W)
        for p, g in zip(model.parameters(), grads[rank], strict=True):
            p.grad = dev_from(g, p.shape)
        ddp.finish_gradient_sync()
        assert not scaler.unscale_(_Opt())
        scaler.update()
        want = o.ddp_pipeline(grads, dts, numels, cap, rank, 1.0 / 2.0**8)
        for i, p in enumerate(model.parameters()):
            got = host_bits(p.grad)
            assert got.size == numels[i]
            assert same_bits(got, want["grads"][i]), f"step {step} param {i}: " + first_mismatch(got, want["grads"][i])
        for b, bucket in enumerate(ddp._buckets):
            assert same_bits(host_bits(bucket.buffer), want["reduced"][b]), f"step {step} bucket {b}"


@pytest.mark.parametrize("cap", [1e-6, 0.001, 25.0])
def test_frozen_parameters_stay_out_of_the_buckets(rng, cap):
    """Parameters that do not require gradients are not bucketed (ddp.py:146): the buckets hold the
    trainable ones only, in their reverse order, and a frozen parameter's gradient is left as the
    caller set it.  Trainable gradients bit for bit against the oracle over the trainable list."""
    shapes = [(33,), (64, 8), (5,), (130,), (1,), (7, 9)]
    frozen = {1, 4}
    W, rank = 4, 3
    model = Flat(shapes)
    for i, p in enumerate(model.parameters()):
        p.requires_grad_(i not in frozen)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap)
    trainable = [i for i in range(len(shapes)) if i not in frozen]
    bucketed = [id(p) for b in ddp._buckets for p in b.params]
    params = list(model.parameters())
    assert sorted(bucketed) == sorted(id(params[i]) for i in trainable)
    grads = synthetic_grads(rng, [shapes[i] for i in trainable], W, torch.float32, 2.0**10)
    dts = [o.F32] * len(trainable)
    stage_peers(ddp, grads, dts, rank, W)
    marker = torch.full((64, 8), 7.0, device=DEV)
    params[1].grad = marker  # a frozen parameter's gradient, set by the caller: untouched
    for k, i in enumerate(trainable):
        params[i].grad = dev_from(grads[rank][k], shapes[i])
    ddp.finish_gradient_sync()
    want = o.ddp_pipeline(grads, dts, [int(np.prod(shapes[i])) for i in trainable], cap, rank, None)
    for k, i in enumerate(trainable):
        got = host_bits(params[i].grad)
        assert same_bits(got, want["grads"][k]), f"param {i}: " + first_mismatch(got, want["grads"][k])
    assert params[1].grad is marker and bool((marker == 7.0).all()) and params[4].grad is None


class _TiedLM(nn.Module):
    """An embedding whose weight is also the output projection's (a tied LM head): one parameter,
    two uses in forward, one accumulated gradient."""

    def __init__(self, vocab: int = 50, h: int = 16):
        super().__init__()
        g = torch.Generator().manual_seed(5)
        self.emb = nn.Embedding(vocab, h)
        self.mid = nn.Linear(h, h)
        self.head = nn.Linear(h, vocab, bias=False)
        self.head.weight = self.emb.weight
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g) * 0.1)

    def forward(self, ids):
        return self.head(torch.tanh(self.mid(self.emb(ids)))).logsumexp(-1).mean()


@pytest.mark.parametrize("cap,overlap", [(1e-6, True), (25.0, True), (25.0, False)])
def test_tied_parameter_is_reduced_once(cap, overlap):
    """A parameter used twice in forward is bucketed once (``parameters()`` yields it once), its hook
    fires once per backward, and it is averaged once: with the peers' contributions zero, every
    gradient is this rank's own backward gradient times 1/W, bit for bit (W a power of two)."""
    W, rank = 4, 0
    model = _TiedLM().to(DEV)
    params = list(model.parameters())
    assert len(params) == 3
    captured: dict[int, torch.Tensor] = {}
    for p in params:
        p.register_post_accumulate_grad_hook(lambda q: captured.__setitem__(id(q), q.grad.detach().clone()))
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, overlap_with_backward=overlap)
    assert sum(len(b.params) for b in ddp._buckets) == 3
    ids = torch.randint(0, 50, (4, 9), generator=torch.Generator().manual_seed(2)).to(DEV)
    ddp(ids).backward()
    for p in params:
        want = captured[id(p)] * (1.0 / W)
        assert torch.equal(p.grad, want)


class _WithUnused(nn.Module):
    def __init__(self):
        super().__init__()
        g = torch.Generator().manual_seed(9)
        self.a = nn.Linear(8, 8)
        self.unused = nn.Linear(8, 8)  # never called: its hooks never fire
        self.b = nn.Linear(8, 1)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g))

    def forward(self, x):
        return self.b(torch.tanh(self.a(x))).square().mean()


@pytest.mark.parametrize("cap,overlap", [(1e-6, True), (25.0, True), (1e-6, False)])
def test_unused_parameter_gets_the_average_of_the_peers(rng, cap, overlap):
    """A parameter that takes no part in forward: its bucket is flushed at the end of backward
    with zeros for this rank (ddp.py:87-88) and it receives a fresh gradient holding the average
    (ddp.py:98-99) -- here of the peers' staged contributions; every other gradient is this
    rank's averaged with the peers'.  Bit for bit against the oracle with this rank's captured
    gradients and None for the unused ones."""
    W, rank = 4, 1
    model = _WithUnused().to(DEV)
    params = list(model.parameters())
    unused = {id(p) for p in model.unused.parameters()}
    captured: dict[int, torch.Tensor] = {}
    for p in params:
        p.register_post_accumulate_grad_hook(lambda q: captured.__setitem__(id(q), q.grad.detach().clone()))
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, overlap_with_backward=overlap)
    shapes = [tuple(p.shape) for p in params]
    peers = synthetic_grads(rng, shapes, W, torch.float32, 1.0)
    stage_peers(ddp, peers, [o.F32] * len(params), rank, W)
    x = torch.randn(6, 8, generator=torch.Generator().manual_seed(4)).to(DEV)
    ddp(x).backward()
    own = [None if id(p) in unused else host_bits(captured[id(p)]) for p in params]
    grads = [own if r == rank else peers[r] for r in range(W)]
    want = o.ddp_pipeline(grads, [o.F32] * len(params), [p.numel() for p in params], cap, rank, None)
    for i, p in enumerate(params):
        assert p.grad is not None
        got = host_bits(p.grad)
        assert same_bits(got, want["grads"][i]), f"param {i}: " + first_mismatch(got, want["grads"][i])


def test_bucket_caps_give_identical_grads(rng):
    """cfg2's property at small scale: 1 B, 25 MB and one giant bucket agree exactly."""
    shapes = [(300, 7), (11,), (1024,), (5, 5), (2048, 3), (9,)]
    W, rank = 4, 3
    grads = synthetic_grads(rng, shapes, W, torch.float32, 1.0)
    results = []
    for cap in (1e-6, 25.0, 1e6):
        model = Flat(shapes)
        ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap)
        stage_peers(ddp, grads, [o.F32] * len(shapes), rank, W)
        for p, g in zip(model.parameters(), grads[rank], strict=True):
            p.grad = dev_from(g, p.shape)
        ddp.finish_gradient_sync()
        results.append([host_bits(p.grad) for p in model.parameters()])
    for other in results[1:]:
        for a, b in zip(results[0], other, strict=True):
            assert np.array_equal(a, b)


def _capture_hook(store):
    def hook(p):
        store[id(p)] = p.grad.detach().clone()

    return hook


@pytest.mark.parametrize("comm_stream", [False, True])
@pytest.mark.parametrize("W", [2, 4])
@pytest.mark.parametrize("cap,overlap", [(25.0, True), (1e-6, True), (1e6, True), (25.0, False)])
def test_backward_matches_full_batch_and_oracle(W, cap, overlap, comm_stream):
    """Reference tests/test_ddp.py:32-77 on one GPU: rank r's DDP grads == full-batch grads.

    With ``comm_stream`` the bucket pipelines run on a dedicated stream while
    backward continues on the default one; the result must not change by a bit."""
    c = tiny_gpt.Config()
    ids, tgt = tiny_gpt.batch(c, 8)
    full = tiny_gpt.GPT(c).to(DEV)
    _, loss = full(ids.to(DEV), tgt.to(DEV))
    loss.backward()
    expected = [p.grad.detach().clone() for p in full.parameters()]

    # Each replica's local gradient on its chunk of the batch.
    replica = []
    for r in range(W):
        m = tiny_gpt.GPT(c).to(DEV)
        _, l_r = m(ids.chunk(W)[r].to(DEV), tgt.chunk(W)[r].to(DEV))
        l_r.backward()
        replica.append([host_bits(p.grad) for p in m.parameters()])

    rank = W - 1
    model = tiny_gpt.GPT(c).to(DEV)
    captured: dict[int, torch.Tensor] = {}
    for p in model.parameters():
        p.register_post_accumulate_grad_hook(_capture_hook(captured))  # runs before DDP's hook
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, overlap_with_backward=overlap,
              comm_stream=comm_stream)
    dts = [o.F32] * len(expected)
    stage_peers(ddp, replica, dts, rank, W)
    _, l = ddp(ids.chunk(W)[rank].to(DEV), tgt.chunk(W)[rank].to(DEV))
    l.backward()

    own = [host_bits(captured[id(p)]) for p in model.parameters()]
    grads_in = [own if r == rank else replica[r] for r in range(W)]
    want = o.ddp_pipeline(grads_in, dts, [p.numel() for p in model.parameters()], cap, rank, None)
    for i, (p, e) in enumerate(zip(model.parameters(), expected, strict=True)):
        assert same_bits(host_bits(p.grad), want["grads"][i]), f"param {i}"
        diff = (p.grad - e).abs().max().item()
        denom = max(e.abs().max().item(), 1.0)
        assert diff / denom <= 2e-5, f"param {i}: relative error {diff / denom:.3e}"


def test_comm_stream_carries_every_launch(monkeypatch):
    """With a caller's stream every pack and fused reduction is enqueued on it, never on
    the default stream, and the default stream sees the results after backward returns."""
    from minidist import _native

    seen = []
    # position of the stream argument in each entry point's Python binding
    for name, at in (("pack", 5), ("pack_planned", 3), ("allreduce_unpack", 7), ("allreduce_unpack_planned", 3),
                     ("pack_allreduce_unpack", 10), ("pack_allreduce_unpack_planned", 4)):
        orig = getattr(_native, name)

        def spy(*a, _orig=orig, _name=name, _at=at):
            seen.append((_name, a[_at]))
            return _orig(*a)

        monkeypatch.setattr(_native, name, spy)
    c = tiny_gpt.Config()
    W, rank = 4, 2
    ids, tgt = tiny_gpt.batch(c, 8)
    replica = []
    for r in range(W):
        m = tiny_gpt.GPT(c).to(DEV)
        _, l_r = m(ids.chunk(W)[r].to(DEV), tgt.chunk(W)[r].to(DEV))
        l_r.backward()
        replica.append([host_bits(p.grad) for p in m.parameters()])
    side = torch.cuda.Stream(DEV)

    scale = 2.0**10
    peers = [[(g * scale).astype(g.dtype) for g in row] for row in replica]
    dts = [o.F32] * len(replica[0])

    def run(stream):
        model = tiny_gpt.GPT(c).to(DEV)
        captured: dict[int, torch.Tensor] = {}
        for p in model.parameters():
            p.register_post_accumulate_grad_hook(_capture_hook(captured))  # runs before DDP's hook
        scaler = DistributedGradScaler(init_scale=scale)
        ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=0.01, grad_scaler=scaler,
                  comm_stream=stream)
        stage_peers(ddp, peers, dts, rank, W)
        _, l = ddp(ids.chunk(W)[rank].to(DEV), tgt.chunk(W)[rank].to(DEV))
        scaler.scale_loss(l).backward()

        class _Opt:
            param_groups = [{"params": list(model.parameters())}]

        found = scaler.unscale_(_Opt())
        own = [host_bits(captured[id(p)]) for p in model.parameters()]
        want = o.ddp_pipeline([own if r == rank else peers[r] for r in range(W)], dts,
                              [p.numel() for p in model.parameters()], 0.01, rank, 1.0 / scale)
        assert not found and not want["found_inf"]
        for i, p in enumerate(model.parameters()):
            assert same_bits(host_bits(p.grad), want["grads"][i]), f"param {i}"
        return len(ddp._buckets)

    nb = run(side)
    launches = list(seen)
    assert nb > 2 and len(launches) >= 2
    assert {s for _, s in launches} == {side.cuda_stream}
    assert side.cuda_stream != torch.cuda.current_stream(DEV).cuda_stream
    seen.clear()
    run(False)
    assert {s for _, s in seen} == {torch.cuda.current_stream(DEV).cuda_stream}


@pytest.mark.parametrize("n_params", [10, 60])
@pytest.mark.parametrize("comm_stream", [False, True])
def test_new_gradient_tensors_every_step(rng, n_params, comm_stream, monkeypatch):
    """``zero_grad(set_to_none=True)``: every step brings new gradient tensors.

    10 gradients fit one kernel-argument table (their pointer columns are
    patched, the tables are built once); 60 need a device plan (rebuilt and
    re-uploaded each step).  Every step is bit-exact against the oracle."""
    from minidist import ddp as ddp_mod

    builds = []
    orig_build = ddp_mod._RunPlan._build
    monkeypatch.setattr(ddp_mod._RunPlan, "_build", lambda self, *a: (builds.append(1), orig_build(self, *a))[1])
    W, rank = 4, 1
    shapes = [(int(rng.integers(1, 300)),) if i % 3 else (int(rng.integers(1, 40)), 33) for i in range(n_params)]
    model = Flat(shapes)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=1e6, comm_stream=comm_stream)
    numels = [int(np.prod(s)) for s in shapes]
    keep = []  # old gradients stay alive, so every step's gradients sit at new addresses
    for step in range(3):
        grads = synthetic_grads(rng, shapes, W, torch.float32, 1.0)
        stage_peers(ddp, grads, [o.F32] * n_params, rank, W)
        keep.append([p.grad for p in model.parameters()])
        for p, g in zip(model.parameters(), grads[rank], strict=True):
            p.grad = dev_from(g, p.shape)
        ddp.finish_gradient_sync()
        want = o.ddp_pipeline(grads, [o.F32] * n_params, numels, 1e6, rank, None)
        for i, p in enumerate(model.parameters()):
            assert same_bits(host_bits(p.grad), want["grads"][i]), f"step {step} param {i}"
    assert len(builds) == (1 if n_params <= 48 else 3)


@pytest.mark.parametrize("comm_stream", [False, True])
def test_set_to_none_backward_steps(comm_stream):
    """Three overlapped backwards with the gradients dropped in between: per-bucket
    launches during backward, new gradient tensors every step, oracle-exact each time."""
    c = tiny_gpt.Config()
    W, rank = 4, 3
    ids, tgt = tiny_gpt.batch(c, 8)
    replica = []
    for r in range(W):
        m = tiny_gpt.GPT(c).to(DEV)
        _, l_r = m(ids.chunk(W)[r].to(DEV), tgt.chunk(W)[r].to(DEV))
        l_r.backward()
        replica.append([host_bits(p.grad) for p in m.parameters()])
    model = tiny_gpt.GPT(c).to(DEV)
    captured: dict[int, torch.Tensor] = {}
    for p in model.parameters():
        p.register_post_accumulate_grad_hook(_capture_hook(captured))
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=0.01, comm_stream=comm_stream)
    dts = [o.F32] * len(replica[0])
    numels = [p.numel() for p in model.parameters()]
    for step in range(3):
        peers = [[(g * (step + 1)).astype(g.dtype) for g in row] for row in replica]
        stage_peers(ddp, peers, dts, rank, W)
        for p in model.parameters():
            p.grad = None
        _, l = ddp(ids.chunk(W)[rank].to(DEV), tgt.chunk(W)[rank].to(DEV))
        l.backward()
        own = [host_bits(captured[id(p)]) for p in model.parameters()]
        want = o.ddp_pipeline([own if r == rank else peers[r] for r in range(W)], dts, numels, 0.01, rank, None)
        for i, p in enumerate(model.parameters()):
            assert same_bits(host_bits(p.grad), want["grads"][i]), f"step {step} param {i}"


def test_graph_replays_match_eager(rng):
    """capture_graphs: every replay is bit-exact with the eager launches on the same inputs.

    Eager work and host syncs run between replays.  The scaler alternates two
    found-inf flags, so even and odd steps have graphs of their own; a graph is
    re-captured when the scale backs off (found-inf at step 2) and when the
    gradients move (set to None before step 4), and replayed otherwise."""
    W, rank, init = 4, 1, 2.0**10
    shapes = [(int(rng.integers(1, 300)),) if i % 3 else (int(rng.integers(1, 40)), 33) for i in range(60)]
    numels = [int(np.prod(s)) for s in shapes]
    runs = {}
    for graphs in (False, True):
        model = Flat(shapes)
        scaler = DistributedGradScaler(init_scale=init, growth_interval=1000)
        ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=0.02, grad_scaler=scaler,
                  capture_graphs=graphs)
        runs[graphs] = (model, scaler, ddp)
    step_rng = np.random.default_rng(77)
    captured = []
    for step in range(6):
        grads = synthetic_grads(step_rng, shapes, W, torch.float32, init)
        if step == 2:
            grads[(rank + 1) % W][5] = grads[(rank + 1) % W][5].copy()
            grads[(rank + 1) % W][5][0] = np.float32(np.inf)
        results = {}
        for graphs, (model, scaler, ddp) in runs.items():
            stage_peers(ddp, grads, [o.F32] * len(shapes), rank, W)
            keep = [p.grad for p in model.parameters()]  # alive, so new gradients get new addresses
            for p, g in zip(model.parameters(), grads[rank], strict=True):
                if step == 4:
                    p.grad = None
                if p.grad is None:
                    p.grad = dev_from(g, p.shape)
                else:
                    p.grad.copy_(dev_from(g, p.shape))  # same tensors: the graph replays
            ddp.finish_gradient_sync()
            if graphs:  # the graph of this step's flag
                flag = scaler._flags[DEV][scaler._parity]
                captured.append(id(ddp._graphs[(0, len(ddp._buckets), flag.data_ptr())][1]))

            class _Opt:
                param_groups = [{"params": list(model.parameters())}]

            found = scaler.unscale_(_Opt())
            scaler.update()
            results[graphs] = (found, [host_bits(p.grad) for p in model.parameters()])
            # unrelated eager work and a host sync between replays
            x = torch.randn(1 << 16, device=DEV)
            assert torch.isfinite(x.sum()).item()
        del keep
        # the step's scale: 2^10 until the backoff at the end of step 2, 2^9 after
        want = o.ddp_pipeline(grads, [o.F32] * len(shapes), numels, 0.02, rank, 1.0 / (init if step <= 2 else init / 2))
        assert results[True][0] == results[False][0] == want["found_inf"] == (step == 2)
        for i in range(len(shapes)):
            assert same_bits(results[True][1][i], results[False][1][i]), f"step {step} param {i}"
            assert same_bits(results[True][1][i], want["grads"][i]), f"step {step} param {i} vs oracle"
    # even steps: captured at 0, replayed at 2, re-captured at 4 (new gradients); odd steps: captured
    # at 1, re-captured at 3 (scale backed off at the end of step 2) and 5 (new gradients)
    assert captured[0] == captured[2] and len({captured[i] for i in (0, 1, 3, 4, 5)}) == 5
    assert runs[True][2]._graphs and not runs[False][2]._graphs


@pytest.mark.parametrize("cap", [25.0, 0.01])
def test_graph_launches_during_backward(cap):
    """capture_graphs with per-bucket launches from the backward hooks: three steps, oracle-exact."""
    c = tiny_gpt.Config()
    W, rank = 4, 0
    ids, tgt = tiny_gpt.batch(c, 8)
    replica = []
    for r in range(W):
        m = tiny_gpt.GPT(c).to(DEV)
        _, l_r = m(ids.chunk(W)[r].to(DEV), tgt.chunk(W)[r].to(DEV))
        l_r.backward()
        replica.append([host_bits(p.grad) for p in m.parameters()])
    model = tiny_gpt.GPT(c).to(DEV)
    captured: dict[int, torch.Tensor] = {}
    for p in model.parameters():
        p.register_post_accumulate_grad_hook(_capture_hook(captured))
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, capture_graphs=True)
    dts = [o.F32] * len(replica[0])
    numels = [p.numel() for p in model.parameters()]
    for step in range(3):
        stage_peers(ddp, replica, dts, rank, W)
        for p in model.parameters():
            if p.grad is not None:
                p.grad.zero_()  # accumulate into the same tensors: replays after the first step
        _, l = ddp(ids.chunk(W)[rank].to(DEV), tgt.chunk(W)[rank].to(DEV))
        l.backward()
        own = [host_bits(captured[id(p)]) for p in model.parameters()]
        want = o.ddp_pipeline([own if r == rank else replica[r] for r in range(W)], dts, numels, cap, rank, None)
        for i, p in enumerate(model.parameters()):
            assert same_bits(host_bits(p.grad), want["grads"][i]), f"step {step} param {i}"
    assert len(ddp._graphs) >= 1


def test_capture_graphs_argument_is_checked():
    with pytest.raises(ValueError):
        DDP(Flat([(4,)]), process_group=ResidentGroup(2, 0, DEV), capture_graphs=True, comm_stream=True)


def test_comm_stream_argument_is_checked():
    with pytest.raises(TypeError):
        DDP(Flat([(4,)]), process_group=ResidentGroup(2, 0, DEV), comm_stream="yes")


@pytest.mark.parametrize("explicit_finish", [False, True])
def test_no_sync_accumulation_then_sync(explicit_finish):
    """Reference tests/test_ddp.py:80-100: two half-batches under no_sync + synced == full step.
    ``explicit_finish``: both halves under no_sync, then ``finish_gradient_sync()`` flushes every
    bucket, as the reference trainer does around a pipeline schedule (examples/train_gpt.py:211-215)."""
    c = tiny_gpt.Config()
    W, rank = 2, 0
    ids, tgt = tiny_gpt.batch(c, 8)
    full = tiny_gpt.GPT(c).to(DEV)
    _, loss = full(ids.to(DEV), tgt.to(DEV))
    loss.backward()
    expected = [p.grad.detach().clone() for p in full.parameters()]
    replica = []
    for r in range(W):
        m = tiny_gpt.GPT(c).to(DEV)
        for half in zip(ids.chunk(W)[r].chunk(2), tgt.chunk(W)[r].chunk(2), strict=True):
            _, l_r = m(half[0].to(DEV), half[1].to(DEV))
            (l_r / 2).backward()
        replica.append([host_bits(p.grad) for p in m.parameters()])
    model = tiny_gpt.GPT(c).to(DEV)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV))
    stage_peers(ddp, replica, [o.F32] * len(expected), rank, W)
    halves = list(zip(ids.chunk(W)[rank].chunk(2), tgt.chunk(W)[rank].chunk(2), strict=True))
    with ddp.no_sync():
        _, l = ddp(halves[0][0].to(DEV), halves[0][1].to(DEV))
        (l / 2).backward()
        if explicit_finish:
            _, l = ddp(halves[1][0].to(DEV), halves[1][1].to(DEV))
            (l / 2).backward()
    if explicit_finish:
        ddp.finish_gradient_sync()
    else:
        _, l = ddp(halves[1][0].to(DEV), halves[1][1].to(DEV))
        (l / 2).backward()
    for p, e in zip(model.parameters(), expected, strict=True):
        rel = (p.grad - e).abs().max().item() / max(e.abs().max().item(), 1.0)
        assert rel <= 2e-5


def test_non_contiguous_gradient_is_rejected():
    """The pack kernels read each gradient as one flat span: a strided gradient is refused with an
    error before anything is launched."""
    model = Flat([(64, 32), (32,)])
    ddp = DDP(model, process_group=ResidentGroup(2, 0, DEV))
    w, b = list(model.parameters())
    w.grad = torch.zeros(32, 64, device=DEV).t()
    b.grad = torch.zeros(32, device=DEV)
    assert not w.grad.is_contiguous()
    with pytest.raises(RuntimeError, match="not a dense"):
        ddp.finish_gradient_sync()


def test_bucket_layout_matches_reference_invariants():
    c = tiny_gpt.Config()
    ddp = DDP(tiny_gpt.GPT(c).to(DEV), process_group=ResidentGroup(2, 0, DEV), bucket_cap_mb=0.05)
    summary = ddp.bucket_summary()
    assert len(summary) > 1
    assert [b[0] for b in summary] == list(range(len(summary)))
    for _, n, mb in summary:
        assert mb <= 0.05 or n == 1
    params = list(ddp.module.parameters())
    assert ddp._buckets[0].params[0] is params[-1]
    nbytes = [p.numel() * p.element_size() for p in params]
    layout = o.build_buckets(nbytes, 0.05)
    index = {id(p): i for i, p in enumerate(params)}
    assert [[index[id(p)] for p in b.params] for b in ddp._buckets] == layout


# ---------------------------------------------------------------------------
# Grad scaler (reference tests/test_amp.py) on the GPU
# ---------------------------------------------------------------------------


def _linear():
    torch.manual_seed(0)
    m = torch.nn.Linear(4, 4).to(DEV)
    return m, torch.optim.SGD(m.parameters(), lr=0.1)


def test_overflow_skips_and_backs_off():
    m, opt = _linear()
    scaler = DistributedGradScaler(init_scale=1024.0)
    for p in m.parameters():
        p.grad = torch.ones_like(p)
    next(iter(m.parameters())).grad[0, 0] = float("inf")
    before = [p.detach().clone() for p in m.parameters()]
    assert not scaler.step(opt)
    scaler.update()
    for p, b in zip(m.parameters(), before, strict=True):
        assert torch.equal(p.detach(), b)
    assert scaler.scale == 512.0 and scaler.num_skipped == 1


def test_clean_steps_grow_the_scale():
    m, opt = _linear()
    scaler = DistributedGradScaler(init_scale=1024.0, growth_interval=2)
    for _ in range(2):
        for p in m.parameters():
            p.grad = torch.full_like(p, 2.0) * scaler.scale
        assert scaler.step(opt)
        scaler.update()
    assert scaler.scale == 2048.0 and scaler.num_skipped == 0


def test_unscale_is_idempotent():
    m, opt = _linear()
    scaler = DistributedGradScaler(init_scale=256.0)
    for p in m.parameters():
        p.grad = torch.full_like(p, 3.0) * scaler.scale
    assert not scaler.unscale_(opt)
    scaler.unscale_(opt)
    for p in m.parameters():
        assert torch.equal(p.grad, torch.full_like(p.grad, 3.0))


@pytest.mark.parametrize("inject", [None, "f32", "bf16", "f16"])
def test_scaler_unscale_over_mixed_dtypes_matches_oracle(rng, inject):
    """``scaler.unscale_`` on its own (no DDP), over an optimizer whose gradients come in fp32,
    bf16 and fp16 across two param groups (one launch per dtype): every gradient and the
    found-inf decision bit for bit against the oracle (amp.py:201-219), with an inf in one
    dtype's gradient or none."""
    S = 2.0**12
    dts = [torch.float32, torch.bfloat16, torch.float16, torch.float32, torch.bfloat16]
    sizes = [300, 77, 4100, 1, 65]
    params = [nn.Parameter(torch.zeros(n, dtype=dt, device=DEV)) for n, dt in zip(sizes, dts, strict=True)]
    hosts = [o.from_f32((rng.standard_normal(n) * 1e-2 * S).astype(np.float32), odt(dt))
             for n, dt in zip(sizes, dts, strict=True)]
    if inject is not None:
        k = {"f32": 0, "bf16": 1, "f16": 2}[inject]
        hosts[k] = hosts[k].copy()
        hosts[k][5] = np.uint16(0x7F80) if inject == "bf16" else np.inf
    for p, h in zip(params, hosts, strict=True):
        p.grad = dev_from(h, p.shape)

    class _Opt:
        param_groups = [{"params": params[:2]}, {"params": params[2:]}]

    scaler = DistributedGradScaler(init_scale=S)
    found = scaler.unscale_(_Opt())
    want, want_found = o.unscale_found_inf(hosts, [odt(dt) for dt in dts], 1.0 / S)
    assert found == want_found == (inject is not None)
    for p, w in zip(params, want, strict=True):
        assert same_bits(host_bits(p.grad), w), first_mismatch(host_bits(p.grad), w)


def test_mixed_overflow_history_final_scale():
    m, opt = _linear()
    scaler = DistributedGradScaler(init_scale=4096.0, growth_interval=2)
    for bad in [True, False, False, True, True]:
        for p in m.parameters():
            p.grad = torch.ones_like(p)
        if bad:
            next(iter(m.parameters())).grad[0, 0] = float("nan")
        scaler.step(opt)
        scaler.update()
    assert scaler.scale == 1024.0


@pytest.mark.parametrize("inject", [False, True])
def test_fused_unscale_in_ddp_unpack(rng, inject):
    """DDP(grad_scaler=...) unscales in its unpack; the scaler then skips those grads."""
    shapes = [(100, 3), (17,), (4096,), (2,)]
    W, rank, S = 4, 1, 2.0**16
    model = Flat(shapes)
    extra = nn.Parameter(torch.full((5,), 3.0 * S, device=DEV))  # optimizer param outside DDP
    scaler = DistributedGradScaler(init_scale=S)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=0.01, grad_scaler=scaler)
    grads = synthetic_grads(rng, shapes, W, torch.float32, S)
    if inject:
        grads[(rank + 1) % W][2][123] = np.float32(np.inf)
    stage_peers(ddp, grads, [o.F32] * 4, rank, W)
    for p, g in zip(model.parameters(), grads[rank], strict=True):
        p.grad = dev_from(g, p.shape)
    extra.grad = torch.full((5,), 3.0 * S, device=DEV)
    opt = torch.optim.SGD(list(model.parameters()) + [extra], lr=0.0)
    ddp.finish_gradient_sync()
    found = scaler.unscale_(opt)
    want = o.ddp_pipeline(grads, [o.F32] * 4, [int(np.prod(s)) for s in shapes], 0.01, rank, 1.0 / S)
    for i, p in enumerate(model.parameters()):
        assert same_bits(host_bits(p.grad), want["grads"][i])
    assert torch.equal(extra.grad, torch.full((5,), 3.0, device=DEV))
    assert found == want["found_inf"] == inject
    with pytest.raises(RuntimeError):
        ddp.finish_gradient_sync()  # second sync before update(): refused
    scaler.update()



# ---------------------------------------------------------------------------
# reduce_dtype: bf16 / fp16 gradients accumulated in fp32 buckets (the Llama-7B configuration, cfg4, at
# small scale)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("W,rank", [(2, 1), (8, 5), (3, 0)])
@pytest.mark.parametrize("cap", [1e-6, 0.01, 25.0])
@pytest.mark.parametrize("inject", [False, True])
def test_reduce_dtype_widening_bitwise(rng, dtype, W, rank, cap, inject):
    """Widening buckets == the reference chain with an fp32 bucket (copy_, mul_(1/W), SUM, copy_, unscale)."""
    shapes = [(33,), (64, 8), (5,), (130,), (1,), (7, 9), (256, 4), (3,)]
    S = 2.0**12 if dtype == torch.bfloat16 else 2.0**10
    model = Flat(shapes, dtype)
    scaler = DistributedGradScaler(init_scale=S)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, grad_scaler=scaler,
              reduce_dtype=torch.float32)
    assert all(b.widening and b.buffer is None for b in ddp._buckets)
    grads = synthetic_grads(rng, shapes, W, dtype, S)
    grads[rank][2] = None
    if inject:  # +inf in a peer's 16-bit gradient
        grads[(rank + 1) % W][5][7] = np.uint16(0x7F80) if dtype == torch.bfloat16 else np.float16(np.inf)
    dts = [odt(dtype)] * len(shapes)
    stage_peers(ddp, grads, dts, rank, W)
    for p, g in zip(model.parameters(), grads[rank], strict=True):
        p.grad = None if g is None else dev_from(g, p.shape)
    opt = torch.optim.SGD(model.parameters(), lr=0.0)
    ddp.finish_gradient_sync()
    found = scaler.unscale_(opt)
    want = o.ddp_pipeline(grads, dts, [int(np.prod(s)) for s in shapes], cap, rank, 1.0 / S, bucket_dtype=o.F32)
    for i, p in enumerate(model.parameters()):
        assert p.grad.dtype == dtype
        got = host_bits(p.grad)
        assert same_bits(got, want["grads"][i]), f"param {i}: " + first_mismatch(got, want["grads"][i])
    for b, bucket in enumerate(ddp._buckets):
        assert bucket.buffer.dtype == torch.float32 and bucket.wire.dtype == dtype
        assert same_bits(host_bits(bucket.buffer), want["reduced"][b])
    assert found == want["found_inf"] == inject
    scaler.update()


def test_reduce_dtype_on_matching_params_is_the_plain_path(rng):
    """fp32 parameters with reduce_dtype=fp32: ordinary (non-widening) buckets, same results."""
    shapes = [(300, 7), (11,), (1024,)]
    W, rank = 4, 2
    grads = synthetic_grads(rng, shapes, W, torch.float32, 1.0)
    model = Flat(shapes)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=0.01, reduce_dtype=torch.float32)
    assert not any(b.widening for b in ddp._buckets)
    stage_peers(ddp, grads, [o.F32] * 3, rank, W)
    for p, g in zip(model.parameters(), grads[rank], strict=True):
        p.grad = dev_from(g, p.shape)
    ddp.finish_gradient_sync()
    want = o.ddp_pipeline(grads, [o.F32] * 3, [int(np.prod(s)) for s in shapes], 0.01, rank, None)
    for i, p in enumerate(model.parameters()):
        assert same_bits(host_bits(p.grad), want["grads"][i])


class MixedFlat(nn.Module):
    """Parameters whose dtypes cycle through fp32, bf16 and fp16 (a partially cast model)."""

    DTYPES = (torch.float32, torch.bfloat16, torch.float16)

    def __init__(self, shapes, offset=0):
        super().__init__()
        self.ps = nn.ParameterList([
            nn.Parameter(torch.zeros(s, dtype=self.DTYPES[(i + offset) % 3], device=DEV)) for i, s in enumerate(shapes)
        ])


@pytest.mark.parametrize("W,rank", [(2, 0), (4, 3), (8, 5)])
@pytest.mark.parametrize("cap", [1e-6, 0.004, 1e6])
@pytest.mark.parametrize("offset", [0, 1, 2])
def test_mixed_dtype_buckets_bitwise(rng, W, rank, cap, offset):
    """A bucket takes its first parameter's dtype (ddp.py:83-84); every other gradient is cast into it on
    pack (`copy_`, ddp.py:90) and back on unpack (ddp.py:100-101), then unscaled in its own dtype."""
    shapes = [(33,), (64, 8), (5,), (130,), (1,), (7, 9), (256, 4), (3,), (500,), (2, 2)]
    S = 2.0**8
    model = MixedFlat(shapes, offset)
    dtypes = [p.dtype for p in model.parameters()]
    scaler = DistributedGradScaler(init_scale=S)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, grad_scaler=scaler)
    grads = []
    for r in range(W):
        grads.append([o.from_f32((rng.standard_normal(int(np.prod(s))) * 1e-2 * S).astype(np.float32), odt(d))
                      for s, d in zip(shapes, dtypes, strict=True)])
    dts = [odt(d) for d in dtypes]
    stage_peers(ddp, grads, dts, rank, W)
    for p, g in zip(model.parameters(), grads[rank], strict=True):
        p.grad = dev_from(g, p.shape)
    ddp.finish_gradient_sync()

    class _Opt:
        param_groups = [{"params": list(model.parameters())}]

    found = scaler.unscale_(_Opt())
    want = o.ddp_pipeline(grads, dts, [int(np.prod(s)) for s in shapes], cap, rank, 1.0 / S)
    if cap == 1e6:
        assert len({b.dtype for b in ddp._buckets}) == 1 and len(ddp._buckets) == 1
    for i, p in enumerate(model.parameters()):
        assert p.grad.dtype == dtypes[i]
        got = host_bits(p.grad)
        assert same_bits(got, want["grads"][i]), f"param {i} ({dtypes[i]}): " + first_mismatch(got, want["grads"][i])
    for b, bucket in enumerate(ddp._buckets):
        assert bucket.buffer.dtype == bucket.params[0].dtype
        assert same_bits(host_bits(bucket.buffer), want["reduced"][b]), f"bucket {b}"
    assert found == want["found_inf"]


def test_current_stream_lookup_follows_torch():
    """The launch path finds the current stream by its raw handle (minidist._native.current_stream):
    it is the stream torch.cuda.current_stream names, inside and outside stream contexts, for
    streams made and dropped in turn, and for a device given without an index."""
    from minidist import _native

    assert _native.current_stream(DEV) == torch.cuda.current_stream(DEV)
    for _ in range(4):
        s = torch.cuda.Stream(device=DEV)
        with torch.cuda.stream(s):
            got = _native.current_stream(DEV)
            assert got == s and got.cuda_stream == s.cuda_stream
            assert _native.current_stream(torch.device("cuda")) == s
        del s
        assert _native.current_stream(DEV) == torch.cuda.current_stream(DEV)
