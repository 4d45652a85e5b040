"""What DDP and FSDP record in ``comm.comm_stats`` during real steps on the GPU.

The reference instruments every collective (minidist/comm.py:50-113, formulas
at :232-233, :247-248, :263-264) and publishes the measured bytes as the
numbers worth trusting (README.md "Communication accounting": 4 ranks, a
6.9M-parameter GPT).  Here the same accounting comes from the one-GPU path:
the fused DDP launch over a ResidentGroup records one all-reduce per bucket,
and FSDP one all-gather per unshard and one reduce-scatter per unit.  Each
test runs real steps (forward, backward, optimizer step) inside
``record_comm()`` and checks the counters three ways:

* entry by entry against the reference formulas applied to layouts derived
  independently here -- the oracle's bucket partition (ddp.py:175-190) and
  the unit partition (fsdp.py:315-357: one unit per Block, the rest in the
  root unit);
* the per-collective and total bus MB against the README's published table,
  whose model is recovered from it: 6 layers, h=256, vocab 4096, context 128
  (6,868,992 parameters: 2·(3/4)·P·4 bytes = 39.30 MB, the DDP row);
* FSDP's 52.9 MB below the naive 59.0 MB: the root unit is not resharded
  after forward (fsdp.py:343-354), so it skips its backward all-gather; with
  ``reshard_root_after_forward=True`` the step records the full 59.0 MB.
"""

from __future__ import annotations

import pytest
import torch

import tiny_gpt
from minidist import DDP, FSDP, MixedPrecisionPolicy, ResidentGroup, comm
from oracle import gradpath as o

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
MB = 1024**2

# The model of the README's accounting table (recovered from its numbers; see the module docstring).
README_MODEL = tiny_gpt.Config(vocab_size=4096, block_size=128, n_layer=6, n_head=4, n_embd=256)
README_W = 4
README_TABLE = {  # strategy -> per-collective bus MB/step/rank, total comm MB
    "ddp": ({"all_reduce": "39.3"}, "39.3"),
    "fsdp": ({"all_gather": "33.2", "reduce_scatter": "19.7"}, "52.9"),
    "fsdp-bf16": ({"all_gather": "16.6", "reduce_scatter": "19.7"}, "36.3"),
}


def _step(model, opt, ids, tgt):
    """One step as the reference's bench_parallelism.py:118-122 runs it."""
    opt.zero_grad(set_to_none=True)
    _, loss = model(ids, tgt)
    loss.backward()
    opt.step()


def _table(stats: comm.CommStats) -> tuple[dict[str, str], str]:
    """The README's formatting of one row (bench_parallelism.py:130-134, :216)."""
    per = {name: f"{bus / MB:.1f}" for name, _, _, bus in stats.as_rows()}
    return per, f"{stats.total_bus_bytes() / MB:.1f}"


def _ddp_expected(params: list[torch.nn.Parameter], W: int, cap_mb: float, wire_bytes: int | None = None):
    """(count, payload, bus) of the all-reduces of one synchronised DDP step: one per bucket of
    the oracle's partition, payload = the bucket's bytes, bus = int(2(W-1)/W * payload)."""
    sizes = [p.numel() * p.element_size() for p in params]
    payload = bus = 0
    layout = o.build_buckets(sizes, cap_mb)
    for idx in layout:
        nb = sum(params[i].numel() * (wire_bytes or params[i].element_size()) for i in idx)
        payload += nb
        bus += int(2 * (W - 1) / W * nb)
    return len(layout), payload, bus


def _rows(stats: comm.CommStats) -> dict[str, tuple[int, int, int]]:
    return {name: (count, payload, bus) for name, count, payload, bus in stats.as_rows()}


@pytest.mark.parametrize("overlap", [True, False])
def test_ddp_step_records_the_readme_accounting(overlap):
    """A real DDP step on rank 1 of 4: one all-reduce per bucket with the reference's payload and
    bus bytes, 39.3 MB as the README's ddp (overlap) and ddp-no-overlap rows print."""
    c, W = README_MODEL, README_W
    model = tiny_gpt.GPT(c).to(DEV)
    ddp = DDP(model, process_group=ResidentGroup(W, 1, DEV), bucket_cap_mb=25.0, overlap_with_backward=overlap)
    opt = torch.optim.AdamW(ddp.parameters(), lr=1e-4)
    ids, tgt = tiny_gpt.batch(c, 2, seed=5)
    ids, tgt = ids.to(DEV), tgt.to(DEV)
    _step(ddp, opt, ids, tgt)  # warmup, outside the record (bench_parallelism.py:124-125)
    with comm.record_comm() as stats:
        _step(ddp, opt, ids, tgt)
    params = list(model.parameters())
    assert sum(p.numel() for p in params) == 6_868_992
    want = _ddp_expected(params, W, 25.0)
    assert _rows(stats) == {"all_reduce": want}
    assert want[1] == 6_868_992 * 4
    assert _table(stats) == README_TABLE["ddp"]


def test_ddp_gpt2_small_w8_records_every_bucket():
    """cfg1 (GPT-2-124M, W=8, 25 MB): the flush of all 18 buckets records 18 all-reduces, payload
    the model's 497,759,232 bytes, bus the sum over buckets of int(2·7/8·payload)."""
    from minidist import workloads as wl

    specs = wl.gpt_specs(**wl.GPT2_SMALL)
    model = wl.SpecModule(specs, DEV)
    ddp = DDP(model, process_group=ResidentGroup(8, 3, DEV), bucket_cap_mb=25.0)
    for b in range(len(ddp._buckets)):
        for row in ddp.bucket_replicas(b):
            row.zero_()
    for p in model.parameters():
        p.grad = torch.zeros_like(p)
    with comm.record_comm() as stats:
        ddp.finish_gradient_sync()
    torch.cuda.synchronize()
    count, payload, bus = _ddp_expected(list(model.parameters()), 8, 25.0)
    assert (count, payload) == (18, 497_759_232)
    assert _rows(stats) == {"all_reduce": (count, payload, bus)}
    per_bucket = [int(2 * 7 / 8 * b.numel * 4) for b in ddp._buckets]
    assert sum(per_bucket) == bus


def test_ddp_widening_buckets_record_the_wire_bytes():
    """bf16 parameters with fp32 buckets (``reduce_dtype``): each all-reduce records the bytes a
    peer sends -- its bf16 gradients, 2 per element, which is also what the reference's bf16
    bucket (ddp.py:84, bucket dtype = first parameter's) records -- not the fp32 bucket's 4."""
    c, W = tiny_gpt.Config(n_layer=3), 4
    model = tiny_gpt.GPT(c).to(DEV).to(torch.bfloat16)
    ddp = DDP(model, process_group=ResidentGroup(W, 0, DEV), bucket_cap_mb=0.01, reduce_dtype=torch.float32)
    assert all(b.widening for b in ddp._buckets) and len(ddp._buckets) > 1
    ids, tgt = tiny_gpt.batch(c, 2, seed=6)
    with comm.record_comm() as stats:
        _, loss = ddp(ids.to(DEV), tgt.to(DEV))
        loss.backward()
    assert _rows(stats) == {"all_reduce": _ddp_expected(list(model.parameters()), W, 0.01, wire_bytes=2)}


def test_ddp_records_nothing_without_communication():
    """Under ``no_sync`` nothing is launched and nothing recorded (ddp.py:202-203); the synchronised
    step that follows records the usual all-reduces.  A world of one never communicates
    (comm.py:229-231, ddp.py:155-156)."""
    c, W = tiny_gpt.Config(), 2
    ids, tgt = tiny_gpt.batch(c, 2, seed=7)
    ids, tgt = ids.to(DEV), tgt.to(DEV)
    model = tiny_gpt.GPT(c).to(DEV)
    ddp = DDP(model, process_group=ResidentGroup(W, 0, DEV))
    with comm.record_comm() as stats:
        with ddp.no_sync():
            ddp(ids, tgt)[1].backward()
        assert stats.as_rows() == []
        ddp(ids, tgt)[1].backward()
    assert _rows(stats) == {"all_reduce": _ddp_expected(list(model.parameters()), W, 25.0)}
    single = DDP(tiny_gpt.GPT(c).to(DEV), process_group=ResidentGroup(1, 0, DEV))
    with comm.record_comm() as stats:
        single(ids, tgt)[1].backward()
    assert stats.as_rows() == []


def _fsdp_expected(model: tiny_gpt.GPT, W: int, gather_bytes: int, reshard_root: bool, reduce_bytes: int = 4):
    """Rows of one synchronised FSDP step: every Block unit is gathered for its forward and again
    for its backward, the root unit (the remaining parameters) once -- twice when it is resharded
    after forward too; one reduce-scatter of the padded fp32 buffer per unit."""
    blocks = [sum(p.numel() for p in b.parameters()) for b in model.blocks]
    root = sum(p.numel() for p in model.parameters()) - sum(blocks)
    padded = [(n + W - 1) // W * W for n in blocks + [root]]
    gathers = [n for n in padded[:-1] for _ in range(2)] + [padded[-1]] * (2 if reshard_root else 1)
    ag = (len(gathers), sum(n * gather_bytes for n in gathers),
          sum(int((W - 1) / W * n * gather_bytes) for n in gathers))
    rs = (len(padded), sum(n * reduce_bytes for n in padded), sum(int((W - 1) / W * n * reduce_bytes) for n in padded))
    return {"all_gather": ag, "reduce_scatter": rs}


@pytest.mark.parametrize("strategy", ["fsdp", "fsdp-bf16"])
@pytest.mark.parametrize("unit_batch", [1, 3])
def test_fsdp_step_records_the_readme_accounting(strategy, unit_batch):
    """A real FSDP step (units = Blocks, fp32 reduction) on rank 2 of 4: 13 all-gathers (the root
    unit's one, each Block's two) and 7 reduce-scatters, the README's fsdp / fsdp-bf16 rows
    (33.2 + 19.7 = 52.9 MB; 16.6 + 19.7 = 36.3 MB).  Batched issue (``unit_batch``) records the
    same per-unit collectives."""
    c, W = README_MODEL, README_W
    param_dtype = torch.bfloat16 if strategy == "fsdp-bf16" else torch.float32
    model = tiny_gpt.GPT(c).to(DEV)
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, 2, DEV),
                mixed_precision=MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32),
                unit_batch=unit_batch)
    opt = torch.optim.AdamW(fsdp.parameters(), lr=1e-4)
    ids, tgt = tiny_gpt.batch(c, 2, seed=8)
    ids, tgt = ids.to(DEV), tgt.to(DEV)
    _step(fsdp, opt, ids, tgt)
    with comm.record_comm() as stats:
        _step(fsdp, opt, ids, tgt)
    want = _fsdp_expected(model, W, 2 if param_dtype == torch.bfloat16 else 4, reshard_root=False)
    assert want["all_gather"][0] == 13 and want["reduce_scatter"][0] == 7
    assert _rows(stats) == want
    assert _table(stats) == README_TABLE[strategy]


def test_fsdp_root_unit_skips_one_all_gather():
    """The README's 52.9 MB against the naive 59.0 MB (1.5 x DDP's 39.3): resharding the root unit
    after forward as well gives it a backward all-gather, and the step then records the naive
    figure exactly."""
    c, W = README_MODEL, README_W
    totals = {}
    for reshard_root in (False, True):
        model = tiny_gpt.GPT(c).to(DEV)
        fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, 0, DEV),
                    reshard_root_after_forward=reshard_root)
        ids, tgt = tiny_gpt.batch(c, 2, seed=9)
        with comm.record_comm() as stats:
            fsdp(ids.to(DEV), tgt.to(DEV))[1].backward()
        assert _rows(stats) == _fsdp_expected(model, W, 4, reshard_root)
        totals[reshard_root] = f"{stats.total_bus_bytes() / MB:.1f}"
    assert totals == {False: "52.9", True: "59.0"}


def test_fsdp_no_sync_defers_the_reduce_scatters():
    """Under ``no_sync`` the units still gather (forward and backward) but reduce nothing; the flush
    (``finish_gradient_sync``, fsdp.py:462-470) then records one reduce-scatter per unit."""
    c, W = tiny_gpt.Config(n_layer=2), 2
    model = tiny_gpt.GPT(c).to(DEV)
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(W, 1, DEV))
    ids, tgt = tiny_gpt.batch(c, 2, seed=10)
    want = _fsdp_expected(model, W, 4, reshard_root=False)
    with comm.record_comm() as stats:
        with fsdp.no_sync():
            fsdp(ids.to(DEV), tgt.to(DEV))[1].backward()
        assert _rows(stats) == {"all_gather": want["all_gather"]}
        fsdp.finish_gradient_sync()
    assert _rows(stats) == want
