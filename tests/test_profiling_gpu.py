"""minidist.profiling on traces the torch profiler actually records on the GPU.

The reference reads what ``torch.profiler`` recorded (minidist/profiling.py:
``summarize_collectives`` :161-180, ``analyze_trace`` :305-362).  Here real
DDP and FSDP steps run under :func:`minidist.profiling.profile_steps` on
``cuda:0`` and the kernel names the profiler recorded are classified.  The
expected counts come from a different source: every call the Python layer
makes into libmdx.so is counted by a proxy in front of the loaded library,
and each launching entry point issues one dispatch of a known kind at these
sizes (a fused all-reduce, a reduce-scatter share, a copy; a zero-span pack
that only clears the scaler's flag is a flag clear).  So a kernel renamed,
or named differently by this tracer than by rocprofv3, fails here.
"""

from __future__ import annotations

import collections

import pytest
import torch

import tiny_gpt
from minidist import DDP, FSDP, DistributedGradScaler, MixedPrecisionPolicy, ResidentGroup
from minidist import _native as nat
from minidist import profiling as P

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

# Launching entry point -> the kind of the one dispatch it issues here.
_KIND_OF_CALL = {
    "mdx_pack_allreduce_unpack": "all_reduce",
    "mdx_pack_allreduce_unpack_planned": "all_reduce",
    "mdx_pack_allreduce_unpack_planned_noalloc": "all_reduce",
    "mdx_allreduce_unpack": "all_reduce",
    "mdx_allreduce_unpack_wide": "all_reduce",
    "mdx_allreduce_unpack_planned": "all_reduce",
    "mdx_allreduce_sum": "all_reduce",
    "mdx_reduce_scatter_share": "reduce_scatter",
    "mdx_reduce_scatter_share_multi": "reduce_scatter",
    "mdx_reduce_scatter_share_multi_planned": "reduce_scatter",
    "mdx_pack": "bucket_copy",
    "mdx_pack_planned": "bucket_copy",
    "mdx_unpack": "bucket_copy",
    "mdx_unpack_planned": "bucket_copy",
    "mdx_unscale_found_inf": "bucket_copy",
    "mdx_cast_f32_bf16": "bucket_copy",
}


class _CountingLib:
    """Forwards to the loaded library and counts the launching calls while ``on``."""

    def __init__(self, real):
        self._real = real
        self.on = False
        self.kinds: collections.Counter[str] = collections.Counter()

    def __getattr__(self, name):
        fn = getattr(self._real, name)
        kind = _KIND_OF_CALL.get(name)
        if kind is None:
            return fn

        def call(*args):
            if self.on:
                if name == "mdx_pack" and args[1] == 0:  # no spans: only the flag clear, if any
                    if args[6] is not None:
                        self.kinds["flag_clear"] += 1
                else:
                    self.kinds[kind] += 1
            return fn(*args)

        return call


@pytest.fixture
def counting(monkeypatch):
    proxy = _CountingLib(nat.lib())
    monkeypatch.setattr(nat, "_lib", proxy)
    return proxy


def _profile(step, proxy, tmp_path, name, num_steps=6, wait=1, warmup=2):
    """Run the steps under the profiler; count the library calls of the recorded (active) steps."""

    def fn(i):
        proxy.on = i >= wait + warmup
        step()
        proxy.on = False
        torch.cuda.synchronize()  # every kernel of the step has finished before the profiler moves on

    trace = tmp_path / f"{name}.json"
    prof = P.profile_steps(fn, num_steps=num_steps, warmup=warmup, wait=wait, trace_path=trace)
    torch.cuda.synchronize()
    names = sorted({e.key for e in prof.key_averages() if P.is_collective(e.key)})
    print(f"{name}: recorded path kernels: {names}", flush=True)
    return prof, trace


def _check(prof, trace, proxy):
    rows = {r.kind: r for r in P.summarize_collectives(prof)}
    got = {k: r.count for k, r in rows.items()}
    assert got == dict(proxy.kinds), f"profiler {got} vs library calls {dict(proxy.kinds)}"
    assert all(r.device_time_us > 0 for r in rows.values())
    table = P.format_collective_table(rows.values())
    for kind in got:
        assert kind in table
    report = P.analyze_trace(trace)
    assert report.device == "cuda"
    assert report.num_comm_events == sum(proxy.kinds.values())
    assert set(report.per_kind_s) == set(got) and all(v > 0 for v in report.per_kind_s.values())
    assert report.num_compute_events > 0 and report.compute_s > 0  # the model's own kernels
    assert 0.0 <= report.overlap_fraction <= 1.0 and report.exposed_comm_s <= report.comm_s
    return got


def test_ddp_steps_recorded_by_the_profiler(counting, tmp_path):
    """DDP over a 4-way ResidentGroup with small buckets, the scaler fused in, overlapped with
    backward: the fused pack + all-reduce + unpack dispatches are the recorded all_reduce kernels."""
    c = tiny_gpt.Config(n_layer=2)
    model = tiny_gpt.GPT(c).to(DEV)
    scaler = DistributedGradScaler(init_scale=2.0**10)
    ddp = DDP(model, process_group=ResidentGroup(4, 1, DEV), bucket_cap_mb=0.02, grad_scaler=scaler)
    assert len(ddp._buckets) > 2
    opt = torch.optim.SGD(ddp.parameters(), lr=1e-3)
    ids, tgt = (t.to(DEV) for t in tiny_gpt.batch(c, 4, seed=3))

    def step():
        opt.zero_grad(set_to_none=True)
        _, loss = ddp(ids, tgt)
        scaler.scale_loss(loss).backward()
        scaler.step(opt)
        scaler.update()

    prof, trace = _profile(step, counting, tmp_path, "ddp")
    got = _check(prof, trace, counting)
    assert got.get("all_reduce", 0) >= 3  # three active steps, at least one launch each


@pytest.mark.parametrize("param_dtype,unit_batch", [(torch.bfloat16, 1), (torch.float32, 2)])
def test_fsdp_steps_recorded_by_the_profiler(counting, tmp_path, param_dtype, unit_batch):
    """FSDP over a 4-way ResidentGroup: the gather casts and peer-slot copies are the recorded
    bucket_copy kernels, the shares the reduce_scatter kernels (one per unit per step, or one per
    batch of units)."""
    c = tiny_gpt.Config(n_layer=3)
    model = tiny_gpt.GPT(c).to(DEV)
    fsdp = FSDP(model, unit_types=(tiny_gpt.Block,), process_group=ResidentGroup(4, 2, DEV),
                mixed_precision=MixedPrecisionPolicy(param_dtype=param_dtype, reduce_dtype=torch.float32),
                unit_batch=unit_batch)
    opt = torch.optim.SGD(fsdp.parameters(), lr=1e-3)
    ids, tgt = (t.to(DEV) for t in tiny_gpt.batch(c, 4, seed=4))

    def step():
        opt.zero_grad(set_to_none=True)
        _, loss = fsdp(ids, tgt)
        loss.backward()
        opt.step()

    prof, trace = _profile(step, counting, tmp_path, f"fsdp_{unit_batch}")
    got = _check(prof, trace, counting)
    units = len(fsdp._units)
    if unit_batch == 1:
        assert got["reduce_scatter"] == 3 * units
    assert got["bucket_copy"] > 0 and got["reduce_scatter"] > 0
