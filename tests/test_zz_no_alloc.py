"""The allocation-free fused launch, mdx_pack_allreduce_unpack_planned_noalloc, on the GPU.

It must do exactly what mdx_pack_allreduce_unpack_planned does with a
caller-allocated device copy of the same plan.  Each case builds the same
seeded inputs twice, launches the existing entry point on one copy and the
allocation-free one on the other, and compares every output bit for bit:
this rank's packed row, the bucket, the gradients (and the sentinels around
them), the found-inf flag and the next step's flag.  Both are also checked
against the oracle.  Two calls in a row share the library's per-GPU buffer,
the second with a smaller plan, so a stale tail of the first plan must not
leak into the second.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from minidist import _native as nat
from oracle import gradpath as o
from test_kernels_gpu import DEV, code, stream, to_host
from test_pack_fused_gpu import _case, _check

pytestmark = pytest.mark.gpu


def _plan(c, W, rank, wdt, bdt):
    reps = [r.data_ptr() for r in c["reps"]]
    return nat.plan_pack_allreduce_unpack(reps, rank, code(wdt), c["runs"], c["out"].data_ptr(), code(bdt),
                                          nat.f32(1.0 / W), DEV)


def _outputs(c, flag, nxt):
    return ([to_host(r) for r in c["reps"]], to_host(c["out"]), [to_host(d) for d in c["dsts"]],
            int(flag.item()), int(nxt.item()))


def _same(a, b) -> bool:
    return a.dtype == b.dtype and a.shape == b.shape and a.tobytes() == b.tobytes()


@pytest.mark.parametrize("first,second", [
    ((o.F32, o.F32, 8, 3, 150, 3000), (o.BF16, o.F32, 4, 1, 20, 700)),
    ((o.BF16, o.BF16, 16, 15, 200, 2000), (o.F16, o.F16, 2, 0, 3, 5000)),
])
def test_noalloc_matches_planned_twice(first, second):
    inv = nat.f32(2.0**-10)
    for k, (wdt, bdt, W, rank, n_grads, max_numel) in enumerate((first, second)):
        print(f"noalloc call {k + 1}: wire {wdt} bucket {bdt} W={W} rank={rank} grads={n_grads}", flush=True)
        numels = [int(x) for x in np.random.default_rng(10 + k).integers(1, max_numel, n_grads)]
        ref = _case(np.random.default_rng(100 + k), wdt, bdt, W, rank, numels, null_every=7, in_place_every=5)
        new = _case(np.random.default_rng(100 + k), wdt, bdt, W, rank, numels, null_every=7, in_place_every=5)
        plan_ref = _plan(ref, W, rank, wdt, bdt)
        plan_new = _plan(new, W, rank, wdt, bdt)
        assert plan_new.host.nbytes <= nat.NOALLOC_SCRATCH_BYTES
        flags = [torch.tensor([0], dtype=torch.int32, device=DEV) for _ in range(2)]
        nexts = [torch.tensor([1], dtype=torch.int32, device=DEV) for _ in range(2)]
        nat.pack_allreduce_unpack_planned(plan_ref, inv, flags[0].data_ptr(), nexts[0].data_ptr(), stream())
        nat.pack_allreduce_unpack_planned_noalloc(plan_new, inv, flags[1].data_ptr(), nexts[1].data_ptr(), stream())
        torch.cuda.synchronize()
        got_ref, got_new = _outputs(ref, flags[0], nexts[0]), _outputs(new, flags[1], nexts[1])
        for r, (a, b) in enumerate(zip(got_ref[0], got_new[0], strict=True)):
            assert _same(a, b), f"call {k + 1}: replica row {r} differs"
        assert _same(got_ref[1], got_new[1]), f"call {k + 1}: bucket differs"
        for g, (a, b) in enumerate(zip(got_ref[2], got_new[2], strict=True)):
            assert _same(a, b), f"call {k + 1}: gradient {g} differs"
        assert got_ref[3:] == got_new[3:], f"call {k + 1}: flags differ"
        assert got_new[4] == 0
        _check(new, numels, W, rank, wdt, bdt, inv, flags[1])

