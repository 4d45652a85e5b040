"""Pack fused into the all-reduce + unpack (mdx_pack_allreduce_unpack), on the GPU, bit for bit.

One dispatch does what ``_Bucket.gather_into_buffer`` (minidist/ddp.py:75-92),
``comm.all_reduce`` (minidist/comm.py:223-234), ``scatter_from_buffer``
(ddp.py:94-102) and ``unscale_`` (minidist/amp.py:212-213) do in turn.  Each
test builds seeded inputs with sentinel gaps, runs the entry point through the
C ABI and checks every output against the oracle: this rank's packed row
(what the peers would read), the bucket (the rank-ordered sum), the gradients
(converted, unscaled), the found-inf flag and the next step's flag, which the
call clears; the peers' rows and every gap must be untouched.  NaN payloads
are not compared (every NaN equals every NaN); every other bit is.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import first_mismatch, same_bits
from minidist import _native as nat
from oracle import gradpath as o
from test_kernels_gpu import DEV, SENTINEL, code, empty_dev, esize, stream, to_dev, to_host, values

pytestmark = pytest.mark.gpu


def _layout(rng, numels, start=3):
    offs, off = [], start
    for n in numels:
        offs.append(off)
        off += n + int(rng.integers(0, 3))
    return offs, off + 4


def _want(src_host, peers_host, a, n, W, rank, wdt, bdt, inv_scale):
    """The reference chain for one gradient: pack, rank-ordered SUM, copy_ into .grad, unscale.

    Returns (packed row, bucket sum, gradient).  ``src_host`` None is a missing
    gradient (ddp.py:87-88 zero-fills its slice)."""
    raw = o.zeros(n, wdt) if src_host is None else src_host
    if wdt == bdt:  # gather_into_buffer: copy_ then mul_(1/W) in the bucket dtype (ddp.py:90-91)
        packed = raw.copy() if W == 1 else o.mul_scalar(raw, wdt, 1.0 / W)
        xs = [packed if r == rank else peers_host[r][a : a + n] for r in range(W)]
    else:  # widening: the raw 16-bit gradient travels; every contribution is widened, then x 1/W
        packed = raw.copy()
        xs = [o.mul_scalar(o.convert(packed if r == rank else peers_host[r][a : a + n], wdt, o.F32), o.F32, 1.0 / W)
              for r in range(W)]
    acc = o.allreduce_sum(xs, bdt)
    g = o.convert(acc, bdt, wdt)
    if inv_scale != 1.0:
        g = o.mul_scalar(g, wdt, inv_scale)
    return packed, acc, g


def _case(rng, wdt, bdt, W, rank, numels, null_every=4, in_place_every=3):
    """Replicas (rank's row full of sentinels), bucket, gradient sources and destinations."""
    offs, extent = _layout(rng, numels)
    peers_host = [values(rng, extent, wdt, scale=1e3) for _ in range(W)]
    reps = [to_dev(h) for h in peers_host]
    reps[rank] = empty_dev(extent, wdt)  # the pack writes it; gaps must keep their sentinel
    out = empty_dev(extent, bdt)
    srcs, dsts, shifts, rows, src_hosts = [], [], [], [], []
    for k, (a, n) in enumerate(zip(offs, numels, strict=True)):
        s = int(rng.integers(0, 3))  # gradient views at odd element offsets
        dst = empty_dev(n + 3, wdt)
        if null_every and k % null_every == null_every - 1:
            src_host, src_ptr, src = None, 0, None
        elif in_place_every and k % in_place_every == 0:  # the gradient is its own source
            src_host = values(rng, n, wdt, scale=1e3)
            host = to_host(dst)
            host[s : s + n] = src_host
            dst = to_dev(host)
            src, src_ptr = dst, dst.data_ptr() + s * esize(wdt)
        else:
            src_host = values(rng, n, wdt, scale=1e3)
            src = to_dev(np.concatenate([o.zeros(1, wdt), src_host]))
            src_ptr = src.data_ptr() + esize(wdt)
        rows.append((a, n, src_ptr, dst.data_ptr() + s * esize(wdt)))
        srcs.append(src)
        dsts.append(dst)
        shifts.append(s)
        src_hosts.append(src_host)
    return dict(offs=offs, extent=extent, peers_host=peers_host, reps=reps, out=out, srcs=srcs, dsts=dsts,
                shifts=shifts, src_hosts=src_hosts, runs=nat.pack_runs_array(rows))


def _check(c, numels, W, rank, wdt, bdt, inv_scale, flag, write_out=True):
    any_bad = False
    row_want = to_host(empty_dev(c["extent"], wdt))
    out_want = to_host(empty_dev(c["extent"], bdt))
    for k, (a, n) in enumerate(zip(c["offs"], numels, strict=True)):
        packed, acc, g = _want(c["src_hosts"][k], c["peers_host"], a, n, W, rank, wdt, bdt, inv_scale)
        row_want[a : a + n] = packed
        out_want[a : a + n] = acc
        any_bad |= bool((~o.isfinite(g, wdt)).any())
        got = to_host(c["dsts"][k])
        s = c["shifts"][k]
        assert same_bits(got[s : s + n], g), f"gradient {k}: " + first_mismatch(got[s : s + n], g)
        gaps = np.concatenate([got[:s], got[s + n :]])
        assert np.all(gaps == SENTINEL[wdt]), f"gradient {k} wrote outside its view"
    got_row = to_host(c["reps"][rank])
    assert same_bits(got_row, row_want), "packed row: " + first_mismatch(got_row, row_want)
    got_out = to_host(c["out"])
    want = out_want if write_out else to_host(empty_dev(c["extent"], bdt))
    assert same_bits(got_out, want), "bucket: " + first_mismatch(got_out, want)
    for r in range(W):
        if r != rank:
            assert same_bits(to_host(c["reps"][r]), c["peers_host"][r]), f"peer row {r} was written"
    assert bool(flag.item()) == any_bad


PAIRS = [(o.F32, o.F32), (o.BF16, o.BF16), (o.F16, o.F16), (o.BF16, o.F32), (o.F16, o.F32)]


@pytest.mark.parametrize("wdt,bdt", PAIRS)
@pytest.mark.parametrize("W,rank", [(1, 0), (2, 1), (3, 0), (4, 2), (8, 0), (8, 5), (16, 15)])
@pytest.mark.parametrize("inv_scale,write_out", [(1.0, True), (2.0**-16, True), (1.0 / 3, False)])
def test_pack_allreduce_unpack_matches_oracle(rng, wdt, bdt, W, rank, inv_scale, write_out):
    numels = [1, 7, 64, 4096, 3, 12345, 256, 5, 8, 9, 1000]
    c = _case(rng, wdt, bdt, W, rank, numels)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nxt = torch.ones(1, dtype=torch.int32, device=DEV)
    nat.pack_allreduce_unpack(
        [r.data_ptr() for r in c["reps"]], rank, code(wdt), c["runs"], c["out"].data_ptr() if write_out else None,
        code(bdt), nat.f32(1.0 / W), nat.f32(inv_scale), flag.data_ptr(), nxt.data_ptr(), stream(),
    )
    _check(c, numels, W, rank, wdt, bdt, inv_scale, flag, write_out)
    assert nxt.item() == 0


@pytest.mark.parametrize("wdt,bdt", PAIRS)
@pytest.mark.parametrize("W,rank", [(8, 3), (5, 4), (2, 0)])
def test_pack_allreduce_unpack_planned_matches_direct(rng, wdt, bdt, W, rank):
    """150 gradients: several kernel-argument dispatches directly, one dispatch through a plan;
    the plan is reusable (the second launch gives the same results again)."""
    numels = [int(x) for x in rng.integers(1, 3000, 150)]
    c = _case(rng, wdt, bdt, W, rank, numels, null_every=0, in_place_every=0)
    reps = [r.data_ptr() for r in c["reps"]]
    plan = nat.plan_pack_allreduce_unpack(reps, rank, code(wdt), c["runs"], c["out"].data_ptr(), code(bdt),
                                          nat.f32(1.0 / W), DEV)
    for _ in range(2):
        flag = torch.zeros(1, dtype=torch.int32, device=DEV)
        nxt = torch.ones(1, dtype=torch.int32, device=DEV)
        nat.pack_allreduce_unpack_planned(plan, nat.f32(2.0**-10), flag.data_ptr(), nxt.data_ptr(), stream())
        _check(c, numels, W, rank, wdt, bdt, 2.0**-10, flag)
        assert nxt.item() == 0
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nat.pack_allreduce_unpack(reps, rank, code(wdt), c["runs"], c["out"].data_ptr(), code(bdt), nat.f32(1.0 / W),
                              nat.f32(2.0**-10), flag.data_ptr(), None, stream())
    _check(c, numels, W, rank, wdt, bdt, 2.0**-10, flag)


def test_pack_allreduce_unpack_run_past_the_run_limit(rng):
    """A gradient longer than one run (2^26 elements) is cut into runs whose offsets line up."""
    n = (1 << 26) + 1000
    W, rank = 2, 1
    peers_host = [np.full(n + 8, 0.5, np.float32), None]
    reps = [to_dev(peers_host[0]), empty_dev(n + 8, o.F32)]
    src = torch.arange(n, dtype=torch.float32, device=DEV).remainder_(1024.0)
    out = empty_dev(n + 8, o.F32)
    runs = nat.pack_runs_array([(4, n, src.data_ptr(), src.data_ptr())])
    want = src.detach().clone()
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nat.pack_allreduce_unpack([r.data_ptr() for r in reps], rank, nat.MDX_F32, runs, out.data_ptr(), nat.MDX_F32,
                              0.5, 1.0, flag.data_ptr(), None, stream())
    packed = want * 0.5  # exact: halving integers below 1024
    assert torch.equal(reps[1][4 : 4 + n], packed)
    assert torch.equal(out[4 : 4 + n], packed + 0.5)
    assert torch.equal(src, packed + 0.5)
    assert torch.all(reps[1][:4] == float(SENTINEL[o.F32])) and torch.all(reps[1][4 + n :] == float(SENTINEL[o.F32]))
    assert flag.item() == 0


@pytest.mark.parametrize("copy_plan", [False, True])
def test_plan_larger_than_one_dispatch(rng, copy_plan):
    """A plan of more than 2^22 workgroups (the slice a dispatch takes; 2^30 + 2^20 fp32 elements
    in three gradients) goes out as several dispatches: every element is checked against the same
    IEEE ops in torch on the device, and windows at the ends and across the first slice boundary
    (workgroup 2^22 of 256 elements) against the oracle.  ``copy_plan`` runs the pack's copy plan
    (mdx_pack_planned, x 1/2) instead of the fused plan."""
    W, rank, inv = 2, 1, 2.0**-10
    numels = [(1 << 29) - 3, (1 << 29) + (1 << 20) - 1000, 1003]
    offs = [1, 1 + numels[0] + 2, 1 + numels[0] + 2 + numels[1] + 5]
    extent = offs[-1] + numels[-1] + 3
    gen = torch.Generator(device=DEV).manual_seed(77)
    grads = [torch.randn(n, device=DEV, generator=gen) for n in numels]
    if copy_plan:
        dst = torch.full((extent,), float(SENTINEL[o.F32]), device=DEV)
        plan = nat.plan_spans(nat.spans_array([(g.data_ptr(), dst.data_ptr() + 4 * a, n)
                                               for g, a, n in zip(grads, offs, numels)]),
                              nat.MDX_F32, nat.MDX_F32, DEV)
        nat.pack_planned(plan, nat.f32(1.0 / W), False, stream())
        for g, a, n in zip(grads, offs, numels):
            assert torch.equal(dst[a : a + n], g * 0.5)
        windows = [(0, 0, 4096), (1, (1 << 30) - numels[0] - 4096, 8192), (2, 0, numels[2])]
        for k, lo, m in windows:
            want = o.mul_scalar(to_host(grads[k][lo : lo + m]), o.F32, 1.0 / W)
            got = to_host(dst[offs[k] + lo : offs[k] + lo + m])
            assert same_bits(got, want), first_mismatch(got, want)
        return
    peer = torch.randn(extent, device=DEV, generator=gen)
    own = torch.full((extent,), float(SENTINEL[o.F32]), device=DEV)
    out = torch.full((extent,), float(SENTINEL[o.F32]), device=DEV)
    runs = nat.pack_runs_array([(a, n, g.data_ptr(), g.data_ptr()) for g, a, n in zip(grads, offs, numels)])
    plan = nat.plan_pack_allreduce_unpack([peer.data_ptr(), own.data_ptr()], rank, nat.MDX_F32, runs, out.data_ptr(),
                                          nat.MDX_F32, nat.f32(1.0 / W), DEV)
    windows = [(0, 0, 4096), (1, (1 << 30) - numels[0] - 4096, 8192), (2, 0, numels[2])]
    before = [(k, lo, m, to_host(grads[k][lo : lo + m])) for k, lo, m in windows]
    packed = [g * 0.5 for g in grads]
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nxt = torch.ones(1, dtype=torch.int32, device=DEV)
    nat.pack_allreduce_unpack_planned(plan, nat.f32(inv), flag.data_ptr(), nxt.data_ptr(), stream())
    for g, pk, a, n in zip(grads, packed, offs, numels):
        assert torch.equal(own[a : a + n], pk)
        acc = peer[a : a + n] + pk
        assert torch.equal(out[a : a + n], acc)
        assert torch.equal(g, acc * inv)
    for k, lo, m, src_host in before:
        a = offs[k] + lo
        peers_host = [to_host(peer[a : a + m]), None]
        want_row, want_acc, want_g = _want(src_host, peers_host, 0, m, W, rank, o.F32, o.F32, inv)
        for got, want in ((own[a : a + m], want_row), (out[a : a + m], want_acc), (grads[k][lo : lo + m], want_g)):
            got = to_host(got)
            assert same_bits(got, want), first_mismatch(got, want)
    assert flag.item() == 0 and nxt.item() == 0


@pytest.mark.parametrize("planned", [False, True])
def test_pack_allreduce_unpack_nothing_to_do_still_clears(planned):
    reps = [torch.zeros(64, device=DEV) for _ in range(2)]
    nxt = torch.ones(1, dtype=torch.int32, device=DEV)
    runs = nat.pack_runs_array([(0, 0, 0, 0)])
    if planned:
        plan = nat.plan_pack_allreduce_unpack([r.data_ptr() for r in reps], 0, nat.MDX_F32, runs, None,
                                              nat.MDX_F32, 0.5, DEV)
        nat.pack_allreduce_unpack_planned(plan, 1.0, None, nxt.data_ptr(), stream())
    else:
        nat.pack_allreduce_unpack([r.data_ptr() for r in reps], 0, nat.MDX_F32, runs, None, nat.MDX_F32, 0.5, 1.0,
                                  None, nxt.data_ptr(), stream())
    assert nxt.item() == 0


def test_pack_allreduce_unpack_rejects_bad_arguments():
    L = nat.lib()
    reps = [torch.zeros(1024, device=DEV) for _ in range(2)]
    ptrs = nat._ptrs([r.data_ptr() for r in reps])
    out = torch.zeros(1024, device=DEV)
    g = torch.zeros(100, device=DEV)
    flag = torch.zeros(2, dtype=torch.int32, device=DEV)

    def call(runs, rank=0, wdt=nat.MDX_F32, bdt=nat.MDX_F32, out_ptr=None, found=None, clear=None):
        return L.mdx_pack_allreduce_unpack(ptrs, 2, rank, wdt, runs.ctypes.data, len(runs),
                                           out_ptr if out_ptr is not None else out.data_ptr(), bdt, 0.5, 1.0,
                                           found, clear, None)

    ok = nat.pack_runs_array([(0, 100, g.data_ptr(), g.data_ptr())])
    assert call(ok, rank=2) == -3  # MDX_EWORLD
    assert call(ok, wdt=nat.MDX_F32, bdt=nat.MDX_BF16) == -2  # MDX_EDTYPE: no narrowing bucket
    assert call(ok, wdt=nat.MDX_BF16, bdt=nat.MDX_F16) == -2
    assert call(ok, out_ptr=reps[1].data_ptr() + 64) == -4  # MDX_EALIAS: bucket overlaps a replica
    on_row = nat.pack_runs_array([(0, 100, g.data_ptr(), reps[1].data_ptr() + 256)])
    assert call(on_row) == -4  # gradient inside a replica's reduced extent (400 bytes)
    shifted = nat.pack_runs_array([(0, 50, g.data_ptr(), g.data_ptr() + 8)])
    assert call(shifted) == -4  # source partially overlaps its gradient
    src_in_out = nat.pack_runs_array([(0, 50, out.data_ptr(), g.data_ptr())])
    assert call(src_in_out) == -4  # source inside the bucket
    assert call(ok, found=flag.data_ptr(), clear=flag.data_ptr()) == -4  # the flag it sets cannot be cleared
    bad_order = nat.pack_runs_array([(50, 10, g.data_ptr(), g.data_ptr()), (40, 5, 0, g.data_ptr() + 400)])
    assert call(bad_order) == -1  # MDX_EINVAL
    no_grad = nat.pack_runs_array([(0, 10, g.data_ptr(), 0)])
    assert call(no_grad) == -1  # MDX_EINVAL
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0 and torch.count_nonzero(reps[0]).item() == 0


# ---------------------------------------------------------------------------
# Through DDP: the packed row, the bucket and the scaler's alternating flags
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype,reduce_dtype", [(torch.float32, None), (torch.bfloat16, None),
                                                (torch.bfloat16, torch.float32), (torch.float16, torch.float32)])
def test_ddp_step_leaves_packed_row_and_averaged_bucket(rng, dtype, reduce_dtype):
    """After finish_gradient_sync this rank's contribution row holds what its pack wrote (the
    bucket the peers would read) and the bucket holds the average, as the reference's bucket
    does after its in-place all-reduce (ddp.py:243-247, 269-273)."""
    from minidist import DDP, ResidentGroup
    from test_ddp_gpu import Flat, odt, stage_peers, synthetic_grads, dev_from, host_bits

    W, rank = 4, 2
    shapes = [(33,), (64, 8), (5,), (130,), (7, 9)]
    model = Flat(shapes, dtype)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=0.001, reduce_dtype=reduce_dtype)
    grads = synthetic_grads(rng, shapes, W, dtype, 2.0**10)
    dts = [odt(dtype)] * len(shapes)
    stage_peers(ddp, grads, dts, rank, W)
    for p, g in zip(model.parameters(), grads[rank], strict=True):
        p.grad = dev_from(g, p.shape)
    ddp.finish_gradient_sync()
    assert any(st for plan in ddp._plans.values() for st in plan.packed_calls)  # the fused pack ran
    params = list(model.parameters())
    index = {id(p): i for i, p in enumerate(params)}
    want = o.ddp_pipeline(grads, dts, [p.numel() for p in params], 0.001, rank, None,
                          **({"bucket_dtype": odt(reduce_dtype)} if reduce_dtype else {}))
    for b, bucket in enumerate(ddp._buckets):
        idxs = [index[id(p)] for p in bucket.params]
        wire_dtype, prescaled = ddp.bucket_wire_format(b)
        packed = o.pack([grads[rank][i] for i in idxs], [dts[i] for i in idxs], [params[i].numel() for i in idxs],
                        odt(wire_dtype), 1.0 / W if prescaled else 1.0)
        assert same_bits(host_bits(ddp.bucket_replicas(b)[rank]), packed), f"bucket {b} packed row"
        assert same_bits(host_bits(bucket.buffer), want["reduced"][b]), f"bucket {b} average"
    for i, p in enumerate(params):
        assert same_bits(host_bits(p.grad), want["grads"][i]), f"param {i}"


@pytest.mark.parametrize("dtype,reduce_dtype", [(torch.float32, None), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("n_params,cap", [(5, 0.001), (70, 25.0)])
@pytest.mark.parametrize("inf", [False, True])
@pytest.mark.parametrize("launch", ["eager", "comm_stream", "graphs"])
def test_ddp_without_bucket_average(rng, dtype, reduce_dtype, n_params, cap, inf, launch):
    """``keep_bucket_average=False``: the same step as the default -- gradients, found-inf and this
    rank's packed rows bit for bit, and against the oracle -- while every bucket keeps the sentinel
    it held before the step.  Small runs go through kernel-argument tables (one bucket per launch),
    70 gradients in one bucket through a device plan; fp32 and widening bf16 -> fp32 buckets; eager
    launches, a dedicated communication stream, and graph replay."""
    from minidist import DDP, DistributedGradScaler, ResidentGroup
    from test_ddp_gpu import Flat, odt, stage_peers, synthetic_grads, dev_from, host_bits

    W, rank, S = 4, 3, 2.0**10
    shapes = [(int(rng.integers(1, 300)),) if k % 3 else (int(rng.integers(1, 40)), 7) for k in range(n_params)]
    grads = synthetic_grads(rng, shapes, W, dtype, S)
    if inf:
        grads[1][n_params // 2] = grads[1][n_params // 2].copy()
        grads[1][n_params // 2][0] = o.from_f32(np.array([np.inf], np.float32), odt(dtype))[0]
    dts = [odt(dtype)] * len(shapes)
    states = []
    for keep in (True, False):
        model = Flat(shapes, dtype)
        scaler = DistributedGradScaler(init_scale=S)
        ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap, reduce_dtype=reduce_dtype,
                  grad_scaler=scaler, keep_bucket_average=keep, comm_stream=launch == "comm_stream",
                  capture_graphs=launch == "graphs")
        stage_peers(ddp, grads, dts, rank, W)
        for b in ddp._buckets:
            b.buffer.fill_(-3.25)
        for p, g in zip(model.parameters(), grads[rank], strict=True):
            p.grad = dev_from(g, p.shape)
        ddp.finish_gradient_sync()
        planned = any(st.plan is not None for plan in ddp._plans.values() for st in plan.packed_calls)
        assert planned == (n_params > 48)

        class _Opt:
            param_groups = [{"params": list(model.parameters())}]

        found = scaler.unscale_(_Opt())
        states.append((
            [host_bits(p.grad) for p in model.parameters()],
            [host_bits(ddp.bucket_replicas(i)[rank]) for i in range(len(ddp._buckets))],
            [b.buffer.detach().clone() for b in ddp._buckets],
            found,
        ))
    (g_keep, r_keep, b_keep, f_keep), (g_skip, r_skip, b_skip, f_skip) = states
    want = o.ddp_pipeline(grads, dts, [int(np.prod(s)) for s in shapes], cap, rank, 1.0 / S,
                          **({"bucket_dtype": odt(reduce_dtype)} if reduce_dtype else {}))
    assert f_keep == f_skip == want["found_inf"] == inf
    for i in range(len(shapes)):
        assert same_bits(g_skip[i], g_keep[i]) and same_bits(g_skip[i], want["grads"][i]), f"param {i}"
    for k in range(len(r_keep)):
        assert same_bits(r_skip[k], r_keep[k]), f"bucket {k} packed row"
        assert same_bits(host_bits(b_keep[k]), want["reduced"][k]), f"bucket {k} average (default)"
        assert bool((b_skip[k] == -3.25).all()), f"bucket {k} was written"


@pytest.mark.parametrize("graphs", [False, True])
def test_found_inf_flags_alternate_across_steps(rng, graphs):
    """Each step reports its own overflow: the fused pack of step s clears the flag of step s+1,
    so an inf in steps 1, 2 and 4 (and none in 0, 3, 5, 6) is seen exactly there."""
    from minidist import DDP, DistributedGradScaler, ResidentGroup
    from test_ddp_gpu import Flat, stage_peers, synthetic_grads, dev_from, host_bits

    W, rank, init = 4, 1, 2.0**10
    shapes = [(40,), (9, 7), (300,), (2,)]
    numels = [int(np.prod(s)) for s in shapes]
    model = Flat(shapes)
    scaler = DistributedGradScaler(init_scale=init, growth_interval=1000)
    ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=25.0, grad_scaler=scaler,
              capture_graphs=graphs)
    scale = init
    for step in range(7):
        grads = synthetic_grads(rng, shapes, W, torch.float32, scale)
        bad = step in (1, 2, 4)
        if bad:  # on a peer in step 1, on this rank in steps 2 and 4
            who = (rank + 1) % W if step == 1 else rank
            grads[who][2] = grads[who][2].copy()
            grads[who][2][7] = np.float32(np.inf if step != 4 else np.nan)
        stage_peers(ddp, grads, [o.F32] * len(shapes), rank, W)
        for p, g in zip(model.parameters(), grads[rank], strict=True):
            if p.grad is None:
                p.grad = dev_from(g, p.shape)
            else:
                p.grad.copy_(dev_from(g, p.shape))
        ddp.finish_gradient_sync()

        class _Opt:
            param_groups = [{"params": list(model.parameters())}]

        found = scaler.unscale_(_Opt())
        want = o.ddp_pipeline(grads, [o.F32] * len(shapes), numels, 25.0, rank, 1.0 / scale)
        assert found == want["found_inf"] == bad, f"step {step}"
        for i, p in enumerate(model.parameters()):
            assert same_bits(host_bits(p.grad), want["grads"][i]), f"step {step} param {i}"
        scaler.update()
        scale = scaler.scale


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_bucket_sequence_leaves_the_fused_state(rng, dtype):
    """The reference's per-bucket sequence (ddp.py:243-247, 269-273) -- ``gather_into_buffer(1/W)``,
    ``comm.all_reduce`` of the returned buffer, ``scatter_from_buffer`` -- over a ResidentGroup:
    the gradients equal the oracle's, and the rows and buckets end as DDP's fused launch leaves
    them (the packed contribution in this rank's row, the average in the bucket)."""
    from minidist import DDP, ResidentGroup, comm
    from test_ddp_gpu import Flat, odt, stage_peers, synthetic_grads, dev_from, host_bits

    W, rank, cap = 4, 2, 0.001
    shapes = [(33,), (64, 8), (5,), (130,), (7, 9), (3,)]
    dts = [odt(dtype)] * len(shapes)
    numels = [int(np.prod(s)) for s in shapes]
    grads = synthetic_grads(rng, shapes, W, dtype, 2.0**10)
    states = []
    for manual in (True, False):
        model = Flat(shapes, dtype)
        ddp = DDP(model, process_group=ResidentGroup(W, rank, DEV), bucket_cap_mb=cap)
        stage_peers(ddp, grads, dts, rank, W)
        for p, g in zip(model.parameters(), grads[rank], strict=True):
            p.grad = dev_from(g, p.shape)
        if manual:
            for b in ddp._buckets:
                buf = b.gather_into_buffer(1.0 / W)
                comm.all_reduce(buf, group=ddp.process_group, async_op=True).wait()
                b.scatter_from_buffer()
        else:
            ddp.finish_gradient_sync()
        states.append((
            [host_bits(p.grad) for p in model.parameters()],
            [host_bits(b.buffer) for b in ddp._buckets],
            [host_bits(ddp.bucket_replicas(i)[rank]) for i in range(len(ddp._buckets))],
        ))
    want = o.ddp_pipeline(grads, dts, numels, cap, rank, None)
    (g_m, b_m, r_m), (g_f, b_f, r_f) = states
    for i in range(len(shapes)):
        assert same_bits(g_m[i], want["grads"][i]), f"param {i}"
        assert same_bits(g_f[i], g_m[i]), f"param {i}"
    for k in range(len(b_m)):
        assert same_bits(b_m[k], want["reduced"][k]), f"bucket {k}"
        assert same_bits(b_f[k], b_m[k]) and same_bits(r_f[k], r_m[k]), f"bucket {k}"
