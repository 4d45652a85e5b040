"""Host-side logic and the C ABI surface, on the CPU (no kernel is launched).

* libmdx.so loads and exports every function include/mdx.h declares, and the
  ctypes table binds exactly those;
* argument checks return their MDX_E* codes before anything is launched;
* byte accounting, precision resolution, the scaler's state machine, the DDP
  bucket layout (on meta tensors, at the real GPT-2 shapes) and the loud
  failure on CPU tensors.
"""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest
import torch
from torch import nn

from conftest import ROOT
from minidist import _native as nat
from minidist import comm
from minidist.amp import DistributedGradScaler, resolve_precision
from minidist.ddp import DistributedDataParallel
from minidist import workloads as w
from oracle import gradpath as o

HEADER = ROOT / "include" / "mdx.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^MDX_API\s+(?:int|const char\*)\s+(mdx_\w+)\(", text, flags=re.M))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert names == set(nat.SIGNATURES), "ctypes table and header disagree"
    lib = nat.lib()
    for name in names:
        assert hasattr(lib, name), name
    assert lib.mdx_abi_version() == nat.ABI_VERSION


_C_TO_CTYPES = {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "float": ctypes.c_float}


def _ctype_of(decl: str):
    """The ctypes type a C parameter (or return) declaration passes as: any pointer is an address."""
    decl = " ".join(decl.replace("*", " * ").split())
    if "*" in decl:
        return ctypes.c_char_p if decl.startswith("const char *") and decl.count("*") == 1 else ctypes.c_void_p
    base = decl.split()[0] if decl.split()[0] != "const" else decl.split()[1]
    return _C_TO_CTYPES[base]


def test_ctypes_signatures_follow_the_header_prototypes():
    """Every argument the Python binding passes has the C type, position and count of the prototype
    in include/mdx.h (a float passed where an int is declared, or a missing argument, would be read
    as garbage by the library without any error)."""
    protos = re.findall(r"^MDX_API\s+(int|const char\*)\s+(mdx_\w+)\(([^)]*)\);", HEADER.read_text(), flags=re.M)
    assert {name for _, name, _ in protos} == set(nat.SIGNATURES)
    for ret, name, params in protos:
        params = " ".join(params.split())
        args = [] if params in ("", "void") else [_ctype_of(p.rsplit(" ", 1)[0] if not p.endswith("*") else p)
                                                   for p in (q.strip() for q in params.split(","))]
        want_ret, want_args = nat.SIGNATURES[name]
        assert _ctype_of(ret) is want_ret, f"{name}: returns {ret}"
        assert list(want_args) == args, f"{name}: header {params!r}"
    # the reference-side bindings shown in INTEGRATION.md declare the same argument lists
    shown = re.findall(r"_lib\.(mdx_\w+)\.argtypes = (\[[^\]]*\])", (ROOT / "INTEGRATION.md").read_text())
    assert len(shown) >= 5
    for name, listed in shown:
        assert eval(listed, {"ctypes": ctypes}) == list(nat.SIGNATURES[name][1]), f"INTEGRATION.md: {name}"


def test_exported_symbols_are_only_the_abi():
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", str(nat.LIB_PATH)], capture_output=True, text=True)
    if out.returncode != 0:
        pytest.skip("nm unavailable")
    text_syms = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    assert text_syms == declared_functions()


def test_strerror_names_every_mdx_code():
    for code_, frag in [(0, "success"), (-1, "invalid"), (-2, "dtype"), (-3, "world"), (-4, "overlap"),
                        (-7, "reduction op")]:
        assert frag in nat.strerror(code_)
    assert "unknown" in nat.strerror(-99)


def _span(src, dst, n):
    return nat.spans_array([(src, dst, n)])


def test_argument_checks_happen_before_any_launch():
    L = nat.lib()
    P = ctypes.c_void_p
    # dtype
    assert L.mdx_pack(None, 0, 9, 0, 1.0, 0, None, None) == -2
    assert L.mdx_unpack(None, 0, 0, 5, 1.0, None, None) == -2
    assert L.mdx_unscale_found_inf(None, 0, 3, 1.0, None, None) == -2
    # counts and NULLs
    assert L.mdx_pack(None, -1, 0, 0, 1.0, 0, None, None) == -1
    assert L.mdx_pack(None, 3, 0, 0, 1.0, 0, None, None) == -1
    s = _span(0, 0, 10)  # dst NULL with numel > 0
    assert L.mdx_pack(s.ctypes.data, 1, 0, 0, 1.0, 0, None, None) == -1
    s = _span(0, 4096, 10)  # unpack needs a source
    assert L.mdx_unpack(s.ctypes.data, 1, 0, 0, 1.0, None, None) == -1
    s = _span(0, 4096, -1)
    assert L.mdx_pack(s.ctypes.data, 1, 0, 0, 1.0, 0, None, None) == -1
    assert L.mdx_cast_f32_bf16(None, None, -1, None) == -1
    assert L.mdx_cast_f32_bf16(P(4096), P(4096 + 8), 16, None) == -4  # overlapping cast
    # zero-length work is a no-op that succeeds without a device
    assert L.mdx_pack(None, 0, 0, 0, 1.0, 0, None, None) == 0
    assert L.mdx_cast_f32_bf16(None, None, 0, None) == 0
    # world / rank
    reps = (ctypes.c_void_p * 2)(4096, 8192)
    offs = (ctypes.c_int64 * 1)(0)
    nums = (ctypes.c_int64 * 1)(8)
    assert L.mdx_allreduce_sum(reps, 0, 0, offs, nums, 1, P(4096), None) == -3
    assert L.mdx_allreduce_sum(reps, 17, 0, offs, nums, 1, P(4096), None) == -3
    bad_offs = (ctypes.c_int64 * 2)(8, 0)  # runs must increase
    bad_nums = (ctypes.c_int64 * 2)(4, 4)
    assert L.mdx_allreduce_sum(reps, 2, 0, bad_offs, bad_nums, 2, P(4096), None) == -1
    assert L.mdx_allreduce_sum(reps, 2, 0, offs, nums, 1, P(4096 + 4), None) == -4  # partial overlap
    runs = nat.grad_runs_array([(0, 8, 1 << 20)])
    assert L.mdx_allreduce_unpack(reps, 0, 0, runs.ctypes.data, 1, None, 0, 1.0, None, None) == -3
    assert L.mdx_allreduce_unpack(reps, 2, 0, runs.ctypes.data, 1, None, 4, 1.0, None, None) == -2
    assert L.mdx_allreduce_unpack(reps, 2, 0, None, 1, None, 0, 1.0, None, None) == -1
    null_grad = nat.grad_runs_array([(0, 8, 0)])
    assert L.mdx_allreduce_unpack(reps, 2, 0, null_grad.ctypes.data, 1, None, 0, 1.0, None, None) == -1
    into_replica = nat.grad_runs_array([(0, 8, 8192 + 4)])
    assert L.mdx_allreduce_unpack(reps, 2, 0, into_replica.ctypes.data, 1, None, 0, 1.0, None, None) == -4
    assert L.mdx_allreduce_unpack(reps, 2, 0, None, 0, None, 0, 1.0, None, None) == 0
    pc = nat.pieces_array([(4096, 0, 8)])
    peers = (ctypes.c_void_p * 2)(0, 8192)
    assert L.mdx_reduce_scatter_share(pc.ctypes.data, 1, peers, 2, 2, 0, 0, 1, P(1 << 20), 0, 0, 1.0, None, None) == -3
    assert L.mdx_reduce_scatter_share(pc.ctypes.data, 1, peers, 2, 0, 0, 7, 1, P(1 << 20), 0, 0, 1.0, None, None) == -2
    assert L.mdx_reduce_scatter_share(pc.ctypes.data, 1, peers, 2, 0, 0, 0, 1, P(8192), 0, 0, 1.0, None, None) == -4
    # fp16 (MDX_F16 = 2) is an element type of every entry point; widening is only bf16 / fp16 -> fp32
    assert nat.MDX_F16 == 2
    assert L.mdx_pack(None, 0, 2, 0, 1.0, 0, None, None) == 0
    assert L.mdx_unscale_found_inf(None, 0, 2, 1.0, None, None) == 0
    assert L.mdx_allreduce_unpack(reps, 2, 2, None, 0, None, 2, 1.0, None, None) == 0
    assert L.mdx_allreduce_unpack_wide(reps, 2, 2, runs.ctypes.data, 1, None, 2, 2, 0.5, 1.0, None, None) == -2
    assert L.mdx_allreduce_unpack_wide(reps, 2, 0, runs.ctypes.data, 1, None, 0, 2, 0.5, 1.0, None, None) == -2
    # dtypes 2 pass the dtype check; the out-of-range rank is what is rejected (nothing launches)
    assert L.mdx_reduce_scatter_share(pc.ctypes.data, 1, peers, 2, 2, 2, 2, 1, P(1 << 20), 2, 0, 1.0, None,
                                      None) == -3
    # the non-SUM all-reduce: op, then mdx_allreduce_sum's checks
    assert L.mdx_allreduce_op(reps, 2, 0, 4, offs, nums, 1, P(4096), None) == nat.MDX_EOP
    assert L.mdx_allreduce_op(reps, 2, 0, -1, offs, nums, 1, P(4096), None) == nat.MDX_EOP
    for op in (nat.MDX_OP_PRODUCT, nat.MDX_OP_MIN, nat.MDX_OP_MAX, nat.MDX_OP_SUM):
        assert L.mdx_allreduce_op(reps, 2, 9, op, offs, nums, 1, P(4096), None) == -2
        assert L.mdx_allreduce_op(reps, 17, 0, op, offs, nums, 1, P(4096), None) == -3
        assert L.mdx_allreduce_op(reps, 2, 0, op, bad_offs, bad_nums, 2, P(4096), None) == -1
        assert L.mdx_allreduce_op(reps, 2, 0, op, offs, nums, 1, P(4096 + 4), None) == -4  # partial overlap
        assert L.mdx_allreduce_op(reps, 2, 0, op, offs, nums, 1, None, None) == -1
        assert L.mdx_allreduce_op(reps, 2, 2, op, offs, nums, 0, None, None) == 0  # nothing to reduce


# ---------------------------------------------------------------------------
# comm
# ---------------------------------------------------------------------------


def test_comm_stats_formulas_match_reference():
    """minidist/comm.py:65-72: all-reduce 2(W-1)/W N, all-gather / reduce-scatter (W-1)/W N."""
    grp = comm.ResidentGroup(4, 1, "cpu")
    with comm.record_comm() as stats:
        comm.comm_stats.add("all_reduce", 1000, int(2 * 3 / 4 * 1000))
    assert stats.as_rows() == [("all_reduce", 1, 1000, 1500)]
    assert stats.total_bus_bytes() == 1500
    assert not comm.comm_stats.enabled
    assert comm.get_world_size(grp) == 4 and comm.get_rank(grp) == 1
    assert comm.get_world_size(None) == 1 and comm.get_rank(None) == 0
    assert comm.all_reduce(torch.zeros(3), group=None) is None  # world 1 short-circuit


def test_dropped_ddp_frees_its_module_and_removes_its_hooks():
    """A parameter's post-accumulate-grad hooks are not visited by the cycle collector, so a
    wrapper reachable from them would keep its module, buckets and resident arenas alive for
    good.  Dropping the wrapper frees it at once and takes its hooks off a module that lives on."""
    import gc
    import weakref

    from minidist import DDP, DistributedGradScaler

    class Flat(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.ps = torch.nn.ParameterList([torch.nn.Parameter(torch.zeros(100)) for _ in range(3)])

    def make():
        m = Flat()
        d = DDP(m, process_group=comm.ResidentGroup(2, 1, "cpu"), bucket_cap_mb=1e-6,
                grad_scaler=DistributedGradScaler())
        return weakref.ref(m.ps[0]), weakref.ref(d)

    wp, wd = make()
    assert wd() is None and wp() is None  # no cycle at all: reference counting frees both
    m = Flat()
    d = DDP(m, process_group=comm.ResidentGroup(2, 1, "cpu"))
    assert all(len(p._post_accumulate_grad_hooks) == 1 for p in m.parameters())
    del d
    gc.collect()
    assert all(not p._post_accumulate_grad_hooks for p in m.parameters())


def test_resident_group_validates_its_shape():
    with pytest.raises(ValueError):
        comm.ResidentGroup(0)
    with pytest.raises(ValueError):
        comm.ResidentGroup(17, device="cpu")
    with pytest.raises(ValueError):
        comm.ResidentGroup(4, 4, "cpu")


def test_resident_group_symmetric_rows_cpu_layout():
    grp = comm.ResidentGroup(3, 2, "cpu")
    own = grp.zeros(10, torch.float32)
    reps = grp.replicas(own[3:7])
    assert len(reps) == 3 and reps[2].data_ptr() == own[3:7].data_ptr()
    assert all(r.numel() == 4 for r in reps)
    assert len({r.data_ptr() for r in reps}) == 3
    with pytest.raises(RuntimeError):
        grp.replicas(torch.zeros(4))
    # views with no elements (an empty bucket) are still places in the buffer, whose data_ptr()
    # torch reports as 0: each is found at its offset, and its replicas are empty too
    for lo in (0, 4, 10):
        empty = own[lo:lo]
        assert empty.data_ptr() == 0 and grp._locate(empty)[1] == lo
        assert [r.numel() for r in grp.replicas(empty)] == [0, 0, 0]
    nothing = grp.zeros(0, torch.float32)
    assert grp._locate(nothing)[1] == 0 and grp.row_addresses(nothing)[2] != 0


# ---------------------------------------------------------------------------
# amp (host logic; kernels are exercised on the GPU)
# ---------------------------------------------------------------------------


def test_resolve_precision():
    """Reference tests/test_amp.py:123-134."""
    assert not resolve_precision("fp32", torch.device("cpu")).enabled
    bf16 = resolve_precision("bf16", torch.device("cpu"))
    assert bf16.dtype == torch.bfloat16 and not bf16.needs_grad_scaler
    assert resolve_precision("auto", torch.device("cpu")).dtype == torch.bfloat16
    with pytest.raises(ValueError):
        resolve_precision("fp16", torch.device("cpu"))
    with pytest.raises(ValueError):
        resolve_precision("int4", torch.device("cpu"))


def test_disabled_scaler_is_transparent():
    """Reference tests/test_amp.py:137-143."""
    model = nn.Linear(4, 4)
    opt = torch.optim.SGD(model.parameters(), lr=0.1)
    scaler = DistributedGradScaler(enabled=False)
    loss = torch.tensor(2.0)
    assert scaler.scale_loss(loss) is loss
    assert scaler.scale == 1.0
    for p in model.parameters():
        p.grad = torch.ones_like(p)
    assert scaler.step(opt)


@pytest.mark.parametrize(
    "init,interval,found,final",
    [(1024.0, 2000, [True], 512.0), (1024.0, 2, [False, False], 2048.0), (4096.0, 2, [True, False, False, True, True], 1024.0)],
)
def test_scaler_state_machine_matches_oracle(init, interval, found, final):
    s = DistributedGradScaler(init_scale=init, growth_interval=interval)
    ref = o.ScalerState(scale=init, growth_interval=interval)
    for f in found:
        s._found_inf_this_step, s._unscaled = f, True  # what unscale_ would have decided
        s.update()
        ref.update(f)
        assert s.scale == ref.scale
        assert not s._unscaled
    assert s.scale == final
    assert set(s.state_dict()) == {"scale", "good_steps", "num_skipped", "num_steps"}


def test_scaler_checkpoint_round_trip_and_summary():
    """state_dict / load_state_dict carry the state machine across a restart (amp.py:164-176): a
    scaler restored mid-history continues exactly as the uninterrupted one; summary() is the
    reference's line, and an old checkpoint without the counters loads with them at zero."""
    history = [True, False, False, False, True, False, False, False, False]
    whole = DistributedGradScaler(init_scale=2.0**10, growth_interval=3)
    first = DistributedGradScaler(init_scale=2.0**10, growth_interval=3)

    def run(s, found):
        s.num_steps += 1  # what step() counts
        s.num_skipped += int(found)
        s._found_inf_this_step, s._unscaled = found, True  # what unscale_ would have decided
        s.update()

    for f in history[:4]:
        run(whole, f)
        run(first, f)
    resumed = DistributedGradScaler(init_scale=1.0, growth_interval=3)
    resumed.load_state_dict(first.state_dict())
    for f in history[4:]:
        run(whole, f)
        run(resumed, f)
        assert resumed.state_dict() == whole.state_dict()
    assert whole.summary() == f"scale={whole.scale:g}  skipped=2/9 (22.2%)"
    old = DistributedGradScaler()
    old.load_state_dict({"scale": 256.0, "good_steps": 1})
    assert old.state_dict() == {"scale": 256.0, "good_steps": 1, "num_skipped": 0, "num_steps": 0}


# ---------------------------------------------------------------------------
# DDP layout (meta tensors: real GPT-2 shapes without allocating them)
# ---------------------------------------------------------------------------


class MetaParams(nn.Module):
    def __init__(self, specs):
        super().__init__()
        self.ps = nn.ParameterList([nn.Parameter(torch.empty(s.shape, device="meta", dtype=s.dtype)) for s in specs])


@pytest.mark.parametrize("cfg,W,cap", [(w.GPT2_SMALL, 8, 25.0), (w.GPT2_MEDIUM, 4, 1e-6), (w.GPT2_MEDIUM, 4, 1e6), (w.TINY_GPT, 4, 25.0)])
def test_ddp_layout_matches_oracle_at_real_shapes(cfg, W, cap):
    specs = w.gpt_specs(**cfg)
    ddp = DistributedDataParallel(MetaParams(specs), process_group=comm.ResidentGroup(W, 0, "meta"), bucket_cap_mb=cap)
    layout = o.build_buckets([s.nbytes for s in specs], cap)
    assert [len(b.params) for b in ddp._buckets] == [len(b) for b in layout]
    assert [b.numel for b in ddp._buckets] == [sum(specs[i].numel for i in b) for b in layout]
    assert ddp.world_size == W


def test_ddp_bucket_summary_and_passthrough():
    """bucket_summary() (ddp.py:296-302): (index, parameters, MiB of their bytes) per bucket in launch
    order; attributes the wrapper does not have come from the wrapped module (ddp.py:304-313)."""
    specs = w.gpt_specs(**w.TINY_GPT)
    module = MetaParams(specs)
    module.vocab_size = 1024
    ddp = DistributedDataParallel(module, process_group=comm.ResidentGroup(4, 0, "meta"), bucket_cap_mb=0.5)
    layout = o.build_buckets([sp.nbytes for sp in specs], 0.5)
    assert ddp.bucket_summary() == [(k, len(b), sum(specs[i].nbytes for i in b) / 2**20) for k, b in enumerate(layout)]
    assert ddp.vocab_size == 1024 and ddp.ps is module.ps
    with pytest.raises(AttributeError):
        ddp.no_such_attribute


def test_bucket_spans_are_the_oracle_partition():
    """DDP's partition (index ranges over the reversed parameters) against the oracle's restatement
    of ddp.py:175-190, over every list of up to 5 sizes from a small alphabet and several caps."""
    import itertools

    from minidist.ddp import bucket_spans

    for k in range(6):
        for sizes in itertools.product((0, 1, 3, 4, 9), repeat=k):
            for cap_mb in (0.0, 2 / 2**20, 4 / 2**20, 9 / 2**20, 1.0):
                nbytes = list(sizes)
                want = o.build_buckets(nbytes, cap_mb)
                n = len(nbytes)
                spans = bucket_spans(nbytes[::-1], int(cap_mb * 1024 * 1024))
                assert [[n - 1 - j for j in range(a, b)] for a, b in spans] == want, (sizes, cap_mb)


def test_two_shot_shares_partition_the_extent():
    """Every element of [lo, hi) belongs to exactly one rank's share, shares follow rank order,
    and every share but the last non-empty one is a whole number of align elements; checked
    element by element against ceil-sized blocks of the extent."""
    rng = np.random.default_rng(3)
    cases = [(0, 0, 4, 64), (5, 5, 3, 64), (0, 1, 8, 64), (10, 11, 1, 64), (0, 64 * 8, 8, 64),
             (0, 64 * 8 + 1, 8, 64), (7, 1000, 3, 64), (0, 100, 16, 1)]
    cases += [(int(lo), int(lo + n), int(w), int(a)) for lo, n, w, a in
              zip(rng.integers(0, 10**6, 200), rng.integers(0, 5000, 200), rng.integers(1, 17, 200),
                  rng.choice([1, 4, 64, 128], 200))]
    for lo, hi, world, align in cases:
        shares = comm.two_shot_shares(lo, hi, world, align)
        assert len(shares) == world
        # elements per share: the smallest multiple of align whose W copies cover the extent (searched)
        block = align
        while world * block < hi - lo:
            block += align
        owner = np.full(hi - lo, -1)
        for j, (a, b) in enumerate(shares):
            assert lo <= a <= b <= hi
            assert (owner[a - lo : b - lo] == -1).all()
            owner[a - lo : b - lo] = j
            if b < hi:
                assert (b - a) % align == 0
        want = (np.arange(hi - lo) // block) if hi > lo else np.zeros(0, int)
        assert (owner == want).all(), (lo, hi, world, align)
        assert [a for a, _ in shares] == sorted(a for a, _ in shares)


def test_clip_grad_runs_against_element_map():
    """The clipped parts of a run table address exactly the window's elements, each at its own
    gradient byte (0 = no gradient stays 0), in run order; the parts over every share of a
    two-shot extent put every element of every run back exactly once."""
    rng = np.random.default_rng(11)
    for trial in range(60):
        n_runs = int(rng.integers(0, 12))
        rows, pos = [], int(rng.integers(0, 50))
        for _ in range(n_runs):
            pos += int(rng.integers(0, 9))  # gaps between runs (bucket padding)
            n = int(rng.integers(0, 300))
            grad = 0 if rng.random() < 0.2 else int(rng.integers(1, 2**40)) * 256
            rows.append((pos, n, grad))
            pos += n
        runs = nat.grad_runs_array(rows)
        esize = int(rng.choice([2, 4]))

        def element_map(table):
            m = {}
            for off, n, g in table.tolist():
                for k in range(n):
                    assert off + k not in m
                    m[off + k] = 0 if g == 0 else g + k * esize
            return m

        full = element_map(runs)
        lo = int(rng.integers(0, pos + 2))
        hi = int(rng.integers(lo, pos + 3))
        part = comm.clip_grad_runs(runs, lo, hi, esize)
        assert part.dtype == nat.GRAD_RUN_DTYPE and (part["numel"] > 0).all()
        assert list(part["offset"]) == sorted(part["offset"])
        assert element_map(part) == {i: g for i, g in full.items() if lo <= i < hi}
        if full:
            xlo, xhi = min(full), max(full) + 1
            world = int(rng.integers(1, 9))
            merged: dict[int, int] = {}
            for a, b in comm.two_shot_shares(xlo, xhi, world, 64):
                got = element_map(comm.clip_grad_runs(runs, a, b, esize))
                assert not set(got) & set(merged)
                merged.update(got)
            assert merged == full


def test_interleave_spans_covers_each_span_in_round_robin_chunks():
    """Chunks copy exactly the bytes of the spans (each source byte to its own destination byte),
    none longer than the chunk size, ordered round-robin across the spans."""
    rng = np.random.default_rng(5)
    for trial in range(80):
        ses, des = int(rng.choice([1, 2, 4])), int(rng.choice([1, 2, 4]))
        chunk = int(rng.choice([1, 8, 64, 1000]))
        spans = [(int(rng.integers(1, 2**30)) * 8, int(rng.integers(1, 2**30)) * 8, int(rng.integers(0, 700)))
                 for _ in range(int(rng.integers(0, 6)))]
        out = comm.interleave_spans(spans, ses, des, chunk)
        step = max(1, chunk // ses)
        assert all(0 < n <= step for _, _, n in out)
        want = {(s + k * ses, d + k * des) for s, d, n in spans for k in range(n)}
        got = [(s + k * ses, d + k * des) for s, d, n in out for k in range(n)]
        assert len(got) == len(set(got)) and set(got) == want
        # round-robin: (chunk index, span index) of the output chunks increases lexicographically
        order = []
        for s, d, n in out:
            j = next(j for j, (s0, d0, n0) in enumerate(spans) if s0 <= s < s0 + n0 * ses and d - d0 == (s - s0) // ses * des)
            order.append(((s - spans[j][0]) // ses // step, j))
        assert order == sorted(order) and len(set(order)) == len(order)


def test_ddp_segments_bound_each_allocation():
    """Buckets grouped into allocations of at most ``limit`` bytes: in order, every bucket once at an
    aligned offset, no segment over the limit, a new segment only when the next bucket would not
    fit; one allocation without a limit; a bucket larger than the limit refused."""
    from minidist.ddp import _Bucket, _segments

    rng = np.random.default_rng(9)
    for trial in range(200):
        n = int(rng.integers(1, 30))
        numels = [int(x) for x in rng.integers(1, 5000, n)]
        buckets = [_Bucket(k, [nn.Parameter(torch.empty(m, device="meta"))]) for k, m in enumerate(numels)]
        align, esize = int(rng.choice([64, 128])), int(rng.choice([2, 4]))
        limit = int(rng.integers(max(numels) * esize, 4 * 5000 * esize + 1))
        segs = _segments(buckets, align, esize, limit)
        assert [b for seg in segs for b, _ in seg] == buckets
        for k, seg in enumerate(segs):
            assert seg and seg[0][1] == 0
            assert all(off % align == 0 for _, off in seg)
            assert all(o2 >= o1 + b1.numel for (b1, o1), (_, o2) in zip(seg, seg[1:]))
            last, off = seg[-1]
            assert (off + last.numel) * esize <= limit
            if k + 1 < len(segs):  # the next segment's first bucket did not fit here
                nxt = segs[k + 1][0][0]
                padded_end = off + -(-last.numel // align) * align
                assert (padded_end + nxt.numel) * esize > limit
        assert len(_segments(buckets, align, esize, None)) == 1
        with pytest.raises(ValueError, match="bucket_cap_mb"):
            _segments(buckets, align, esize, max(numels) * esize - 1)


def test_fsdp_ipc_segments_bound_each_allocation():
    """FSDP's units over an IpcGroup: in order, each at an aligned offset of its segment's two buffers,
    no buffer past ``segment_bytes``, a new segment only when the next unit would not fit; a unit
    exactly ``segment_bytes`` long fits alone; one larger is refused with the size it needs."""
    from types import SimpleNamespace

    from minidist.fsdp import _ARENA_ALIGN_ELEMS, _attach_ipc_rows

    class _Rows:  # IpcGroup.zeros / row_addresses, on the CPU
        def __init__(self, limit):
            self.segment_bytes, self.sizes = limit, []

        def zeros(self, numel, dtype):
            self.sizes.append(numel * torch.empty((), dtype=dtype).element_size())
            return torch.zeros(numel, dtype=dtype)

        def row_addresses(self, row):
            return [row.data_ptr(), row.data_ptr() + (1 << 40)]

    rng = np.random.default_rng(11)
    for trial in range(200):
        W, dtype = int(rng.integers(1, 9)), [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]
        es = 4 if dtype == torch.float32 else 2
        units = []
        for k in range(int(rng.integers(1, 12))):
            shard = int(rng.integers(0, 3000))
            units.append(SimpleNamespace(name=f"u{k}", padded_numel=shard * W, shard_numel=shard))
        need = max(u.padded_numel for u in units) * es
        limit = need if trial % 5 == 0 else int(rng.integers(max(need, 1), 3 * need + 2))
        group = _Rows(limit)
        rows = _attach_ipc_rows(units, group, dtype)
        assert len(group.sizes) == 2 * len(rows) and max(group.sizes) <= limit
        segs = [[u for u in units if u.segment == s] for s in range(len(rows))]
        assert [u for seg in segs for u in seg] == units
        for s, seg in enumerate(segs):
            assert seg[0].arena_offset == 0 and all(u.arena_offset % _ARENA_ALIGN_ELEMS == 0 for u in seg)
            assert all(u._ipc.grads.numel() == u.padded_numel and u._ipc.shard.numel() == u.shard_numel for u in seg)
            assert all(u._ipc.grad_ptrs[1] - u._ipc.grad_ptrs[0] == 1 << 40 for u in seg)
            if s + 1 < len(segs):  # the next segment's first unit did not fit in this one
                end = seg[-1].arena_offset + -(-seg[-1].padded_numel // _ARENA_ALIGN_ELEMS) * _ARENA_ALIGN_ELEMS
                assert (end + segs[s + 1][0].padded_numel) * es > limit
        if need:
            with pytest.raises(ValueError, match=f"needs {need} bytes of gradient rows, more than the group's "
                                                 f"segment_bytes \\({need - 1}\\)"):
                _attach_ipc_rows(units, _Rows(need - 1), dtype)


def test_ipc_group_checks_its_algorithm():
    with pytest.raises(ValueError, match="algorithm"):
        comm.IpcGroup(None, "cpu", algorithm="ring")
    for bad in (0, -1, 1 << 31):
        with pytest.raises(ValueError, match="segment_bytes"):
            comm.IpcGroup(None, "cpu", segment_bytes=bad)


def test_ddp_refuses_graph_capture_over_an_ipc_group(tmp_path):
    """An IpcGroup's collectives wait on the host for the peers: no graph can hold them, so DDP
    refuses capture_graphs over one before anything is allocated (a one-rank gloo group here)."""
    import torch.distributed as dist

    dist.init_process_group("gloo", init_method=f"file://{tmp_path / 'store'}", rank=0, world_size=1)
    try:
        group = comm.IpcGroup(dist.group.WORLD, "cpu")
        assert "two_shot" not in repr(group) and group.plans_reductions and not group.symmetric_targets
        with pytest.raises(ValueError, match="not an IpcGroup"):
            DistributedDataParallel(nn.Linear(2, 2), process_group=group, capture_graphs=True)
    finally:
        dist.destroy_process_group()


def test_fsdp_unit_batch_is_checked():
    """unit_batch must be a positive int (rejected before any work)."""
    from minidist import FSDP

    for bad in (0, -1, 2.0):
        with pytest.raises(ValueError, match="positive int"):
            FSDP(nn.Linear(2, 2), unit_batch=bad)


def _broadcast_worker(rank: int, store: str, out_dir: str) -> None:
    import os

    import torch.distributed as dist

    from minidist.ddp import _broadcasts_buffer

    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=2)
    try:
        def module():
            m = nn.Linear(3, 2)
            with torch.no_grad():
                for p in m.parameters():
                    p.fill_(10 + rank)
            m.register_buffer("f", torch.full((2,), 20.0 + rank))
            m.register_buffer("i", torch.full((2,), 30 + rank, dtype=torch.int64))
            m.register_buffer("u", torch.full((2,), 40 + rank, dtype=torch.uint8))
            return m

        out = {}
        sub = dist.new_group([0, 1])
        for tag, group, src, flt in (("ddp_default", None, 1, _broadcasts_buffer),
                                     ("ddp_sub", sub, 1, _broadcasts_buffer),
                                     ("fsdp_sub", sub, 0, None)):
            m = module()
            comm.broadcast_module_state(m, group, src, buffer_filter=flt)
            out[tag] = np.array([m.weight[0, 0].item(), m.bias[0].item(), m.f[0].item(), m.i[0].item(), m.u[0].item()])
        np.savez(os.path.join(out_dir, f"bcast_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


def test_module_state_broadcast_rules(tmp_path):
    """The construction-time sync over a real two-rank gloo group: DDP broadcasts parameters and
    floating-point / int32 / int64 / bool buffers from group rank ``src`` (from rank 0 on the
    default group, whatever ``src``), ddp.py:160-173; FSDP every parameter and buffer from group
    rank 0, fsdp.py:307-313."""
    import torch.multiprocessing as mp

    mp.spawn(_broadcast_worker, args=(str(tmp_path / "store"), str(tmp_path)), nprocs=2, join=True)
    for r in range(2):
        with np.load(tmp_path / f"bcast_r{r}.npz", allow_pickle=False) as d:
            assert list(d["ddp_default"]) == [10, 10, 20, 30, 40 + r]  # rank 0's; uint8 buffer untouched
            assert list(d["ddp_sub"]) == [11, 11, 21, 31, 40 + r]  # group rank 1's
            assert list(d["fsdp_sub"]) == [10, 10, 20, 30, 40]  # every buffer, group rank 0's


def test_out_of_scope_names_say_so():
    import minidist

    with pytest.raises(ImportError, match="does not provide"):
        minidist.ParallelMesh  # noqa: B018
    with pytest.raises(AttributeError):
        minidist.no_such_thing  # noqa: B018


def test_cpu_tensors_fail_loudly():
    model = nn.Linear(3, 3)
    ddp = DistributedDataParallel(model, process_group=comm.ResidentGroup(2, 0, "cpu"))
    for p in model.parameters():
        p.grad = torch.ones_like(p)
    with pytest.raises(RuntimeError, match="HIP kernels"):
        ddp.finish_gradient_sync()


def test_span_table_layout_is_the_c_struct():
    a = nat.spans_array([(1, 2, 3)])
    assert a.itemsize == 24 and a.tobytes() == np.array([1, 2, 3], dtype="<i8").tobytes()
    b = nat.pieces_array([(5, 6, 7)])
    assert b.itemsize == 24


# ---------------------------------------------------------------------------
# Device plans: building is host-only work
# ---------------------------------------------------------------------------


def _plan_header(buf: np.ndarray) -> dict:
    h = buf.view(np.int32)
    q = buf.view(np.int64)
    # PlanHeader (csrc/mdx_internal.h): 12 int32 fields, replicas[16] and out (uint64), then the
    # int64 offsets first_block, head, numel, a, b, pos, the total size and the hint offset.
    return {"magic": int(h[0]) & 0xFFFFFFFF, "kind": int(h[1]), "count": int(h[2]), "blocks": int(h[3]),
            "rank": int(h[10]), "off_first_block": int(q[23]), "bytes": int(q[29]), "off_hint": int(q[30])}


HINT_SHIFT = 6  # kHintShift: one run hint per 64 workgroups


def _plan_runs(buf: np.ndarray) -> tuple[np.ndarray, np.ndarray, dict]:
    h = _plan_header(buf)
    raw = buf.view(np.uint8)
    fb = raw[h["off_first_block"] : h["off_first_block"] + 4 * (h["count"] + 1)].view(np.int32)
    groups = (h["blocks"] + (1 << HINT_SHIFT) - 1) >> HINT_SHIFT
    hint = raw[h["off_hint"] : h["off_hint"] + 4 * (groups + 1)].view(np.int32)
    return fb, hint, h


def _hinted_run(fb: np.ndarray, hint: np.ndarray, blk: int) -> int:
    """The kernels' find_run_hinted, step for step: binary search in [hint[g], hint[g+1]]."""
    g = blk >> HINT_SHIFT
    lo, hi = int(hint[g]), int(hint[g + 1]) + 1
    while hi - lo > 1:
        mid = (lo + hi) >> 1
        if fb[mid] <= blk:
            lo = mid
        else:
            hi = mid
    return lo


def test_plan_spans_sizing_and_layout():
    L = nat.lib()
    # 150 spans (more than one kernel-argument batch), 16-byte aligned, 4096 fp32 each
    rows = [(0x10000000 + i * 65536, 0x40000000 + i * 65536, 4096) for i in range(150)]
    spans = nat.spans_array(rows)
    size = ctypes.c_int64(0)
    assert L.mdx_plan_spans(spans.ctypes.data, 150, 0, 0, None, ctypes.byref(size)) == nat.MDX_ESIZE
    need = size.value
    assert need > 150 * 36
    buf = np.zeros((need + 7) // 8, dtype=np.uint64)
    small = ctypes.c_int64(need - 8)
    assert L.mdx_plan_spans(spans.ctypes.data, 150, 0, 0, buf.ctypes.data, ctypes.byref(small)) == nat.MDX_ESIZE
    cap = ctypes.c_int64(buf.nbytes)
    assert L.mdx_plan_spans(spans.ctypes.data, 150, 0, 0, buf.ctypes.data, ctypes.byref(cap)) == 0
    h = _plan_header(buf)
    assert h["magic"] == 0x5058444D and h["kind"] == 1 and h["count"] == 150
    # one 16-byte fragment (4 fp32) per lane: 4096 fp32 = 16 one-wave workgroups per span
    assert h["blocks"] == 150 * 16
    assert h["bytes"] == need and h["off_hint"] + 4 * ((2400 >> HINT_SHIFT) + 2) <= need


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_plan_run_hints_resolve_every_workgroup(seed):
    """Every workgroup's hinted lookup lands on the run brute force assigns it.

    Run sizes mix one-workgroup runs (many runs per hint group) with runs of
    hundreds of workgroups (many groups per run)."""
    L = nat.lib()
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 400))
    sizes = np.where(rng.random(n) < 0.6, rng.integers(1, 1024, n), rng.integers(1, 1 << 20, n))
    rows, addr = [], 0x10000000
    for k in sizes:
        rows.append((addr, addr + (1 << 34), int(k)))
        addr += (int(k) * 4 + 255) // 256 * 256
    spans = nat.spans_array(rows)
    size = ctypes.c_int64(0)
    assert L.mdx_plan_spans(spans.ctypes.data, n, 0, 0, None, ctypes.byref(size)) == nat.MDX_ESIZE
    buf = np.zeros((size.value + 7) // 8, dtype=np.uint64)
    cap = ctypes.c_int64(buf.nbytes)
    assert L.mdx_plan_spans(spans.ctypes.data, n, 0, 0, buf.ctypes.data, ctypes.byref(cap)) == 0
    fb, hint, h = _plan_runs(buf)
    assert h["count"] == n and fb[0] == 0 and fb[-1] == h["blocks"] and np.all(np.diff(fb) >= 1)
    brute = np.searchsorted(fb, np.arange(h["blocks"]), side="right") - 1
    got = np.array([_hinted_run(fb, hint, b) for b in range(h["blocks"])])
    assert np.array_equal(got, brute)


@pytest.mark.parametrize("seed", [0, 1])
def test_plan_builders_on_random_tables(seed):
    """Every plan builder on random tables (fake device addresses, aligned or not, runs from empty to
    past the 2^26-element run limit, bad dtypes and worlds): each call returns a documented code; a
    size query followed by a build into exactly that many bytes succeeds, and one 8 bytes short is
    refused with MDX_ESIZE.  (The same tables also ran against a build with the host code under
    AddressSanitizer and UndefinedBehaviorSanitizer, clean.)"""
    import random

    L = nat.lib()
    rng = random.Random(seed)
    codes = {0, -2, -3, -4, -5}
    base = 1 << 40

    def ptr(aligned=True):
        return base + rng.randrange(1 << 30) * 256 + (0 if aligned else rng.choice([2, 4, 8, 12]))

    def numel():
        return rng.choice([0, 1, 63, 64, 4096, 100_003, (1 << 26) - 1, (1 << 26) + 5])

    def dt():
        return rng.choice([0, 1, 2, 0, 1, 2, 7])

    def check(fn, *args):
        size = ctypes.c_int64(0)
        rc = fn(*args, None, ctypes.byref(size))
        assert rc in codes, rc
        if rc != nat.MDX_ESIZE:
            return
        buf = np.zeros((size.value + 7) // 8 + 1, dtype=np.uint64)
        short = ctypes.c_int64(size.value - 8)
        assert fn(*args, buf.ctypes.data, ctypes.byref(short)) == nat.MDX_ESIZE
        exact = ctypes.c_int64(size.value)
        assert fn(*args, buf.ctypes.data, ctypes.byref(exact)) == 0

    for _ in range(400):
        kind = rng.randrange(4)
        k = rng.randrange(0, 60)
        if kind == 0:
            spans = np.array([(ptr(rng.random() > 0.2), ptr(rng.random() > 0.2), numel()) for _ in range(k)],
                             dtype=nat.SPAN_DTYPE)
            check(L.mdx_plan_spans, nat._ptr(spans), k, dt(), dt())
            continue
        if kind == 3:
            W = rng.choice([1, 2, 4, 8, 16])
            pieces = np.array([(ptr() if rng.random() > 0.1 else 0, rng.randrange(1 << 20) * 8,
                                rng.choice([0, 1, 5000, 1 << 20])) for _ in range(k)], dtype=nat.PIECE_DTYPE)
            outs = nat._ptrs([ptr() for _ in range(k)]) if k else None
            check(L.mdx_plan_reduce_scatter_share_multi, nat._ptr(pieces), outs, k,
                  nat._ptrs([ptr() for _ in range(W)]), W, rng.randrange(W), dt())
            continue
        W = rng.choice([0, 1, 2, 3, 8, 16, 17])
        reps = nat._ptrs([ptr() for _ in range(max(W, 1))])
        off, rows = 0, []
        for _ in range(k):
            m = numel() if rng.random() < 0.3 else rng.randrange(5000)
            rows.append((off, m, ptr(rng.random() > 0.2)))
            off += m + rng.choice([0, 128])
        out = ptr() if rng.random() < 0.7 else None
        if kind == 1:
            runs = np.array(rows, dtype=nat.GRAD_RUN_DTYPE)
            check(L.mdx_plan_allreduce_unpack, reps, W, dt(), nat._ptr(runs), k, out, dt())
        else:
            runs = np.array([(a, m, ptr(rng.random() > 0.2), g) for a, m, g in rows], dtype=nat.PACK_RUN_DTYPE)
            check(L.mdx_plan_pack_allreduce_unpack, reps, W, rng.randrange(max(W, 1)), dt(), nat._ptr(runs), k,
                  out, dt(), ctypes.c_float(0.125))


def test_plan_allreduce_unpack_builds_and_rejects_overlap():
    L = nat.lib()
    reps = (ctypes.c_void_p * 8)(*[0x100000000 + r * (1 << 24) for r in range(8)])
    runs = nat.grad_runs_array([(i * 1024, 1000, 0x900000000 + i * 8192) for i in range(100)])
    size = ctypes.c_int64(0)
    rc = L.mdx_plan_allreduce_unpack(reps, 8, 0, runs.ctypes.data, 100, reps[0], 0, None, ctypes.byref(size))
    assert rc == nat.MDX_ESIZE
    buf = np.zeros((size.value + 7) // 8, dtype=np.uint64)
    cap = ctypes.c_int64(buf.nbytes)
    assert L.mdx_plan_allreduce_unpack(reps, 8, 0, runs.ctypes.data, 100, reps[0], 0, buf.ctypes.data, ctypes.byref(cap)) == 0
    h = _plan_header(buf)
    assert h["kind"] == 2 and h["count"] == 100 and h["blocks"] == 100 * 4  # 250 fragments per run, 64 per one-wave workgroup
    bad = nat.grad_runs_array([(0, 16, 0x100000000 + 8)])  # gradient inside replica 0
    assert L.mdx_plan_allreduce_unpack(reps, 8, 0, bad.ctypes.data, 1, reps[0], 0, buf.ctypes.data, ctypes.byref(cap)) == -4


def test_planned_launch_rejects_bad_plans_before_launch():
    L = nat.lib()
    junk = np.zeros(64, dtype=np.uint64)
    assert L.mdx_pack_planned(junk.ctypes.data, junk.ctypes.data, 1.0, 0, None, None) == -1  # no magic
    assert L.mdx_pack_planned(None, None, 1.0, 0, None, None) == -1
    spans = nat.spans_array([(0, 0x40000000, 64)])  # a zero-source span
    size = ctypes.c_int64(junk.nbytes)
    assert L.mdx_plan_spans(spans.ctypes.data, 1, 0, 0, junk.ctypes.data, ctypes.byref(size)) == 0
    assert L.mdx_unpack_planned(junk.ctypes.data, junk.ctypes.data, 1.0, None, None) == -1  # unpack needs sources
    assert L.mdx_allreduce_unpack_planned(junk.ctypes.data, junk.ctypes.data, 1.0, None, None) == -1  # wrong kind


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits (code 2) with a message that says so,
    before anything touches a GPU."""
    import subprocess
    import sys

    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr or "single" in res.stderr
    assert res.stdout.strip() == ""


def test_host_grad_ptrs_helper_matches_python():
    """The native gather of gradient addresses (minidist._hostptrs) equals p.grad.data_ptr() per
    parameter, 0 where .grad is None, for Parameters and plain tensors, and rejects non-tensors."""
    import torch

    from minidist import _hostptrs

    ps = [torch.nn.Parameter(torch.zeros(i + 1)) for i in range(40)]
    for i, p in enumerate(ps):
        if i % 3:
            p.grad = torch.randn(i + 1)
    views = torch.zeros(100)
    ps[5].grad = views[7:13]  # a view: the address of its first element
    want = [0 if p.grad is None else p.grad.data_ptr() for p in ps]
    assert _hostptrs.grad_ptrs(ps) == want
    assert _hostptrs.grad_ptrs([]) == []
    with pytest.raises(TypeError):
        _hostptrs.grad_ptrs([ps[0], 3])
    with pytest.raises(TypeError):
        _hostptrs.grad_ptrs(tuple(ps))
    # torch's own error for a gradient without storage comes back as a Python error, as it does from
    # p.grad.data_ptr(), instead of ending the process
    ps[2].grad = torch.zeros(3).to_sparse()
    with pytest.raises(RuntimeError, match="storage"):
        _hostptrs.grad_ptrs(ps)


def test_new_entry_points_check_arguments_before_any_launch():
    """The multi-unit share, its plan, the allocation-free launch, the IPC calls and the host-flag
    address refuse bad arguments with their MDX_E* codes before touching a device."""
    L = nat.lib()
    P = ctypes.c_void_p
    pieces = nat.pieces_array([(4096, 0, 8), (0, 8, 8)])
    outs = (ctypes.c_void_p * 2)(1 << 20, (1 << 20) + 32)
    peers = (ctypes.c_void_p * 2)(1 << 24, 1 << 25)
    args = (pieces.ctypes.data, outs, 2, peers)
    assert L.mdx_reduce_scatter_share_multi(*args, 2, 0, 7, 0, 1, 0, 0, 1.0, None, None) == -2  # dtype
    assert L.mdx_reduce_scatter_share_multi(*args, 2, 2, 0, 0, 1, 0, 0, 1.0, None, None) == -3  # rank
    bad_outs = (ctypes.c_void_p * 2)(1 << 20, 0)
    assert L.mdx_reduce_scatter_share_multi(pieces.ctypes.data, bad_outs, 2, peers, 2, 0, 0, 0, 1, 0, 0, 1.0, None,
                                            None) == -1  # NULL destination
    over_row = (ctypes.c_void_p * 2)(1 << 20, (1 << 25) + 8)
    assert L.mdx_reduce_scatter_share_multi(pieces.ctypes.data, over_row, 2, peers, 2, 0, 0, 0, 1, 0, 0, 1.0, None,
                                            None) == -4  # a destination over peer 1's row
    over_each_other = (ctypes.c_void_p * 2)(1 << 20, (1 << 20) + 16)
    assert L.mdx_reduce_scatter_share_multi(pieces.ctypes.data, over_each_other, 2, peers, 2, 0, 0, 0, 1, 0, 0, 1.0,
                                            None, None) == -4
    assert L.mdx_reduce_scatter_share_multi(None, None, 0, peers, 2, 0, 0, 0, 1, 0, 0, 1.0, None, None) == 0
    size = ctypes.c_int64(0)
    assert L.mdx_plan_reduce_scatter_share_multi(*args, 2, 0, 9, None, ctypes.byref(size)) == -2
    assert L.mdx_plan_reduce_scatter_share_multi(*args, 2, 0, 1, None, ctypes.byref(size)) == nat.MDX_ESIZE
    assert size.value > 0
    assert L.mdx_reduce_scatter_share_multi_planned(None, None, 1, 0, 1.0, None, None) == -1
    assert L.mdx_pack_allreduce_unpack_planned_noalloc(None, 1.0, None, None, None) == -1
    junk = np.zeros(64, dtype=np.uint64)  # not a plan
    assert L.mdx_pack_allreduce_unpack_planned_noalloc(junk.ctypes.data, 1.0, None, None, None) == -1
    assert L.mdx_ipc_export(None, None) == -1
    assert L.mdx_ipc_open(None, None) == -1
    assert L.mdx_ipc_close(None) == -1
    h = nat.IpcHandle()
    h.alloc_bytes = 1 << 31  # a shared allocation of 2 GiB or more is refused
    assert L.mdx_ipc_open(ctypes.byref(h), ctypes.byref(P())) == nat.MDX_ESIZE
    assert L.mdx_host_device_address(None, ctypes.byref(P())) == -1
    assert "256 KiB" in nat.strerror(nat.MDX_ESCRATCH)


def test_noalloc_rejects_oversize_plan_and_aliased_flags():
    """A plan beyond MDX_NOALLOC_SCRATCH_BYTES is refused with MDX_ESCRATCH, and found_inf ==
    clear_flag with MDX_EALIAS, both before any HIP call: the addresses here are made up and
    never touched (no GPU in this process).  The Python copy of the limit is the header's."""
    limit = re.search(r"#define MDX_NOALLOC_SCRATCH_BYTES \((\d+) \* (\d+)\)", HEADER.read_text())
    assert limit is not None and int(limit[1]) * int(limit[2]) == nat.NOALLOC_SCRATCH_BYTES
    base = 1 << 40
    reps = [base + r * (1 << 30) for r in range(2)]

    def plan(n_runs):
        runs = nat.pack_runs_array([(4 * k, 1, base + (1 << 36) + 64 * k, base + (1 << 37) + 64 * k)
                                    for k in range(n_runs)])
        size = ctypes.c_int64(0)
        rc = nat.lib().mdx_plan_pack_allreduce_unpack(nat._ptrs(reps), 2, 0, nat.MDX_F32, nat._ptr(runs), n_runs,
                                                      base + (1 << 38), nat.MDX_F32, 0.5, None, ctypes.byref(size))
        assert rc == nat.MDX_ESIZE
        host = np.zeros((size.value + 7) // 8, dtype=np.uint64)
        cap = ctypes.c_int64(host.nbytes)
        nat.check(nat.lib().mdx_plan_pack_allreduce_unpack(nat._ptrs(reps), 2, 0, nat.MDX_F32, nat._ptr(runs),
                                                           n_runs, base + (1 << 38), nat.MDX_F32, 0.5,
                                                           host.ctypes.data, ctypes.byref(cap)), "plan")
        return host, size.value

    host, nbytes = plan(9000)  # about 32 bytes per run: well past 256 KiB
    assert nbytes > nat.NOALLOC_SCRATCH_BYTES
    flag, other = ctypes.c_void_p(base + (1 << 39)), ctypes.c_void_p(base + (1 << 39) + 256)
    L = nat.lib()
    rc = L.mdx_pack_allreduce_unpack_planned_noalloc(host.ctypes.data, 1.0, flag, other, None)
    assert rc == nat.MDX_ESCRATCH, nat.strerror(rc)
    assert "256 KiB" in nat.strerror(rc)
    small, nbytes = plan(16)
    assert nbytes <= nat.NOALLOC_SCRATCH_BYTES
    for h in (host, small):
        rc = L.mdx_pack_allreduce_unpack_planned_noalloc(h.ctypes.data, 1.0, flag, flag, None)
        assert rc == nat.MDX_EALIAS, nat.strerror(rc)


def test_cfg1_plan_fits_the_allocation_free_buffer():
    """The fused plan of GPT-2-124M's 148 gradients in 18 buckets (the headline step) is well under
    MDX_NOALLOC_SCRATCH_BYTES; the plan is built on the host from addresses alone."""
    specs = w.gpt_specs(**w.GPT2_SMALL)
    layout = o.build_buckets([s.nbytes for s in specs[::-1]], 25.0)
    rows, off = [], 0
    base = 1 << 40
    rev = specs[::-1]
    for idx in layout:
        for i in idx:
            n = rev[i].numel
            rows.append((off, n, base + (1 << 36) + 4 * off, base + (1 << 37) + 4 * off))
            off += n
        off = (off + 63) // 64 * 64
    runs = nat.pack_runs_array(rows)
    reps = (ctypes.c_void_p * 8)(*[base + r * (1 << 31) for r in range(8)])
    size = ctypes.c_int64(0)
    rc = nat.lib().mdx_plan_pack_allreduce_unpack(reps, 8, 0, nat.MDX_F32, runs.ctypes.data, len(rows),
                                                  ctypes.c_void_p(base + (1 << 38)), nat.MDX_F32, 0.125, None,
                                                  ctypes.byref(size))
    assert rc == nat.MDX_ESIZE
    assert 8 * 1024 < size.value < nat.NOALLOC_SCRATCH_BYTES // 4
    print(f"cfg1 fused plan: {size.value} bytes")
