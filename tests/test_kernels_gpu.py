"""Kernel parity on the GPU: every libmdx entry point vs the oracle, bit for bit.

Each test builds seeded inputs on the host, runs the entry point through the C
ABI (minidist._native is a ctypes shim over include/mdx.h) on ``cuda:0``,
copies the result back and compares it with oracle/gradpath.py.  NaN payloads
are not compared (every NaN equals every NaN); every other bit is.  Buffers
carry sentinel gaps so that a write outside a span shows up.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from conftest import bf16_bits_torch, first_mismatch, load_golden, same_bits
from minidist import _native as nat
from oracle import gradpath as o

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
SENTINEL_F32 = np.float32(-7.25)
SENTINEL_BF16 = np.uint16(0x4242)
SENTINEL = {o.F32: SENTINEL_F32, o.BF16: SENTINEL_BF16, o.F16: np.float16(-3.5)}
CODE = {o.F32: nat.MDX_F32, o.BF16: nat.MDX_BF16, o.F16: nat.MDX_F16}
DTYPES = [o.F32, o.BF16, o.F16]


def code(dt: str) -> int:
    return CODE[dt]


def to_dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).to(DEV).view(torch.bfloat16)
    if a.dtype == np.float16:
        return torch.from_numpy(a.copy()).to(DEV)
    return torch.from_numpy(a.astype(np.float32)).to(DEV)


def to_host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().astype(np.uint16)
    return t.numpy().copy()


def empty_dev(n: int, dt: str) -> torch.Tensor:
    if dt == o.BF16:
        return torch.full((n,), int(SENTINEL_BF16.view(np.int16)), dtype=torch.int16, device=DEV).view(torch.bfloat16)
    if dt == o.F16:
        return torch.full((n,), float(SENTINEL[o.F16]), dtype=torch.float16, device=DEV)
    return torch.full((n,), float(SENTINEL_F32), dtype=torch.float32, device=DEV)


def stream() -> int:
    return torch.cuda.current_stream(DEV).cuda_stream


def values(rng, n: int, dt: str, specials: bool = True, scale: float = 1.0) -> np.ndarray:
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    if specials and n:
        if dt == o.F16:  # fp16's own edges: subnormals, the largest finite value, the smallest normal
            pool = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 6e-8, -1e-5, 65504.0, -60000.0, 6.1035e-5],
                            np.float32)
        else:
            pool = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-40, 3.4e38, -3.39e38, 1.2e-38],
                            np.float32)
        idx = rng.integers(0, n, max(1, n // 50))
        x[idx] = pool[rng.integers(0, len(pool), idx.size)]
    return o.from_f32(x, dt)


def esize(dt: str) -> int:
    return o.itemsize(dt)


# ---------------------------------------------------------------------------
# pack / unpack / unscale (the copy kernel)
# ---------------------------------------------------------------------------

SIZES = [0, 1, 2, 3, 7, 8, 15, 16, 17, 63, 64, 65, 255, 256, 1000, 4095, 4096, 4097, 12345, 70001]


def _span_case(rng, sdt, ddt, null_every=0, n_spans=None):
    """Random spans: misaligned sources (sub-views), misaligned packed destinations."""
    n_spans = n_spans or len(SIZES)
    sizes = [SIZES[i % len(SIZES)] for i in range(n_spans)]
    rng.shuffle(sizes)
    srcs, rows_host = [], []
    dst_off, offs = 0, []
    for k, n in enumerate(sizes):
        shift = int(rng.integers(0, 8))
        host = values(rng, n + shift, sdt)
        t = to_dev(host)
        null = null_every and k % null_every == 0
        srcs.append((t, shift, host[shift:], null))
        dst_off += int(rng.integers(0, 4))  # gap keeps a sentinel
        offs.append(dst_off)
        dst_off += n
    dst = empty_dev(dst_off + 5, ddt)
    rows = []
    for (t, shift, host, null), off, n in zip(srcs, offs, sizes, strict=True):
        src_ptr = 0 if null else t.data_ptr() + shift * esize(sdt)
        rows.append((src_ptr, dst.data_ptr() + off * esize(ddt), n))
        rows_host.append((None if null else host, off, n))
    return srcs, dst, rows, rows_host


@pytest.mark.parametrize("sdt", DTYPES)
@pytest.mark.parametrize("ddt", DTYPES)
@pytest.mark.parametrize("scale,divide", [(1.0, False), (1.0 / 8, False), (1.0 / 3, False), (3.0, True), (8.0, True)])
def test_pack_matches_oracle(rng, sdt, ddt, scale, divide):
    srcs, dst, rows, rows_host = _span_case(rng, sdt, ddt, null_every=5)
    nat.pack(nat.spans_array(rows), code(sdt), code(ddt), nat.f32(scale), divide, stream())
    got = to_host(dst)
    want = np.full(got.shape, SENTINEL[ddt], dtype=got.dtype)
    for host, off, n in rows_host:
        v = o.zeros(n, ddt) if host is None else o.convert(host, sdt, ddt)
        if scale != 1.0:
            v = o.div_scalar(v, ddt, int(scale)) if divide else o.mul_scalar(v, ddt, scale)
        want[off : off + n] = v
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize(
    "bdt,gdt",
    [(o.F32, o.F32), (o.BF16, o.BF16), (o.F32, o.BF16), (o.F16, o.F16), (o.F32, o.F16), (o.F16, o.F32),
     (o.BF16, o.F16)],
)
@pytest.mark.parametrize("inv_scale", [1.0, 2.0**-16, 1.0 / 3])
def test_unpack_unscale_found_inf_matches_oracle(rng, bdt, gdt, inv_scale):
    n_total = sum(SIZES) + 64
    bucket_host = values(rng, n_total, bdt, specials=False, scale=1e3)
    bucket = to_dev(bucket_host)
    grads, rows, expect = [], [], []
    off = 0
    for n in SIZES:
        off += int(rng.integers(0, 3))
        g = empty_dev(n + 3, gdt)
        shift = int(rng.integers(0, 3))
        grads.append(g)
        rows.append((bucket.data_ptr() + off * esize(bdt), g.data_ptr() + shift * esize(gdt), n))
        expect.append((g, shift, bucket_host[off : off + n]))
        off += n
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nat.unpack(nat.spans_array(rows), code(bdt), code(gdt), nat.f32(inv_scale), flag.data_ptr(), stream())
    any_bad = False
    for g, shift, src in expect:
        v = o.convert(src, bdt, gdt)
        if inv_scale != 1.0:
            v = o.mul_scalar(v, gdt, inv_scale)
        any_bad |= bool((~o.isfinite(v, gdt)).any())
        got = to_host(g)
        assert same_bits(got[shift : shift + len(src)], v), first_mismatch(got[shift : shift + len(src)], v)
        sent = got[:shift].tolist() + got[shift + len(src) :].tolist()
        assert all(s == SENTINEL[gdt] for s in sent)
    assert bool(flag.item()) == any_bad


def test_unpack_flags_only_when_nonfinite(rng):
    clean = to_dev(values(rng, 5000, o.F32, specials=False))
    out = empty_dev(5000, o.F32)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nat.unpack(nat.spans_array([(clean.data_ptr(), out.data_ptr(), 5000)]), 0, 0, 1.0, flag.data_ptr(), stream())
    assert flag.item() == 0
    for bad in (np.inf, -np.inf, np.nan):
        h = values(rng, 5000, o.F32, specials=False)
        h[4321] = bad
        t = to_dev(h)
        nat.unpack(nat.spans_array([(t.data_ptr(), out.data_ptr(), 5000)]), 0, 0, 1.0, flag.data_ptr(), stream())
        assert flag.item() == 1
        flag.zero_()
    # fp32 value finite, bf16 result overflows: counts
    h = np.full(64, 3.40e38, np.float32)
    t = to_dev(h)
    ob = empty_dev(64, o.BF16)
    nat.unpack(nat.spans_array([(t.data_ptr(), ob.data_ptr(), 64)]), 0, 1, 1.0, flag.data_ptr(), stream())
    assert flag.item() == 1
    # fp32 value finite, fp16 result overflows (65520 rounds to inf): counts; 65519 does not
    flag.zero_()
    oh = empty_dev(64, o.F16)
    for v, want in ((65519.0, 0), (65520.0, 1)):
        t = to_dev(np.full(64, v, np.float32))
        nat.unpack(nat.spans_array([(t.data_ptr(), oh.data_ptr(), 64)]), 0, nat.MDX_F16, 1.0, flag.data_ptr(),
                   stream())
        assert flag.item() == want, v


@pytest.mark.parametrize("dt", DTYPES)
def test_unscale_in_place_matches_oracle(rng, dt):
    hosts = [values(rng, n, dt, scale=2.0**10 if dt == o.F16 else 2.0**16) for n in SIZES]
    devs = [to_dev(h) for h in hosts]
    rows = [(t.data_ptr(), t.data_ptr(), t.numel()) for t in devs]
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nat.unscale_found_inf(nat.spans_array(rows), code(dt), nat.f32(2.0**-16), flag.data_ptr(), stream())
    want, found = o.unscale_found_inf(hosts, [dt] * len(hosts), 2.0**-16)
    for t, w in zip(devs, want, strict=True):
        assert same_bits(to_host(t), w), first_mismatch(to_host(t), w)
    assert bool(flag.item()) == found


# ---------------------------------------------------------------------------
# W-way all-reduce
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("W", [1, 2, 3, 4, 5, 8, 16])
def test_allreduce_sum_matches_oracle(rng, dt, W):
    runs = [(3, 1), (17, 4096), (5000, 3), (70000, 12345)]  # (offset, numel), increasing
    extent = runs[-1][0] + runs[-1][1] + 9
    reps_host = [values(rng, extent, dt, scale=1e-2) for _ in range(W)]
    reps = [to_dev(h) for h in reps_host]
    out = empty_dev(extent, dt)
    nat.allreduce_sum(
        [r.data_ptr() for r in reps], code(dt), [a for a, _ in runs], [n for _, n in runs], out.data_ptr(), stream()
    )
    got = to_host(out)
    want = np.full(extent, SENTINEL[dt], dtype=got.dtype)
    for a, n in runs:
        want[a : a + n] = o.allreduce_sum([h[a : a + n] for h in reps_host], dt)
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("W,k", [(8, 0), (8, 5), (4, 3)])
def test_allreduce_in_place_on_one_replica(rng, W, k):
    n = 1 << 20
    reps_host = [values(rng, n, o.F32, specials=False) for _ in range(W)]
    reps = [to_dev(h) for h in reps_host]
    nat.allreduce_sum([r.data_ptr() for r in reps], nat.MDX_F32, [0], [n], reps[k].data_ptr(), stream())
    want = o.allreduce_sum(reps_host, o.F32)
    assert same_bits(to_host(reps[k]), want)
    for r in range(W):
        if r != k:
            assert same_bits(to_host(reps[r]), reps_host[r])


def test_allreduce_full_bucket_exact_sum_property(rng):
    """A 25 MiB fp32 bucket, W = 8: short-mantissa inputs make the exact sum the answer."""
    W, n = 8, 25 * 1024 * 1024 // 4
    ks = rng.integers(-(2**16), 2**16, (W, n), dtype=np.int64)
    reps = [to_dev((k * 2.0**-10).astype(np.float32)) for k in ks]
    out = torch.empty(n, dtype=torch.float32, device=DEV)
    nat.allreduce_sum([r.data_ptr() for r in reps], nat.MDX_F32, [0], [n], out.data_ptr(), stream())
    want = (ks.sum(axis=0) * 2.0**-10).astype(np.float32)
    assert np.array_equal(to_host(out), want)


@pytest.mark.parametrize(
    "bdt,gdt",
    [(o.F32, o.F32), (o.BF16, o.BF16), (o.F32, o.BF16), (o.BF16, o.F32), (o.F16, o.F16), (o.F32, o.F16),
     (o.F16, o.F32), (o.BF16, o.F16), (o.F16, o.BF16)],
)
@pytest.mark.parametrize("W", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("inv_scale,write_out", [(1.0, True), (2.0**-16, True), (1.0 / 3, False)])
def test_allreduce_unpack_matches_oracle(rng, bdt, gdt, W, inv_scale, write_out):
    """Fused SUM + unpack + unscale + found-inf == allreduce_sum, unpack (copy_), mul_, isfinite."""
    numels = [1, 7, 64, 4096, 3, 12345, 256, 5]
    offs, off = [], 5
    for n in numels:
        offs.append(off)
        off += n + int(rng.integers(0, 3))
    extent = off + 4
    reps_host = [values(rng, extent, bdt, scale=1e3) for _ in range(W)]
    reps = [to_dev(h) for h in reps_host]
    rank = W // 2
    grads = [empty_dev(n + 2, gdt) for n in numels]
    shifts = [int(rng.integers(0, 3)) for _ in numels]
    runs = nat.grad_runs_array(
        [(a, n, g.data_ptr() + s * esize(gdt)) for a, n, g, s in zip(offs, numels, grads, shifts, strict=True)]
    )
    before = to_host(reps[rank])
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nat.allreduce_unpack(
        [r.data_ptr() for r in reps], code(bdt), runs, reps[rank].data_ptr() if write_out else None, code(gdt),
        nat.f32(inv_scale), flag.data_ptr(), stream(),
    )
    any_bad = False
    want_out = before.copy()
    for a, n, g, s in zip(offs, numels, grads, shifts, strict=True):
        acc = o.allreduce_sum([h[a : a + n] for h in reps_host], bdt)
        want_out[a : a + n] = acc
        v = o.convert(acc, bdt, gdt)
        if inv_scale != 1.0:
            v = o.mul_scalar(v, gdt, inv_scale)
        any_bad |= bool((~o.isfinite(v, gdt)).any())
        got = to_host(g)
        assert same_bits(got[s : s + n], v), first_mismatch(got[s : s + n], v)
        sent = np.concatenate([got[:s], got[s + n :]])
        assert np.all(sent == SENTINEL[gdt])
    got_out = to_host(reps[rank])
    assert same_bits(got_out, want_out if write_out else before), first_mismatch(got_out, want_out)
    for r in range(W):
        if r != rank:
            assert same_bits(to_host(reps[r]), reps_host[r])
    assert bool(flag.item()) == any_bad


@pytest.mark.parametrize("wide", [False, True])
def test_allreduce_unpack_plan_larger_than_one_dispatch(wide):
    """The two-dispatch pipeline's planned all-reduce + unpack over more than 2^22 workgroups, sent
    as several dispatches: W = 8 fp32 contributions (256 elements per workgroup), or 8 bf16
    contributions widened, x 1/8 and summed into an fp32 bucket (512 per workgroup).  Every element
    is checked against the same IEEE ops in torch on the device: the rank-ordered sum, then the
    gradient converted and unscaled."""
    W, inv = 8, 2.0**-10
    per_block = 512 if wide else 256
    n = (1 << 22) * per_block + (1 << 18)
    wdt = torch.bfloat16 if wide else torch.float32
    gen = torch.Generator(device=DEV).manual_seed(91)
    reps = [torch.randn(n + 8, device=DEV, generator=gen).to(wdt) for _ in range(W)]
    out = torch.empty(n + 8, dtype=torch.float32, device=DEV)
    grad = torch.empty(n, dtype=wdt, device=DEV)
    runs = nat.grad_runs_array([(4, n, grad.data_ptr())])
    ptrs = [r.data_ptr() for r in reps]
    if wide:
        plan = nat.plan_allreduce_unpack_wide(ptrs, nat.MDX_BF16, runs, out.data_ptr(), nat.MDX_F32, nat.MDX_BF16,
                                              nat.f32(1.0 / W), DEV)
    else:
        plan = nat.plan_allreduce_unpack(ptrs, nat.MDX_F32, runs, out.data_ptr(), nat.MDX_F32, DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nat.allreduce_unpack_planned(plan, nat.f32(inv), flag.data_ptr(), stream())
    acc = None
    for r in reps:
        x = r[4 : 4 + n].float()
        x = x * (1.0 / W) if wide else x  # exact: a power of two on normal values
        acc = x if acc is None else acc + x
        del x
    assert torch.equal(out[4 : 4 + n], acc)
    want = (acc.to(wdt).float() * inv).to(wdt) if wide else acc * inv
    assert torch.equal(grad, want)
    assert flag.item() == 0


def test_allreduce_unpack_rejects_grad_overlapping_a_replica():
    reps = [torch.zeros(1024, device=DEV) for _ in range(2)]
    runs = nat.grad_runs_array([(0, 16, reps[1][4:].data_ptr())])  # inside the reduced extent
    with pytest.raises(RuntimeError, match="overlaps"):
        nat.allreduce_unpack([r.data_ptr() for r in reps], 0, runs, None, 0, 1.0, None, stream())


# ---------------------------------------------------------------------------
# reduce-scatter share
# ---------------------------------------------------------------------------


@pytest.mark.parametrize(
    "idt,rdt,sdt",
    [(o.BF16, o.F32, o.F32), (o.F32, o.F32, o.F32), (o.BF16, o.BF16, o.F32), (o.BF16, o.F32, o.BF16),
     (o.F32, o.BF16, o.BF16), (o.F16, o.F32, o.F32), (o.F16, o.F16, o.F32), (o.F16, o.F32, o.F16),
     (o.F16, o.F16, o.F16), (o.F32, o.F16, o.F32), (o.BF16, o.F16, o.BF16), (o.F16, o.BF16, o.F32)],
)
@pytest.mark.parametrize("W,rank", [(1, 0), (2, 1), (3, 2), (4, 0), (8, 5)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_reduce_scatter_share_matches_oracle(rng, idt, rdt, sdt, W, rank, accumulate):
    _share_case(rng, [7, 12, 5, 33, 640, 3, 4099, 1], idt, rdt, sdt, W, rank, accumulate)


@pytest.mark.parametrize("k", range(7))
@pytest.mark.parametrize("idt", [o.BF16, o.F32])
def test_reduce_scatter_share_piece_counts(rng, k, idt):
    """Rank 0's shard covers k whole parameters and part of one more: k + 1 pieces, across the
    one-piece, few-piece (up to 4) and full kernel-argument tables."""
    numels = [37 + 64 * i for i in range(k)]
    numels.append(sum(numels) + 4100 + 8 * k)
    _share_case(rng, numels, idt, o.F32, o.F32, 2, 0, k % 2 == 1)


@pytest.mark.parametrize("seed", range(40))
def test_reduce_scatter_share_fuzz(seed):
    """Seeded random shares: 1-10 parameters of 1-5000 elements, W in [2, 16], any rank, fp32 / bf16 /
    fp16 contributions into an fp32 shard, with or without accumulation -- shards of one piece, a
    few pieces or many, against the oracle."""
    r = np.random.default_rng(1000 + seed)
    W = int(r.integers(2, 17))
    rank = int(r.integers(0, W))
    numels = [int(x) for x in r.integers(1, 5000, int(r.integers(1, 11)))]
    idt = (o.F32, o.BF16, o.F16)[seed % 3]
    _share_case(r, numels, idt, o.F32, o.F32, W, rank, seed % 2 == 1)


def _share_case(rng, numels, idt, rdt, sdt, W, rank, accumulate):
    total = sum(numels)
    S = (total + W - 1) // W
    P = S * W
    grads = []
    for r in range(W):
        grads.append([None if (r + i) % 5 == 3 else values(rng, n, idt, scale=1e-3) for i, n in enumerate(numels)])
    # own pieces: straight from this rank's per-param tensors (as FSDP does)
    own_devs = [None if g is None else to_dev(g) for g in grads[rank]]
    lo, hi = rank * S, rank * S + S
    pieces, off, cursor = [], 0, lo
    for t, n in zip(own_devs, numels, strict=True):
        a, b = max(off, lo), min(off + n, hi)
        if a < b:
            ptr = 0 if t is None else t.data_ptr() + (a - off) * esize(idt)
            pieces.append((ptr, a - lo, b - a))
            cursor = b
        off += n
    if cursor < hi:
        pieces.append((0, cursor - lo, hi - cursor))
    flats = [o.fsdp_flatten(g, idt, numels, P, idt) for g in grads]
    peer_devs = [to_dev(f) for f in flats]
    peers = [peer_devs[r][lo:].data_ptr() for r in range(W)]
    prev_host = values(rng, S, sdt, specials=False, scale=1e-3)
    shard = to_dev(prev_host) if accumulate else empty_dev(S, sdt)
    nat.reduce_scatter_share(
        nat.pieces_array(pieces), peers, rank, code(idt), code(rdt), True, shard.data_ptr(), code(sdt),
        accumulate, 1.0, None, stream(),
    )
    want = o.fsdp_reduce_scatter_share(grads, idt, numels, rank, rdt, sdt, existing=prev_host if accumulate else None)
    got = to_host(shard)
    assert same_bits(got, want), first_mismatch(got, want)


# ---------------------------------------------------------------------------
# fp32 -> bf16 cast
# ---------------------------------------------------------------------------


def test_cast_structured_sweep():
    hi = np.arange(1 << 16, dtype=np.uint32) << np.uint32(16)
    lows = np.array(
        [0x0000, 0x0001, 0x3FFF, 0x7FFE, 0x7FFF, 0x8000, 0x8001, 0xBFFF, 0xFFFE, 0xFFFF, 0x1234, 0x9ABC],
        dtype=np.uint32,
    )
    x = (hi[:, None] | lows[None, :]).reshape(-1).view(np.float32)
    src = to_dev(x)
    dst = empty_dev(x.size, o.BF16)
    nat.cast_f32_bf16(src.data_ptr(), dst.data_ptr(), x.size, stream())
    got = to_host(dst)
    want = o.bf16_from_f32(x)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_cast_matches_golden_and_ties():
    d = load_golden("bf16_cast.npz")
    for x, want in ((d["x_bits"].view(np.float32), d["y_bits"]), o.bf16_tie_cases()):
        src = to_dev(np.ascontiguousarray(x))
        dst = empty_dev(x.size, o.BF16)
        nat.cast_f32_bf16(src.data_ptr(), dst.data_ptr(), x.size, stream())
        assert np.array_equal(to_host(dst), want), first_mismatch(to_host(dst), want)


def test_cast_exhaustive():
    """All 2^32 fp32 bit patterns, in 16 dispatches of 2^28, through mdx_cast_f32_bf16 against
    the oracle's rounding (bf16_bits_torch, evaluated on the device): every non-NaN input,
    ties, subnormals and overflow to inf included, and every NaN -> 0xFFFF."""
    chunk = 1 << 28
    for c in range(16):
        u = torch.arange(c * chunk, (c + 1) * chunk, dtype=torch.int64, device=DEV)
        x = (u - ((u >> 31) << 32)).to(torch.int32).view(torch.float32)
        dst = torch.empty(chunk, dtype=torch.int16, device=DEV)
        nat.cast_f32_bf16(x.data_ptr(), dst.data_ptr(), chunk, stream())
        got = dst.to(torch.int64) & 0xFFFF
        want = bf16_bits_torch(u)
        bad = torch.nonzero(got != want)
        if bad.numel():
            i = int(bad[0])
            pytest.fail(
                f"chunk {c}: {bad.numel()} mismatches; first input {int(u[i]):#010x} -> "
                f"{int(got[i]):#06x}, want {int(want[i]):#06x}"
            )
        del u, x, dst, got, want, bad


@pytest.mark.parametrize("sdt,ddt", [(o.F32, o.BF16), (o.F32, o.F16), (o.BF16, o.F32), (o.F32, o.F32)])
def test_single_span_pack_every_misalignment(rng, sdt, ddt):
    """One span per call (the one-run kernel-argument table): source and destination at every
    element offset 0-7 of a 16-byte line, lengths from 1 to a few thousand, x 1/8 -- the
    alignment head, the vector body and the ragged tail, against the oracle; the destination's
    neighbours keep their sentinels."""
    for so in range(8):
        for do in range(8):
            n = int(rng.integers(1, 3000)) if (so + do) % 3 else int(rng.integers(1, 24))
            x = values(rng, n + 16, sdt, scale=4.0)
            src = to_dev(x)
            dst = empty_dev(n + 16, ddt)
            nat.pack(nat.spans_array([(src.data_ptr() + so * esize(sdt), dst.data_ptr() + do * esize(ddt), n)]),
                     code(sdt), code(ddt), nat.f32(0.125), False, stream())
            got = to_host(dst)
            want = o.mul_scalar(o.convert(x[so : so + n], sdt, ddt), ddt, 0.125)
            assert same_bits(got[do : do + n], want), (so, do, n, first_mismatch(got[do : do + n], want))
            assert np.all(got[:do] == SENTINEL[ddt]) and np.all(got[do + n :] == SENTINEL[ddt]), (so, do, n)


def _cast_f16(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 through the pack entry point (one span, scale 1): the gather cast for
    param_dtype = float16.  Returns the fp16 bit patterns."""
    src = to_dev(np.ascontiguousarray(x))
    dst = empty_dev(x.size, o.F16)
    nat.pack(nat.spans_array([(src.data_ptr(), dst.data_ptr(), x.size)]), nat.MDX_F32, nat.MDX_F16, 1.0, False,
             stream())
    return to_host(dst).view(np.uint16)


def test_cast_f16_structured_sweep():
    """Every (sign, exponent, top-14 mantissa) pattern x low bits deciding ties from bit 9 up,
    NaN bits included, against the oracle's integer restatement."""
    hi = np.arange(1 << 23, dtype=np.uint32) << np.uint32(9)
    lows = np.array([0x000, 0x001, 0x0FF, 0x100, 0x101, 0x1FF], dtype=np.uint32)
    x = (hi[:, None] | lows[None, :]).reshape(-1).view(np.float32)
    got = _cast_f16(x)
    want = o.f16_from_f32(x).view(np.uint16)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_cast_f16_matches_golden():
    d = load_golden("f16_cast.npz")
    got = _cast_f16(d["x_bits"].view(np.float32))
    assert np.array_equal(got, d["y_bits"]), first_mismatch(got, d["y_bits"])


# ---------------------------------------------------------------------------
# Golden replays through the raw ABI
# ---------------------------------------------------------------------------


TORCH = {o.F32: torch.float32, o.BF16: torch.bfloat16, o.F16: torch.float16}


def _golden_dtype(name) -> str:
    name = str(name)
    return o.BF16 if "bfloat16" in name else (o.F16 if "float16" in name else o.F32)


@pytest.mark.parametrize("name", ["ddp_f32_w4.npz", "ddp_f32_w3_inf.npz", "ddp_bf16_w8.npz", "ddp_f16_w4_inf.npz"])
def test_golden_ddp_replay(name):
    d = load_golden(name)
    W, rank = int(d["W"]), int(d["rank"])
    numels = [int(n) for n in d["numels"]]
    dt = _golden_dtype(d["dtype"])
    layout = json.loads(str(d["layout"]))
    scale = float(d["scale"])
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    for b, idxs in enumerate(layout):
        bn = sum(numels[i] for i in idxs)
        reps = [torch.zeros(bn + 8, dtype=TORCH[dt], device=DEV) for _ in range(W)]
        keep = []
        for r in range(W):
            rows, off = [], 0
            for i in idxs:
                g = d.get(f"grad_r{r}_p{i}")
                t = None if g is None else to_dev(g)
                keep.append(t)
                rows.append((0 if t is None else t.data_ptr(), reps[r].data_ptr() + off * esize(dt), numels[i]))
                off += numels[i]
            nat.pack(nat.spans_array(rows), code(dt), code(dt), nat.f32(1.0 / W), False, stream())
        nat.allreduce_sum([x.data_ptr() for x in reps], code(dt), [0], [bn], reps[rank].data_ptr(), stream())
        got = to_host(reps[rank])[:bn]
        assert same_bits(got, d[f"reduced_b{b}"]), f"bucket {b}: " + first_mismatch(got, d[f"reduced_b{b}"])
        rows, outs, off = [], [], 0
        for i in idxs:
            g = empty_dev(numels[i], dt)
            outs.append((i, g))
            rows.append((reps[rank].data_ptr() + off * esize(dt), g.data_ptr(), numels[i]))
            off += numels[i]
        nat.unpack(nat.spans_array(rows), code(dt), code(dt), nat.f32(1.0 / scale), flag.data_ptr(), stream())
        for i, g in outs:
            assert same_bits(to_host(g), d[f"unscaled_p{i}"]), f"param {i}"
    assert bool(flag.item()) == bool(d["found_inf"])


# ---------------------------------------------------------------------------
# ABI argument checks that need device pointers
# ---------------------------------------------------------------------------


def test_allreduce_rejects_partial_overlap():
    a = torch.zeros(1024, device=DEV)
    b = torch.zeros(1024, device=DEV)
    out = a[8:]
    with pytest.raises(RuntimeError, match="overlaps"):
        nat.allreduce_sum([a.data_ptr(), b.data_ptr()], nat.MDX_F32, [0], [1000], out.data_ptr(), stream())


def test_reduce_scatter_rejects_shard_overlapping_a_peer():
    peers = torch.zeros((2, 256), device=DEV)
    own = torch.zeros(128, device=DEV)
    with pytest.raises(RuntimeError, match="overlaps"):
        nat.reduce_scatter_share(
            nat.pieces_array([(own.data_ptr(), 0, 128)]), [0, peers[1].data_ptr()], 0, 0, 0, True,
            peers[1, 64:].data_ptr(), 0, False, 1.0, None, stream(),
        )


# ---------------------------------------------------------------------------
# Device plans: one dispatch for any number of runs
# ---------------------------------------------------------------------------


def test_pack_and_unpack_planned_match_direct(rng):
    """150 spans (beyond one kernel-argument batch) through a device plan, vs the oracle."""
    sizes = [int(x) for x in rng.integers(0, 3000, 150)]
    srcs = [to_dev(values(rng, n + 1, o.F32))[1:] for n in sizes]  # odd offsets: misaligned sources
    offs, off = [], 0
    for n in sizes:
        offs.append(off)
        off += n
    bucket = empty_dev(off + 3, o.F32)
    rows = [(s.data_ptr(), bucket.data_ptr() + a * 4, n) for s, a, n in zip(srcs, offs, sizes, strict=True)]
    plan = nat.plan_spans(nat.spans_array(rows), 0, 0, DEV)
    nat.pack_planned(plan, nat.f32(1.0 / 8), False, stream())
    got = to_host(bucket)
    for s, a, n in zip(srcs, offs, sizes, strict=True):
        want = o.mul_scalar(to_host(s), o.F32, 1.0 / 8)
        assert same_bits(got[a : a + n], want)
    # unpack back into bf16 gradients with unscale + found-inf
    grads = [empty_dev(n, o.BF16) for n in sizes]
    urows = [(bucket.data_ptr() + a * 4, g.data_ptr(), n) for g, a, n in zip(grads, offs, sizes, strict=True)]
    uplan = nat.plan_spans(nat.spans_array(urows), 0, 1, DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nat.unpack_planned(uplan, nat.f32(0.5), flag.data_ptr(), stream())
    bad = False
    for g, a, n in zip(grads, offs, sizes, strict=True):
        want = o.mul_scalar(o.convert(got[a : a + n], o.F32, o.BF16), o.BF16, 0.5)
        bad |= bool((~o.isfinite(want, o.BF16)).any())
        assert same_bits(to_host(g), want)
    assert bool(flag.item()) == bad


@pytest.mark.parametrize(
    "W,bdt,gdt",
    [(8, o.F32, o.F32), (4, o.F32, o.BF16), (3, o.BF16, o.BF16), (4, o.F16, o.F16), (8, o.F32, o.F16)],
)
def test_allreduce_unpack_planned_matches_oracle(rng, W, bdt, gdt):
    numels = [int(x) for x in rng.integers(1, 5000, 120)]
    offs, off = [], 0
    for n in numels:
        offs.append(off)
        off += n + int(rng.integers(0, 3))
    reps_host = [values(rng, off, bdt, scale=1e3) for _ in range(W)]
    reps = [to_dev(h) for h in reps_host]
    grads = [empty_dev(n, gdt) for n in numels]
    runs = nat.grad_runs_array([(a, n, g.data_ptr()) for a, n, g in zip(offs, numels, grads, strict=True)])
    plan = nat.plan_allreduce_unpack([r.data_ptr() for r in reps], code(bdt), runs, reps[0].data_ptr(), code(gdt), DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    for _ in range(2):  # a plan is reusable; the second launch reduces the first one's output
        before = [to_host(r) for r in reps]
        nat.allreduce_unpack_planned(plan, nat.f32(2.0**-10), flag.data_ptr(), stream())
        want0 = before[0].copy()
        for a, n, g in zip(offs, numels, grads, strict=True):
            acc = o.allreduce_sum([b[a : a + n] for b in before], bdt)
            want0[a : a + n] = acc
            v = o.mul_scalar(o.convert(acc, bdt, gdt), gdt, 2.0**-10)
            assert same_bits(to_host(g), v)
        assert same_bits(to_host(reps[0]), want0)


# ---------------------------------------------------------------------------
# Widening fused all-reduce + unpack (bf16 contributions, fp32 bucket)
# ---------------------------------------------------------------------------


def _wide_want(reps_host, a, n, W, gdt, inv_scale, wdt=o.BF16):
    """The reference chain for an fp32 bucket of 16-bit gradients: copy_ (widen), mul_(1/W), SUM, copy_, mul_."""
    xs = [o.mul_scalar(o.convert(h[a : a + n], wdt, o.F32), o.F32, 1.0 / W) for h in reps_host]
    acc = o.allreduce_sum(xs, o.F32)
    v = o.convert(acc, o.F32, gdt)
    if inv_scale != 1.0:
        v = o.mul_scalar(v, gdt, inv_scale)
    return acc, v


@pytest.mark.parametrize("wdt,gdt", [(o.BF16, o.BF16), (o.BF16, o.F32), (o.F16, o.F16), (o.F16, o.F32),
                                     (o.BF16, o.F16)])
@pytest.mark.parametrize("W", [1, 2, 3, 8, 16])
@pytest.mark.parametrize("inv_scale,write_out", [(1.0, True), (2.0**-12, True), (1.0 / 3, False)])
def test_allreduce_unpack_wide_matches_oracle(rng, wdt, gdt, W, inv_scale, write_out):
    numels = [1, 7, 64, 4096, 3, 12345, 256, 5, 8, 9]
    offs, off = [], 3
    for n in numels:
        offs.append(off)
        off += n + int(rng.integers(0, 3))
    extent = off + 4
    reps_host = [values(rng, extent, wdt, scale=1e3) for _ in range(W)]
    reps = [to_dev(h) for h in reps_host]
    out = empty_dev(extent, o.F32)
    out_before = to_host(out)
    grads = [empty_dev(n + 2, gdt) for n in numels]
    shifts = [int(rng.integers(0, 3)) for _ in numels]
    runs = nat.grad_runs_array(
        [(a, n, g.data_ptr() + s * esize(gdt)) for a, n, g, s in zip(offs, numels, grads, shifts, strict=True)]
    )
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    nat.allreduce_unpack_wide(
        [r.data_ptr() for r in reps], code(wdt), runs, out.data_ptr() if write_out else None, nat.MDX_F32,
        code(gdt), nat.f32(1.0 / W), nat.f32(inv_scale), flag.data_ptr(), stream(),
    )
    any_bad = False
    want_out = out_before.copy()
    for a, n, g, s in zip(offs, numels, grads, shifts, strict=True):
        acc, v = _wide_want(reps_host, a, n, W, gdt, inv_scale, wdt)
        want_out[a : a + n] = acc
        any_bad |= bool((~o.isfinite(v, gdt)).any())
        got = to_host(g)
        assert same_bits(got[s : s + n], v), first_mismatch(got[s : s + n], v)
        sent = np.concatenate([got[:s], got[s + n :]])
        assert np.all(sent == SENTINEL[gdt])
    got_out = to_host(out)
    assert same_bits(got_out, want_out if write_out else out_before), first_mismatch(got_out, want_out)
    for r in range(W):
        assert same_bits(to_host(reps[r]), reps_host[r])
    assert bool(flag.item()) == any_bad


@pytest.mark.parametrize("W,wdt,gdt", [(8, o.BF16, o.BF16), (4, o.BF16, o.F32), (5, o.BF16, o.BF16),
                                       (8, o.F16, o.F16), (3, o.F16, o.F32)])
def test_allreduce_unpack_wide_planned_matches_oracle(rng, W, wdt, gdt):
    numels = [int(x) for x in rng.integers(1, 5000, 120)]
    offs, off = [], 0
    for n in numels:
        offs.append(off)
        off += n + int(rng.integers(0, 3))
    reps_host = [values(rng, off, wdt, scale=1e3) for _ in range(W)]
    reps = [to_dev(h) for h in reps_host]
    out = empty_dev(off, o.F32)
    grads = [empty_dev(n, gdt) for n in numels]
    runs = nat.grad_runs_array([(a, n, g.data_ptr()) for a, n, g in zip(offs, numels, grads, strict=True)])
    plan = nat.plan_allreduce_unpack_wide(
        [r.data_ptr() for r in reps], code(wdt), runs, out.data_ptr(), nat.MDX_F32, code(gdt),
        nat.f32(1.0 / W), DEV,
    )
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    for _ in range(2):  # reusable: the second launch gives the same result
        nat.allreduce_unpack_planned(plan, nat.f32(2.0**-10), flag.data_ptr(), stream())
        got_out = to_host(out)
        bad = False
        for a, n, g in zip(offs, numels, grads, strict=True):
            acc, v = _wide_want(reps_host, a, n, W, gdt, 2.0**-10, wdt)
            bad |= bool((~o.isfinite(v, gdt)).any())
            assert same_bits(got_out[a : a + n], acc)
            assert same_bits(to_host(g), v)
        assert bool(flag.item()) == bad


def test_allreduce_unpack_wide_rejects_bad_dtypes_and_overlap():
    reps = [torch.zeros(1024, dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    out = torch.zeros(1024, device=DEV)
    g = torch.zeros(16, dtype=torch.bfloat16, device=DEV)
    runs = nat.grad_runs_array([(0, 16, g.data_ptr())])
    ptrs = [r.data_ptr() for r in reps]
    with pytest.raises(RuntimeError, match="dtype"):  # only bf16 / fp16 -> fp32 widens
        nat.allreduce_unpack_wide(ptrs, nat.MDX_F32, runs, out.data_ptr(), nat.MDX_F32, 1, 0.5, 1.0, None, stream())
    with pytest.raises(RuntimeError, match="dtype"):
        nat.allreduce_unpack_wide(ptrs, nat.MDX_BF16, runs, out.data_ptr(), nat.MDX_BF16, 1, 0.5, 1.0, None, stream())
    with pytest.raises(RuntimeError, match="dtype"):
        nat.allreduce_unpack_wide(ptrs, nat.MDX_BF16, runs, out.data_ptr(), nat.MDX_F16, 1, 0.5, 1.0, None, stream())
    with pytest.raises(RuntimeError, match="overlaps"):  # the fp32 bucket may not alias a bf16 row
        nat.allreduce_unpack_wide(ptrs, nat.MDX_BF16, runs, reps[0].data_ptr(), nat.MDX_F32, 1, 0.5, 1.0, None,
                                  stream())


@pytest.mark.parametrize("name", ["ddp_bf16_f32bucket_w8.npz", "ddp_f16_f32bucket_w8.npz"])
def test_golden_widening_replay(name):
    """The fixture replays torch's chain for an fp32 bucket of 16-bit grads; the wide kernel must match it."""
    d = load_golden(name)
    wdt = _golden_dtype(d["dtype"])
    W, rank = int(d["W"]), int(d["rank"])
    numels = [int(n) for n in d["numels"]]
    layout = json.loads(str(d["layout"]))
    scale = float(d["scale"])
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    for b, idxs in enumerate(layout):
        bn = sum(numels[i] for i in idxs)
        reps = [torch.zeros(bn + 8, dtype=TORCH[wdt], device=DEV) for _ in range(W)]
        keep = []
        for r in range(W):
            rows, off = [], 0
            for i in idxs:
                g = d.get(f"grad_r{r}_p{i}")
                t = None if g is None else to_dev(g)
                keep.append(t)
                rows.append((0 if t is None else t.data_ptr(), reps[r].data_ptr() + off * 2, numels[i]))
                off += numels[i]
            nat.pack(nat.spans_array(rows), code(wdt), code(wdt), 1.0, False, stream())
        out = empty_dev(bn, o.F32)
        grads, rows, off = [], [], 0
        for i in idxs:
            g = empty_dev(numels[i], wdt)
            grads.append((i, g))
            rows.append((off, numels[i], g.data_ptr()))
            off += numels[i]
        nat.allreduce_unpack_wide(
            [x.data_ptr() for x in reps], code(wdt), nat.grad_runs_array(rows), out.data_ptr(), nat.MDX_F32,
            code(wdt), nat.f32(1.0 / W), nat.f32(1.0 / scale), flag.data_ptr(), stream(),
        )
        got = to_host(out)
        assert same_bits(got, d[f"reduced_b{b}"]), f"bucket {b}: " + first_mismatch(got, d[f"reduced_b{b}"])
        for i, g in grads:
            assert same_bits(to_host(g), d[f"unscaled_p{i}"]), f"param {i}"
    assert bool(flag.item()) == bool(d["found_inf"])


@pytest.mark.parametrize("n_spans", [0, 3, 150])
@pytest.mark.parametrize("planned", [False, True])
def test_pack_clears_the_flag(rng, n_spans, planned):
    """clear_flag: the pack also sets the found-inf flag to 0 in stream order -- with nothing to
    copy, over several kernel-argument batches, or through a plan -- and copies exactly as without it."""
    sizes = [int(x) for x in rng.integers(1, 700, n_spans)]
    srcs = [to_dev(values(rng, n, o.F32)) for n in sizes]
    dst = empty_dev(sum(sizes) + 1, o.F32)
    rows, off = [], 0
    for s, n in zip(srcs, sizes, strict=True):
        rows.append((s.data_ptr(), dst.data_ptr() + off * 4, n))
        off += n
    flag = torch.ones(1, dtype=torch.int32, device=DEV)
    other = torch.ones(1, dtype=torch.int32, device=DEV)
    if planned and n_spans:
        plan = nat.plan_spans(nat.spans_array(rows), 0, 0, DEV)
        nat.pack_planned(plan, nat.f32(0.25), False, stream(), flag.data_ptr())
    else:
        nat.pack(nat.spans_array(rows), 0, 0, nat.f32(0.25), False, stream(), flag.data_ptr())
    assert flag.item() == 0 and other.item() == 1
    got, off = to_host(dst), 0
    for s, n in zip(srcs, sizes, strict=True):
        assert same_bits(got[off : off + n], o.mul_scalar(to_host(s), o.F32, 0.25))
        off += n
    assert same_bits(got[off:], np.full(len(got) - off, SENTINEL_F32, dtype=np.float32))


# ---------------------------------------------------------------------------
# multi-unit reduce-scatter share (finish_gradient_sync's flush of many units)
# ---------------------------------------------------------------------------


def _multi_share_case(rng, units, idt, W, rank, accumulate, sdt=o.F32, rdt=o.F32):
    """Units laid out one after another in shared contribution rows; each unit's shard result
    goes to a tensor of its own.  Returns the pieces, destinations, rows and the expected shards."""
    layouts, base = [], 0
    for numels in units:
        total = sum(numels)
        S = (total + W - 1) // W
        layouts.append((numels, S, S * W, base))
        base += S * W + int(rng.integers(0, 5))  # units need not be packed back to back
    rows_host = [o.zeros(base, idt) for _ in range(W)]
    grads_all, pieces, outs, shards, wants, prevs, own_keep = [], [], [], [], [], [], []
    for u, (numels, S, P, off0) in enumerate(layouts):
        grads = [[None if (r + i + u) % 5 == 3 else values(rng, n, idt, scale=1e-3) for i, n in enumerate(numels)]
                 for r in range(W)]
        grads_all.append(grads)
        for r in range(W):
            rows_host[r][off0 : off0 + P] = o.fsdp_flatten(grads[r], idt, numels, P, idt)
        own_devs = [None if g is None else to_dev(g) for g in grads[rank]]
        own_keep.append(own_devs)
        prev = values(rng, S, sdt, specials=False, scale=1e-3)
        shard = to_dev(prev) if accumulate else empty_dev(S, sdt)
        shards.append(shard)
        prevs.append(prev)
        lo, hi = rank * S, rank * S + S
        off, cursor = 0, lo
        for t, n in zip(own_devs, numels, strict=True):
            a, b = max(off, lo), min(off + n, hi)
            if a < b:
                ptr = 0 if t is None else t.data_ptr() + (a - off) * esize(idt)
                pieces.append((ptr, off0 + a, b - a))
                outs.append(shard.data_ptr() + (a - lo) * esize(sdt))
                cursor = b
            off += n
        if cursor < hi:
            pieces.append((0, off0 + cursor, hi - cursor))
            outs.append(shard.data_ptr() + (cursor - lo) * esize(sdt))
        wants.append(o.fsdp_reduce_scatter_share(grads, idt, numels, rank, rdt, sdt,
                                                 existing=prev if accumulate else None))
    row_devs = [to_dev(h) for h in rows_host]
    return dict(pieces=nat.pieces_array(pieces), outs=outs, rows=row_devs, shards=shards, wants=wants,
                prevs=prevs, keep=own_keep)


@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("idt", [o.BF16, o.F32, o.F16])
@pytest.mark.parametrize("W,rank", [(2, 1), (3, 0), (8, 5), (16, 9)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_reduce_scatter_share_multi_matches_oracle(rng, planned, idt, W, rank, accumulate):
    """Sixty units of 1-8 parameters (at least one piece each: more than one kernel-argument table)
    reduced in one call, each unit's shard against the oracle; the plan form does it in one dispatch
    and is launched twice (the second launch must give the same bits again, from fresh inputs)."""
    units = [[int(x) for x in rng.integers(1, 3000, int(rng.integers(1, 9)))] for _ in range(60)]
    c = _multi_share_case(rng, units, idt, W, rank, accumulate)
    peers = [r.data_ptr() for r in c["rows"]]
    assert len(c["pieces"]) > 48
    if planned:
        plan = nat.plan_reduce_scatter_share_multi(c["pieces"], c["outs"], peers, rank, code(idt), DEV)
        for launch in range(2):
            if launch:  # restore the shards and launch the same plan again
                for sh, prev in zip(c["shards"], c["prevs"], strict=True):
                    sh.copy_(to_dev(prev) if accumulate else empty_dev(sh.numel(), o.F32))
            nat.reduce_scatter_share_multi_planned(plan, True, accumulate, 1.0, None, stream())
            for u, (sh, want) in enumerate(zip(c["shards"], c["wants"], strict=True)):
                got = to_host(sh)
                assert same_bits(got, want), f"launch {launch} unit {u}: " + first_mismatch(got, want)
    else:
        nat.reduce_scatter_share_multi(c["pieces"], c["outs"], peers, rank, code(idt), nat.MDX_F32, True,
                                       nat.MDX_F32, accumulate, 1.0, None, stream())
        for u, (sh, want) in enumerate(zip(c["shards"], c["wants"], strict=True)):
            got = to_host(sh)
            assert same_bits(got, want), f"unit {u}: " + first_mismatch(got, want)


@pytest.mark.parametrize("sdt,rdt", [(o.BF16, o.F32), (o.F16, o.F32), (o.F32, o.BF16)])
def test_reduce_scatter_share_multi_other_dtypes(rng, sdt, rdt):
    """Low-precision shards (keep_low_precision_shard) and a bf16 reduction go through the
    kernel-argument form of the multi-unit share, against the oracle."""
    units = [[int(x) for x in rng.integers(1, 2000, int(rng.integers(1, 6)))] for _ in range(6)]
    W, rank = 4, 3
    c = _multi_share_case(rng, units, o.BF16, W, rank, False, sdt=sdt, rdt=rdt)
    peers = [r.data_ptr() for r in c["rows"]]
    nat.reduce_scatter_share_multi(c["pieces"], c["outs"], peers, rank, nat.MDX_BF16, code(rdt), True, code(sdt),
                                   False, 1.0, None, stream())
    for u, (sh, want) in enumerate(zip(c["shards"], c["wants"], strict=True)):
        got = to_host(sh)
        assert same_bits(got, want), f"unit {u}: " + first_mismatch(got, want)


def test_reduce_scatter_share_multi_rejects_overlaps():
    """A destination over a contribution row, over a piece's own data or over another
    destination is refused before anything is launched; the plan rejects non-fp32 shards."""
    rows = [torch.zeros(4096, device=DEV) for _ in range(2)]
    own = torch.zeros(1024, device=DEV)
    out = torch.zeros(2048, device=DEV)
    peers = [r.data_ptr() for r in rows]
    pieces = nat.pieces_array([(own.data_ptr(), 0, 512), (0, 512, 512)])
    for outs in ([rows[0].data_ptr(), out.data_ptr()], [out.data_ptr(), own.data_ptr()],
                 [out.data_ptr(), out.data_ptr() + 4 * 100]):
        rc = nat.lib().mdx_reduce_scatter_share_multi(
            nat._ptr(pieces), nat._ptrs(outs), 2, nat._ptrs(peers), 2, 1, nat.MDX_F32, nat.MDX_F32, 1,
            nat.MDX_F32, 0, 1.0, None, stream())
        assert rc == nat.MDX_EALIAS, nat.strerror(rc)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0
