"""Pin the CPU oracle (oracle/gradpath.py) before it is trusted as the checker.

Each oracle function is checked against something other than itself: the
golden fixtures (torch CPU replays of the reference's ATen chains), torch CPU
ops on fresh inputs, hand-built answers, the reference's own known-answer
tests, and invariants that fix the result uniquely.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN, bf16_bits_torch, first_mismatch, load_golden, same_bits
from oracle import gradpath as o


TORCH_DTYPE = {o.F32: torch.float32, o.BF16: torch.bfloat16, o.F16: torch.float16}


def _torch_bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().astype(np.uint16)
    return t.numpy().copy()


def _from_bits(a: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == o.BF16:
        return torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16)
    if dtype == o.F16:
        return torch.from_numpy(np.asarray(a, dtype=np.float16).copy())
    return torch.from_numpy(np.asarray(a, dtype=np.float32).copy())


def _golden_dtype(name) -> str:
    name = str(name)
    return o.BF16 if "bfloat16" in name else (o.F16 if "float16" in name else o.F32)


# ---------------------------------------------------------------------------
# bf16 conversion
# ---------------------------------------------------------------------------


def test_bf16_hand_built_ties_and_specials():
    x, want = o.bf16_tie_cases()
    got = o.bf16_from_f32(x)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_bf16_matches_golden_fixture():
    d = load_golden("bf16_cast.npz")
    got = o.bf16_from_f32(d["x_bits"].view(np.float32))
    assert np.array_equal(got, d["y_bits"]), first_mismatch(got, d["y_bits"])


def test_bf16_structured_sweep_matches_torch():
    """Every (sign, exponent, top-7 mantissa) pattern x the low halves that decide rounding."""
    hi = np.arange(1 << 16, dtype=np.uint32) << np.uint32(16)
    lows = np.array([0x0000, 0x0001, 0x3FFF, 0x7FFF, 0x8000, 0x8001, 0xBFFF, 0xFFFF], dtype=np.uint32)
    u = (hi[:, None] | lows[None, :]).reshape(-1)
    x = u.view(np.float32)
    got = o.bf16_from_f32(x)
    want = _torch_bits(torch.from_numpy(x.copy()).to(torch.bfloat16))
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_bf16_torch_restatement_matches_oracle(rng):
    """The integer torch form used by the exhaustive device test equals the oracle on every
    (sign, exponent, top-7 mantissa) pattern x tie-deciding low halves, and on random patterns."""
    hi = np.arange(1 << 16, dtype=np.uint32) << np.uint32(16)
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x4000, 0xC000], dtype=np.uint32)
    u = np.concatenate([(hi[:, None] | lows[None, :]).reshape(-1), rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint32)])
    got = bf16_bits_torch(torch.from_numpy(u.astype(np.int64))).numpy().astype(np.uint16)
    want = o.bf16_from_f32(u.view(np.float32))
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_bf16_widening_is_exact_roundtrip():
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = o.f32_from_bf16(b)
    nan = np.isnan(f)
    assert np.array_equal(o.bf16_from_f32(f)[~nan], b[~nan])
    assert np.all(o.bf16_from_f32(f)[nan] == 0xFFFF)


# ---------------------------------------------------------------------------
# fp16 conversion
# ---------------------------------------------------------------------------


def _f16_cases() -> tuple[np.ndarray, np.ndarray]:
    """Hand-built fp32 inputs with their fp16 answers, worked out from the format:
    ties at mantissa bit 12 (normal) or at the subnormal quantum, the overflow
    threshold 65520, the smallest subnormal, signed zero, inf and NaN."""
    cases = [
        (0x3F800000, 0x3C00),  # 1.0
        (0x3F801000, 0x3C00),  # 1 + half ulp: tie -> even (0x3C00)
        (0x3F803000, 0x3C02),  # 1 + 1.5 ulp: tie -> even (0x3C02)
        (0x3F801001, 0x3C01),  # just above the tie rounds up
        (0x3F800FFF, 0x3C00),  # just below the tie rounds down
        (0x477FE000, 0x7BFF),  # 65504, the largest finite fp16
        (0x477FEFFF, 0x7BFF),  # just below 65520 stays finite
        (0x477FF000, 0x7C00),  # 65520: tie between 65504 and 2^16 -> even = inf
        (0x7F7FFFFF, 0x7C00),  # FLT_MAX -> inf
        (0x38800000, 0x0400),  # 2^-14, smallest normal
        (0x387FC000, 0x03FF),  # 2^-14 - 2^-24: the largest subnormal, exact
        (0x387FD000, 0x03FF),  # 2^-14 - 3 * 2^-26: below the tie rounds down
        (0x387FE000, 0x0400),  # 2^-14 - 2^-25: tie between 0x3FF and 0x400 -> even (0x400)
        (0x387FF000, 0x0400),  # 2^-14 - 2^-26: above the tie rounds up
        (0x33800000, 0x0001),  # 2^-24, the smallest subnormal
        (0x33000000, 0x0000),  # 2^-25: tie between 0 and 2^-24 -> even (0)
        (0x33000001, 0x0001),  # just above 2^-25 rounds up
        (0x33C00000, 0x0002),  # 1.5 * 2^-24: tie -> even (2)
        (0x34200000, 0x0002),  # 2.5 * 2^-24: tie -> even (2)
        (0x00000001, 0x0000),  # fp32 subnormal -> +0
        (0x80000000, 0x8000),  # -0
        (0xC0000000, 0xC000),  # -2
        (0x7F800000, 0x7C00),  # +inf
        (0xFF800000, 0xFC00),  # -inf
        (0x7FC00000, 0x7E00),  # qNaN
        (0xFFC12345, 0xFE09),  # negative NaN: sign and top mantissa bits kept, quieted
        (0x7F800001, 0x7E00),  # sNaN with a low payload: quieted, payload bits below 13 dropped
    ]
    x = np.array([c[0] for c in cases], dtype=np.uint32).view(np.float32)
    y = np.array([c[1] for c in cases], dtype=np.uint16)
    return x, y


def test_f16_hand_built_ties_and_specials():
    x, want = _f16_cases()
    got = o.f16_from_f32(x).view(np.uint16)
    assert np.array_equal(got, want), first_mismatch(got, want)
    t = x.copy()
    assert np.array_equal(_torch_bits(torch.from_numpy(t).to(torch.float16)).view(np.uint16), want)


def test_f16_matches_golden_fixture():
    d = load_golden("f16_cast.npz")
    got = o.f16_from_f32(d["x_bits"].view(np.float32)).view(np.uint16)
    assert np.array_equal(got, d["y_bits"]), first_mismatch(got, d["y_bits"])


def test_f16_structured_sweep_matches_torch_and_numpy():
    """Every (sign, exponent, top-14 mantissa) pattern x low bits that decide ties at
    any position from mantissa bit 9 up (normal results tie at bit 12, subnormal
    ones at bits 13-23)."""
    hi = np.arange(1 << 23, dtype=np.uint32) << np.uint32(9)
    lows = np.array([0x000, 0x001, 0x0FF, 0x100, 0x101, 0x1FF], dtype=np.uint32)
    for part in np.array_split(hi, 8):
        u = (part[:, None] | lows[None, :]).reshape(-1)
        x = u.view(np.float32)
        got = o.f16_from_f32(x).view(np.uint16)
        want = _torch_bits(torch.from_numpy(x.copy()).to(torch.float16)).view(np.uint16)
        assert np.array_equal(got, want), first_mismatch(got, want)
        nan = np.isnan(x)
        with np.errstate(over="ignore"):
            lib = x[~nan].astype(np.float16).view(np.uint16)
        assert np.array_equal(got[~nan], lib)


def test_f16_widening_is_exact_roundtrip():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    f = o.f32_from_f16(h)
    nan = np.isnan(f)
    assert np.array_equal(o.f16_from_f32(f).view(np.uint16)[~nan], h.view(np.uint16)[~nan])
    # torch widens alike; it also quiets signalling NaNs, whose payloads no test compares
    assert same_bits(f, _torch_bits(torch.from_numpy(h.copy()).float()))


# ---------------------------------------------------------------------------
# Scalar ops vs torch CPU (the ATen ops the reference calls)
# ---------------------------------------------------------------------------


def _random_with_specials(rng, n: int) -> np.ndarray:
    x = (rng.standard_normal(n) * 10.0 ** rng.integers(-40, 38, n)).astype(np.float32)
    pool = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-40, 3.4e38, 1.17549435e-38], np.float32)
    idx = rng.integers(0, n, n // 10)
    x[idx] = pool[rng.integers(0, len(pool), idx.size)]
    return x


@pytest.mark.parametrize("dtype", [o.F32, o.BF16, o.F16])
@pytest.mark.parametrize("scale", [1.0 / 8, 1.0 / 3, 1.0 / 7, 2.0**-16, 1e-3])
def test_mul_scalar_matches_torch(rng, dtype, scale):
    x = o.from_f32(_random_with_specials(rng, 20000), dtype)
    got = o.mul_scalar(x, dtype, scale)
    want = _torch_bits(_from_bits(x, dtype).clone().mul_(scale))
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("dtype", [o.F32, o.BF16, o.F16])
@pytest.mark.parametrize("w", [2, 3, 5, 8])
def test_div_scalar_matches_torch(rng, dtype, w):
    x = o.from_f32(_random_with_specials(rng, 20000), dtype)
    got = o.div_scalar(x, dtype, w)
    want = _torch_bits(_from_bits(x, dtype).clone().div_(w))
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("src", [o.F32, o.BF16, o.F16])
@pytest.mark.parametrize("dst", [o.F32, o.BF16, o.F16])
def test_convert_matches_torch_copy(rng, src, dst):
    x = o.from_f32(_random_with_specials(rng, 20000), src)
    got = o.convert(x, src, dst)
    want = _torch_bits(torch.empty(x.size, dtype=TORCH_DTYPE[dst]).copy_(_from_bits(x, src)))
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("dtype", [o.F32, o.BF16, o.F16])
@pytest.mark.parametrize("W", [2, 3, 8, 16])
def test_allreduce_sum_matches_torch_sequential_add(rng, dtype, W):
    contribs = [o.from_f32(_random_with_specials(rng, 5000), dtype) for _ in range(W)]
    got = o.allreduce_sum(contribs, dtype)
    acc = _from_bits(contribs[0], dtype).clone()
    for c in contribs[1:]:
        acc = acc.add_(_from_bits(c, dtype)) if dtype == o.F32 else acc + _from_bits(c, dtype)
    assert same_bits(got, _torch_bits(acc)), first_mismatch(got, _torch_bits(acc))


TORCH_FOLD = {"max": torch.maximum, "min": torch.minimum, "product": torch.mul}


@pytest.mark.parametrize("dtype", [o.F32, o.BF16, o.F16])
@pytest.mark.parametrize("W", [1, 2, 3, 8, 16])
@pytest.mark.parametrize("op", ["max", "min", "product"])
def test_allreduce_op_matches_torch_chain(rng, dtype, W, op):
    """The rank-ordered fold against torch CPU's own maximum / minimum / mul on the same tensors:
    special values (NaN, +-inf, +-0, subnormals, overflow) and repeated values among the ranks.
    For MAX and MIN the sign of a zero is compared separately (closed form below): torch answers
    a tie of -0 and +0 differently in its scalar and vectorised loops."""
    contribs = [o.from_f32(_random_with_specials(rng, 6000), dtype) for _ in range(W)]
    if W > 1:
        contribs[1][:500] = contribs[0][:500]  # ties between ranks
    got = o.allreduce_op(contribs, dtype, op)
    acc = _from_bits(contribs[0], dtype).clone()
    for c in contribs[1:]:
        acc = TORCH_FOLD[op](acc, _from_bits(c, dtype))
    want = _torch_bits(acc)
    if op != "product":
        got, want = _unsigned_zeros(got, dtype), _unsigned_zeros(want, dtype)
    assert same_bits(got, want), first_mismatch(got, want)


def _unsigned_zeros(a: np.ndarray, dtype: str) -> np.ndarray:
    a = np.array(a, copy=True)
    a[o.to_f32(a, dtype) == 0] = o.zeros(1, dtype)[0]
    return a


def test_allreduce_op_closed_forms(rng):
    """Without NaNs MAX and MIN are numpy's max and min reductions (by value); products of signed
    powers of two are exact; a tie of -0 and +0 is +0 under MAX and -0 under MIN in either rank
    order (IEEE 754-2019 maximum / minimum), and -0 with -0 stays -0."""
    x = rng.standard_normal((5, 4000)).astype(np.float32) * 1e3
    contribs = list(x)
    assert np.array_equal(o.allreduce_op(contribs, o.F32, "max"), x.max(axis=0))
    assert np.array_equal(o.allreduce_op(contribs, o.F32, "min"), x.min(axis=0))
    k = rng.integers(-20, 20, (6, 4000))
    sign = rng.choice([-1.0, 1.0], (6, 4000))
    p = (sign * 2.0 ** k).astype(np.float32)
    want = (sign.prod(axis=0) * 2.0 ** k.sum(axis=0)).astype(np.float32)
    assert np.array_equal(o.allreduce_op(list(p), o.F32, "product"), want)
    for dtype in (o.F32, o.BF16, o.F16):
        z, nz = o.from_f32(np.array([0.0], np.float32), dtype), o.from_f32(np.array([-0.0], np.float32), dtype)
        for op, want_neg in (("max", False), ("min", True)):
            for pair in ([nz, z], [z, nz], [nz, z, nz]):
                got = o.to_f32(o.allreduce_op(pair, dtype, op), dtype)
                assert got[0] == 0 and bool(np.signbit(got[0])) == want_neg, (dtype, op, pair)
            both = o.to_f32(o.allreduce_op([nz, nz], dtype, op), dtype)
            assert np.signbit(both[0])
    nan = o.allreduce_op([np.array([1.0, np.nan], np.float32), np.array([np.nan, 2.0], np.float32)], o.F32, "max")
    assert np.isnan(nan).all()


@pytest.mark.parametrize("W", [2, 3, 7, 8, 16])
def test_allreduce_sum_of_short_mantissa_copies_is_exact(rng, W):
    """Inputs k * 2^-10 with |k| < 2^16 keep every partial sum exact in fp32, so the
    rank-ordered sum of W distinct contributions equals their exact integer sum."""
    ks = rng.integers(-(2**16), 2**16, (W, 10000))
    contribs = [(k * 2.0**-10).astype(np.float32) for k in ks]
    got = o.allreduce_sum(contribs, o.F32)
    assert np.array_equal(got, (ks.sum(axis=0) * 2.0**-10).astype(np.float32))


def test_unscale_found_inf_matches_torch(rng):
    grads = [_random_with_specials(rng, n) for n in (17, 1000, 3)]
    grads.append(np.ones(8, np.float32))
    dts = [o.F32] * len(grads)
    got, found = o.unscale_found_inf(grads, dts, 1.0 / 65536)
    f = torch.zeros(1)
    for g, want in zip(grads, got, strict=True):
        t = torch.from_numpy(g.copy()).mul_(1.0 / 65536)
        f += (~torch.isfinite(t)).any().to(f.dtype)
        assert same_bits(want, t.numpy())
    assert found == bool(f.item() > 0)
    _, found_clean = o.unscale_found_inf([np.ones(4, np.float32)], [o.F32], 0.5)
    assert not found_clean


def test_found_inf_sees_bf16_overflow_of_a_finite_fp32_value():
    big = np.array([3.40e38], np.float32)  # finite in fp32, above the bf16 rounding threshold 3.396e38
    b = o.convert(big, o.F32, o.BF16)
    _, found = o.unscale_found_inf([b], [o.BF16], 1.0)
    assert found


def test_unscale_found_inf_f16_matches_torch(rng):
    """fp16 gradients (the loss scaler's own format, amp.py:1-30): unscale + isfinite."""
    grads = [o.from_f32((rng.standard_normal(n) * 3000).astype(np.float32), o.F16) for n in (40, 1000)]
    grads[1][7] = np.float16(np.inf)
    grads.append(o.from_f32(np.array([70000.0, 1.0], np.float32), o.F16))  # overflows to inf when cast
    got, found = o.unscale_found_inf(grads, [o.F16] * 3, 1.0 / 1024)
    f = torch.zeros(1)
    for g, want in zip(grads, got, strict=True):
        t = torch.from_numpy(g.copy()).mul_(1.0 / 1024)
        f += (~torch.isfinite(t)).any().to(f.dtype)
        assert same_bits(want, t.numpy())
    assert found and bool(f.item() > 0)
    _, clean = o.unscale_found_inf(grads[:1], [o.F16], 1.0 / 1024)
    assert not clean


# ---------------------------------------------------------------------------
# DDP bucketer
# ---------------------------------------------------------------------------


def _check_greedy_partition(nbytes, cap_mb, buckets):
    """The three properties that define the greedy reverse-order partition uniquely."""
    cap = int(cap_mb * 1024 * 1024)
    flat = [i for b in buckets for i in b]
    assert flat == list(reversed(range(len(nbytes)))), "buckets must tile the reversed parameter list"
    for b in buckets:
        assert len(b) >= 1
        assert sum(nbytes[i] for i in b) <= cap or len(b) == 1, "over cap without being a singleton"
    for b, nxt in zip(buckets, buckets[1:]):
        assert sum(nbytes[i] for i in b) + nbytes[nxt[0]] > cap, "a flush happened that the cap did not force"


@pytest.mark.parametrize("seed", range(20))
def test_build_buckets_is_the_greedy_partition(seed):
    r = np.random.default_rng(seed)
    nbytes = [int(x) for x in r.integers(1, 5000, r.integers(1, 40))]
    cap_mb = float(r.choice([1e-6, 1e-3, 2e-3, 5e-3, 1e6]))
    _check_greedy_partition(nbytes, cap_mb, o.build_buckets(nbytes, cap_mb))


def test_build_buckets_brute_force_tiny():
    """Exhaustive: every list of up to 6 sizes in {1,2,3} with caps 0..6 bytes."""
    import itertools

    for n in range(1, 7):
        for sizes in itertools.product([1, 2, 3], repeat=n):
            for cap in range(0, 7):
                cap_mb = cap / (1024 * 1024)
                _check_greedy_partition(list(sizes), cap_mb, o.build_buckets(list(sizes), cap_mb))


def test_cap_one_byte_gives_one_bucket_per_param_and_huge_cap_one_bucket():
    nbytes = [4 * n for n in (10, 1, 300, 7)]
    assert o.build_buckets(nbytes, 1e-6) == [[3], [2], [1], [0]]  # int(1.048576) = 1 byte
    assert o.build_buckets(nbytes, 1e6) == [[3, 2, 1, 0]]


def test_reference_layout_invariants_on_the_test_gpt():
    """tests/test_ddp.py:103-121 on GPTConfig(vocab=64, block=16, n_layer=2, n_embd=32), cap 0.05 MB."""
    from minidist import workloads as w

    specs = w.gpt_specs(n_layer=2, n_embd=32, vocab=64, ctx=16, untied_head=True)
    nbytes = [s.nbytes for s in specs]
    buckets = o.build_buckets(nbytes, 0.05)
    assert len(buckets) > 1
    assert buckets[0][0] == len(specs) - 1  # bucket 0 starts from the last parameter
    _check_greedy_partition(nbytes, 0.05, buckets)


def test_cfg_bucket_counts():
    from minidist import workloads as w

    s1 = w.gpt_specs(**w.GPT2_SMALL)
    assert w.total_numel(s1) == 124_439_808
    lay = o.build_buckets([s.nbytes for s in s1], 25.0)
    # reverse order ends ..., wte (147.24 MiB, alone), wpe (3 MiB, alone)
    assert len(lay) == 18 and lay[-2] == [1] and lay[-1] == [0]
    s2 = w.gpt_specs(**w.GPT2_MEDIUM)
    assert w.total_numel(s2) == 354_823_168
    assert [len(o.build_buckets([s.nbytes for s in s2], c)) for c in (1e-6, 25.0, 1e6)] == [292, 74, 1]
    assert w.total_numel(w.llama_specs()) == 6_738_415_616


def _golden_ddp_inputs(d):
    W, rank = int(d["W"]), int(d["rank"])
    numels = [int(n) for n in d["numels"]]
    dt = _golden_dtype(d["dtype"])
    grads = [[d.get(f"grad_r{r}_p{i}") for i in range(len(numels))] for r in range(W)]
    return W, rank, numels, dt, grads


DDP_GOLDEN = ["ddp_f32_w4.npz", "ddp_f32_w3_inf.npz", "ddp_bf16_w8.npz", "ddp_bf16_f32bucket_w8.npz",
              "ddp_f16_w4_inf.npz", "ddp_f16_f32bucket_w8.npz"]


@pytest.mark.parametrize("name", DDP_GOLDEN)
def test_ddp_pipeline_matches_golden(name):
    d = load_golden(name)
    W, rank, numels, dt, grads = _golden_ddp_inputs(d)
    bdt = _golden_dtype(d["bucket_dtype"])
    res = o.ddp_pipeline(
        grads, [dt] * len(numels), numels, float(d["cap_mb"]), rank, 1.0 / float(d["scale"]), bucket_dtype=bdt
    )
    assert res["layout"] == json.loads(str(d["layout"]))
    for b, red in enumerate(res["reduced"]):
        assert same_bits(red, d[f"reduced_b{b}"]), f"bucket {b}: " + first_mismatch(red, d[f"reduced_b{b}"])
    for i, g in enumerate(res["grads"]):
        assert same_bits(g, d[f"unscaled_p{i}"]), f"param {i}: " + first_mismatch(g, d[f"unscaled_p{i}"])
    assert res["found_inf"] == bool(d["found_inf"])


def test_ddp_pipeline_is_cap_invariant(rng):
    """Elementwise fixed-order arithmetic: bucketing cannot change any value (cfg2's property)."""
    numels = [int(n) for n in rng.integers(1, 300, 15)]
    W = 4
    grads = [[(rng.standard_normal(n) * 1e-3).astype(np.float32) for n in numels] for _ in range(W)]
    outs = [o.ddp_pipeline(grads, [o.F32] * len(numels), numels, cap, 2, 2.0**-16)["grads"] for cap in (1e-6, 1e-3, 1e6)]
    for other in outs[1:]:
        for a, b in zip(outs[0], other, strict=True):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------------------
# Loss scaler
# ---------------------------------------------------------------------------


def test_scaler_known_answers():
    kat = json.loads((GOLDEN / "scaler_kat.json").read_text())
    s = o.ScalerState(scale=kat["overflow_skips"]["init_scale"])
    stepped = s.step(True)
    s.update(True)
    assert not stepped and s.scale == 512.0 and s.num_skipped == 1

    k = kat["clean_growth"]
    s = o.ScalerState(scale=k["init_scale"], growth_interval=k["growth_interval"])
    for f in k["found"]:
        assert s.step(f)
        s.update(f)
    assert s.scale == k["scale_after"] and s.num_skipped == 0

    k = kat["mixed_history"]
    s = o.ScalerState(scale=k["init_scale"], growth_interval=k["growth_interval"])
    for f in k["found"]:
        s.step(f)
        s.update(f)
    assert s.scale == k["scale_after"]
    assert s.history == [2048.0, 2048.0, 4096.0, 2048.0, 1024.0]


def test_scaler_min_scale_floor():
    s = o.ScalerState(scale=2.0, min_scale=1.0)
    for _ in range(5):
        s.update(True)
    assert s.scale == 1.0


# ---------------------------------------------------------------------------
# FSDP unit
# ---------------------------------------------------------------------------


def test_fsdp_layout_closed_form_and_invariants():
    from minidist import workloads as w

    assert o.fsdp_layout([7, 12, 5], 4) == (24, 6, 24)
    assert o.fsdp_layout([7, 12, 6], 4) == (25, 7, 28)
    blk = w.gpt_block_specs(0, 1600)
    total, S, P = o.fsdp_layout([s.numel for s in blk], 8)
    assert (total, S, P) == (30_740_800, 3_842_600, 30_740_800)
    # tests/test_fsdp.py:130-149: one unit per block + root, local <= 1.25 * full / W
    specs = w.gpt_specs(n_layer=3, n_embd=32, vocab=64, ctx=16, untied_head=True)
    units = [[s.numel for s in specs if s.name.startswith(f"blocks.{i}.")] for i in range(3)]
    units.append([s.numel for s in specs if not s.name.startswith("blocks.")])
    full = sum(s.numel for s in specs)
    for W in (2, 4):
        local = sum(o.fsdp_layout(u, W)[1] for u in units)
        assert local <= full / W * 1.25
    assert len(units) == 3 + 1


FSDP_GOLDEN = ["fsdp_bf16_w4.npz", "fsdp_bf16_w3.npz", "fsdp_f32_w2.npz", "fsdp_bf16red_w4.npz",
               "fsdp_f16_w4.npz", "fsdp_f16red_w3.npz"]


@pytest.mark.parametrize("name", FSDP_GOLDEN)
def test_fsdp_reduce_scatter_and_cast_match_golden(name):
    d = load_golden(name)
    W = int(d["W"])
    numels = [int(n) for n in d["numels"]]
    gdt = _golden_dtype(d["grad_dtype"])
    rdt = _golden_dtype(d["reduce_dtype"])
    cdt = _golden_dtype(d["cast_dtype"]) if "cast_dtype" in d else o.BF16
    grads = [[d.get(f"grad_r{r}_p{i}") for i in range(len(numels))] for r in range(W)]
    S = int(d["S"])
    for rank in range(W):
        got = o.fsdp_reduce_scatter_share(grads, gdt, numels, rank, rdt, o.F32)
        assert same_bits(got, d[f"shard_grad_r{rank}"]), first_mismatch(got, d[f"shard_grad_r{rank}"])
        acc = o.fsdp_reduce_scatter_share(grads, gdt, numels, rank, rdt, o.F32, existing=d[f"prev_r{rank}"])
        assert same_bits(acc, d[f"shard_grad_acc_r{rank}"])
        cast = o.fsdp_gather_cast(d["master_flat"][rank * S : (rank + 1) * S], cdt)
        assert same_bits(cast, d[f"gather_cast_r{rank}"])


def test_fsdp_world1_is_plain_flatten(rng):
    numels = [3, 4]
    g = [[rng.standard_normal(n).astype(np.float32) for n in numels]]
    got = o.fsdp_reduce_scatter_share(g, o.F32, numels, 0)
    assert np.array_equal(got, np.concatenate(g[0]))
