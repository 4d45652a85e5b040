"""CPU oracle for minidist's per-rank gradient-communication path.

TEST INFRASTRUCTURE ONLY.  This module is the checker, never the thing that is
measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``minidist`` + ``libmdx.so``) never calls into it and has no CPU fallback.

It restates, element by element and in numpy, the arithmetic the reference
performs with ATen ops.  Every function cites the reference lines it follows
(paths relative to the reference repository root).  Conventions:

* fp32 arrays are ``np.float32``; bf16 arrays are ``np.uint16`` bit patterns;
  fp16 arrays are ``np.float16`` (only ever converted, never computed in).
* ATen evaluates bf16 and fp16 arithmetic in an fp32 "opmath" type and rounds
  the result back once per op; Python scalars passed to ``mul_`` are first
  rounded to fp32.  Both facts were probed against torch 2.10 CPU and are what
  the helpers below implement.
* The fp32 -> bf16 conversion is IEEE round-to-nearest-even; every NaN maps to
  ``0xFFFF`` (torch 2.10's vectorised CPU conversion, the one the reference's
  gloo path runs).
* The fp32 -> fp16 conversion is IEEE round-to-nearest-even with fp16
  subnormals and overflow to +-inf; a NaN keeps its sign and the top ten
  mantissa bits, with the quiet bit set (torch 2.10 CPU).

Pins (each function is checked by ``tests/test_oracle.py`` against something
other than itself):

=========================  ===================================================
function                   pinned by
=========================  ===================================================
bf16_from_f32              torch CPU ``.to(bfloat16)`` over a structured sweep
                           of every (sign, exponent, high mantissa) pattern x
                           the rounding-relevant low halves; hand-built ties
f16_from_f32               torch CPU ``.to(float16)`` and numpy's
                           ``astype(float16)`` (non-NaN) over a structured
                           sweep of every (sign, exponent, top 14 mantissa
                           bits) x low bits; hand-built ties, subnormals and
                           overflow; the golden fixture
build_buckets              brute-force enumeration on tiny configs, the
                           layout invariants of tests/test_ddp.py:103-121 and
                           the closed-form cfg1/cfg2 bucket counts
pack / unpack              torch CPU ``copy_`` + ``mul_`` on the same inputs;
                           identity round trip
allreduce_sum              torch CPU sequential ``add_`` (fp32) and bf16 ``+``;
                           exact closed form W*x for power-of-two W
allreduce_op               torch CPU ``maximum`` / ``minimum`` / ``mul`` chains
                           over special values; numpy's max / min reductions
                           and exact power-of-two products
unscale_found_inf          torch CPU ``mul_`` + ``isfinite``; special values
ScalerState                known answers of tests/test_amp.py:19-104
fsdp_layout                closed form ceil(total/W); tests/test_fsdp.py
                           invariants
fsdp_reduce_scatter_share  torch CPU op sequence of fsdp.py:218-237 with an
                           explicit rank-ordered sum
=========================  ===================================================

The only thing left unpinned at bit level is the summation order inside
gloo/NCCL's all-reduce, which the reference delegates to the backend
(minidist/comm.py:234); the oracle fixes it to rank order 0..W-1.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

F32 = "f32"
BF16 = "bf16"
F16 = "f16"
_ITEMSIZE = {F32: 4, BF16: 2, F16: 2}

BF16_NAN = np.uint16(0xFFFF)


# ---------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------


def itemsize(dtype: str) -> int:
    return _ITEMSIZE[dtype]


def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even; NaN -> 0xFFFF.

    Follows the conversion behind ``Tensor.to(torch.bfloat16)`` at
    minidist/fsdp.py:180 and bf16 ``copy_`` at minidist/ddp.py:90,101.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    bias = np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    r = ((u.astype(np.uint64) + bias) >> np.uint64(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r[nan] = BF16_NAN
    return r


def f32_from_bf16(b: np.ndarray) -> np.ndarray:
    """bf16 bits -> fp32 (exact widening)."""
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(
        np.float32
    )


def f16_from_f32(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16, round to nearest even, in integer arithmetic.

    Follows ``Tensor.to(torch.float16)`` / fp16 ``copy_`` (the casts at
    minidist/fsdp.py:180 with ``param_dtype=torch.float16`` and
    minidist/ddp.py:90,101 for fp16 gradients).  Normal results rebias the
    exponent (127 -> 15) and round at mantissa bit 13; results below 2^-14
    are the significand (implicit bit included) shifted right by
    126 - exponent with the same ties-to-even rule; from 65520 up
    everything rounds to +-inf; a NaN becomes sign | 0x7E00 | mantissa >> 13.
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (u >> 16) & 0x8000
    a = u & 0x7FFFFFFF
    r = a - 0x38000000  # exponent 127 -> 15
    normal = (r + 0xFFF + ((r >> 13) & 1)) >> 13
    e = a >> 23
    m = (a & 0x7FFFFF) | 0x800000
    shift = np.clip(126 - e, 14, 25)
    q = m >> shift
    rem = m & ((1 << shift) - 1)
    half = 1 << (shift - 1)
    sub = q + ((rem > half) | ((rem == half) & ((q & 1) == 1)))
    out = np.where(a >= 0x38800000, normal, sub)
    out = np.where(a >= 0x477FF000, 0x7C00, out)
    out = np.where(a > 0x7F800000, 0x7E00 | ((a >> 13) & 0x3FF), out)
    return (sign | out).astype(np.uint16).view(np.float16)


def f32_from_f16(h: np.ndarray) -> np.ndarray:
    """fp16 -> fp32 (exact widening; numpy's conversion, subnormals included)."""
    return np.ascontiguousarray(h, dtype=np.float16).astype(np.float32)


def to_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == BF16:
        return f32_from_bf16(a)
    if dtype == F16:
        return f32_from_f16(a)
    return np.asarray(a, dtype=np.float32)


def from_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == BF16:
        return bf16_from_f32(a)
    if dtype == F16:
        return f16_from_f32(a)
    return np.asarray(a, dtype=np.float32)


def convert(a: np.ndarray, src: str, dst: str) -> np.ndarray:
    """``dst_tensor.copy_(src_tensor)`` across dtypes."""
    if src == dst:
        return np.array(a, copy=True)
    return from_f32(to_f32(a, src), dst)


def zeros(n: int, dtype: str) -> np.ndarray:
    return np.zeros(n, dtype={BF16: np.uint16, F16: np.float16}.get(dtype, np.float32))


def mul_scalar(a: np.ndarray, dtype: str, scale: float) -> np.ndarray:
    """``t.mul_(python_float)``: scalar rounded to fp32, product in fp32, rounded to dtype."""
    s = np.float32(scale)
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        return from_f32(to_f32(a, dtype) * s, dtype)


def div_scalar(a: np.ndarray, dtype: str, divisor: int) -> np.ndarray:
    """``t.div_(int)``: true fp32 division, rounded to dtype (minidist/fsdp.py:227)."""
    d = np.float32(divisor)
    with np.errstate(over="ignore", invalid="ignore", under="ignore", divide="ignore"):
        return from_f32(to_f32(a, dtype) / d, dtype)


def add(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    """``a + b`` in ``dtype`` with fp32 opmath (one rounding per add)."""
    with np.errstate(over="ignore", invalid="ignore"):
        return from_f32(to_f32(a, dtype) + to_f32(b, dtype), dtype)


def isfinite(a: np.ndarray, dtype: str) -> np.ndarray:
    return np.isfinite(to_f32(a, dtype))


# ---------------------------------------------------------------------------
# DDP bucketer (minidist/ddp.py)
# ---------------------------------------------------------------------------


def build_buckets(nbytes: list[int], cap_mb: float) -> list[list[int]]:
    """Greedy reverse-order bucketing; returns parameter indices per bucket.

    minidist/ddp.py:175-190: ``cap_bytes = int(cap_mb * 1024 * 1024)``; walk the
    parameters in reverse; flush when the bucket is non-empty and adding the
    next tensor would exceed the cap (so an oversize tensor sits alone).
    """
    cap_bytes = int(cap_mb * 1024 * 1024)
    buckets: list[list[int]] = []
    current: list[int] = []
    current_bytes = 0
    for i in reversed(range(len(nbytes))):
        pb = nbytes[i]
        if current and current_bytes + pb > cap_bytes:
            buckets.append(current)
            current, current_bytes = [], 0
        current.append(i)
        current_bytes += pb
    if current:
        buckets.append(current)
    return buckets


def bucket_offsets(numels: list[int]) -> tuple[list[int], int]:
    """Element offsets of each parameter in its bucket (minidist/ddp.py:61-66)."""
    offs, off = [], 0
    for n in numels:
        offs.append(off)
        off += n
    return offs, off


def pack(
    grads: list[np.ndarray | None],
    grad_dtypes: list[str],
    numels: list[int],
    bucket_dtype: str,
    scale: float,
) -> np.ndarray:
    """Flatten grads into one bucket, then multiply by ``scale``.

    minidist/ddp.py:82-92: buffer dtype = first parameter's dtype; ``zero_()``
    for a missing grad, ``copy_`` otherwise; then ``buffer.mul_(scale)``.
    """
    offs, total = bucket_offsets(numels)
    flat = zeros(total, bucket_dtype)
    for g, gd, off, n in zip(grads, grad_dtypes, offs, numels, strict=True):
        if g is not None:
            flat[off : off + n] = convert(g.reshape(-1), gd, bucket_dtype)
    return mul_scalar(flat, bucket_dtype, scale)


def allreduce_sum(contribs: list[np.ndarray], dtype: str) -> np.ndarray:
    """SUM all-reduce arithmetic, fixed rank order 0..W-1.

    minidist/comm.py:234 hands this to the backend; the oracle pins the order
    to ``acc = c0; acc += c1; ...`` with one rounding per add in ``dtype``.
    """
    acc = np.array(contribs[0], copy=True)
    for c in contribs[1:]:
        acc = add(acc, c, dtype)
    return acc


QUIET_NAN_BITS = {F32: 0x7FC00000, BF16: 0x7FC0, F16: 0x7E00}


def _bits(a: np.ndarray, dtype: str) -> np.ndarray:
    """The stored bit patterns of an oracle array (uint32 for fp32, uint16 otherwise)."""
    a = np.asarray(a)
    return a.view(np.uint32) if dtype == F32 else a.view(np.uint16)


def _from_bits_of(u: np.ndarray, dtype: str) -> np.ndarray:
    return u.view(np.float32) if dtype == F32 else (u if dtype == BF16 else u.view(np.float16))


def allreduce_op(contribs: list[np.ndarray], dtype: str, op: str) -> np.ndarray:
    """all_reduce with ``op`` in {"product", "min", "max"}, fixed rank order 0..W-1.

    minidist/comm.py:223-234 forwards ``op`` to the backend; the oracle folds
    ``acc = f(acc, c_r)`` in ``dtype`` with ``f`` the IEEE 754-2019 operations
    that torch's ``maximum`` / ``minimum`` and ``mul`` compute on the CPU:
    ``maximum`` / ``minimum`` -- NaN when either is NaN, else the larger /
    smaller value, where -0 < +0 (torch itself returns its first operand on a
    tie of -0 and +0 in its scalar loop and its second in its vectorised one;
    the IEEE rule makes the fold independent of rank order); ``mul`` -- the
    fp32 product rounded once to ``dtype``.  A NaN from maximum / minimum is
    the dtype's quiet NaN.
    """
    if op not in ("product", "min", "max"):
        raise ValueError(f"allreduce_op: unknown op {op!r}")
    acc = np.array(contribs[0], copy=True)
    for c in contribs[1:]:
        c = np.asarray(c)
        a, b = to_f32(acc, dtype), to_f32(c, dtype)
        if op == "product":
            with np.errstate(over="ignore", invalid="ignore", under="ignore"):
                acc = from_f32(a * b, dtype)
            continue
        # equal values have equal bits except the zeros: -0 & +0 = +0 (max), -0 | +0 = -0 (min)
        ua, ub = _bits(acc, dtype), _bits(c, dtype)
        tie = (ua & ub) if op == "max" else (ua | ub)
        res = _from_bits_of(np.where(a < b, ub, np.where(b < a, ua, tie)) if op == "max"
                            else np.where(b < a, ub, np.where(a < b, ua, tie)), dtype)
        nan = np.isnan(a) | np.isnan(b)
        if nan.any():
            bits = QUIET_NAN_BITS[dtype]
            if dtype == F32:
                res[nan] = np.array([bits], dtype=np.uint32).view(np.float32)[0]
            elif dtype == BF16:
                res[nan] = np.uint16(bits)
            else:
                res[nan] = np.array([bits], dtype=np.uint16).view(np.float16)[0]
        acc = res
    return acc


def unpack(
    flat: np.ndarray, bucket_dtype: str, numels: list[int], grad_dtypes: list[str | None]
) -> list[np.ndarray]:
    """Bucket -> per-parameter grads (minidist/ddp.py:94-102).

    ``grad_dtypes[i] is None`` means ``p.grad`` was None, so the reference
    clones the bucket slice (bucket dtype); otherwise ``copy_`` casts.
    """
    offs, _ = bucket_offsets(numels)
    out = []
    for off, n, gd in zip(offs, numels, grad_dtypes, strict=True):
        sl = flat[off : off + n]
        out.append(np.array(sl, copy=True) if gd is None else convert(sl, bucket_dtype, gd))
    return out


def unscale_found_inf(
    grads: list[np.ndarray | None], dtypes: list[str], inv_scale: float
) -> tuple[list[np.ndarray | None], bool]:
    """Per-grad ``mul_(inv_scale)`` then ``any(!isfinite)`` (minidist/amp.py:201-219)."""
    out: list[np.ndarray | None] = []
    found = False
    for g, d in zip(grads, dtypes, strict=True):
        if g is None:
            out.append(None)
            continue
        u = mul_scalar(g, d, inv_scale)
        found = found or bool((~isfinite(u, d)).any())
        out.append(u)
    return out, found


def ddp_pipeline(
    replica_grads: list[list[np.ndarray | None]],
    param_dtypes: list[str],
    numels: list[int],
    cap_mb: float,
    rank: int,
    inv_scale: float | None,
    bucket_dtype: str | None = None,
) -> dict:
    """The whole per-rank bucket pipeline for one step.

    pack(1/W) per replica (ddp.py:243-244) -> rank-ordered SUM (comm.py:234)
    -> unpack into rank ``rank``'s grads (ddp.py:269-273) -> optional
    unscale + found-inf (amp.py:201-219).  Grads are assumed to carry their
    parameter's dtype.  The bucket dtype is the first parameter's
    (ddp.py:84) unless ``bucket_dtype`` overrides it; a parameter without a
    gradient gets one of its own dtype.  Returns the layout, the reduced
    buckets, and the final grads of ``rank`` with their dtypes.
    """
    W = len(replica_grads)
    nbytes = [n * itemsize(d) for n, d in zip(numels, param_dtypes, strict=True)]
    layout = build_buckets(nbytes, cap_mb)
    final: list[np.ndarray | None] = [None] * len(numels)
    final_dtypes: list[str] = list(param_dtypes)
    reduced_buckets = []
    for idxs in layout:
        bdt = bucket_dtype or param_dtypes[idxs[0]]
        bn = [numels[i] for i in idxs]
        packed = [
            pack([replica_grads[r][i] for i in idxs], [param_dtypes[i] for i in idxs], bn, bdt, 1.0 / W)
            for r in range(W)
        ]
        red = allreduce_sum(packed, bdt)
        reduced_buckets.append(red)
        own = [param_dtypes[i] for i in idxs]
        for i, g in zip(idxs, unpack(red, bdt, bn, own), strict=True):
            final[i] = g
    found = None
    if inv_scale is not None:
        final, found = unscale_found_inf(final, final_dtypes, inv_scale)
    return {
        "layout": layout,
        "reduced": reduced_buckets,
        "grads": final,
        "grad_dtypes": final_dtypes,
        "found_inf": found,
    }


# ---------------------------------------------------------------------------
# Loss scaler state machine (minidist/amp.py)
# ---------------------------------------------------------------------------


@dataclass
class ScalerState:
    """Restatement of DistributedGradScaler's host arithmetic (amp.py:135-258)."""

    scale: float = 2.0**16
    growth_factor: float = 2.0
    backoff_factor: float = 0.5
    growth_interval: int = 2000
    min_scale: float = 1.0
    good_steps: int = 0
    num_skipped: int = 0
    num_steps: int = 0
    history: list = field(default_factory=list)

    def step(self, found_inf: bool) -> bool:
        """amp.py:223-238: count the step; skip it when the group found an inf."""
        self.num_steps += 1
        if found_inf:
            self.num_skipped += 1
            return False
        return True

    def update(self, found_inf: bool) -> None:
        """amp.py:240-258: backoff on overflow, growth after a clean interval."""
        if found_inf:
            self.scale = max(self.min_scale, self.scale * self.backoff_factor)
            self.good_steps = 0
        else:
            self.good_steps += 1
            if self.good_steps >= self.growth_interval:
                self.scale *= self.growth_factor
                self.good_steps = 0
        self.history.append(self.scale)


# ---------------------------------------------------------------------------
# FSDP flat-parameter unit (minidist/fsdp.py)
# ---------------------------------------------------------------------------


def fsdp_layout(numels: list[int], world: int) -> tuple[int, int, int]:
    """(total, shard_numel, padded_numel) -- minidist/fsdp.py:132-136."""
    total = sum(numels)
    shard = (total + world - 1) // world
    return total, shard, shard * world


def fsdp_gather_cast(flat_shard_f32: np.ndarray, param_dtype: str) -> np.ndarray:
    """``flat_shard.to(param_dtype)`` before the all-gather (fsdp.py:178-180)."""
    if param_dtype == F32:
        return np.array(flat_shard_f32, dtype=np.float32, copy=True)
    return from_f32(flat_shard_f32, param_dtype)


def fsdp_flatten(
    grads: list[np.ndarray | None], grad_dtype: str, numels: list[int], padded: int, reduce_dtype: str
) -> np.ndarray:
    """``buf = zeros(padded, reduce_dtype)`` + per-grad ``copy_`` (fsdp.py:218-223)."""
    buf = zeros(padded, reduce_dtype)
    off = 0
    for g, n in zip(grads, numels, strict=True):
        if g is not None:
            buf[off : off + n] = convert(g.reshape(-1), grad_dtype, reduce_dtype)
        off += n
    return buf


def fsdp_reduce_scatter_share(
    replica_grads: list[list[np.ndarray | None]],
    grad_dtype: str,
    numels: list[int],
    rank: int,
    reduce_dtype: str = F32,
    shard_dtype: str = F32,
    existing: np.ndarray | None = None,
) -> np.ndarray:
    """This rank's shard gradient after reduce_scatter_grads (fsdp.py:215-237).

    buf_r = flatten(grads_r) in reduce_dtype; if W > 1: buf_r /= W (true
    division), out = sum_r buf_r[rank*S:(rank+1)*S] in rank order; else out =
    buf.  ``out.to(shard_dtype)`` then set, or ``add_`` into ``existing``.
    """
    W = len(replica_grads)
    _, S, P = fsdp_layout(numels, W)
    bufs = [fsdp_flatten(g, grad_dtype, numels, P, reduce_dtype) for g in replica_grads]
    if W > 1:
        bufs = [div_scalar(b, reduce_dtype, W) for b in bufs]
        out = allreduce_sum([b[rank * S : (rank + 1) * S] for b in bufs], reduce_dtype)
    else:
        out = bufs[0]
    out = convert(out, reduce_dtype, shard_dtype)
    if existing is not None:
        out = add(existing, out, shard_dtype)
    return out


def bf16_tie_cases() -> tuple[np.ndarray, np.ndarray]:
    """Hand-built fp32 inputs with their RNE bf16 answers (independent of the formula).

    Halfway points between adjacent bf16 values round to the even neighbour;
    one ulp above/below a halfway point rounds away/toward.
    """
    one = 0x3F800000
    cases = [
        (one, 0x3F80),            # 1.0 exact
        (one | 0x8000, 0x3F80),   # 1 + half ulp: tie -> even (0x3F80)
        (one | 0x18000, 0x3F82),  # 1 + 1.5 ulp: tie -> even (0x3F82)
        (one | 0x8001, 0x3F81),   # just above the tie rounds up
        (one | 0x7FFF, 0x3F80),   # just below the tie rounds down
        (0x7F7FFFFF, 0x7F80),     # FLT_MAX overflows to +inf
        (0x7F7F7FFF, 0x7F7F),     # largest value that stays finite
        (0x7F7F8000, 0x7F80),     # tie at the top rounds to even = inf
        (0x00000001, 0x0000),     # smallest subnormal rounds to +0
        (0x00008000, 0x0000),     # subnormal tie -> even (0)
        (0x00018000, 0x0002),     # subnormal tie -> even (2)
        (0x80000000, 0x8000),     # -0
        (0x7F800000, 0x7F80),     # +inf
        (0xFF800000, 0xFF80),     # -inf
        (0x7FC00000, 0xFFFF),     # qNaN
        (0xFFC00001, 0xFFFF),     # negative NaN with payload
        (0x7F800001, 0xFFFF),     # sNaN
    ]
    x = np.array([c[0] for c in cases], dtype=np.uint32).view(np.float32)
    y = np.array([c[1] for c in cases], dtype=np.uint16)
    return x, y


def is_pow2(w: int) -> bool:
    return w > 0 and (w & (w - 1)) == 0


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


__all__ = [
    "F32", "BF16", "itemsize", "bf16_from_f32", "f32_from_bf16", "to_f32", "from_f32", "convert",
    "zeros", "mul_scalar", "div_scalar", "add", "isfinite", "build_buckets", "bucket_offsets",
    "pack", "allreduce_sum", "unpack", "unscale_found_inf", "ddp_pipeline", "ScalerState",
    "fsdp_layout", "fsdp_gather_cast", "fsdp_flatten", "fsdp_reduce_scatter_share",
    "bf16_tie_cases", "is_pow2", "ceil_div",
]
