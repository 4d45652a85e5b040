"""Write the golden fixtures under tests/golden/ (run from the repo root).

The reference (minidist) ships no data files, so these vectors are produced by
replaying the reference's *ATen op chains* with torch CPU tensors -- the same
library calls, in the same order, that its Python issues -- on small seeded
inputs.  This is independent of the numpy oracle in oracle/gradpath.py, which
the CPU tests check against these files.  The reference package itself is not
imported; each chain below cites the lines it replays.

  python tests/golden/make_golden.py          # writes the fixtures that are missing
  python tests/golden/make_golden.py --force  # rewrites every fixture
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent

DDP_NUMELS = [3, 64, 5, 130, 1, 33, 256, 7, 96, 2, 513, 40]
FSDP_NUMELS = [7, 12, 5, 33, 64, 3]


def _bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().astype(np.uint16)
    return t.numpy().copy()  # fp32 -> float32, fp16 -> float16


def _specials(g: torch.Generator, n: int) -> torch.Tensor:
    pool = torch.tensor(
        [0.0, -0.0, 1e-40, -1e-42, 3.0e38, -3.0e38, 1.0, 2.0**-126, 7.5e-39, 65504.0], dtype=torch.float32
    )
    return pool[torch.randint(0, len(pool), (n,), generator=g)]


def _specials_f16(g: torch.Generator, n: int) -> torch.Tensor:
    """fp16's own edge values: subnormals, the largest finite value, the smallest normal."""
    pool = torch.tensor(
        [0.0, -0.0, 6e-8, -1.2e-7, 60000.0, -65504.0, 1.0, 2.0**-14, 3.0e-5, 65504.0], dtype=torch.float32
    )
    return pool[torch.randint(0, len(pool), (n,), generator=g)]


# ---------------------------------------------------------------------------
# bf16 cast (fsdp.py:178-180 `flat_shard.to(param_dtype)`)
# ---------------------------------------------------------------------------


def bf16_cast() -> dict:
    g = torch.Generator().manual_seed(11)
    words = [
        0x3F800000, 0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF, 0x7F7FFFFF, 0x7F7F7FFF,
        0x7F7F8000, 0x00000001, 0x00008000, 0x00018000, 0x80000000, 0x7F800000, 0xFF800000,
        0x7FC00000, 0xFFC00001, 0x7F800001, 0x807FFFFF, 0x00FF8000, 0x80008000,
    ]
    rand = torch.randint(0, 2**32, (4000,), generator=g, dtype=torch.int64)
    # bias half of the random words to rounding boundaries
    rand[:2000] = (rand[:2000] & ~0xFFFF) | torch.tensor([0x7FFF, 0x8000, 0x8001, 0x0000])[
        torch.randint(0, 4, (2000,), generator=g)
    ]
    u = np.concatenate([np.array(words, dtype=np.uint32), rand.numpy().astype(np.uint32)])
    x = torch.from_numpy(u.view(np.float32).copy())
    return {"x_bits": u, "y_bits": _bits(x.to(torch.bfloat16))}


# ---------------------------------------------------------------------------
# fp16 cast (fsdp.py:178-180 `flat_shard.to(param_dtype)` with param_dtype=float16)
# ---------------------------------------------------------------------------


def f16_cast() -> dict:
    g = torch.Generator().manual_seed(17)
    words = [
        0x3F800000, 0x3F801000, 0x3F803000, 0x3F801001, 0x3F800FFF,  # 1.0; ties at mantissa bit 12
        0x477FE000, 0x477FEFFF, 0x477FF000, 0x477FFFFF, 0x47800000,  # 65504 .. the overflow threshold
        0x38800000, 0x387FF000, 0x387FE000, 0x387FFFFF,  # 2^-14 and just below (subnormal -> normal)
        0x33800000, 0x33000000, 0x33000001, 0x32FFFFFF, 0x33C00000, 0x34200000,  # 2^-24, 2^-25 ties
        0x00000001, 0x80000000, 0x7F800000, 0xFF800000, 0x7F7FFFFF,
        0x7FC00000, 0xFFC12345, 0x7F800001, 0x7FA00000,  # NaNs: quiet, payload, signalling
    ]
    rand = torch.randint(0, 2**32, (4000,), generator=g, dtype=torch.int64)
    # exponents that land in fp16's range, low bits at rounding boundaries
    rand[:2000] = ((rand[:2000] & 0x807FFFFF) | (torch.randint(100, 145, (2000,), generator=g) << 23)) & ~0x3F
    u = np.concatenate([np.array(words, dtype=np.uint32), rand.numpy().astype(np.uint32)])
    x = torch.from_numpy(u.view(np.float32).copy())
    return {"x_bits": u, "y_bits": x.to(torch.float16).view(torch.int16).numpy().view(np.uint16)}


# ---------------------------------------------------------------------------
# DDP bucket pipeline + unscale (ddp.py:75-102,175-190,243-274; amp.py:201-219)
# ---------------------------------------------------------------------------


def _build_buckets(nbytes: list[int], cap_mb: float) -> list[list[int]]:
    cap_bytes = int(cap_mb * 1024 * 1024)
    buckets, cur, cur_b = [], [], 0
    for i in reversed(range(len(nbytes))):
        if cur and cur_b + nbytes[i] > cap_bytes:
            buckets.append(cur)
            cur, cur_b = [], 0
        cur.append(i)
        cur_b += nbytes[i]
    if cur:
        buckets.append(cur)
    return buckets


def ddp_case(
    dtype: torch.dtype, W: int, rank: int, cap_mb: float, scale: float, seed: int, inject_inf: bool,
    bucket_dtype: torch.dtype | None = None,
) -> dict:
    """``bucket_dtype`` replays a bucket whose dtype differs from the gradients'
    (the first parameter's dtype in the reference, ddp.py:84): ``copy_`` then
    widens on pack and rounds on unpack."""
    bucket_dtype = bucket_dtype or dtype
    g = torch.Generator().manual_seed(seed)
    n_params = len(DDP_NUMELS)
    grads: list[list[torch.Tensor | None]] = []
    for r in range(W):
        row = []
        for i, n in enumerate(DDP_NUMELS):
            t = torch.randn(n, generator=g) * 1e-2 * scale
            k = max(1, n // 8)
            idx = torch.randint(0, n, (k,), generator=g)
            if dtype == torch.float16:
                t[idx] = _specials_f16(g, k)
            else:
                t[idx] = _specials(g, k) * (1.0 if dtype == torch.float32 else 1e-30)
            row.append(t.to(dtype))
        grads.append(row)
    grads[rank][4] = None  # this rank's param 4 got no gradient (zero-filled, then cloned)
    if inject_inf:
        grads[(rank + 1) % W][6][17] = float("inf")
    itemsize = torch.empty((), dtype=dtype).element_size()
    layout = _build_buckets([n * itemsize for n in DDP_NUMELS], cap_mb)
    final: list[torch.Tensor | None] = [None] * n_params
    reduced = []
    for idxs in layout:
        numel = sum(DDP_NUMELS[i] for i in idxs)
        packed = []
        for r in range(W):
            buf = torch.zeros(numel, dtype=bucket_dtype)  # ddp.py:83-84
            off = 0
            for i in idxs:
                flat = buf[off : off + DDP_NUMELS[i]]
                if grads[r][i] is None:
                    flat.zero_()  # ddp.py:87-88
                else:
                    flat.copy_(grads[r][i].reshape(-1))  # ddp.py:90
                off += DDP_NUMELS[i]
            buf.mul_(1.0 / W)  # ddp.py:91
            packed.append(buf)
        acc = packed[0].clone()
        for r in range(1, W):
            acc.add_(packed[r])  # rank-ordered SUM (comm.py:234)
        reduced.append(acc)
        off = 0
        for i in idxs:
            sl = acc[off : off + DDP_NUMELS[i]]
            if grads[rank][i] is None:
                # ddp.py:98-99; torch only accepts a gradient of the parameter dtype
                final[i] = sl.clone() if bucket_dtype == dtype else torch.empty(sl.shape, dtype=dtype).copy_(sl)
            else:
                final[i] = grads[rank][i].clone().copy_(sl)  # ddp.py:100-101
            off += DDP_NUMELS[i]
    unscaled = []
    found_inf = torch.zeros(1)
    for t in final:  # amp.py:208-213
        u = t.clone().mul_(1.0 / scale)
        found_inf += (~torch.isfinite(u)).any().to(found_inf.dtype)
        unscaled.append(u)
    out = {
        "W": W, "rank": rank, "cap_mb": cap_mb, "scale": scale, "dtype": str(dtype),
        "bucket_dtype": str(bucket_dtype),
        "numels": np.array(DDP_NUMELS), "found_inf": bool(found_inf.item() > 0),
        "layout": json.dumps(layout),
    }
    for r in range(W):
        for i in range(n_params):
            if grads[r][i] is not None:
                out[f"grad_r{r}_p{i}"] = _bits(grads[r][i])
    for b, t in enumerate(reduced):
        out[f"reduced_b{b}"] = _bits(t)
    for i in range(n_params):
        out[f"final_p{i}"] = _bits(final[i])
        out[f"unscaled_p{i}"] = _bits(unscaled[i])
    return out


# ---------------------------------------------------------------------------
# FSDP unit: gather cast and reduce_scatter_grads (fsdp.py:130-151,172-241)
# ---------------------------------------------------------------------------


def fsdp_case(W: int, grad_dtype: torch.dtype, reduce_dtype: torch.dtype, seed: int,
              cast_dtype: torch.dtype = torch.bfloat16) -> dict:
    """``cast_dtype`` is the gather dtype (MixedPrecisionPolicy.param_dtype)."""
    g = torch.Generator().manual_seed(seed)
    total = sum(FSDP_NUMELS)
    S = (total + W - 1) // W  # fsdp.py:135
    P = S * W
    master_flat = torch.zeros(P)
    master_flat[:total] = torch.randn(total, generator=g) * 0.02
    out = {"W": W, "S": S, "P": P, "numels": np.array(FSDP_NUMELS), "grad_dtype": str(grad_dtype),
           "reduce_dtype": str(reduce_dtype), "master_flat": master_flat.numpy().copy()}
    if cast_dtype != torch.bfloat16:
        out["cast_dtype"] = str(cast_dtype)
    for r in range(W):
        out[f"gather_cast_r{r}"] = _bits(master_flat[r * S : (r + 1) * S].clone().to(cast_dtype))
    grads = []
    for r in range(W):
        row = []
        for i, n in enumerate(FSDP_NUMELS):
            if (r + i) % 5 == 3:
                row.append(None)  # missing grad -> stays zero in buf
                continue
            t = (torch.randn(n, generator=g) * 1e-3).to(grad_dtype)
            row.append(t)
            out[f"grad_r{r}_p{i}"] = _bits(t)
        grads.append(row)
    bufs = []
    for r in range(W):
        buf = torch.zeros(P, dtype=reduce_dtype)  # fsdp.py:218
        off = 0
        for i, n in enumerate(FSDP_NUMELS):
            if grads[r][i] is not None:
                buf[off : off + n].copy_(grads[r][i].reshape(-1))  # fsdp.py:222
            off += n
        if W > 1:
            buf.div_(W)  # fsdp.py:227
        bufs.append(buf)
    for rank in range(W):
        acc = bufs[0][rank * S : (rank + 1) * S].clone()
        for r in range(1, W):
            acc.add_(bufs[r][rank * S : (rank + 1) * S])  # rank-ordered reduce-scatter SUM
        shard_grad = acc.to(torch.float32)  # fsdp.py:233
        out[f"shard_grad_r{rank}"] = _bits(shard_grad)
        prev = torch.randn(S, generator=g) * 1e-3
        out[f"prev_r{rank}"] = prev.numpy().copy()
        out[f"shard_grad_acc_r{rank}"] = _bits(prev.clone().add_(shard_grad))  # fsdp.py:237
    return out


FIXTURES = {
    "bf16_cast.npz": bf16_cast,
    "f16_cast.npz": f16_cast,
    "ddp_f32_w4.npz": lambda: ddp_case(torch.float32, W=4, rank=1, cap_mb=0.001, scale=2.0**16, seed=5,
                                       inject_inf=False),
    "ddp_f32_w3_inf.npz": lambda: ddp_case(torch.float32, W=3, rank=2, cap_mb=0.002, scale=2.0**10, seed=6,
                                           inject_inf=True),
    "ddp_bf16_w8.npz": lambda: ddp_case(torch.bfloat16, W=8, rank=5, cap_mb=0.0005, scale=2.0**12, seed=7,
                                        inject_inf=False),
    "ddp_bf16_f32bucket_w8.npz": lambda: ddp_case(torch.bfloat16, W=8, rank=3, cap_mb=0.0005, scale=2.0**12,
                                                  seed=13, inject_inf=True, bucket_dtype=torch.float32),
    "ddp_f16_w4_inf.npz": lambda: ddp_case(torch.float16, W=4, rank=2, cap_mb=0.0005, scale=2.0**10, seed=14,
                                           inject_inf=True),
    "ddp_f16_f32bucket_w8.npz": lambda: ddp_case(torch.float16, W=8, rank=6, cap_mb=0.0005, scale=2.0**10,
                                                 seed=15, inject_inf=False, bucket_dtype=torch.float32),
    "fsdp_bf16_w4.npz": lambda: fsdp_case(4, torch.bfloat16, torch.float32, seed=8),
    "fsdp_bf16_w3.npz": lambda: fsdp_case(3, torch.bfloat16, torch.float32, seed=9),
    "fsdp_f32_w2.npz": lambda: fsdp_case(2, torch.float32, torch.float32, seed=10),
    "fsdp_bf16red_w4.npz": lambda: fsdp_case(4, torch.bfloat16, torch.bfloat16, seed=12),
    "fsdp_f16_w4.npz": lambda: fsdp_case(4, torch.float16, torch.float32, seed=16, cast_dtype=torch.float16),
    "fsdp_f16red_w3.npz": lambda: fsdp_case(3, torch.float16, torch.float16, seed=18, cast_dtype=torch.float16),
}


def main() -> None:
    force = "--force" in sys.argv[1:]
    for name, make in FIXTURES.items():
        if force or not (HERE / name).exists():
            np.savez_compressed(HERE / name, **make())
    # Scaler known answers from the reference's tests/test_amp.py.
    kat = {
        "overflow_skips": {"init_scale": 1024.0, "found": [True], "scale_after": 512.0, "num_skipped": 1,
                           "source": "tests/test_amp.py:19-43"},
        "clean_growth": {"init_scale": 1024.0, "growth_interval": 2, "found": [False, False],
                         "scale_after": 2048.0, "num_skipped": 0, "source": "tests/test_amp.py:46-59"},
        "mixed_history": {"init_scale": 4096.0, "growth_interval": 2,
                          "found": [True, False, False, True, True], "scale_after": 1024.0,
                          "source": "tests/test_amp.py:83-104 (nan on rank 0, nobody, nobody, rank 1, rank 1)"},
        "unscale_value": {"init_scale": 256.0, "grad": 3.0 * 256.0, "unscaled": 3.0,
                          "source": "tests/test_amp.py:62-80"},
    }
    (HERE / "scaler_kat.json").write_text(json.dumps(kat, indent=1) + "\n")


if __name__ == "__main__":
    main()
