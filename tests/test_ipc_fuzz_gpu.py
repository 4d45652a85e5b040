"""Seeded random DDP pipelines over IPC-mapped rows: W processes on the one GPU (comm.IpcGroup).

Each case draws W in [2, 4], one- or two-shot, the gradient dtype (fp32, bf16
or fp16, the 16-bit ones optionally widened into fp32 buckets), 10-30
parameters of ragged shapes (some empty), a bucket cap from one bucket per
parameter to a single bucket, the symmetric-buffer segment size (so that the
buckets spread over one or several buffers), DDP's communication stream or
not, and the fused scaler or not.  Every rank draws every rank's gradients from
the same seed, with rare special values and, on some ranks, parameters that
received no gradient.  Two steps run (new gradient tensors in the second).
Every rank's gradients and buckets are checked bit for bit against the oracle's
rank-ordered pipeline (``oracle.gradpath.ddp_pipeline``) over all ranks'
gradients, and the found-inf decision against the oracle's.  The reference
hands each bucket to ``dist.all_reduce`` (minidist/comm.py:223-234,
ddp.py:243-274).
"""

from __future__ import annotations

import os
from datetime import timedelta

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp
from torch import nn

from conftest import first_mismatch, same_bits
from minidist import DDP, DistributedGradScaler, IpcGroup
from oracle import gradpath as o

pytestmark = pytest.mark.gpu
SPECIALS = np.array([np.inf, -np.inf, np.nan, 1e-45, -1e-40, 0.0, -0.0], dtype=np.float32)
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
STEPS = 2


def _case(seed: int) -> dict:
    """The whole case, drawn from ``seed`` alone (the parent and every rank draw the same)."""
    rng = np.random.default_rng(41000 + seed)
    dtype = DTYPES[int(rng.integers(0, 3))]
    widening = dtype != torch.float32 and bool(rng.random() < 0.5)
    gdt = {torch.bfloat16: o.BF16, torch.float16: o.F16}.get(dtype, o.F32)
    W = int(rng.integers(2, 5))
    algorithm = ["one_shot", "two_shot"][int(rng.integers(0, 2))]
    n_params = int(rng.integers(10, 31))
    shapes = []
    for _ in range(n_params):
        u = rng.random()
        shapes.append((0,) if u < 0.1 else (int(rng.integers(1, 5000)),) if u < 0.8
                      else (int(rng.integers(1, 60)), int(rng.integers(1, 50))))
    numels = [int(np.prod(s)) for s in shapes]
    esize = 4 if dtype == torch.float32 or widening else 2
    nbytes = [n * (4 if dtype == torch.float32 else 2) for n in numels]
    total_mb = sum(nbytes) / 2**20
    cap = float(rng.choice([1e-6, total_mb / 5, total_mb / 2, 1e6]))
    # segments: the default, or small enough that the buckets spread over several buffers
    largest = max(sum(numels[i] for i in idxs) for idxs in o.build_buckets(nbytes, cap))
    small = max(256, (largest * esize + 255) // 256 * 256, int(rng.integers(1, 5)) * 16384)
    segment_bytes = [1 << 30, small][int(rng.integers(0, 2))]
    use_scaler = bool(rng.random() < 0.6)
    scale = 2.0 ** int(rng.integers(0, 14 if dtype != torch.float16 else 10)) if use_scaler else 1.0
    comm_stream = bool(rng.random() < 0.4)
    grads = []  # [step][rank][param]
    for _ in range(STEPS):
        per_rank = []
        for _ in range(W):
            row = []
            for n in numels:
                g = (rng.standard_normal(n) * 1e-3 * scale).astype(np.float32)
                if n and rng.random() < 0.04:
                    g[int(rng.integers(0, n))] = SPECIALS[int(rng.integers(0, len(SPECIALS)))]
                row.append(o.from_f32(g, gdt))
            for i in rng.integers(0, n_params, int(rng.integers(0, 3))):  # never received on this rank
                row[int(i)] = None
            per_rank.append(row)
        grads.append(per_rank)
    return dict(dtype=dtype, widening=widening, gdt=gdt, W=W, algorithm=algorithm, shapes=shapes, numels=numels,
                cap=cap, segment_bytes=segment_bytes, use_scaler=use_scaler, scale=scale, comm_stream=comm_stream,
                grads=grads)


def _describe(seed: int, c: dict) -> str:
    return (f"ipc fuzz seed {seed}: W={c['W']} {c['algorithm']} {c['dtype']} widening={c['widening']} "
            f"params={len(c['shapes'])} cap={c['cap']:.3g} MB segment={c['segment_bytes']} "
            f"comm_stream={c['comm_stream']} scale={c['scale']:g}")


class _Flat(nn.Module):
    def __init__(self, shapes, dtype, dev):
        super().__init__()
        self.ps = nn.ParameterList([nn.Parameter(torch.zeros(s, dtype=dtype, device=dev)) for s in shapes])


def _to_dev(a: np.ndarray, shape, dev) -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(dev).view(shape)
    return torch.from_numpy(a.copy()).to(dev).view(shape)


def _host_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().reshape(-1).cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def _worker(rank: int, world: int, store: str, out_dir: str, seed: int) -> None:
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world,
                            timeout=timedelta(seconds=60))
    try:
        c = _case(seed)
        group = IpcGroup(dist.group.WORLD, dev, algorithm=c["algorithm"], segment_bytes=c["segment_bytes"])
        model = _Flat(c["shapes"], c["dtype"], dev)
        params = list(model.parameters())
        scaler = DistributedGradScaler(init_scale=c["scale"], process_group=group) if c["use_scaler"] else None
        ddp = DDP(model, process_group=group, bucket_cap_mb=c["cap"], grad_scaler=scaler,
                  reduce_dtype=torch.float32 if c["widening"] else None, comm_stream=c["comm_stream"])

        class _Opt:
            param_groups = [{"params": params}]

        out = {"buckets": np.array(len(ddp._buckets)), "segments": np.array(len({b.segment for b in ddp._buckets}))}
        for step in range(STEPS):
            for p, g in zip(params, c["grads"][step][rank], strict=True):
                p.grad = None if g is None else _to_dev(g, p.shape, dev)
            ddp.finish_gradient_sync()
            if scaler is not None:
                out[f"found_{step}"] = np.array(scaler.unscale_(_Opt()))
                scaler.update()
                out[f"scale_after_{step}"] = np.array(scaler.scale)
            torch.cuda.synchronize()
            for i, p in enumerate(params):
                out[f"grad_{step}_{i}"] = _host_bits(p.grad)
            for b, bucket in enumerate(ddp._buckets):
                out[f"bucket_{step}_{b}"] = _host_bits(bucket.buffer[: bucket.numel])
        group.release()
        np.savez(os.path.join(out_dir, f"fuzz_r{rank}.npz"), **out)
    finally:
        dist.destroy_process_group()


@pytest.mark.parametrize("seed", range(12))
def test_random_ipc_pipeline_matches_oracle(tmp_path, seed):
    c = _case(seed)
    case = _describe(seed, c)
    print(case, flush=True)
    W = c["W"]
    mp.spawn(_worker, args=(W, str(tmp_path / "store"), str(tmp_path), seed), nprocs=W, join=True)
    res = []
    for r in range(W):
        with np.load(tmp_path / f"fuzz_r{r}.npz", allow_pickle=False) as d:
            res.append({k: d[k] for k in d.files})
    n = len(c["numels"])
    print(f"  {int(res[0]['buckets'])} buckets in {int(res[0]['segments'])} symmetric buffer(s)", flush=True)
    scaler = o.ScalerState(scale=c["scale"])  # a step that found an inf halves the next step's scale
    for step in range(STEPS):
        for rank in range(W):
            want = o.ddp_pipeline(c["grads"][step], [c["gdt"]] * n, c["numels"], c["cap"], rank,
                                  1.0 / scaler.scale if c["use_scaler"] else None,
                                  bucket_dtype=o.F32 if c["widening"] else None)
            assert int(res[rank]["buckets"]) == len(want["layout"]), case
            if c["use_scaler"]:
                assert bool(res[rank][f"found_{step}"]) == want["found_inf"], f"{case} step {step} rank {rank}"
            for i in range(n):
                got = res[rank][f"grad_{step}_{i}"]
                assert same_bits(got, want["grads"][i]), (
                    f"{case} step {step} rank {rank} param {i}: " + first_mismatch(got, want["grads"][i]))
            for b, red in enumerate(want["reduced"]):
                got = res[rank][f"bucket_{step}_{b}"]
                assert same_bits(got, red), f"{case} step {step} rank {rank} bucket {b}: " + first_mismatch(got, red)
        if c["use_scaler"]:
            scaler.update(want["found_inf"])
            assert all(float(res[r][f"scale_after_{step}"]) == scaler.scale for r in range(W)), case
