"""The reference's CPU gradient path (torch CPU ops + gloo), for the CPU baseline.

TEST / MEASUREMENT INFRASTRUCTURE ONLY: bench.py's ``cpu_baseline`` leg times
this restatement on the host cores; nothing in the product calls it.

W processes (``torch.multiprocessing.spawn``, gloo over a FileStore, the
pattern of the reference's tests/common.py:26-60) each hold one replica's
gradients and run, per step, the reference's op sequence.

DDP (``run``; GPT configurations in fp32, Llama-7B layers in bf16 with fp32
buckets -- FSDP's reduce_dtype arithmetic applied to DDP buckets, as the GPU
path's cfg4 does):

* per bucket, in bucket order: per-parameter ``copy_`` into the flat buffer,
  ``mul_(1/W)``, async ``all_reduce(SUM)``  (minidist/ddp.py:75-92,243-247);
* ``wait`` then per-parameter ``copy_`` back (ddp.py:265-273);
* per gradient ``mul_(1/S)`` and ``found_inf += (~isfinite(g)).any()``, then
  ``all_reduce(MAX)`` and ``.item()`` (minidist/amp.py:201-219).

FSDP (``run_fsdp``; GPT-2-XL block units, cfg3), per unit:

* the unshard cast ``flat_shard.to(bfloat16)`` (minidist/fsdp.py:178-180);
* ``buf = zeros(padded, float32)``, per-parameter ``copy_`` of the bf16
  gradients, ``buf.div_(W)``, ``reduce_scatter_tensor(out, buf)``,
  ``out.to(float32)`` as the shard gradient (fsdp.py:215-235).

The unshard's all-gather is not timed: the GPU measurement of the same
configuration (the gather cast into this rank's slot and the reduce-scatter
share) does not include the peers' gather either.

The step overwrites the gradients in place, as the reference's does; every
step (warmup and timed) starts again from the same pristine gradients, copied
back outside the timed region, so that every timed step works on the same
normal-range values (not on gradients halved and unscaled step after step
into subnormals and zeros).

Timing: ``perf_counter`` around the step bracketed by barriers, max over
ranks, with Python's garbage collector paused over the timed steps.  Prints one JSON line.

    python -m oracle.gloo_path --config gpt2-small --world 8 --steps 3 --warmup 1 --threads 2
    python -m oracle.gloo_path --config llama-7b --layers 1 --world 8 --steps 3 --threads 2
    python -m oracle.gloo_path --fsdp --units 4 --world 8 --steps 3 --threads 2
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import torch
import torch.distributed as dist
import torch.multiprocessing as mp

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "distributed-training-framework_amd"))

from minidist import workloads as wl  # noqa: E402  (parameter tables only)

from .gradpath import build_buckets  # noqa: E402


def model_specs(cfg: dict, layers: int | None = None, layers_only: bool = False) -> list:
    """The parameter table of a configuration; ``layers`` keeps only the first ``layers`` blocks
    (GPT) or decoder layers (Llama) next to the embeddings, norms and head (``layers_only``: next
    to the norms only): a bounded sample."""
    if "ffn" in cfg:
        specs = wl.llama_specs(**cfg)
        prefix, big = "layers.", ("embed.weight", "lm_head.weight")
    else:
        specs = wl.gpt_specs(**cfg)
        prefix, big = "blocks.", ("embedding.wpe", "embedding.wte.weight", "lm_head.head.weight")
    if layers is not None:
        specs = [s for s in specs if not s.name.startswith(prefix) or int(s.name.split(".")[1]) < layers]
        if layers_only:
            specs = [s for s in specs if s.name not in big]
    return specs


def _worker(rank, world, store, cfg, steps, warmup, threads, cap_mb, scale, out_path, layers, grads_path=None,
            layers_only=False):
    torch.set_num_threads(threads)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world)
    specs = model_specs(cfg, layers, layers_only)
    g = torch.Generator().manual_seed(1234 + 7919 * rank)
    # bf16 parameters (Llama) sum in fp32 buckets; fp32 parameters in fp32 buckets
    pristine = [(torch.randn(s.numel, generator=g) * (1e-3 * scale)).to(s.dtype) for s in specs]
    grads = [t.clone() for t in pristine]
    layout = build_buckets([s.nbytes for s in specs], cap_mb)
    buffers = [torch.zeros(sum(specs[i].numel for i in idx), dtype=torch.float32) for idx in layout]
    inv_w, inv_s = 1.0 / world, 1.0 / scale

    def step() -> bool:
        works = []
        for idx, buf in zip(layout, buffers):
            off = 0
            for i in idx:
                n = specs[i].numel
                buf[off : off + n].copy_(grads[i])
                off += n
            buf.mul_(inv_w)
            works.append(dist.all_reduce(buf, async_op=True))
        for idx, buf, work in zip(layout, buffers, works):
            work.wait()
            off = 0
            for i in idx:
                n = specs[i].numel
                grads[i].copy_(buf[off : off + n])
                off += n
        found = torch.zeros(1)
        for t in grads:
            t.mul_(inv_s)
            found += (~torch.isfinite(t)).any().to(found.dtype)
        dist.all_reduce(found, op=dist.ReduceOp.MAX)
        return bool(found.item() > 0)

    def restore() -> None:
        for t, t0 in zip(grads, pristine):
            t.copy_(t0)

    for _ in range(warmup):
        restore()
        step()
    times = []
    gc.collect()
    gc.disable()  # as in the GPU measurement: no collector pause inside a timed step
    for _ in range(steps):
        restore()
        dist.barrier()
        t0 = time.perf_counter()
        step()
        dist.barrier()
        times.append(time.perf_counter() - t0)
    gc.enable()
    t = torch.tensor(times, dtype=torch.float64)
    dist.all_reduce(t, op=dist.ReduceOp.MAX)
    if rank == 0:
        numel = sum(s.numel for s in specs)
        Path(out_path).write_text(
            json.dumps({"step_s": t.tolist(), "numel": numel, "buckets": len(layout)})
        )
        if grads_path is not None:  # checking runs: rank 0's gradients after the last step
            torch.save([gr.clone() for gr in grads], grads_path)
    dist.barrier()
    dist.destroy_process_group()


def run(world: int, steps: int, warmup: int, threads: int, cfg: dict, cap_mb: float = 25.0,
        scale: float = 2.0**16, layers: int | None = None, grads_path: str | None = None,
        layers_only: bool = False) -> dict:
    """Time the path; with ``grads_path``, rank 0's final gradients are saved there (torch.save)."""
    with tempfile.TemporaryDirectory() as tmp:
        store = os.path.join(tmp, "store")
        out = os.path.join(tmp, "out.json")
        mp.spawn(
            _worker,
            args=(world, store, cfg, steps, warmup, threads, cap_mb, scale, out, layers, grads_path, layers_only),
            nprocs=world,
            join=True,
        )
        res = json.loads(Path(out).read_text())
    step_s = sorted(res["step_s"])
    med = step_s[len(step_s) // 2]
    return {
        "world": world,
        "threads_per_rank": threads,
        "cores": world * threads,
        "numel": res["numel"],
        "buckets": res["buckets"],
        "best_ms": step_s[0] * 1e3,
        "median_ms": med * 1e3,
        "steps": steps,
    }


def _fsdp_worker(rank, world, store, h, units, steps, warmup, threads, out_path, check_path=None):
    torch.set_num_threads(threads)
    dist.init_process_group("gloo", init_method=f"file://{store}", rank=rank, world_size=world)
    numels = [s.numel for s in wl.gpt_block_specs(0, h)]
    total = sum(numels)
    S = (total + world - 1) // world  # fsdp.py:132-136
    P = S * world
    g = torch.Generator().manual_seed(4321 + 7919 * rank)
    masters = [torch.randn(S, generator=g) * 0.02 for _ in range(units)]
    grads = [[(torch.randn(n, generator=g) * 1e-3).to(torch.bfloat16) for n in numels] for _ in range(units)]
    gathered: list = [None] * units
    shard_grads: list = [None] * units

    def step() -> None:
        for u in range(units):
            gathered[u] = masters[u].to(torch.bfloat16)  # unshard's cast (fsdp.py:178-180)
            buf = torch.zeros(P, dtype=torch.float32)  # reduce_scatter_grads (fsdp.py:218-235)
            off = 0
            for t, n in zip(grads[u], numels):
                buf[off : off + n].copy_(t.reshape(-1))
                off += n
            buf.div_(world)
            out = torch.empty(S, dtype=torch.float32)
            dist.reduce_scatter_tensor(out, buf)
            shard_grads[u] = out.to(torch.float32)

    for _ in range(warmup):
        step()
    times = []
    gc.collect()
    gc.disable()
    for _ in range(steps):
        dist.barrier()
        t0 = time.perf_counter()
        step()
        dist.barrier()
        times.append(time.perf_counter() - t0)
    gc.enable()
    t = torch.tensor(times, dtype=torch.float64)
    dist.all_reduce(t, op=dist.ReduceOp.MAX)
    if rank == 0:
        Path(out_path).write_text(json.dumps({"step_s": t.tolist(), "shard_numel": S, "padded_numel": P}))
    if check_path is not None:  # checking runs: every rank's inputs and rank 0's results
        torch.save({"masters": masters, "grads": grads, "gathered": gathered, "shard_grads": shard_grads},
                   f"{check_path}.{rank}")
    dist.barrier()
    dist.destroy_process_group()


def run_fsdp(world: int, units: int, steps: int, warmup: int, threads: int, h: int = 1600,
             total_units: int = 48, check_path: str | None = None) -> dict:
    """Time ``units`` GPT-2-XL block units per step (a bounded sample of ``total_units``); the
    per-step figure for all units is the sample's median scaled by total_units / units."""
    with tempfile.TemporaryDirectory() as tmp:
        store = os.path.join(tmp, "store")
        out = os.path.join(tmp, "out.json")
        mp.spawn(_fsdp_worker, args=(world, store, h, units, steps, warmup, threads, out, check_path),
                 nprocs=world, join=True)
        res = json.loads(Path(out).read_text())
    step_s = sorted(res["step_s"])
    med = step_s[len(step_s) // 2]
    scale = total_units / units
    return {
        "world": world,
        "threads_per_rank": threads,
        "cores": world * threads,
        "shard_numel": res["shard_numel"],
        "units_timed": units,
        "best_ms": step_s[0] * 1e3 * scale,
        "median_ms": med * 1e3 * scale,
        "steps": steps,
        "note": f"{units} of {total_units} units timed per step, scaled by {total_units}/{units}",
    }


CONFIGS = {"tiny": wl.TINY_GPT, "gpt2-small": wl.GPT2_SMALL, "gpt2-medium": wl.GPT2_MEDIUM, "llama-7b": wl.LLAMA_7B}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="gpt2-small", choices=sorted(CONFIGS))
    ap.add_argument("--world", type=int, default=8)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--threads", type=int, default=2)
    ap.add_argument("--layers", type=int, default=None,
                    help="time only the first LAYERS blocks / decoder layers (plus embeddings, norms and head) and "
                         "scale the step time to the whole model by element count")
    ap.add_argument("--layers-only", action="store_true",
                    help="with --layers: leave the embeddings and head out of the timed sample too")
    ap.add_argument("--scale", type=float, default=2.0**16, help="loss scale the gradients carry")
    ap.add_argument("--fsdp", action="store_true", help="the FSDP unit path (GPT-2-XL block units) instead of DDP")
    ap.add_argument("--units", type=int, default=4, help="--fsdp: units timed per step (of 48)")
    args = ap.parse_args()
    if args.fsdp:
        print(json.dumps(run_fsdp(args.world, args.units, args.steps, args.warmup, args.threads)))
        return
    cfg = CONFIGS[args.config]
    res = run(args.world, args.steps, args.warmup, args.threads, cfg, scale=args.scale, layers=args.layers,
              layers_only=args.layers_only)
    if args.layers is not None:
        full = wl.total_numel(model_specs(cfg))
        factor = full / res["numel"]
        what = "layers" + ("" if args.layers_only else " with the embeddings and head")
        res["note"] = (f"first {args.layers} {what} timed ({res['numel']:,} of {full:,} elements), scaled by "
                       f"element count x{factor:.2f}")
        res["sample_ms"] = res["median_ms"]
        res["best_ms"] *= factor
        res["median_ms"] *= factor
        res["numel"] = full
    print(json.dumps(res))


if __name__ == "__main__":
    main()
