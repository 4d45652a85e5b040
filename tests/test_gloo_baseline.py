"""The CPU baseline runner (oracle/gloo_path.py) computes the reference path's result.

bench.py times this runner as the reference's CPU path.  Here two gloo ranks
(spawned processes, CPU only) run one step on the tiny GPT configuration and
rank 0's gradients are compared bit for bit with oracle.ddp_pipeline on the
same seeded gradients: with two ranks the backend's sum a + b is the same in
either order, so nothing is left to the backend.
"""

from __future__ import annotations

import numpy as np
import torch

from minidist import workloads as wl
from oracle import gloo_path
from oracle import gradpath as o


def test_two_rank_gloo_step_matches_oracle(tmp_path):
    W, scale, cap = 2, 2.0**16, 0.05  # a small cap: several buckets
    cfg = dict(n_layer=2, n_embd=64, vocab=128, ctx=32)
    specs = wl.gpt_specs(**cfg)
    path = str(tmp_path / "grads.pt")
    res = gloo_path.run(W, steps=1, warmup=0, threads=1, cfg=cfg, cap_mb=cap, scale=scale, grads_path=path)
    assert res["numel"] == wl.total_numel(specs) and res["buckets"] > 2
    got = torch.load(path, weights_only=True)
    replica = []
    for r in range(W):  # the runner's generator recipe
        g = torch.Generator().manual_seed(1234 + 7919 * r)
        replica.append([(torch.randn(s.numel, generator=g) * (1e-3 * scale)).numpy() for s in specs])
    want = o.ddp_pipeline(replica, [o.F32] * len(specs), [s.numel for s in specs], cap, 0, 1.0 / scale)
    assert not want["found_inf"]
    for i, (a, b) in enumerate(zip(got, want["grads"], strict=True)):
        assert np.array_equal(a.numpy().view(np.uint32), b.view(np.uint32)), f"param {i}"


def test_every_timed_step_starts_from_pristine_gradients(tmp_path):
    """Warmup and timed steps each restore the seeded gradients first: after one warmup and
    three timed steps rank 0 holds one application of the pipeline, not four."""
    W, scale, cap = 2, 2.0**16, 0.05
    cfg = dict(n_layer=1, n_embd=32, vocab=64, ctx=16)
    specs = wl.gpt_specs(**cfg)
    path = str(tmp_path / "grads.pt")
    gloo_path.run(W, steps=3, warmup=1, threads=1, cfg=cfg, cap_mb=cap, scale=scale, grads_path=path)
    got = torch.load(path, weights_only=True)
    replica = []
    for r in range(W):
        g = torch.Generator().manual_seed(1234 + 7919 * r)
        replica.append([(torch.randn(s.numel, generator=g) * (1e-3 * scale)).numpy() for s in specs])
    want = o.ddp_pipeline(replica, [o.F32] * len(specs), [s.numel for s in specs], cap, 0, 1.0 / scale)
    for i, (a, b) in enumerate(zip(got, want["grads"], strict=True)):
        assert np.array_equal(a.numpy().view(np.uint32), b.view(np.uint32)), f"param {i}"


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).numpy().astype(np.uint16)


def test_llama_layer_sample_bf16_grads_fp32_buckets_match_oracle(tmp_path):
    """The cfg4 baseline path: bf16 gradients widened into fp32 buckets, averaged, narrowed back
    and unscaled in bf16 -- rank 0's gradients bit for bit against the oracle (W = 2)."""
    W, scale, cap = 2, 2.0**12, 0.01
    cfg = dict(n_layer=2, h=32, ffn=64, vocab=50)
    specs = gloo_path.model_specs(cfg, layers=1)
    assert len(specs) == 1 + 9 + 2  # embedding, one decoder layer, norm and head
    path = str(tmp_path / "grads.pt")
    res = gloo_path.run(W, steps=2, warmup=1, threads=1, cfg=cfg, cap_mb=cap, scale=scale, layers=1,
                        grads_path=path)
    assert res["numel"] == wl.total_numel(specs) and res["buckets"] > 2
    got = torch.load(path, weights_only=True)
    replica = []
    for r in range(W):
        g = torch.Generator().manual_seed(1234 + 7919 * r)
        replica.append([_bf16_bits((torch.randn(s.numel, generator=g) * (1e-3 * scale)).to(torch.bfloat16))
                        for s in specs])
    want = o.ddp_pipeline(replica, [o.BF16] * len(specs), [s.numel for s in specs], cap, 0, 1.0 / scale,
                          bucket_dtype=o.F32)
    for i, (a, b) in enumerate(zip(got, want["grads"], strict=True)):
        assert a.dtype == torch.bfloat16 and np.array_equal(_bf16_bits(a), b), f"param {i}"


def test_fsdp_units_match_oracle(tmp_path):
    """The cfg3 baseline path on a small block unit (h = 24, W = 2): every rank's bf16 gather cast
    and reduce-scatter shard gradient bit for bit against the oracle."""
    W, h, units = 2, 24, 2
    path = str(tmp_path / "fsdp")
    res = gloo_path.run_fsdp(W, units, steps=2, warmup=1, threads=1, h=h, total_units=units, check_path=path)
    numels = [s.numel for s in wl.gpt_block_specs(0, h)]
    total, S, P = o.fsdp_layout(numels, W)
    assert res["shard_numel"] == S and res["units_timed"] == units
    saved = [torch.load(f"{path}.{r}", weights_only=True) for r in range(W)]
    for rank in range(W):
        for u in range(units):
            master = saved[rank]["masters"][u].numpy()
            assert np.array_equal(_bf16_bits(saved[rank]["gathered"][u]), o.fsdp_gather_cast(master, o.BF16))
            grads = [[_bf16_bits(t) for t in saved[r]["grads"][u]] for r in range(W)]
            want = o.fsdp_reduce_scatter_share(grads, o.BF16, numels, rank, o.F32, o.F32)
            got = saved[rank]["shard_grads"][u].numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"rank {rank} unit {u}"
