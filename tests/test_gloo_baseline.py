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
