"""Seeded random sweep of the consumer side (global-norm clip and Adam).

Eight tensor lists drawn once from a fixed seed.  Each has 1 to 130 tensors,
so a list can be longer than one launch holds (64 tensors for the norm, 48
for Adam). Sizes are log-uniform up to 300,000 elements, with empty tensors
and sizes next to the 8192-element block chunk mixed in.  Per list, on the
helpers of test_gpu_optim and the same bars (dnn/utils/clip_grad_norm.cu:13-67,
dnn/optimizers/adam_optimizer.cu:11-109):
- the global norm within one binary32 ulp of the oracle's;
- clipping in place bit-exact;
- two Adam steps bit-exact (parameters, m, v) against the oracle, with a
  weight decay and a max norm drawn per list, the clip fused into the update
  or applied beforehand.
"""
import numpy as np
import pytest
import torch

import deepfuse_amd as df
from oracle import pyoracle as orc
from test_gpu_optim import adam_case, rand_list, to_dev, ulps

pytestmark = pytest.mark.gpu


def _draw_lists(count=8, seed=20261204):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        n = int(rng.integers(1, 131))
        sizes = []
        for _ in range(n):
            r = rng.random()
            if r < 0.1:
                sizes.append(0)
            elif r < 0.3:
                sizes.append(8192 + int(rng.integers(-2, 3)))
            else:
                sizes.append(int(np.exp(rng.uniform(0.0, np.log(300_000.0)))))
        out.append(sizes)
    return out


LISTS = _draw_lists()


@pytest.mark.parametrize("idx", range(len(LISTS)))
def test_sweep_norm_clip_adam(dev, idx):
    sizes = LISTS[idx]
    rng = np.random.default_rng(100 + idx)
    host = rand_list(sizes, seed=200 + idx, scale=float(rng.uniform(0.01, 2.0)))
    d = to_dev(host, dev)
    norm = df.grad_norm(d)
    torch.cuda.synchronize()
    nv = norm.item()
    assert ulps(nv, orc.grad_norm(host)) <= 1, f"list {idx}: norm"
    max_norm = float(np.float32(nv * rng.uniform(0.3, 1.5)))
    df.grad_norm(d, clip=max_norm)
    torch.cuda.synchronize()
    expect = [a.copy() for a in host]
    for a in expect:
        orc.clip_scale(a, nv, max_norm)
    for i, (a, t) in enumerate(zip(expect, d)):
        assert np.array_equal(t.cpu().numpy(), a), f"list {idx}: clipped tensor {i} (size {a.size})"
    adam_case(dev, sizes, steps=2, wd=float(rng.choice([0.0, 0.01, 0.1])), max_norm=float(rng.uniform(0.5, 50.0)),
              fused=bool(idx % 2), seed=300 + idx)


def test_sweep_lists_cover_launch_limits():
    assert any(len(s) > 64 for s in LISTS) and any(len(s) < 48 for s in LISTS)
    assert any(0 in s for s in LISTS) and any(8192 in s or 8193 in s for s in LISTS)
