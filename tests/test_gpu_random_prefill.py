"""Randomised parity sweep of the paged prefill attention kernel (needs an MI355X).

Each case draws head_dim, group size, block size, a batch of sequences with
cached-prefix and new-token counts (single new tokens, whole prompts without a
cache, long prefixes that split the key range, ragged batches) and checks every
new token's output against the fp32 oracle (max abs error 2e-3). The draws
cover launches with one and with two column groups per wavefront and launches
with and without key-range splits. Cases are seeded.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from test_gpu_prefill_attention import TOL, build, max_err, oracle, run

pytestmark = pytest.mark.gpu

CASES = 30


def draw(seed):
    rng = np.random.default_rng(5000 + seed)
    d = int(rng.choice([32, 64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4]))
    g = int(rng.choice([1, 2, 3, 7, 8]))
    bs = int(rng.choice([5, 8, 16, 16, 32]))
    b = int(rng.choice([1, 1, 2, 5, 12]))
    kind = rng.integers(0, 4)
    if kind == 0:    # short suffixes over long cached prefixes (splits)
        new = rng.integers(1, 40, size=b)
        cached = rng.integers(500, 4000, size=b)
    elif kind == 1:  # whole prompts, no cache
        new = rng.integers(1, 600, size=b)
        cached = np.zeros(b, dtype=np.int64)
    elif kind == 2:  # ragged mix
        new = rng.integers(1, 300, size=b)
        cached = rng.integers(0, 1500, size=b)
    else:            # one new token (a decode step through the prefill path)
        new = np.ones(b, dtype=np.int64)
        cached = rng.integers(0, 2000, size=b)
    return dict(d=d, hkv=hkv, g=g, bs=bs, new=new.tolist(), cached=cached.tolist())


@pytest.mark.parametrize("seed", range(CASES))
def test_random_prefill(cuda_device, seed):
    c = draw(seed)
    ctx = [a + n for a, n in zip(c["cached"], c["new"])]
    print(f"[random-prefill] seed {seed}: D={c['d']} Hkv={c['hkv']} g={c['g']} bs={c['bs']} "
          f"new={c['new']} cached={c['cached']}", flush=True)
    case = build(c["hkv"] * c["g"], c["hkv"], c["d"], c["bs"], ctx, c["new"], 100 + seed,
                 cuda_device)
    scale = c["d"] ** -0.5
    got = run(case, scale)
    torch.cuda.synchronize()
    err = max_err(got, oracle(case, scale))
    assert err <= TOL, f"seed {seed}: max abs err {err:.3e}"
