"""Randomised parity sweep of the batched decode kernel (needs an MI355X).

Each case draws a batch size (across the one-pair-per-workgroup, stream-K and
fixed-split schedules), lengths (zeros, single tokens, block boundaries, long
tails), head_dim, group size, block size, table padding and, for some cases,
leading blocks shared between neighbouring sequences, then checks a sample of
sequences against the fp32 oracle (max abs error 2e-3) and that zero-length
rows are zero. Cases are seeded, so a failure names a reproducible shape.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from engine import workloads
from engine.kernels.paged_attention import paged_attention_decode_batched
from oracle.paged_attention_oracle import naive_reference_paged_attention

pytestmark = pytest.mark.gpu

TOL = 2e-3
CASES = 40


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    d = int(rng.choice([32, 64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 3, 4, 7, 8, 16]))
    bs = int(rng.choice([1, 8, 12, 16, 16, 32]))
    b = int(rng.choice([1, 3, 17, 64, 130, 300, 1030]))
    kind = rng.integers(0, 4)
    if kind == 0:    # short
        lens = rng.integers(0, 80, size=b)
    elif kind == 1:  # block-boundary lengths
        lens = rng.integers(1, 40, size=b) * bs + rng.integers(-1, 2, size=b)
    elif kind == 2:  # mixed with long tails
        lens = np.where(rng.random(b) < 0.1, rng.integers(1000, 5000, size=b),
                        rng.integers(0, 400, size=b))
    else:            # near-uniform medium
        lens = rng.integers(200, 700, size=b)
    lens = np.clip(lens, 0, 6000)
    if b > 300:  # keep the large-batch cases small
        lens = np.minimum(lens, 300)
    share = bool(rng.random() < 0.4) and bs % 16 == 0
    return dict(d=d, hkv=hkv, g=g, bs=bs, lens=lens.tolist(), share=share, seed=seed)


def build(c, device):
    """A shuffled pool; with share, pairs of neighbours list the same leading blocks."""
    bs, lens = c["bs"], c["lens"]
    rng = np.random.default_rng(c["seed"])
    nblk = [(n + bs - 1) // bs for n in lens]
    total = sum(nblk) + 16
    perm = rng.permutation(total).tolist()
    pos, tables = 0, []
    for i, n in enumerate(nblk):
        if c["share"] and i % 2 == 1 and tables and lens[i - 1] > 0 and lens[i] > 0:
            k = min(len(tables[-1]), n - 1, int(rng.integers(0, 70)))
            row = tables[-1][:k] + perm[pos:pos + n - k]
            pos += n - k
        else:
            row = perm[pos:pos + n]
            pos += n
        tables.append(row)
    width = max(1, max(nblk)) + int(rng.integers(0, 3))
    gen = torch.Generator().manual_seed(c["seed"])
    hq = c["hkv"] * c["g"]
    q = torch.randn(len(lens), hq, c["d"], generator=gen).half()
    k = torch.randn(total, bs, c["hkv"], c["d"], generator=gen).half()
    v = torch.randn(total, bs, c["hkv"], c["d"], generator=gen).half()
    bt = torch.zeros(len(lens), width, dtype=torch.int32)
    for i, row in enumerate(tables):
        bt[i, :len(row)] = torch.tensor(row, dtype=torch.int32)
    return (q.to(device), k.to(device), v.to(device), bt.to(device),
            torch.tensor(lens, dtype=torch.int32, device=device), tables, q, k, v)


@pytest.mark.parametrize("seed", range(CASES))
def test_random_shape(cuda_device, seed):
    c = draw(seed)
    q, k, v, bt, sl, tables, qc, kc, vc = build(c, cuda_device)
    scale = c["d"] ** -0.5
    print(f"[random] seed {seed}: B={len(c['lens'])} D={c['d']} Hkv={c['hkv']} g={c['g']} "
          f"bs={c['bs']} share={c['share']} max_len={max(c['lens'])}", flush=True)
    out = paged_attention_decode_batched(q, k, v, bt, sl, scale)
    torch.cuda.synchronize()
    lens = c["lens"]
    zero = [i for i, n in enumerate(lens) if n == 0]
    if zero:
        assert torch.count_nonzero(out[zero]).item() == 0
    nz = [i for i, n in enumerate(lens) if n > 0]
    rng = np.random.default_rng(seed)
    pick = sorted(set(rng.choice(nz, size=min(6, len(nz)), replace=False).tolist()
                      + [max(nz, key=lambda i: lens[i])])) if nz else []
    if pick:
        want = naive_reference_paged_attention(qc[pick], kc, vc, [tables[i] for i in pick],
                                               [lens[i] for i in pick], scale,
                                               compute_dtype=torch.float32)
        err = (out[pick].float().cpu() - want.float()).abs().max().item()
        assert err <= TOL, f"seed {seed}: max abs err {err:.3e}"


@pytest.mark.parametrize("hkv,g,bs,lens", [
    (1, 2, 4, [6, 10, 24, 300]),      # odd kv-head count: one kv head per workgroup
    (3, 2, 8, [33, 10, 24]),
    (1, 7, 12, [50, 1, 700]),
    (1, 4, 1, [17, 40]),
    (2, 2, 4, [6, 10, 24]),           # small batch: one kv head per workgroup
    (2, 7, 8, [2000, 129, 5]),        # long pair split into stream-K ranges
])
def test_head_dim_32_single_head_tiles_span_blocks(cuda_device, hkv, g, bs, lens):
    """Head_dim 32 with one kv head per workgroup: a 16-row tile is one load
    instruction, and with blocks shorter than 16 tokens each lane's row lies in
    its own block (every lane must look up its own row's block id)."""
    c = dict(d=32, hkv=hkv, g=g, bs=bs, lens=lens, share=False, seed=77 + bs + hkv)
    q, k, v, bt, sl, tables, qc, kc, vc = build(c, cuda_device)
    print(f"[one-head tiles] hkv={hkv} g={g} bs={bs} lens={lens}", flush=True)
    out = paged_attention_decode_batched(q, k, v, bt, sl, 32 ** -0.5)
    torch.cuda.synchronize()
    want = naive_reference_paged_attention(qc, kc, vc, tables, lens, 32 ** -0.5,
                                           compute_dtype=torch.float32)
    err = (out.float().cpu() - want.float()).abs().max().item()
    assert err <= TOL, f"max abs err {err:.3e}"
