"""Parity of batched decode attention where neighbouring sequences share their
leading blocks (needs an MI355X).

The kernel reads such a prefix once per run of sequences (up to eight per
group) and merges each member's prefix and suffix partial results. These cases
vary what that depends on: group sizes below, at and above the member limit,
chains whose shared lengths differ (the group shares the fewest), members with
nothing after the prefix, prefixes longer than the 64 compared table entries,
block sizes 16 and 32, head_dim 32 and 64, query group sizes 1 to 16 (1 to 16
members per 16-column block), one and two kv heads per pair. Batches are padded
to the 64 sequences from which the kernel looks for sharing. Every row is
compared with the fp32 oracle (max abs error 2e-3).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from engine.kernels.paged_attention import paged_attention_decode_batched
from oracle.paged_attention_oracle import naive_reference_paged_attention

pytestmark = pytest.mark.gpu

TOL = 2e-3


# Batches below this size are not searched for shared prefixes (the search costs more
# than small batches save); shorter specs are padded with unshared sequences.
MIN_SEQS = 64


def build(spec, hkv, g, d, bs, seed, device):
    """spec: (length, shared) per sequence; `shared` leading table entries repeat the
    previous sequence's physical block ids, every other block is a fresh shuffled id."""
    rng = np.random.default_rng(seed)
    spec = list(spec) + [(int(rng.integers(1, 400)), 0) for _ in range(MIN_SEQS - len(spec))]
    nblk = [(n + bs - 1) // bs for n, _ in spec]
    total = sum(nblk) + 8
    perm = rng.permutation(total).tolist()
    pos, tables = 0, []
    for (n, sh), nb in zip(spec, nblk):
        prev = tables[-1] if tables else []
        sh = min(sh, nb, len(prev))
        row = prev[:sh] + perm[pos:pos + nb - sh]
        pos += nb - sh
        tables.append(row)
    width = max(1, max(nblk)) + 2
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(len(spec), hkv * g, d, generator=gen).half()
    k = torch.randn(total, bs, hkv, d, generator=gen).half()
    v = torch.randn(total, bs, hkv, d, generator=gen).half()
    bt = torch.zeros(len(spec), width, dtype=torch.int32)
    for i, row in enumerate(tables):
        bt[i, :len(row)] = torch.tensor(row, dtype=torch.int32)
    lens = [n for n, _ in spec]
    return dict(q=q, k=k, v=v, bt=bt, lens=lens, tables=tables, device=device, d=d)


def check(case, name):
    dev = case["device"]
    scale = case["d"] ** -0.5
    args = (case["q"].to(dev), case["k"].to(dev), case["v"].to(dev), case["bt"].to(dev),
            torch.tensor(case["lens"], dtype=torch.int32, device=dev), scale)
    print(f"[shared-prefix] {name}: B={len(case['lens'])}", flush=True)
    out = paged_attention_decode_batched(*args)
    again = paged_attention_decode_batched(*args)
    torch.cuda.synchronize()
    assert torch.equal(out, again), f"{name}: two calls differ"
    want = naive_reference_paged_attention(case["q"], case["k"], case["v"], case["tables"],
                                           case["lens"], scale, compute_dtype=torch.float32)
    err = (out.float().cpu() - want.float()).abs().max().item()
    assert err <= TOL, f"{name}: max abs err {err:.3e}"


def groups(sizes, shared, lens_rng, lo, hi):
    spec = []
    for n in sizes:
        for m in range(n):
            spec.append((int(lens_rng.integers(lo, hi)), 0 if m == 0 else shared))
    return spec


def test_groups_of_eight_and_more_one_kv_head_per_pair(cuda_device):
    # 14 q / 2 kv heads, head_dim 64, block 16: groups of 8, 8, 3, 12 (8 + 4), 1, 2, 6 sharing
    # 64 blocks; 40 sequences x 2 kv heads fill fewer than 256 CUs: one kv head per pair.
    rng = np.random.default_rng(1)
    spec = groups([8, 8, 3, 12, 1, 2, 6], 64, rng, 1100, 3000)
    check(build(spec, 2, 7, 64, 16, 11, cuda_device), "groups, one kv head per pair")


def test_groups_two_kv_heads_per_pair(cuda_device):
    # 160 sequences x 2 kv heads exceed the CUs: two kv heads per pair (prefix items are
    # one kv head each and merge into both heads of a pair).
    rng = np.random.default_rng(2)
    spec = groups([8] * 18 + [5, 3, 1, 1, 2], 64, rng, 1030, 2400)
    check(build(spec, 2, 7, 64, 16, 12, cuda_device), "groups, two kv heads per pair")


def test_chain_shares_the_fewest_blocks(cuda_device):
    # Each sequence shares a different number of blocks with its predecessor: the group's
    # prefix is the fewest (10 blocks); the rest of the longer shares is read per sequence.
    spec = [(2000, 0), (1500, 30), (1800, 20), (1700, 40), (1600, 10), (900, 50), (3000, 0)]
    check(build(spec, 2, 7, 64, 16, 13, cuda_device), "chain")


def test_members_with_nothing_after_the_prefix(cuda_device):
    # Lengths of exactly 64 full blocks, all shared: the leader's and a member's own pairs
    # are empty and their output is the prefix alone.
    spec = [(1024, 0), (1024, 64), (1500, 64), (1024, 64), (700, 0), (2048, 0), (2048, 128)]
    check(build(spec, 2, 7, 64, 16, 14, cuda_device), "empty suffixes")


def test_prefix_longer_than_the_compared_entries(cuda_device):
    # 120 shared blocks: the first 64 are read once, the other 56 per sequence.
    spec = [(3000, 0), (3000, 120), (2500, 120), (4000, 120)] * 3
    check(build(spec, 2, 7, 64, 16, 15, cuda_device), "long prefix")


def test_block_32_head_dim_32(cuda_device):
    # Block 32 (two tiles per block), head_dim 32, 16 q / 4 kv heads (group 4: four members
    # per column block, two blocks for a group of eight).
    rng = np.random.default_rng(3)
    spec = groups([8, 5, 8, 2], 40, rng, 1300, 2600)
    check(build(spec, 4, 4, 32, 32, 16, cuda_device), "block 32, head_dim 32")


@pytest.mark.parametrize("hkv,g", [(8, 1), (2, 3), (4, 2), (1, 16), (2, 8)])
def test_query_group_sizes(cuda_device, hkv, g):
    # Members per 16-column block: 16 // g (16, 5, 8, 1, 2); group size capped at
    # min(8, 4 x that).
    rng = np.random.default_rng(10 + g)
    spec = groups([9, 4, 6], 48, rng, 800, 3000)
    check(build(spec, hkv, g, 64, 16, 20 + g, cuda_device), f"hkv={hkv} g={g}")


def test_short_shares_are_read_per_sequence(cuda_device):
    # Sequences sharing 1, 2 or 40 blocks with their predecessor: too little to pay for a
    # prefix item (the reads saved must outweigh the item's fixed cost), so each is read per
    # sequence; beside them a run of three sharing 64 blocks, which does get a prefix item.
    # Lengths above 128 tiles keep the launch on the stream-K kernel that builds prefix
    # items (shorter tables would take one workgroup per pair, which never shares).
    from engine.kernels import _native

    spec = [(2400, 0), (2300, 2), (2500, 0), (2600, 1), (2800, 0), (2700, 40),
            (3000, 0), (2900, 64), (2200, 64)]
    case = build(spec, 2, 7, 64, 16, 17, cuda_device)
    sched = _native.decode_schedule(len(case["lens"]), 14, 2, 64, 16, case["bt"].shape[1])
    assert sched["path"] == "stream_k" and sched["shared_prefixes"], sched
    check(case, "short shares")
