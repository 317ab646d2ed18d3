"""Seeded inputs of the golden fixtures: fp16 K/V written into shuffled pool blocks.

Shapes follow the reference's GPU tests (tests/test_paged_attention_reference.py:278-285,
:439-485, :540-643): GQA ratios 1, 2, 4, 7, partial last blocks, block sizes 8 and 16, a
2048-token sequence, and a batch with lengths [1, 17, 500, 2000]. Unused pool rows hold large
values so a wrong gather cannot pass.
"""
from __future__ import annotations

import torch

CASES = {
    # name: (num_q_heads, num_kv_heads, head_dim, block_size, lens, seed)
    "mha_37": (8, 8, 32, 16, [37], 201),
    "gqa2_45": (8, 4, 32, 16, [45], 202),
    "gqa7_67": (14, 2, 64, 16, [67], 203),
    "gqa7_32": (14, 2, 64, 16, [32], 204),
    "mqa4_bs8_19": (4, 1, 64, 8, [19], 205),
    "long_2048": (14, 2, 64, 16, [2048], 401),
    "batched_1_17_500_2000": (14, 2, 64, 16, [1, 17, 500, 2000], 601),
    "d128_gqa7": (28, 4, 128, 16, [129, 1000, 5], 701),
}


def build(name):
    hq, hkv, d, bs, lens, seed = CASES[name]
    g = torch.Generator().manual_seed(seed)
    nlog = sum((n + bs - 1) // bs for n in lens)
    nb = 2 * nlog + 5
    k_cache = (torch.randn(nb, bs, hkv, d, generator=g) * 30).half()
    v_cache = (torch.randn(nb, bs, hkv, d, generator=g) * 30).half()
    ids = torch.randperm(nb, generator=g)[:nlog].tolist()
    q = torch.randn(len(lens), hq, d, generator=g).half()
    k_flat, v_flat, tables, pos = [], [], [], 0
    for n in lens:
        kf = torch.randn(n, hkv, d, generator=g).half()
        vf = torch.randn(n, hkv, d, generator=g).half()
        m = (n + bs - 1) // bs
        table = ids[pos:pos + m]
        pos += m
        for j, b in enumerate(table):
            take = min(bs, n - j * bs)
            k_cache[b, :take] = kf[j * bs:j * bs + take]
            v_cache[b, :take] = vf[j * bs:j * bs + take]
        k_flat.append(kf)
        v_flat.append(vf)
        tables.append(table)
    return dict(q=q, k_cache=k_cache, v_cache=v_cache, tables=tables, lens=list(lens),
                k_flat=k_flat, v_flat=v_flat, scale=d ** -0.5)
