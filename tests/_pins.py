"""Checks that pin an attention oracle to mathematics it does not share code with.

Each check takes an oracle with the signature of
oracle.paged_attention_oracle.naive_reference_paged_attention (plus
compute_dtype) and raises AssertionError when it disagrees with:
  * contiguous scaled-dot-product attention (torch SDPA, GQA-enabled) on the
    un-paged K/V the pool was filled from;
  * the repeat_interleave GQA statement the reference's own tests use
    (tests/test_paged_attention_reference.py:136-158);
  * an fp64 brute force written with explicit Python loops and math.exp;
  * special cases: seq_len 1, identical keys, a dominant score;
  * invariance to where blocks sit in the pool and to extra table entries.
Unused pool rows hold large garbage values, so an oracle that reads past a
sequence's length or mis-indexes a block cannot pass by accident.
"""
from __future__ import annotations

import math
import random

import torch
import torch.nn.functional as F


def build_case(num_q_heads, num_kv_heads, head_dim, block_size, seq_lens, seed, dtype=torch.float64,
               slack=2):
    """Flat per-sequence K/V scattered into shuffled blocks of a garbage-filled pool."""
    g = torch.Generator().manual_seed(seed)
    rnd = random.Random(seed)
    nlog = sum((n + block_size - 1) // block_size for n in seq_lens)
    num_blocks = nlog * slack + 3
    k_cache = torch.randn(num_blocks, block_size, num_kv_heads, head_dim, generator=g).to(dtype) * 50
    v_cache = torch.randn(num_blocks, block_size, num_kv_heads, head_dim, generator=g).to(dtype) * 50
    ids = rnd.sample(range(num_blocks), nlog)
    q = torch.randn(len(seq_lens), num_q_heads, head_dim, generator=g).to(dtype)
    k_flats, v_flats, tables, pos = [], [], [], 0
    for n in seq_lens:
        kf = torch.randn(n, num_kv_heads, head_dim, generator=g).to(dtype)
        vf = torch.randn(n, num_kv_heads, head_dim, generator=g).to(dtype)
        nb = (n + block_size - 1) // block_size
        table = ids[pos:pos + nb]
        pos += nb
        for j, b in enumerate(table):
            take = min(block_size, n - j * block_size)
            k_cache[b, :take] = kf[j * block_size:j * block_size + take]
            v_cache[b, :take] = vf[j * block_size:j * block_size + take]
        k_flats.append(kf)
        v_flats.append(vf)
        tables.append(table)
    return q, k_cache, v_cache, tables, list(seq_lens), k_flats, v_flats


def sdpa_closed_form(q, k_flats, v_flats, scale):
    outs = []
    for s in range(q.shape[0]):
        qs = q[s].unsqueeze(0).unsqueeze(2)                 # [1, Hq, 1, D]
        ks = k_flats[s].permute(1, 0, 2).unsqueeze(0)       # [1, Hkv, L, D]
        vs = v_flats[s].permute(1, 0, 2).unsqueeze(0)
        o = F.scaled_dot_product_attention(qs, ks, vs, scale=scale, enable_gqa=True)
        outs.append(o[0, :, 0, :])
    return torch.stack(outs)


def repeat_interleave_form(q, k_flat, v_flat, scale):
    g = q.shape[0] // k_flat.shape[1]
    k = k_flat.repeat_interleave(g, dim=1)
    v = v_flat.repeat_interleave(g, dim=1)
    scores = torch.einsum("hd,shd->hs", q, k) * scale
    return torch.einsum("hs,shd->hd", torch.softmax(scores, dim=-1), v)


def brute_force(q, k_flats, v_flats, scale):
    """Explicit loops in Python floats (fp64)."""
    S, Hq, D = q.shape
    out = torch.zeros(S, Hq, D, dtype=torch.float64)
    for s in range(S):
        kf, vf = k_flats[s].tolist(), v_flats[s].tolist()
        Hkv = len(kf[0])
        g = Hq // Hkv
        qs = q[s].tolist()
        for h in range(Hq):
            kh = h // g
            sc = [scale * sum(qs[h][d] * kf[t][kh][d] for d in range(D)) for t in range(len(kf))]
            m = max(sc)
            w = [math.exp(x - m) for x in sc]
            z = sum(w)
            for d in range(D):
                out[s, h, d] = sum(w[t] * vf[t][kh][d] for t in range(len(kf))) / z
    return out


GQA_SHAPES = [
    # (num_q_heads, num_kv_heads, head_dim, block_size, seq_lens, seed)
    (8, 8, 32, 16, [16, 37, 8], 101),
    (8, 4, 32, 16, [16, 45, 9], 102),
    (14, 2, 64, 16, [13, 32, 67], 103),
    (4, 1, 16, 8, [19, 1, 24], 104),
    (6, 3, 8, 4, [12, 20, 7], 105),
]


def check_sdpa(oracle):
    for hq, hkv, d, bs, lens, seed in GQA_SHAPES:
        q, kc, vc, tables, lens_, kf, vf = build_case(hq, hkv, d, bs, lens, seed)
        scale = d ** -0.5
        got = oracle(q, kc, vc, tables, lens_, scale, compute_dtype=torch.float64)
        want = sdpa_closed_form(q, kf, vf, scale)
        torch.testing.assert_close(got, want, atol=1e-10, rtol=1e-10)


def check_repeat_interleave(oracle):
    for hq, hkv, d, bs, lens, seed in GQA_SHAPES:
        q, kc, vc, tables, lens_, kf, vf = build_case(hq, hkv, d, bs, lens, seed + 1000,
                                                      dtype=torch.float32)
        scale = d ** -0.5
        got = oracle(q, kc, vc, tables, lens_, scale, compute_dtype=torch.float32)
        for s in range(len(lens_)):
            want = repeat_interleave_form(q[s], kf[s], vf[s], scale)
            torch.testing.assert_close(got[s], want, atol=1e-5, rtol=1e-5)


def check_brute_force(oracle):
    q, kc, vc, tables, lens, kf, vf = build_case(4, 2, 3, 2, [5, 2, 1], 7)
    got = oracle(q, kc, vc, tables, lens, 0.7, compute_dtype=torch.float64)
    torch.testing.assert_close(got, brute_force(q, kf, vf, 0.7), atol=1e-12, rtol=1e-12)


def check_special_cases(oracle):
    # seq_len 1: softmax over one token is 1 -> every head returns v_0 of its kv head.
    q, kc, vc, tables, lens, kf, vf = build_case(6, 2, 16, 4, [1], 11)
    got = oracle(q, kc, vc, tables, lens, 0.25, compute_dtype=torch.float64)
    want = vf[0][0].repeat_interleave(3, dim=0)
    torch.testing.assert_close(got[0], want, atol=1e-12, rtol=0)
    # identical keys: uniform weights -> mean of V over the sequence.
    q, kc, vc, tables, lens, kf, vf = build_case(4, 2, 8, 4, [10], 12)
    for j, b in enumerate(tables[0]):
        take = min(4, 10 - 4 * j)
        kc[b, :take] = kf[0][0]
    got = oracle(q, kc, vc, tables, lens, 0.3, compute_dtype=torch.float64)
    torch.testing.assert_close(got[0], vf[0].mean(0).repeat_interleave(2, dim=0), atol=1e-12, rtol=0)
    # one dominant score: output is that token's V.
    q, kc, vc, tables, lens, kf, vf = build_case(2, 1, 4, 4, [9], 13)
    q[0] = torch.tensor([1.0, 0.0, 0.0, 0.0], dtype=q.dtype)
    for j, b in enumerate(tables[0]):
        take = min(4, 9 - 4 * j)
        kc[b, :take] = 0.0
    t_star = 6
    kc[tables[0][t_star // 4], t_star % 4, 0, 0] = 1000.0
    got = oracle(q, kc, vc, tables, lens, 1.0, compute_dtype=torch.float64)
    torch.testing.assert_close(got[0, 0], vf[0][t_star, 0], atol=1e-12, rtol=0)


def check_layout_invariance(oracle):
    """Moving blocks around the pool, adding slack and extra table entries changes nothing."""
    q, kc, vc, tables, lens, kf, vf = build_case(8, 2, 16, 4, [11, 6], 21)
    base = oracle(q, kc, vc, tables, lens, 0.25, compute_dtype=torch.float64)
    nb = kc.shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(5))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb)
    kc2 = torch.cat([kc[perm], torch.randn(7, *kc.shape[1:], dtype=kc.dtype) * 50])
    vc2 = torch.cat([vc[perm], torch.randn(7, *vc.shape[1:], dtype=vc.dtype) * 50])
    tables2 = [[int(inv[b]) for b in t] + [nb + 3, nb + 5] for t in tables]
    moved = oracle(q, kc2, vc2, tables2, lens, 0.25, compute_dtype=torch.float64)
    torch.testing.assert_close(moved, base, atol=1e-12, rtol=0)


ALL_CHECKS = [check_sdpa, check_repeat_interleave, check_brute_force, check_special_cases,
              check_layout_invariance]


def failing_checks(oracle):
    """Names of the checks the oracle fails (empty when it is pinned)."""
    failed = []
    for chk in ALL_CHECKS:
        try:
            chk(oracle)
        except Exception:  # noqa: BLE001  (any failure counts, including crashes)
            failed.append(chk.__name__)
    return failed
