"""The prefix-prefill oracle is pinned by code it does not share (no GPU).

prefix_prefill_attention restates the reference's "full" prefix-cache mode
(engine/kernels/paged_attention_integration.py:459-482): the prompt suffix
attends causally over the cached prefix blocks and itself. The checks below
pin it against (1) the decode oracle when each sequence has one new token,
(2) torch's causal scaled_dot_product_attention over the whole gathered
sequence, whose last rows are the suffix's rows, and (3) an fp64 brute force
with explicit loops. Planted mistakes each fail at least one check.
"""
from __future__ import annotations

import math
import random

import pytest
import torch
import torch.nn.functional as F

import _pins
from oracle.paged_attention_oracle import naive_reference_paged_attention, prefix_prefill_attention

SHAPES = [  # hq, hkv, d, bs, context lengths, new tokens, seed
    (4, 2, 8, 4, [9, 4, 13], [3, 4, 1], 1),
    (6, 3, 16, 8, [40, 17], [17, 5], 2),
    (2, 2, 8, 16, [33], [20], 3),
    (7, 1, 8, 4, [12, 7], [6, 7], 4),
]


def _case(hq, hkv, d, bs, lens, qlens, seed):
    _, kc, vc, tables, lens_, kf, vf = _pins.build_case(hq, hkv, d, bs, lens, seed)
    g = torch.Generator().manual_seed(seed + 100)
    q = torch.randn(sum(qlens), hq, d, generator=g, dtype=torch.float64)
    return q, kc, vc, tables, lens_, kf, vf


def check_one_new_token_is_decode(fn):
    for hq, hkv, d, bs, lens, _, seed in SHAPES:
        q, kc, vc, tables, lens_, _, _ = _case(hq, hkv, d, bs, lens, [1] * len(lens), seed)
        got = fn(q, kc, vc, tables, lens_, [1] * len(lens), d ** -0.5, torch.float64)
        want = naive_reference_paged_attention(q, kc, vc, tables, lens_, d ** -0.5,
                                               compute_dtype=torch.float64)
        torch.testing.assert_close(got, want, atol=1e-10, rtol=1e-10)


def check_last_rows_of_causal_sdpa(fn):
    """Queries at every position of the flat sequence through SDPA(is_causal=True); the new
    tokens are the last rows, so their outputs must match the suffix-only evaluation."""
    for hq, hkv, d, bs, lens, qlens, seed in SHAPES:
        q, kc, vc, tables, lens_, kf, vf = _case(hq, hkv, d, bs, lens, qlens, seed)
        got = fn(q, kc, vc, tables, lens_, qlens, d ** -0.5, torch.float64)
        row = 0
        g = torch.Generator().manual_seed(seed + 7)
        for s, (L, n) in enumerate(zip(lens_, qlens)):
            qfull = torch.randn(L, hq, d, generator=g, dtype=torch.float64)
            qfull[L - n:] = q[row:row + n]
            o = F.scaled_dot_product_attention(
                qfull.permute(1, 0, 2).unsqueeze(0), kf[s].permute(1, 0, 2).unsqueeze(0),
                vf[s].permute(1, 0, 2).unsqueeze(0), is_causal=True, scale=d ** -0.5,
                enable_gqa=True)[0].permute(1, 0, 2)
            torch.testing.assert_close(got[row:row + n], o[L - n:], atol=1e-10, rtol=1e-10)
            row += n


def check_brute_force(fn):
    for hq, hkv, d, bs, lens, qlens, seed in SHAPES[:2]:
        q, kc, vc, tables, lens_, kf, vf = _case(hq, hkv, d, bs, lens, qlens, seed)
        got = fn(q, kc, vc, tables, lens_, qlens, d ** -0.5, torch.float64)
        g = hq // hkv
        row = 0
        for s, (L, n) in enumerate(zip(lens_, qlens)):
            for i in range(n):
                p = L - n + i
                for h in range(hq):
                    kh = h // g
                    sc = [sum(float(q[row + i, h, e]) * float(kf[s][t, kh, e]) for e in range(d))
                          * d ** -0.5 for t in range(p + 1)]
                    mx = max(sc)
                    w = [math.exp(x - mx) for x in sc]
                    tot = sum(w)
                    for e in range(d):
                        o = sum(w[t] * float(vf[s][t, kh, e]) for t in range(p + 1)) / tot
                        assert abs(float(got[row + i, h, e]) - o) < 1e-9
            row += n


CHECKS = [check_one_new_token_is_decode, check_last_rows_of_causal_sdpa, check_brute_force]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_pinned(check):
    check(prefix_prefill_attention)


def _mutant(mutation):
    def fn(q, kc, vc, tables, lens, qlens, scale, compute_dtype=torch.float64):
        hq, d = q.shape[1], q.shape[2]
        hkv, bs = kc.shape[2], kc.shape[1]
        out = torch.zeros(q.shape, dtype=compute_dtype)
        idx = (torch.arange(hq) % hkv) if mutation == "head_modulo" else torch.arange(hq) // (hq // hkv)
        row = 0
        for s, (L, n) in enumerate(zip(lens, qlens)):
            nb = (L + bs - 1) // bs
            ids = torch.tensor(list(tables[s])[:nb])
            k = kc[ids].reshape(nb * bs, hkv, d)[:L].to(compute_dtype)
            v = vc[ids].reshape(nb * bs, hkv, d)[:L].to(compute_dtype)
            sc = torch.einsum("nhd,shd->hns", q[row:row + n].to(compute_dtype), k[:, idx]) * scale
            base = 0 if mutation == "positions_from_suffix" else L - n
            pos = torch.arange(base, base + n).unsqueeze(1)
            keys = torch.arange(L).unsqueeze(0)
            vis = keys < pos if mutation == "mask_excludes_self" else keys <= pos
            if mutation != "no_mask":
                sc = sc.masked_fill(~vis, float("-inf"))
            out[row:row + n] = torch.einsum("hns,shd->nhd", torch.softmax(sc, -1), v[:, idx])
            row += n
        return out
    return fn


def _fails(fn):
    bad = []
    for check in CHECKS:
        try:
            check(fn)
        except (AssertionError, RuntimeError):
            bad.append(check.__name__)
    return bad


def test_unmutated_copy_passes():
    assert _fails(_mutant(None)) == []


@pytest.mark.parametrize("mutation", ["head_modulo", "positions_from_suffix", "mask_excludes_self",
                                      "no_mask"])
def test_mutant_is_caught(mutation):
    assert _fails(_mutant(mutation)), f"no check catches the '{mutation}' mutant"


def test_zero_new_tokens_contribute_no_rows():
    q, kc, vc, tables, lens, _, _ = _case(4, 2, 8, 4, [9, 5], [0, 2], 5)
    out = prefix_prefill_attention(q, kc, vc, tables, lens, [0, 2], 0.3, torch.float64)
    want = prefix_prefill_attention(q, kc, vc, tables[1:], lens[1:], [2], 0.3, torch.float64)
    torch.testing.assert_close(out, want)


def test_shuffled_pool_gives_same_rows():
    """Relocating the blocks (another permutation, another pool) leaves the result unchanged."""
    hq, hkv, d, bs, lens, qlens, seed = SHAPES[1]
    q, kc, vc, tables, lens_, kf, vf = _case(hq, hkv, d, bs, lens, qlens, seed)
    a = prefix_prefill_attention(q, kc, vc, tables, lens_, qlens, 0.25, torch.float64)
    rnd = random.Random(9)
    nb = kc.shape[0]
    perm = list(range(nb))
    rnd.shuffle(perm)
    inv = torch.empty(nb, dtype=torch.long)
    inv[torch.tensor(perm)] = torch.arange(nb)
    kc2, vc2 = kc[torch.tensor(perm)], vc[torch.tensor(perm)]
    tables2 = [[int(inv[b]) for b in t] for t in tables]
    b = prefix_prefill_attention(q, kc2, vc2, tables2, lens_, qlens, 0.25, torch.float64)
    torch.testing.assert_close(a, b, atol=0, rtol=0)
