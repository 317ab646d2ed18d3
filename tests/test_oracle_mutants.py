"""Plausible mistakes planted in copies of the oracle are each caught by a pin check.

A mutant is the oracle's algorithm with one deliberate error; if a pin check
passed on it, that check would not be pinning the oracle.
"""
from __future__ import annotations

import pytest
import torch

import _pins


def _make(mutation):
    def oracle(q, k_cache, v_cache, block_tables, seq_lens, scale, compute_dtype=None):
        num_seqs, num_q_heads, head_dim = q.shape
        num_kv_heads = k_cache.shape[2]
        group = num_q_heads // num_kv_heads
        out = torch.zeros(q.shape, dtype=compute_dtype or q.dtype)
        bs = k_cache.shape[1]
        for s in range(num_seqs):
            n = int(seq_lens[s]) - (1 if mutation == "drop_last_token" else 0)
            ks, vs, rem = [], [], n
            for b in block_tables[s]:
                take = bs if mutation == "full_blocks" else min(bs, rem)
                ks.append(k_cache[b, :take])
                vs.append(v_cache[b, :take])
                rem -= take
                if rem <= 0:
                    break
            k = torch.cat(ks).to(compute_dtype or q.dtype)
            v = torch.cat(vs).to(compute_dtype or q.dtype)
            qs = q[0 if mutation == "first_query" else s].to(compute_dtype or q.dtype)
            if mutation == "head_modulo":
                idx = torch.arange(num_q_heads) % num_kv_heads
            else:
                idx = torch.arange(num_q_heads) // group
            ke, ve = k[:, idx], v[:, idx]
            if mutation == "k_for_v":
                ve = ke
            sc = torch.einsum("hd,shd->hs", qs, ke) * (1.0 if mutation == "no_scale" else scale)
            if mutation == "sign":
                sc = -sc
            p = torch.softmax(sc, dim=0 if mutation == "softmax_dim" else -1)
            out[s] = torch.einsum("hs,shd->hd", p, ve)
        return out
    return oracle


MUTANTS = ["drop_last_token", "full_blocks", "first_query", "head_modulo", "k_for_v",
           "no_scale", "sign", "softmax_dim"]


def test_unmutated_copy_passes():
    assert _pins.failing_checks(_make(None)) == []


@pytest.mark.parametrize("mutation", MUTANTS)
def test_mutant_is_caught(mutation):
    assert _pins.failing_checks(_make(mutation)), f"no pin check catches the '{mutation}' mutant"
