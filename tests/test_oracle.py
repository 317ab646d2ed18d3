"""The CPU oracle is pinned by closed forms, brute force and special cases (no GPU)."""
from __future__ import annotations

import pytest
import torch

import _pins
from oracle.paged_attention_oracle import naive_reference_paged_attention


@pytest.mark.parametrize("check", _pins.ALL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_pinned(check):
    check(naive_reference_paged_attention)


@pytest.mark.parametrize("hq,hkv,d,bs,lens,seed", _pins.GQA_SHAPES)
def test_literal_fp16_path_tracks_fp64(hq, hkv, d, bs, lens, seed):
    """The fp16 path (what the reference runs for fp16 inputs) stays near the fp64 one."""
    q, kc, vc, tables, lens_, _, _ = _pins.build_case(hq, hkv, d, bs, lens, seed, dtype=torch.float32)
    kc = kc / 50  # keep fp16 in range: the garbage rows were scaled up
    vc = vc / 50
    q16, k16, v16 = q.half(), kc.half(), vc.half()
    scale = d ** -0.5
    lit = naive_reference_paged_attention(q16, k16, v16, tables, lens_, scale)
    ref = naive_reference_paged_attention(q16, k16, v16, tables, lens_, scale,
                                          compute_dtype=torch.float64)
    assert lit.dtype == torch.float16
    torch.testing.assert_close(lit.double(), ref, atol=1e-2, rtol=1e-2)


def test_zero_length_sequence_gives_zeros():
    q, kc, vc, tables, lens, _, _ = _pins.build_case(4, 2, 8, 4, [5], 3)
    out = naive_reference_paged_attention(q, kc, vc, tables, [0], 0.5, compute_dtype=torch.float64)
    assert torch.count_nonzero(out) == 0
