"""Golden fixtures (fp64 closed-form outputs on seeded inputs) against the oracle and the kernels."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
from cases import CASES, build  # noqa: E402
from make_golden import input_digest  # noqa: E402

from oracle.paged_attention_oracle import naive_reference_paged_attention  # noqa: E402


def _load(name):
    data = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    case = build(name)
    assert str(data["digest"]) == input_digest(case), "regenerated inputs differ from the fixture's"
    return case, data["expected"]


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_golden(name):
    case, expected = _load(name)
    got = naive_reference_paged_attention(case["q"], case["k_cache"], case["v_cache"], case["tables"],
                                          case["lens"], case["scale"], compute_dtype=torch.float64)
    np.testing.assert_allclose(got.numpy(), expected, atol=1e-9, rtol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_kernels_match_golden(cuda_device, name):
    from engine.kernels.paged_attention import (
        paged_attention_decode_batched,
        paged_attention_decode_v1,
        paged_attention_decode_v2,
        pad_block_tables,
    )

    case, expected = _load(name)
    dev = cuda_device
    q, kc, vc = case["q"].to(dev), case["k_cache"].to(dev), case["v_cache"].to(dev)
    out = paged_attention_decode_batched(
        q, kc, vc, pad_block_tables(case["tables"], device=dev),
        torch.tensor(case["lens"], dtype=torch.int32, device=dev), case["scale"])
    err = np.abs(out.float().cpu().numpy() - expected).max()
    print(f"[golden] {name}: batched max abs err {err:.3e}", flush=True)
    assert err <= 2e-3
    for s, n in enumerate(case["lens"]):
        bt = torch.tensor(case["tables"][s], dtype=torch.int32, device=dev)
        for fn in (paged_attention_decode_v1, paged_attention_decode_v2):
            o = fn(q[s], kc, vc, bt, n, case["scale"])
            assert np.abs(o.float().cpu().numpy() - expected[s]).max() <= 2e-3, fn.__name__
