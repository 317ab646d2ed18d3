"""Decode-step linear layer (pa_linear_f16) against fp32 references (needs an MI355X).

Each epilogue runs at the shapes of a Qwen2.5-0.5B decoder layer at batch 128
(q/k/v with bias, o_proj, the merged gate/up with SwiGLU, down_proj added into
the residual) and at ragged row counts, forced K splits and padded row strides:
- store and add: within one fp16 ulp of the fp64 product (plus bias or the old
  value), plus the fp32 accumulation bound K 2^-24 sum|x||w| that matters only
  near zero -- the kernel accumulates in fp32 and rounds once;
- SwiGLU: with the same K splits, the store epilogue on the merged [gate; up]
  weight yields exactly the fp16 gate and up values the SwiGLU epilogue forms
  (each output summed in the same order), and the store path is pinned above;
  so the SwiGLU output equals silu_mul (pa_silu_mul_f16) of that store output
  bit for bit, and torch's silu(gate) * up within one ulp;
- with K split over workgroups, two calls give the same bits.
"""
from __future__ import annotations

import pytest
import torch

from engine.kernels.paged_attention_integration import linear, silu_mul

pytestmark = pytest.mark.gpu


def ulp16(ref: torch.Tensor) -> torch.Tensor:
    """Spacing of fp16 values at |ref| (subnormal spacing below 2^-14)."""
    a = ref.abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def operands(m, k, n, dev, seed, w_rows=None, x_pad=0, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k + x_pad, generator=g).half()[:, :k]
    w = (torch.randn(w_rows or n, k, generator=g) * scale).half()
    return x.to(dev), w.to(dev)


def ref_mm(x, w):
    return x.float() @ w.float().t()


def ref64(x, w):
    """fp64 product and the fp32 accumulation bound K 2^-24 sum_k |x||w| per entry."""
    exact = x.double() @ w.double().t()
    acc_bound = (x.double().abs() @ w.double().abs().t()) * (x.shape[1] * 2.0 ** -24)
    return exact, acc_bound


@pytest.mark.parametrize("m,k,n,bias,splits", [
    (128, 896, 1152, True, 0),   # q/k/v
    (128, 896, 896, False, 0),   # o_proj
    (1, 896, 896, True, 0),
    (7, 96, 68, True, 3),
    (130, 896, 200, False, 5),
    (257, 64, 4, True, 1),
    (300, 4864, 896, False, 0),
])
def test_store(cuda_device, m, k, n, bias, splits):
    print(f"[linear store] m={m} k={k} n={n} bias={bias} splits={splits}", flush=True)
    x, w = operands(m, k, n, cuda_device, 1 + m + n, x_pad=8 if m % 2 else 0)
    b = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.5).half().to(cuda_device) \
        if bias else None
    y = linear(x, w, b, splits=splits)
    ref, bound = ref64(x, w)
    if bias:
        ref = ref + b.double()
    torch.cuda.synchronize()
    err = (y.double() - ref).abs()
    assert torch.all(err <= ulp16(ref) + bound), f"max err {err.max().item():.3e}"


@pytest.mark.parametrize("m,k,n,splits", [
    (128, 4864, 896, 0),  # down_proj into the residual
    (5, 4864, 896, 7),
    (129, 128, 36, 2),
])
def test_add(cuda_device, m, k, n, splits):
    print(f"[linear add] m={m} k={k} n={n} splits={splits}", flush=True)
    x, w = operands(m, k, n, cuda_device, 7 + m)
    y0 = torch.randn(m, n, generator=torch.Generator().manual_seed(3)).half().to(cuda_device)
    y = y0.clone()
    linear(x, w, out=y, accumulate=True, splits=splits)
    ref, bound = ref64(x, w)
    ref = ref + y0.double()
    torch.cuda.synchronize()
    err = (y.double() - ref).abs()
    assert torch.all(err <= ulp16(ref) + bound), f"max err {err.max().item():.3e}"


@pytest.mark.parametrize("m,k,inter,splits", [
    (128, 896, 4864, 0),  # merged gate/up of the MLP
    (3, 896, 4864, 0),
    (140, 64, 40, 2),
])
def test_swiglu(cuda_device, m, k, inter, splits):
    print(f"[linear swiglu] m={m} k={k} inter={inter} splits={splits}", flush=True)
    x, w = operands(m, k, inter, cuda_device, 11 + m, w_rows=2 * inter, scale=0.1)
    y = linear(x, w, swiglu=True, splits=splits)
    gu = linear(x, w, splits=splits)  # fp16 gate | up, same accumulation order
    same = silu_mul(gu)
    want = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
    ref, bound = ref64(x, w)
    torch.cuda.synchronize()
    assert torch.all((gu.double() - ref).abs() <= ulp16(ref) + bound)
    assert torch.equal(y, same)
    err = (y.double() - want.double()).abs()
    assert torch.all(err <= ulp16(want.double())), f"max err {err.max().item():.3e}"


def test_split_partials_repeatable(cuda_device):
    x, w = operands(128, 4864, 896, cuda_device, 5)
    a = linear(x, w, splits=9)
    b = linear(x, w, splits=9)
    c = linear(x, w, splits=1)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    ref, bound = ref64(x, w)
    assert torch.all((c.double() - ref).abs() <= ulp16(ref) + bound)


def test_matches_library_linear(cuda_device):
    """Same results as torch's fp16 linear up to one ulp where the roundings straddle."""
    x, w = operands(128, 896, 1152, cuda_device, 9)
    b = torch.randn(1152, generator=torch.Generator().manual_seed(1)).half().to(cuda_device)
    y = linear(x, w, b)
    t = torch.nn.functional.linear(x, w, b)
    torch.cuda.synchronize()
    diff = (y.double() - t.double()).abs()
    _, bound = ref64(x, w)
    assert torch.all(diff <= ulp16(t.double()) + 2 * bound)
    assert (diff == 0).float().mean().item() > 0.9
