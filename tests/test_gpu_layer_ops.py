"""The fused decode-step layer pieces match transformers' own ops (needs an MI355X).

rms_norm replaces Qwen2RMSNorm.forward (seven launches) and silu_mul the
act_fn(gate) * up of Qwen2MLP.forward; both keep transformers' roundings, so
the results are bit-identical except where a sum taken in another order lands
on the other side of an fp16 rounding boundary: one unit in the last place of
the normalised value, which the weight product can turn into two, on a small
fraction of values. The fused decoder layer itself is
checked end to end by the decode-step tests (greedy streams and
teacher-forced logits against the unpatched model).
"""
from __future__ import annotations

import pytest
import torch

from engine.kernels.paged_attention_integration import greedy_top2, rms_norm, silu_mul

pytestmark = pytest.mark.gpu


def _ulps(a, b):
    """Distance in fp16 units in the last place (same-sign values)."""
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    return (ai - bi).abs()


@pytest.mark.parametrize("rows,hidden", [(128, 896), (3, 1000), (1, 64), (257, 4864)])
def test_rms_norm_matches_transformers(cuda_device, rows, hidden):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    g = torch.Generator(device=cuda_device).manual_seed(rows + hidden)
    x = (torch.randn(rows, hidden, generator=g, device=cuda_device) * 3).half()
    norm = Qwen2RMSNorm(hidden, eps=1e-6).to(cuda_device).half()
    with torch.no_grad():
        norm.weight.copy_(torch.randn(hidden, generator=g, device=cuda_device).half())
        want = norm(x)
    got = rms_norm(x, norm.weight, norm.variance_epsilon)
    d = _ulps(got, want)
    frac = (d > 0).float().mean().item()
    print(f"[layer-ops] rms_norm {rows}x{hidden}: max {d.max().item()} ulp, {frac:.4%} differ",
          flush=True)
    assert d.max().item() <= 2 and frac < 0.01


def test_rms_norm_of_a_3d_view(cuda_device):
    x = torch.randn(4, 1, 896, device=cuda_device).half()
    w = torch.randn(896, device=cuda_device).half()
    assert torch.equal(rms_norm(x, w, 1e-6), rms_norm(x.view(4, 896), w, 1e-6).view(4, 1, 896))


@pytest.mark.parametrize("rows,inter", [(128, 4864), (5, 100)])
def test_silu_mul_matches_transformers(cuda_device, rows, inter):
    g = torch.Generator(device=cuda_device).manual_seed(rows)
    gu = (torch.randn(rows, 2 * inter, generator=g, device=cuda_device) * 4).half()
    want = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
    got = silu_mul(gu)
    d = _ulps(got, want)
    frac = (d > 0).float().mean().item()
    print(f"[layer-ops] silu_mul {rows}x{inter}: max {d.max().item()} ulp, {frac:.4%} differ",
          flush=True)
    assert d.max().item() <= 1 and frac < 0.02


@pytest.mark.parametrize("rows,hidden", [(128, 896), (2, 3000)])
def test_residual_add_and_rms_norm(cuda_device, rows, hidden):
    """The decoder layer's residual + x in fp16, then the norm of that sum."""
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    g = torch.Generator(device=cuda_device).manual_seed(hidden)
    x = torch.randn(rows, hidden, generator=g, device=cuda_device).half()
    res = (torch.randn(rows, hidden, generator=g, device=cuda_device) * 2).half()
    norm = Qwen2RMSNorm(hidden, eps=1e-6).to(cuda_device).half()
    with torch.no_grad():
        norm.weight.copy_(torch.randn(hidden, generator=g, device=cuda_device).half())
        want_sum = res + x
        want = norm(want_sum)
    got_sum, got = rms_norm(x, norm.weight, norm.variance_epsilon, residual=res)
    assert torch.equal(got_sum, want_sum)
    assert _ulps(got, want).max().item() <= 2


@pytest.mark.parametrize("rows,vocab", [(128, 151936), (3, 1000), (1, 7)])
def test_greedy_top2_matches_torch(cuda_device, rows, vocab):
    g = torch.Generator(device=cuda_device).manual_seed(vocab)
    logits = (torch.randn(rows, vocab, generator=g, device=cuda_device) * 3).half()
    if vocab > 10:
        logits[0, 5] = logits[0, 9] = 100.0  # a tied maximum: first index, margin 0
    idx, top = greedy_top2(logits)
    assert torch.equal(idx, torch.argmax(logits, dim=-1))
    assert torch.equal(top, torch.topk(logits, 2, dim=-1).values.float())
    if vocab > 10:
        assert int(idx[0]) == 5 and float(top[0, 0] - top[0, 1]) == 0.0
