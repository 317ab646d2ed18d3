"""paged_rope_decode_attention (one decode step's attention block in one call)
against paged_rope_kv_write followed by paged_attention_decode_batched on the
same inputs (needs an MI355X).

Both the attention output and the whole K/V pool must be the same bits: the
one-launch kernel rotates q and the new key with the same fp16 operations as
the rotary write kernel, writes the same slot, and attends over the same rows
(the new token's taken from on-chip memory instead of the pool). Shapes cover
the one-launch form (one workgroup per (sequence, kv-head group): one and two
kv heads per pair, head_dim 64 and 128, block 16 and 32) and the two-launch form
(small batches), with zero-length, single-token and block-boundary sequences.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from engine.kernels.paged_attention import paged_attention_decode_batched
from engine.kernels.paged_attention_integration import (
    paged_rope_decode_attention,
    paged_rope_kv_write,
)
from oracle.paged_attention_oracle import naive_reference_paged_attention

pytestmark = pytest.mark.gpu


def make_case(num_seqs, hq, hkv, d, bs, lens, seed, device):
    rng = np.random.default_rng(seed)
    nblk = [max(1, (n + bs - 1) // bs) for n in lens]
    total = sum(nblk) + 4
    perm = rng.permutation(total).tolist()
    width = max(nblk) + 1
    bt = torch.zeros(num_seqs, width, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = torch.tensor(perm[pos:pos + n], dtype=torch.int32)
        pos += n
    gen = torch.Generator().manual_seed(seed)
    kc = torch.randn(total, bs, hkv, d, generator=gen).half()
    vc = torch.randn(total, bs, hkv, d, generator=gen).half()
    # q, k, v as the decode step makes them: views into one projection output.
    qkv = torch.randn(num_seqs, (hq + 2 * hkv) * d, generator=gen).half()
    q = qkv[:, :hq * d].view(num_seqs, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(num_seqs, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(num_seqs, hkv, d)
    ang = torch.rand(num_seqs, d // 2, generator=gen) * 6.0
    cos = torch.cat([ang.cos(), ang.cos()], dim=1).half()
    sin = torch.cat([ang.sin(), ang.sin()], dim=1).half()
    to = lambda t: t.to(device)
    return dict(q=to(q), k=to(k), v=to(v), cos=to(cos), sin=to(sin), kc=to(kc), vc=to(vc),
                bt=to(bt), lens=torch.tensor(lens, dtype=torch.int32, device=device),
                scale=d ** -0.5)


def run_both(c):
    kc1, vc1 = c["kc"].clone(), c["vc"].clone()
    kc2, vc2 = c["kc"].clone(), c["vc"].clone()
    got = paged_rope_decode_attention(c["q"], c["k"], c["v"], c["cos"], c["sin"], kc1, vc1,
                                      c["bt"], c["lens"], c["scale"])
    qr = paged_rope_kv_write(c["q"], c["k"], c["v"], c["cos"], c["sin"], kc2, vc2, c["bt"],
                             c["lens"])
    want = paged_attention_decode_batched(qr, kc2, vc2, c["bt"], c["lens"], c["scale"])
    torch.cuda.synchronize()
    return got, want, (kc1, vc1), (kc2, vc2), qr


def lens_for(n, rng, lo, hi, bs):
    lens = rng.integers(lo, hi, size=n).tolist()
    lens[0] = 0            # no tokens: zero rows, nothing written
    lens[1] = 1            # only the new token
    lens[2] = 3 * bs + 1   # the new token opens a block
    lens[3] = 4 * bs       # the new token closes a block
    return lens


@pytest.mark.parametrize("num_seqs,hq,hkv,d,bs", [
    (128, 14, 2, 64, 16),   # the Qwen2.5-0.5B decode step: one kv head per pair, one launch
    (200, 14, 2, 64, 16),   # pairs of two kv heads, one launch
    (32, 32, 8, 128, 32),   # head_dim 128, block 32, one launch
    (8, 14, 2, 64, 16),     # small batch: the two-launch form
    (96, 12, 4, 32, 16),    # head_dim 32: the two-launch form
])
def test_matches_rope_write_then_attention(cuda_device, num_seqs, hq, hkv, d, bs):
    rng = np.random.default_rng(num_seqs + d)
    lens = lens_for(num_seqs, rng, 64, 1100, bs)
    print(f"[rope-decode] B={num_seqs} hq={hq} hkv={hkv} d={d} bs={bs}", flush=True)
    c = make_case(num_seqs, hq, hkv, d, bs, lens, 7, cuda_device)
    got, want, pool1, pool2, qr = run_both(c)
    assert torch.equal(got, want), "attention output differs from the two-call path"
    assert torch.equal(pool1[0], pool2[0]) and torch.equal(pool1[1], pool2[1]), \
        "pool contents differ from the two-call path"
    assert torch.count_nonzero(got[0]).item() == 0  # the zero-length sequence
    # And against the fp32 oracle over the written pool with the rotated queries.
    sample = [1, 2, 3, num_seqs - 1]
    tables = [c["bt"][i, :(lens[i] + bs - 1) // bs].tolist() for i in sample]
    ref = naive_reference_paged_attention(qr[sample].cpu(), pool2[0].cpu(), pool2[1].cpu(), tables,
                                          [lens[i] for i in sample], c["scale"],
                                          compute_dtype=torch.float32)
    err = (got[sample].float().cpu() - ref).abs().max().item()
    assert err <= 2e-3, f"max abs err {err:.3e}"


def test_repeated_calls_are_bit_identical(cuda_device):
    c = make_case(128, 14, 2, 64, 16, lens_for(128, np.random.default_rng(3), 64, 1100, 16), 9,
                  cuda_device)
    kc, vc = c["kc"].clone(), c["vc"].clone()
    a = paged_rope_decode_attention(c["q"], c["k"], c["v"], c["cos"], c["sin"], kc, vc, c["bt"],
                                    c["lens"], c["scale"])
    b = paged_rope_decode_attention(c["q"], c["k"], c["v"], c["cos"], c["sin"], kc, vc, c["bt"],
                                    c["lens"], c["scale"])
    torch.cuda.synchronize()
    assert torch.equal(a, b)
