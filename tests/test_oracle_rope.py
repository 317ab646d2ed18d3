"""The RoPE restatement of the oracle is pinned against transformers itself (no GPU).

transformers' apply_rotary_pos_emb (5.15.0, pinned by the reference's
requirements.txt:3) is what the reference calls on the new token's q and k
(engine/kernels/paged_attention_integration.py:108-109). The oracle's numpy
restatement must give the same fp16 bits, and satisfy two closed forms.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.paged_attention_oracle import rope_fp16


def _hf_rope(q, k, cos, sin):
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    return apply_rotary_pos_emb(q, k, cos, sin)


def _tables(num_seqs, head_dim, positions, theta=1e6):
    """cos/sin rows [B, 1, D] fp16 the way the model's rotary module builds them."""
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    cfg = Qwen2Config(hidden_size=head_dim * 4, num_attention_heads=4, rope_theta=theta,
                      max_position_embeddings=65536)
    rot = Qwen2RotaryEmbedding(cfg)
    x = torch.zeros(1, dtype=torch.float16)
    pos = torch.tensor(positions, dtype=torch.long).view(num_seqs, 1)
    return rot(x, pos)


@pytest.mark.parametrize("d,hq,hkv,seed", [(64, 14, 2, 0), (128, 28, 4, 1), (32, 8, 8, 2)])
def test_rope_oracle_matches_transformers_bit_for_bit(d, hq, hkv, seed):
    g = torch.Generator().manual_seed(seed)
    B = 9
    positions = [0, 1, 2, 15, 16, 1023, 4096, 32767, 65535][:B]
    cos, sin = _tables(B, d, positions)
    q = (torch.randn(B, hq, 1, d, generator=g) * 3).half()
    k = (torch.randn(B, hkv, 1, d, generator=g) * 3).half()
    q_hf, k_hf = _hf_rope(q, k, cos, sin)
    c = cos.numpy()[:, None]  # [B, 1, 1, D]
    s = sin.numpy()[:, None]
    assert np.array_equal(rope_fp16(q.numpy(), c, s).view(np.int16), q_hf.numpy().view(np.int16))
    assert np.array_equal(rope_fp16(k.numpy(), c, s).view(np.int16), k_hf.numpy().view(np.int16))


def test_rope_oracle_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 64)).astype(np.float16)
    one = np.ones(64, np.float16)
    zero = np.zeros(64, np.float16)
    # Position 0: cos = 1, sin = 0 -> identity.
    assert np.array_equal(rope_fp16(x, one, zero).view(np.int16), x.view(np.int16))
    # cos = 0, sin = 1 (a quarter turn): (x1, x2) -> (-x2, x1), exactly.
    want = np.concatenate([-x[:, 32:], x[:, :32]], axis=1)
    assert np.array_equal(rope_fp16(x, zero, one).view(np.int16), want.view(np.int16))
