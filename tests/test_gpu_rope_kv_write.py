"""The fused rotary-embedding + K/V write is bit-exact against the oracle and transformers.

Reference semantics: transformers' apply_rotary_pos_emb on the new token's q and
k (engine/kernels/paged_attention_integration.py:108-109) and the K/V write loop
(:148-161). The rotated queries and the whole pool are compared bit for bit
with the oracle's rope_fp16 + kv_write_scatter, and the queries also with
transformers' own function run on the GPU.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from engine.kernels.paged_attention_integration import paged_rope_kv_write
from oracle.paged_attention_oracle import kv_write_scatter, rope_fp16

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.cpu().contiguous().view(torch.int16).numpy()


def _rotary(positions, d, theta=1e6):
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    cfg = Qwen2Config(hidden_size=d * 4, num_attention_heads=4, rope_theta=theta,
                      max_position_embeddings=65536)
    rot = Qwen2RotaryEmbedding(cfg)
    pos = torch.tensor(positions, dtype=torch.long).view(-1, 1)
    return rot(torch.zeros(1, dtype=torch.float16), pos)  # [B, 1, D] fp16 each


def _case(num_seqs, hq, hkv, d, bs, seed, lens=None):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    if lens is None:
        lens = rng.integers(1, 300, size=num_seqs).tolist()
    need = sum(max(1, (n + bs - 1) // bs) for n in lens)
    nb = need * 2 + 3
    perm = rng.permutation(nb).tolist()
    tables, at = [], 0
    for n in lens:
        k = max(1, (n + bs - 1) // bs)
        tables.append(perm[at:at + k])
        at += k
    bt = np.zeros((num_seqs, max(len(t) for t in tables)), dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    pool_k = torch.randn(nb, bs, hkv, d, generator=g).half()
    pool_v = torch.randn(nb, bs, hkv, d, generator=g).half()
    # Projection-shaped inputs: [B, 1, H * D] -> view [B, 1, H, D] -> transpose(1, 2).
    qp = (torch.randn(num_seqs, 1, hq * d, generator=g) * 2).half()
    kp = (torch.randn(num_seqs, 1, hkv * d, generator=g) * 2).half()
    vp = torch.randn(num_seqs, 1, hkv * d, generator=g).half()
    cos, sin = _rotary([max(n - 1, 0) for n in lens], d)
    return lens, bt, pool_k, pool_v, qp, kp, vp, cos, sin


def _views(t, heads, d):
    return t.view(t.shape[0], 1, heads, d).transpose(1, 2)  # [B, H, 1, D], strides (H*D, D, H*D, 1)


def _oracle(lens, bt, pk, pv, q, k, v, cos, sin):
    c = cos.numpy()[:, None]  # [B, 1, 1, D]
    s = sin.numpy()[:, None]
    q_rot = rope_fp16(q.numpy(), c, s)[:, :, 0]
    k_rot = rope_fp16(k.numpy(), c, s)[:, :, 0]
    sk, sv = _bits(pk), _bits(pv)
    kv_write_scatter(k_rot.view(np.int16), v.numpy()[:, :, 0].view(np.int16), sk, sv, bt, np.array(lens))
    return q_rot.view(np.int16), sk, sv


@pytest.mark.parametrize("hq,hkv,d,bs", [(14, 2, 64, 16), (28, 4, 128, 16), (8, 8, 32, 8),
                                         (4, 2, 16, 3), (6, 2, 40, 16)])
def test_fused_rope_write_bit_exact(cuda_device, hq, hkv, d, bs):
    lens, bt, pk, pv, qp, kp, vp, cos, sin = _case(41, hq, hkv, d, bs, seed=hq * 100 + d + bs)
    q, k, v = _views(qp, hq, d), _views(kp, hkv, d), _views(vp, hkv, d)
    kd, vd = pk.to(cuda_device), pv.to(cuda_device)
    q_rot = paged_rope_kv_write(_views(qp.to(cuda_device), hq, d), _views(kp.to(cuda_device), hkv, d),
                                _views(vp.to(cuda_device), hkv, d), cos.to(cuda_device),
                                sin.to(cuda_device), kd, vd, torch.from_numpy(bt).to(cuda_device),
                                torch.tensor(lens, dtype=torch.int32, device=cuda_device))
    torch.cuda.synchronize()
    want_q, want_k, want_v = _oracle(lens, bt, pk, pv, q, k, v, cos, sin)
    assert q_rot.shape == (41, hq, d) and q_rot.is_contiguous()
    assert np.array_equal(_bits(q_rot), want_q)
    assert np.array_equal(_bits(kd), want_k)
    assert np.array_equal(_bits(vd), want_v)
    print(f"[rope] hq={hq} hkv={hkv} d={d} bs={bs}: q, K and V pool bit-exact", flush=True)


def test_matches_transformers_on_gpu(cuda_device):
    """Same bits as transformers' apply_rotary_pos_emb computed on the GPU in fp16."""
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    lens, bt, pk, pv, qp, kp, vp, cos, sin = _case(64, 14, 2, 64, 16, seed=7,
                                                   lens=list(range(1, 20000, 312))[:64])
    qd, kdv, vdv = qp.cuda(), kp.cuda(), vp.cuda()
    cd, sd = cos.cuda(), sin.cuda()
    q_hf, k_hf = apply_rotary_pos_emb(_views(qd, 14, 64), _views(kdv, 2, 64), cd, sd)
    kd, vd = pk.cuda(), pv.cuda()
    q_rot = paged_rope_kv_write(_views(qd, 14, 64), _views(kdv, 2, 64), _views(vdv, 2, 64), cd, sd,
                                kd, vd, torch.from_numpy(bt).cuda(),
                                torch.tensor(lens, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(q_rot), _bits(q_hf.squeeze(2)))
    L = np.array(lens)
    ids = bt[np.arange(len(lens)), (L - 1) // 16]
    assert np.array_equal(_bits(kd)[ids, (L - 1) % 16], _bits(k_hf.squeeze(2)))


def test_strided_head_dim_takes_element_path(cuda_device):
    """Inputs whose head_dim stride is not 1 (element path) give the same bits."""
    lens, bt, pk, pv, qp, kp, vp, cos, sin = _case(9, 4, 2, 32, 16, seed=21)
    # Head_dim stride 2: take every other element of a doubled tensor.
    q2 = torch.stack([qp, qp], -1).flatten(-2)[..., ::2]
    k2 = torch.stack([kp, kp], -1).flatten(-2)[..., ::2]
    assert q2.stride(-1) == 2
    q_in = q2.unflatten(-1, (4, 32)).transpose(1, 2)
    k_in = k2.unflatten(-1, (2, 32)).transpose(1, 2)
    assert q_in.stride(-1) == 2
    kd, vd = pk.cuda(), pv.cuda()
    q_rot = paged_rope_kv_write(q_in.cuda(), k_in.cuda(), _views(vp.cuda(), 2, 32), cos.cuda(),
                                sin.cuda(), kd, vd, torch.from_numpy(bt).cuda(),
                                torch.tensor(lens, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    want_q, want_k, want_v = _oracle(lens, bt, pk, pv, _views(qp, 4, 32), _views(kp, 2, 32),
                                     _views(vp, 2, 32), cos, sin)
    assert np.array_equal(_bits(q_rot), want_q)
    assert np.array_equal(_bits(kd), want_k) and np.array_equal(_bits(vd), want_v)


def test_single_sequence_and_missing_slots(cuda_device):
    """A host length for one sequence; rows with L <= 0 or a block past the table write nothing."""
    lens, bt, pk, pv, qp, kp, vp, cos, sin = _case(1, 14, 2, 64, 16, seed=5, lens=[77])
    kd, vd = pk.cuda(), pv.cuda()
    q_rot = paged_rope_kv_write(_views(qp.cuda(), 14, 64), _views(kp.cuda(), 2, 64),
                                _views(vp.cuda(), 2, 64), cos.cuda(), sin.cuda(), kd, vd,
                                torch.from_numpy(bt[0]).cuda(), 77)
    torch.cuda.synchronize()
    want_q, want_k, want_v = _oracle(lens, bt, pk, pv, _views(qp, 14, 64), _views(kp, 2, 64),
                                     _views(vp, 2, 64), cos, sin)
    assert np.array_equal(_bits(q_rot), want_q) and np.array_equal(_bits(kd), want_k)
    lens2, bt2, pk2, pv2, qp2, kp2, vp2, cos2, sin2 = _case(3, 14, 2, 64, 16, seed=6, lens=[20, 40, 60])
    kd2, vd2 = pk2.cuda(), pv2.cuda()
    bad = torch.tensor([0, -5, 60], dtype=torch.int32, device="cuda")  # no slot for rows 0 and 1
    bt_narrow = torch.from_numpy(bt2[:, :1].copy()).cuda()             # row 2's block 3 is past the table
    paged_rope_kv_write(_views(qp2.cuda(), 14, 64), _views(kp2.cuda(), 2, 64), _views(vp2.cuda(), 2, 64),
                        cos2.cuda(), sin2.cuda(), kd2, vd2, bt_narrow, bad)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(kd2), _bits(pk2)) and np.array_equal(_bits(vd2), _bits(pv2))
