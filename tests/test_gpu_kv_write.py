"""The HIP K/V write is bit-exact against the oracle's statements of the reference loop.

Reference semantics: engine/kernels/paged_attention_integration.py:148-161.
The whole pool is compared bit for bit, so the test also shows that nothing
outside the written slots changes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from engine.kernels.paged_attention_integration import paged_kv_write
from oracle.paged_attention_oracle import kv_write_reference, kv_write_scatter

pytestmark = pytest.mark.gpu


def _setup(num_seqs, hkv, d, bs, seed, device, lens=None):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    if lens is None:
        lens = rng.integers(1, 200, size=num_seqs).tolist()
    need = sum((n + bs - 1) // bs for n in lens)
    nb = need * 2 + 3
    perm = rng.permutation(nb).tolist()
    tables, pos = [], 0
    for n in lens:
        k = max(1, (n + bs - 1) // bs)
        tables.append(perm[pos:pos + k])
        pos += k
    width = max(len(t) for t in tables)
    bt = np.zeros((num_seqs, width), dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    pool_k = torch.randn(nb, bs, hkv, d, generator=g).half()
    pool_v = torch.randn(nb, bs, hkv, d, generator=g).half()
    key = torch.randn(num_seqs, hkv, d, generator=g).half()
    val = torch.randn(num_seqs, hkv, d, generator=g).half()
    return lens, tables, bt, pool_k, pool_v, key, val


def _bits(t):
    return t.cpu().contiguous().view(torch.int16).numpy()


@pytest.mark.parametrize("hkv,d,bs", [(2, 64, 16), (4, 128, 16), (8, 32, 8), (2, 64, 1), (3, 40, 5)])
def test_write_matches_oracle_bit_exact(cuda_device, hkv, d, bs):
    lens, tables, bt, pk, pv, key, val = _setup(37, hkv, d, bs, seed=hkv * 1000 + d + bs,
                                                device=cuda_device)
    kd, vd = pk.to(cuda_device), pv.to(cuda_device)
    paged_kv_write(key.to(cuda_device), val.to(cuda_device), kd, vd,
                   torch.from_numpy(bt).to(cuda_device),
                   torch.tensor(lens, dtype=torch.int32, device=cuda_device))
    rk, rv = pk.clone(), pv.clone()
    kv_write_reference(key, val, rk, rv, tables, lens, bs)
    sk, sv = _bits(pk), _bits(pv)
    kv_write_scatter(_bits(key), _bits(val), sk, sv, bt, np.array(lens))
    assert np.array_equal(_bits(rk), sk) and np.array_equal(_bits(rv), sv)  # oracle statements agree
    assert np.array_equal(_bits(kd), sk)
    assert np.array_equal(_bits(vd), sv)


def test_projection_views_and_block_boundaries(cuda_device):
    """key/value as the [B, Hkv, 1, D] transposed views the projections give; lengths on block edges."""
    B, hkv, d, bs = 6, 2, 64, 16
    lens = [1, 16, 17, 32, 33, 48]
    lens_, tables, bt, pk, pv, _, _ = _setup(B, hkv, d, bs, seed=77, device=cuda_device, lens=lens)
    g = torch.Generator().manual_seed(5)
    kproj = torch.randn(B, 1, hkv * d, generator=g).half()
    vproj = torch.randn(B, 1, hkv * d, generator=g).half()
    key_states = kproj.view(B, 1, hkv, d).transpose(1, 2)
    value_states = vproj.view(B, 1, hkv, d).transpose(1, 2)
    kd, vd = pk.to(cuda_device), pv.to(cuda_device)
    paged_kv_write(kproj.to(cuda_device).view(B, 1, hkv, d).transpose(1, 2),
                   vproj.to(cuda_device).view(B, 1, hkv, d).transpose(1, 2), kd, vd,
                   torch.from_numpy(bt).to(cuda_device),
                   torch.tensor(lens, dtype=torch.int32, device=cuda_device))
    rk, rv = pk.clone(), pv.clone()
    kv_write_reference(key_states.squeeze(2), value_states.squeeze(2), rk, rv, tables, lens, bs)
    assert np.array_equal(_bits(kd), _bits(rk)) and np.array_equal(_bits(vd), _bits(rv))


def test_scalar_path_for_strided_sources(cuda_device):
    """Sources with head_dim stride 2 take the element-wise path and stay bit-exact."""
    lens, tables, bt, pk, pv, key, val = _setup(9, 2, 64, 16, seed=8, device=cuda_device)
    kbig = torch.zeros(9, 2, 128, dtype=torch.float16)
    vbig = torch.zeros(9, 2, 128, dtype=torch.float16)
    kbig[..., ::2] = key
    vbig[..., ::2] = val
    kd, vd = pk.to(cuda_device), pv.to(cuda_device)
    paged_kv_write(kbig.to(cuda_device)[..., ::2], vbig.to(cuda_device)[..., ::2], kd, vd,
                   torch.from_numpy(bt).to(cuda_device),
                   torch.tensor(lens, dtype=torch.int32, device=cuda_device))
    rk, rv = pk.clone(), pv.clone()
    kv_write_reference(key, val, rk, rv, tables, lens, 16)
    assert np.array_equal(_bits(kd), _bits(rk)) and np.array_equal(_bits(vd), _bits(rv))


def test_block_table_indexing_with_encoded_patterns(cuda_device):
    """Each written row carries its (sequence, head, element) in its bits, so any indexing slip shows."""
    B, hkv, d, bs = 50, 2, 64, 16
    lens, tables, bt, pk, pv, _, _ = _setup(B, hkv, d, bs, seed=31, device=cuda_device)
    b_idx = torch.arange(B).view(B, 1, 1)
    h_idx = torch.arange(hkv).view(1, hkv, 1)
    e_idx = torch.arange(d).view(1, 1, d)
    code = (b_idx * 1024 + h_idx * 128 + e_idx).to(torch.int16)
    key = code.view(torch.float16)
    val = (code ^ 0x4000).view(torch.float16)
    kd, vd = torch.zeros_like(pk, device=cuda_device), torch.zeros_like(pv, device=cuda_device)
    paged_kv_write(key.to(cuda_device), val.to(cuda_device), kd, vd,
                   torch.from_numpy(bt).to(cuda_device),
                   torch.tensor(lens, dtype=torch.int32, device=cuda_device))
    kb, vb = _bits(kd), _bits(vd)
    for b, n in enumerate(lens):
        pid, off = tables[b][(n - 1) // bs], (n - 1) % bs
        assert np.array_equal(kb[pid, off], code[b].numpy())
        assert np.array_equal(vb[pid, off], (code[b] ^ 0x4000).numpy())
    assert np.count_nonzero(kb) == np.count_nonzero(code.numpy())


def test_rows_without_a_slot_are_skipped(cuda_device):
    """Length 0 rows and slots past the table width leave the pool untouched."""
    lens, tables, bt, pk, pv, key, val = _setup(4, 2, 64, 16, seed=12, device=cuda_device,
                                                lens=[20, 0, 5, 16])
    lens_dev = torch.tensor([20, 0, 5, 16 * bt.shape[1] + 1], dtype=torch.int32, device=cuda_device)
    kd, vd = pk.to(cuda_device), pv.to(cuda_device)
    paged_kv_write(key.to(cuda_device), val.to(cuda_device), kd, vd,
                   torch.from_numpy(bt).to(cuda_device), lens_dev)
    rk, rv = pk.clone(), pv.clone()
    kv_write_reference(key[[0, 2]], val[[0, 2]], rk, rv, [tables[0], tables[2]], [20, 5], 16)
    assert np.array_equal(_bits(kd), _bits(rk)) and np.array_equal(_bits(vd), _bits(rv))


def test_single_sequence_host_length(cuda_device):
    lens, tables, bt, pk, pv, key, val = _setup(1, 2, 64, 16, seed=4, device=cuda_device, lens=[41])
    kd, vd = pk.to(cuda_device), pv.to(cuda_device)
    paged_kv_write(key.to(cuda_device), val.to(cuda_device), kd, vd,
                   torch.from_numpy(bt[0]).to(cuda_device), 41)
    rk, rv = pk.clone(), pv.clone()
    kv_write_reference(key, val, rk, rv, tables, [41], 16)
    assert np.array_equal(_bits(kd), _bits(rk)) and np.array_equal(_bits(vd), _bits(rv))
