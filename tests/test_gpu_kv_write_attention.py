"""paged_decode_kv_write_attention: the new token's K/V write and batched attention in one
call (needs an MI355X).

Reference: the K/V write loop of paged_decode_attention_forward and the
paged_attention_decode_batched call after it
(engine/kernels/paged_attention_integration.py:148-161, :164-171). The fused
call must give the same bits as paged_kv_write followed by
paged_attention_decode_batched on the same inputs -- the output and the whole
pool -- on every schedule: one workgroup per pair (decode_pair_kernel),
stream-K ranges with and without shared prefixes (decode_streamk_kernel),
head_dim 64 and 128, blocks of 16 and 32, and the shapes served by two
launches (head_dim 32, more than 1024 sequences). Invalid lengths (zero, past
the table) are covered too, and one case is checked against the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from engine import workloads
from engine.kernels import _native
from engine.kernels.paged_attention import paged_attention_decode_batched
from engine.kernels.paged_attention_integration import (paged_decode_kv_write_attention,
                                                       paged_kv_write)

pytestmark = pytest.mark.gpu


def _new_rows(w, seed):
    g = torch.Generator(device=w.q.device).manual_seed(seed)
    hkv, d = w.k_cache.shape[2], w.k_cache.shape[3]
    k = torch.randn(w.num_seqs, hkv, d, generator=g, device=w.q.device).half()
    v = torch.randn(w.num_seqs, hkv, d, generator=g, device=w.q.device).half()
    return k, v


def _both(w, seed, name):
    """Outputs and pools of the fused call and of the two calls, on copies of the pool."""
    k, v = _new_rows(w, seed)
    kc2, vc2 = w.k_cache.clone(), w.v_cache.clone()
    sched = _native.decode_schedule(w.num_seqs, w.q.shape[1], w.k_cache.shape[2],
                                    w.k_cache.shape[3], w.k_cache.shape[1],
                                    w.block_tables.shape[1])
    print(f"[kv-write-attention] {name}: {sched}", flush=True)
    paged_kv_write(k, v, w.k_cache, w.v_cache, w.block_tables, w.seq_lens)
    want = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables,
                                          w.seq_lens, w.scale)
    got = paged_decode_kv_write_attention(w.q, k, v, kc2, vc2, w.block_tables, w.seq_lens,
                                          w.scale)
    again = paged_decode_kv_write_attention(w.q, k, v, kc2, vc2, w.block_tables, w.seq_lens,
                                            w.scale)
    torch.cuda.synchronize()
    return got, want, again, kc2, vc2, sched


def _check(w, seed, name):
    got, want, again, kc2, vc2, sched = _both(w, seed, name)
    assert torch.equal(got, again), f"{name}: two fused calls differ"
    assert torch.equal(got, want), (
        f"{name}: fused output differs from write + attention in "
        f"{int((got != want).sum())} values")
    assert torch.equal(kc2.view(torch.int16), w.k_cache.view(torch.int16)), f"{name}: K pool differs"
    assert torch.equal(vc2.view(torch.int16), w.v_cache.view(torch.int16)), f"{name}: V pool differs"
    return sched


def test_pair_per_workgroup_schedule(cuda_device):
    assert _check(workloads.qwen_layer(device=cuda_device, seed=21), 1,
                  "qwen_layer B8")["path"] == "pair_per_workgroup"
    assert _check(workloads.decode_step_layer(128, cuda_device, 22), 2,
                  "decode layer B128")["path"] == "pair_per_workgroup"


def test_stream_k_with_shared_prefixes(cuda_device):
    w = workloads.long_context(device=cuda_device, seed=23, num_seqs=96)
    sched = _check(w, 3, "long_context B96")
    assert sched["path"] == "stream_k" and sched["shared_prefixes"]


def test_stream_k_headline_shape(cuda_device):
    w = workloads.long_context(device=cuda_device, seed=24)
    assert _check(w, 4, "long_context B256")["kv_heads_per_pair"] == 2


def test_stream_k_numerics_shape_and_head_dim_128(cuda_device):
    assert _check(workloads.softmax_stress(device=cuda_device, seed=25), 5,
                  "softmax_stress")["path"] == "stream_k"
    lens = np.random.default_rng(26).integers(1, 3000, size=40).tolist()
    w = workloads.make_random(40, 28, 7, 128, lens, 16, seed=26, device=cuda_device)
    _check(w, 6, "B40 D128 g4")


@pytest.mark.parametrize("bs", [32, 8])
def test_block_sizes(cuda_device, bs):
    # Block 32 takes the fused kernels; block 8 the two launches.
    lens = np.random.default_rng(27 + bs).integers(1, 2600, size=70).tolist()
    w = workloads.make_random(70, 14, 2, 64, lens, bs, seed=27 + bs, device=cuda_device)
    _check(w, 7, f"block {bs}")


def test_two_launch_shapes(cuda_device):
    lens = np.random.default_rng(29).integers(1, 700, size=24).tolist()
    _check(workloads.make_random(24, 8, 2, 32, lens, 16, seed=29, device=cuda_device), 8,
           "head_dim 32")
    lens = np.random.default_rng(30).integers(1, 300, size=1030).tolist()
    w = workloads.make_random(1030, 14, 2, 64, lens, 16, seed=30, device=cuda_device)
    assert _check(w, 9, "1030 sequences")["path"] == "fixed_split"


def test_empty_and_past_table_lengths(cuda_device):
    # Length 0 (nothing written, zero output), a length past the table width (the write is
    # skipped and the attention clamps the length) and one filling the table exactly, next to
    # ordinary ones, on both schedules. Those three rows list blocks no other sequence uses, so
    # that no sequence reads a slot another one writes (a write into a shared block, which the
    # reference's runner refuses).
    for n, name in ((8, "pair"), (300, "stream-K")):
        lens = np.random.default_rng(31 + n).integers(1, 900, size=n).tolist()
        w = workloads.make_random(n, 14, 2, 64, lens, 16, seed=31 + n, device=cuda_device)
        width = w.block_tables.shape[1]
        used = {i for t in w.tables for i in t}
        free = [i for i in range(w.k_cache.shape[0]) if i not in used]
        assert len(free) >= 3 * width
        for r in range(3):
            w.block_tables[r] = torch.tensor(free[r * width:(r + 1) * width], dtype=torch.int32)
        w.seq_lens[0] = 0
        w.seq_lens[1] = width * 16 + 5
        w.seq_lens[2] = width * 16
        got, want, again, kc2, vc2, _ = _both(w, 10 + n, f"edge lengths ({name})")
        assert torch.equal(got, want) and torch.equal(got, again)
        assert torch.count_nonzero(got[0]) == 0
        assert torch.equal(kc2.view(torch.int16), w.k_cache.view(torch.int16))
        assert torch.equal(vc2.view(torch.int16), w.v_cache.view(torch.int16))


def test_against_the_oracle(cuda_device):
    from oracle.paged_attention_oracle import kv_write_scatter, naive_reference_paged_attention

    w = workloads.long_context(device=cuda_device, seed=33, num_seqs=64)
    k, v = _new_rows(w, 11)
    kc_host = w.k_cache.cpu().view(torch.int16).numpy().copy()
    vc_host = w.v_cache.cpu().view(torch.int16).numpy().copy()
    got = paged_decode_kv_write_attention(w.q, k, v, w.k_cache, w.v_cache, w.block_tables,
                                          w.seq_lens, w.scale)
    torch.cuda.synchronize()
    kv_write_scatter(k.cpu().view(torch.int16).numpy(), v.cpu().view(torch.int16).numpy(),
                     kc_host, vc_host, w.block_tables.cpu().numpy(), np.array(w.lens))
    assert np.array_equal(w.k_cache.cpu().view(torch.int16).numpy(), kc_host)
    assert np.array_equal(w.v_cache.cpu().view(torch.int16).numpy(), vc_host)
    kc = torch.from_numpy(kc_host).view(torch.float16)
    vc = torch.from_numpy(vc_host).view(torch.float16)
    want = naive_reference_paged_attention(w.q.cpu(), kc, vc, w.tables, w.lens, w.scale,
                                           compute_dtype=torch.float32)
    err = (got.float().cpu() - want).abs().max().item()
    print(f"[kv-write-attention] oracle: max abs err {err:.3e}", flush=True)
    assert err <= 2e-3
