"""Parity of the HIP decode-attention kernels with the CPU oracle (needs an MI355X).

Gate: max |kernel - oracle| <= 2e-3, where the oracle runs the reference
algorithm in fp32 on the same fp16 inputs and the kernel stores fp16 (fp32
accumulation). The reference's own GPU tests use atol=rtol=1e-2
(tests/test_paged_attention_reference.py:354-360); this gate is tighter.
Cases follow those tests (configurations, seeds, sparse shuffled pools) and add
the measured workload shapes.
"""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from engine import workloads
from engine.kernels.paged_attention import (
    paged_attention_decode,
    paged_attention_decode_batched,
    paged_attention_decode_v1,
    paged_attention_decode_v2,
    pad_block_tables,
)
from oracle.paged_attention_oracle import naive_reference_paged_attention

pytestmark = pytest.mark.gpu

TOL = 2e-3


def oracle32(q, k, v, tables, lens, scale):
    return naive_reference_paged_attention(q.cpu(), k.cpu(), v.cpu(), tables, lens, scale,
                                           compute_dtype=torch.float32)


def max_err(got, want):
    return (got.float().cpu() - want.float()).abs().max().item()


def reference_style_case(hq, hkv, d, bs, seq_len, seed, device, mag=1.0, slack=None):
    """Pool built the way the reference's GPU tests build it (:287-318)."""
    torch.manual_seed(seed)
    random.seed(seed)
    nlog = (seq_len + bs - 1) // bs
    nphys = slack if slack is not None else nlog * 3 + 4
    ids = random.sample(range(nphys), nlog)
    q = torch.randn(hq, d).half() * mag
    kf = torch.randn(seq_len, hkv, d).half() * mag
    vf = torch.randn(seq_len, hkv, d).half()
    kc = torch.zeros(nphys, bs, hkv, d, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    for j, pid in enumerate(ids):
        take = min(bs, seq_len - j * bs)
        kc[pid, :take] = kf[j * bs:j * bs + take]
        vc[pid, :take] = vf[j * bs:j * bs + take]
    return (q.to(device), kc.to(device), vc.to(device),
            torch.tensor(ids, dtype=torch.int32, device=device), ids)


REF_CONFIGS = [
    (8, 8, 32, 16, 37, 201),
    (8, 4, 32, 16, 45, 202),
    (14, 2, 64, 16, 67, 203),
    (14, 2, 64, 16, 32, 204),
    (4, 1, 64, 8, 19, 205),
]


@pytest.mark.parametrize("hq,hkv,d,bs,L,seed", REF_CONFIGS)
def test_v1_matches_oracle(cuda_device, hq, hkv, d, bs, L, seed):
    q, kc, vc, bt, ids = reference_style_case(hq, hkv, d, bs, L, seed, cuda_device)
    out = paged_attention_decode_v1(q, kc, vc, bt, L, d ** -0.5)
    want = oracle32(q.unsqueeze(0), kc, vc, [ids], [L], d ** -0.5)[0]
    assert out.shape == q.shape and out.dtype == torch.float16
    assert max_err(out, want) <= TOL


@pytest.mark.parametrize("hq,hkv,d,bs,L,seed", [(h, k, d, b, L, s + 100) for h, k, d, b, L, s in REF_CONFIGS])
def test_v2_matches_oracle_and_v1(cuda_device, hq, hkv, d, bs, L, seed):
    q, kc, vc, bt, ids = reference_style_case(hq, hkv, d, bs, L, seed, cuda_device)
    o1 = paged_attention_decode_v1(q, kc, vc, bt, L, d ** -0.5)
    o2 = paged_attention_decode_v2(q, kc, vc, bt, L, d ** -0.5)
    want = oracle32(q.unsqueeze(0), kc, vc, [ids], [L], d ** -0.5)[0]
    assert max_err(o2, want) <= TOL
    assert max_err(o2, o1.float().cpu()) <= TOL


def test_long_sequence_2048(cuda_device):
    q, kc, vc, bt, ids = reference_style_case(14, 2, 64, 16, 2048, 401, cuda_device, slack=148)
    o1 = paged_attention_decode_v1(q, kc, vc, bt, 2048, 0.125)
    o2 = paged_attention_decode_v2(q, kc, vc, bt, 2048, 0.125)
    want = oracle32(q.unsqueeze(0), kc, vc, [ids], [2048], 0.125)[0]
    for o in (o1, o2):
        assert torch.isfinite(o).all()
        assert max_err(o, want) <= TOL


def test_large_magnitude_scores(cuda_device):
    """q, k scaled by 10: scaled scores reach hundreds (reference :488-537)."""
    q, kc, vc, bt, ids = reference_style_case(8, 2, 64, 16, 250, 501, cuda_device, mag=10.0,
                                              slack=26)
    o1 = paged_attention_decode_v1(q, kc, vc, bt, 250, 0.125)
    o2 = paged_attention_decode_v2(q, kc, vc, bt, 250, 0.125)
    want = naive_reference_paged_attention(q.cpu().unsqueeze(0), kc.cpu(), vc.cpu(), [ids], [250],
                                           0.125, compute_dtype=torch.float64)[0]
    for o in (o1, o2):
        assert torch.isfinite(o).all()
        assert max_err(o, want) <= TOL


def test_batched_variable_lengths(cuda_device):
    """Lengths [1, 17, 500, 2000] in one launch; also equals a per-sequence v2 loop (:540-643)."""
    torch.manual_seed(601)
    random.seed(601)
    lens = [1, 17, 500, 2000]
    bs, hq, hkv, d = 16, 14, 2, 64
    nphys = sum((n + bs - 1) // bs for n in lens) + 40
    kc = torch.zeros(nphys, bs, hkv, d, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    used, tables, qs = set(), [], []
    for n in lens:
        qs.append(torch.randn(hq, d).half())
        kf, vf = torch.randn(n, hkv, d).half(), torch.randn(n, hkv, d).half()
        nb = (n + bs - 1) // bs
        ids = random.sample([i for i in range(nphys) if i not in used], nb)
        used.update(ids)
        for j, pid in enumerate(ids):
            take = min(bs, n - j * bs)
            kc[pid, :take] = kf[j * bs:j * bs + take]
            vc[pid, :take] = vf[j * bs:j * bs + take]
        tables.append(ids)
    q = torch.stack(qs)
    qd, kd, vd = q.to(cuda_device), kc.to(cuda_device), vc.to(cuda_device)
    out = paged_attention_decode_batched(qd, kd, vd, pad_block_tables(tables, device=cuda_device),
                                         torch.tensor(lens, dtype=torch.int32, device=cuda_device),
                                         d ** -0.5)
    want = oracle32(q, kc, vc, tables, lens, d ** -0.5)
    assert max_err(out, want) <= TOL
    for i, n in enumerate(lens):
        o2 = paged_attention_decode_v2(qd[i], kd, vd, torch.tensor(tables[i], dtype=torch.int32,
                                                                   device=cuda_device), n, d ** -0.5)
        assert max_err(out[i], o2.float().cpu()) <= TOL
    lst = paged_attention_decode(qd, kd, vd, tables, lens, d ** -0.5)
    assert torch.equal(lst, out)


def _check_workload(w, seqs=None, tol=TOL, fp64=False):
    out = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables, w.seq_lens,
                                         w.scale)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    if seqs is None:
        seqs = list(range(w.num_seqs))
    q, k, v, tables, lens = workloads.gather_subset(w, seqs)
    want = naive_reference_paged_attention(q, k, v, tables, lens, w.scale,
                                           compute_dtype=torch.float64 if fp64 else torch.float32)
    err = max_err(out[seqs], want)
    print(f"[parity] {w.name}: {len(seqs)} seqs, max abs err {err:.3e}", flush=True)
    assert err <= tol
    return out


def test_workload_qwen_layer(cuda_device):
    w = workloads.qwen_layer(device=cuda_device, seed=0)
    _check_workload(w)


def test_workload_softmax_stress(cuda_device):
    """q, k ~ N(0, 8^2): scaled scores with sigma ~64; long rows exercise split-K."""
    w = workloads.softmax_stress(device=cuda_device, seed=0)
    _check_workload(w, fp64=True)


@pytest.mark.parametrize("hkv", [28, 14, 7, 4])
def test_workload_gqa_sweep(cuda_device, hkv):
    """Batch 64 x 2048 tokens, 28 q heads, head_dim 128: every sequence against the oracle."""
    w = workloads.gqa_sweep(hkv, device=cuda_device, seed=hkv)
    _check_workload(w)


def test_workload_long_context(cuda_device):
    """The headline shape (batch 256, lognormal lengths to ~19k, groups of 8 sharing prefix
    blocks): every sequence against the oracle."""
    w = workloads.long_context(device=cuda_device, seed=0)
    _check_workload(w)


def _device_cus(device):
    return torch.cuda.get_device_properties(device).multi_processor_count


@pytest.mark.parametrize("extra", [0, 1])
def test_decode_step_layer_at_the_head_group_boundary(cuda_device, extra):
    """One layer's call of the batch-128 decode step (14 q / 2 kv, head_dim 64, lengths
    64 + U[64, 1024]), every row against the oracle. With sequences x kv heads up to the CU
    count each (sequence, kv head) pair runs alone on a workgroup; one sequence more and
    pairs hold both kv heads. Both sides of that boundary are checked: batch CUs/2 (128 on
    MI355X, the decode step's own schedule) and CUs/2 + 1."""
    b = _device_cus(cuda_device) // 2 + extra
    w = workloads.decode_step_layer(b, device=cuda_device, seed=b)
    _check_workload(w)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("bs", [1, 8, 12, 16, 32])
def test_head_dims_and_block_sizes(cuda_device, d, bs):
    lens = [1, bs, bs + 1, 15, 16, 17, 300, 700]
    w = workloads.make_random(len(lens), 4 * 2, 2, d, lens, bs, seed=d * 100 + bs,
                              device=cuda_device)
    _check_workload(w)


@pytest.mark.parametrize("g", [1, 2, 3, 4, 7, 8, 16])
def test_group_sizes(cuda_device, g):
    lens = [5, 64, 257, 1030]
    w = workloads.make_random(len(lens), 2 * g, 2, 64, lens, 16, seed=g, device=cuda_device)
    _check_workload(w)


def test_zero_length_rows_are_zero(cuda_device):
    w = workloads.make_random(3, 14, 2, 64, [0, 40, 0], 16, seed=3, device=cuda_device)
    out = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables, w.seq_lens,
                                         w.scale)
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0
    q, k, v, tables, lens = workloads.gather_subset(w, [1])
    assert max_err(out[1:2], oracle32(q, k, v, tables, lens, w.scale)) <= TOL
    o1 = paged_attention_decode_v1(w.q[0], w.k_cache, w.v_cache, w.block_tables[0], 0, w.scale)
    o2 = paged_attention_decode_v2(w.q[0], w.k_cache, w.v_cache, w.block_tables[0], 0, w.scale)
    assert torch.count_nonzero(o1) == 0 and torch.count_nonzero(o2) == 0


def test_strided_query_and_table_views(cuda_device):
    w = workloads.make_random(4, 14, 2, 64, [33, 100, 7, 513], 16, seed=9, device=cuda_device)
    base = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables, w.seq_lens,
                                          w.scale)
    qbig = torch.zeros(4, 14, 3, 64, dtype=torch.float16, device=cuda_device)
    qbig[:, :, 1] = w.q
    btbig = torch.zeros(4, w.block_tables.shape[1] * 2, dtype=torch.int32, device=cuda_device)
    btbig[:, ::2] = w.block_tables
    out = paged_attention_decode_batched(qbig[:, :, 1], w.k_cache, w.v_cache, btbig[:, ::2],
                                         w.seq_lens, w.scale)
    assert torch.equal(out, base)


@pytest.mark.parametrize("name", ["softmax_stress", "qwen_layer", "long_context"])
def test_repeatable_bits(cuda_device, name):
    """Repeated calls return the same bits: short launches (one pair per workgroup), mid-size
    ones, and the B256 long-context shape where every workgroup walks hundreds of tiles."""
    w = getattr(workloads, name)(device=cuda_device, seed=5)
    a = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables, w.seq_lens, w.scale)
    for _ in range(4):
        b = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables, w.seq_lens,
                                           w.scale)
        assert torch.equal(a, b)


def test_shared_blocks_across_sequences(cuda_device):
    """Several sequences listing the same physical blocks (prefix sharing) read them correctly."""
    w = workloads.long_context(device=cuda_device, seed=1, num_seqs=16)
    _check_workload(w)


@pytest.mark.parametrize("d", [64, 128])
def test_large_batch_fixed_split_path(cuda_device, d):
    """More than 1024 sequences take the fixed 512-token split-K kernel and its merge."""
    rng = np.random.default_rng(d)
    lens = rng.integers(1, 1500, size=1100).tolist()
    lens[0], lens[1], lens[2] = 0, 512, 1537
    w = workloads.make_random(len(lens), 14 if d == 64 else 8, 2, d, lens, 16, seed=d,
                              device=cuda_device)
    out = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables, w.seq_lens,
                                         w.scale)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[0]) == 0
    seqs = list(range(1, len(lens)))  # every row (row 0 is empty and checked above)
    q, k, v, tables, ls = workloads.gather_subset(w, seqs)
    err = max_err(out[seqs], oracle32(q, k, v, tables, ls, w.scale))
    print(f"[parity] fixed-split path D{d}: {len(seqs)} rows, max abs err {err:.3e}", flush=True)
    assert err <= TOL


def _decode_counters(device):
    """The pair-counter region (first 256 KB) of this stream's decode workspace."""
    from engine.kernels import _native

    key = (device.index, torch.cuda.current_stream(device).cuda_stream, _native.WS_DECODE)
    return _native._workspaces[key][:65536 * 4].view(torch.int32)


def test_merge_counters_return_to_zero(cuda_device):
    """Every call leaves the in-kernel merge counters at zero (the next call relies on it)."""
    w = workloads.long_context(device=cuda_device, seed=3, num_seqs=64)
    first = None
    for _ in range(3):
        out = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables,
                                             w.seq_lens, w.scale)
        torch.cuda.synchronize()
        assert torch.count_nonzero(_decode_counters(cuda_device)).item() == 0
        first = out if first is None else first
        assert max_err(out, first.float().cpu()) <= TOL
    _check_workload(w, seqs=[0, 1, 7, 8, 31, 63])


def test_calls_run_on_the_current_stream(cuda_device):
    """The launch goes to the caller's current torch stream (a side stream here): the handle
    the wrapper passes is that stream's, and the result equals the default stream's."""
    from engine.kernels import _native

    w = workloads.qwen_layer(device=cuda_device, seed=5)
    want = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables,
                                          w.seq_lens, w.scale)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=cuda_device)
    with torch.cuda.stream(side):
        assert _native.stream_handle(cuda_device) == side.cuda_stream
        assert _native.stream_handle(torch.device("cuda")) == side.cuda_stream
        got = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables,
                                             w.seq_lens, w.scale)
    side.synchronize()
    assert _native.stream_handle(cuda_device) == torch.cuda.current_stream(cuda_device).cuda_stream
    assert torch.equal(got, want)


def test_paths_interleaved_on_one_stream(cuda_device):
    """Stream-K, fixed-split and two-pass calls alternate on one stream without
    disturbing each other's scratch: each result still matches the oracle."""
    a = workloads.long_context(device=cuda_device, seed=4, num_seqs=32)
    rng = np.random.default_rng(11)
    lens = rng.integers(1, 900, size=1030).tolist()
    big = workloads.make_random(len(lens), 14, 2, 64, lens, 16, seed=12, device=cuda_device)
    q1, kc, vc, bt, ids = reference_style_case(14, 2, 64, 16, 777, 13, cuda_device)
    for _ in range(2):
        _check_workload(a, seqs=[0, 5, 9, 31])
        _check_workload(big, seqs=[0, 1, 515, 1029])
        got = paged_attention_decode_v1(q1, kc, vc, bt, 777, 0.125)
        want = oracle32(q1[None], kc, vc, [ids], [777], 0.125)[0]
        assert max_err(got, want) <= TOL
        assert torch.count_nonzero(_decode_counters(cuda_device)).item() == 0
