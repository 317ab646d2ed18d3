"""pa_decode_batched_noalloc_f16, the entry point that allocates nothing, against
pa_decode_batched_f16 on the same inputs (needs an MI355X).

Both run the same kernels with the same schedule; only where the split-K
scratch lives differs (the library's static array instead of a workspace), so
the outputs must be the same bits. Two calls in a row, the second smaller than
the first: the array keeps the first call's contents, and the second must not
depend on them.
"""
from __future__ import annotations

import pytest
import torch

from engine import workloads
from engine.kernels import _native
from engine.kernels.paged_attention import paged_attention_decode_batched

pytestmark = pytest.mark.gpu


def _noalloc(w, out=None):
    lib = _native.load()
    out = torch.empty_like(w.q) if out is None else out
    nb, bs, hkv, d = w.k_cache.shape
    dev = w.q.device
    status = lib.pa_decode_batched_noalloc_f16(
        w.q.data_ptr(), _native.strides_of(w.q), w.k_cache.data_ptr(), _native.strides_of(w.k_cache),
        w.v_cache.data_ptr(), _native.strides_of(w.v_cache), w.block_tables.data_ptr(),
        _native.strides_of(w.block_tables), w.seq_lens.data_ptr(), out.data_ptr(),
        _native.strides_of(out), w.num_seqs, w.q.shape[1], hkv, d, bs, nb,
        w.block_tables.shape[1], float(w.scale), _native.stream_handle(dev))
    _native.check(status, "pa_decode_batched_noalloc_f16")
    return out


def _with_workspace(w):
    return paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables, w.seq_lens,
                                          w.scale)


def test_noalloc_matches_workspace_entry_on_two_calls(cuda_device):
    # First call: 64 long sequences sharing prefix groups -- stream-K ranges that cut pairs,
    # so partial records and merge counters in the static array are used. Second call, smaller:
    # one Qwen2.5-0.5B layer at batch 8 (one workgroup per pair).
    big = workloads.long_context(device=cuda_device, seed=7, num_seqs=64)
    small = workloads.qwen_layer(device=cuda_device, seed=7)
    for name, w in (("long_context B64", big), ("qwen_layer B8", small)):
        print(f"[no-alloc] {name}", flush=True)
        got = _noalloc(w)
        want = _with_workspace(w)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), f"{name}: no-allocation output differs from the workspace entry"
    # The counters the merge uses were left at zero: a repeat of the large call agrees again.
    assert torch.equal(_noalloc(big), _with_workspace(big))


def test_noalloc_refuses_batches_beyond_its_scratch(cuda_device):
    w = workloads.make_random(1100, 14, 2, 64, [5] * 1100, 16, seed=1, device=cuda_device)
    lib = _native.load()
    with pytest.raises(_native.NativeLibraryError, match="no-allocation"):
        _noalloc(w)
    assert b"1024" in lib.pa_last_error()


def test_noalloc_inside_a_captured_graph(cuda_device):
    """The callers the entry point is for include code under HIP graph capture: one eager
    call (which sets up the device's array and clears its counters), then the call captured
    in a graph and replayed, with other eager work and synchronisations between the
    replays; every replay must give the workspace entry's bits."""
    w = workloads.long_context(device=cuda_device, seed=9, num_seqs=64)
    other = workloads.qwen_layer(device=cuda_device, seed=9)
    want = _with_workspace(w)
    out = torch.empty_like(w.q)
    _noalloc(w, out)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    graph = torch.cuda.CUDAGraph()
    # Inside inference mode, as the decode runner captures its steps: an earlier test's
    # inference-mode work may have made torch's generator state an inference tensor, which
    # capture_begin updates in place.
    with torch.inference_mode(), torch.cuda.graph(graph):
        _noalloc(w, out)
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        print(f"[no-alloc] graph replay {i}", flush=True)
        assert torch.equal(out, want), f"replay {i} differs from the workspace entry"
        _with_workspace(other)  # eager work between the replays
        torch.cuda.synchronize()


def _shared_groups(num_seqs, hkv, g, d, shared_blocks, seed, device):
    """num_seqs sequences of 600-1000 tokens in groups of 8 whose first `shared_blocks`
    table entries are the same physical blocks (a prefix cache's shared prompt)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    bs = 16
    lens = rng.integers(600, 1001, size=num_seqs).tolist()
    need = [(n + bs - 1) // bs for n in lens]
    total = sum(need) + 16
    perm = rng.permutation(total).tolist()
    pos, tables = 0, []
    for i, nb in enumerate(need):
        sh = min(shared_blocks, nb - 1) if i % 8 else 0
        row = tables[i - 1][:sh] + perm[pos:pos + nb - sh] if sh else perm[pos:pos + nb]
        pos += nb - sh
        tables.append(row)
    return workloads.from_tables(tables, lens, hkv * g, hkv, d, bs, total, seed, device)


def test_noalloc_without_room_for_prefix_records(cuda_device):
    """Past the size where shared-prefix records fit the static array (here 120 sequences
    of 8 kv heads, head_dim 64), the entry point reads shared prefixes once per sequence:
    its results stay within the attention tolerance of the oracle, while the workspace
    entry (which builds prefix items) may differ from it in the last bits."""
    from oracle.paged_attention_oracle import naive_reference_paged_attention

    w = _shared_groups(120, 8, 7, 64, 24, 13, cuda_device)
    sched = _native.decode_schedule(120, 56, 8, 64, 16, w.block_tables.shape[1])
    assert sched["path"] == "stream_k" and sched["shared_prefixes"], sched
    got = _noalloc(w)
    ref = _with_workspace(w)
    torch.cuda.synchronize()
    want = naive_reference_paged_attention(w.q.cpu(), w.k_cache.cpu(), w.v_cache.cpu(), w.tables,
                                           w.lens, w.scale, compute_dtype=torch.float32)
    err = (got.float().cpu() - want).abs().max().item()
    err_ws = (ref.float().cpu() - want).abs().max().item()
    differ = int((got != ref).sum().item())
    print(f"[no-alloc] prefix records do not fit: max abs err {err:.3e} (workspace entry "
          f"{err_ws:.3e}); {differ} of {got.numel()} values differ in bits", flush=True)
    assert err <= 2e-3 and err_ws <= 2e-3
