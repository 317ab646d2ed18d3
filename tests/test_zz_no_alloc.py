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


def _noalloc(w):
    lib = _native.load()
    out = torch.empty_like(w.q)
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
