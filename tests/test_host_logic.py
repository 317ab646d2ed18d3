"""Host-side logic of the wrappers (no GPU): table padding and the reference's asserts."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from engine.kernels.paged_attention import (
    paged_attention_decode,
    paged_attention_decode_batched,
    paged_attention_decode_v1,
    paged_attention_decode_v2,
    pad_block_tables,
)
from engine.kernels.paged_attention_integration import PagedAttentionContext, paged_kv_write
from oracle.paged_attention_oracle import pad_block_tables_reference


def test_pad_block_tables_matches_spec():
    tables = [[3, 1, 4], [], [1, 5], SimpleNamespace(physical_block_ids=[9, 2, 6, 5])]
    got = pad_block_tables(tables, device="cpu")
    assert got.dtype == torch.int32 and got.shape == (4, 4)
    np.testing.assert_array_equal(got.numpy(), pad_block_tables_reference(tables))
    np.testing.assert_array_equal(got.numpy(), [[3, 1, 4, 0], [0, 0, 0, 0], [1, 5, 0, 0], [9, 2, 6, 5]])


def test_pad_block_tables_edge_cases():
    assert pad_block_tables([], device="cpu").shape == (0, 0)
    assert pad_block_tables([[], []], device="cpu").shape == (2, 1)  # at least one column
    assert pad_block_tables([(7, 8)], device="cpu").tolist() == [[7, 8]]
    with pytest.raises(TypeError):
        pad_block_tables([{1, 2}], device="cpu")


def _cpu_inputs():
    q = torch.zeros(2, 14, 64, dtype=torch.float16)
    k = torch.zeros(8, 16, 2, 64, dtype=torch.float16)
    bt = torch.zeros(2, 4, dtype=torch.int32)
    lens = torch.tensor([5, 9], dtype=torch.int32)
    return q, k, bt, lens


def test_wrappers_assert_like_the_reference():
    q, k, bt, lens = _cpu_inputs()
    with pytest.raises(AssertionError):
        paged_attention_decode_batched(q, k, k, bt, lens, 0.125)  # CPU tensors
    with pytest.raises(AssertionError):
        paged_attention_decode_v1(q[0], k, k, bt[0], 5, 0.125)
    with pytest.raises(AssertionError):
        paged_attention_decode_v2(q[0], k, k, bt[0], 5, 0.125)
    with pytest.raises(AssertionError):
        paged_attention_decode(q, k, k, [[0], [1]], [5, 9], 0.125)
    with pytest.raises(AssertionError):
        paged_kv_write(q[:, :2], q[:, :2], k, k, bt, lens)


def test_context_builds_padded_tables_and_lengths():
    pool = SimpleNamespace(device=torch.device("cpu"), k_cache=[], v_cache=[])
    ctx = PagedAttentionContext(pool, [[4, 2], SimpleNamespace(physical_block_ids=[7])], [20, 3])
    assert ctx.is_batched
    assert ctx.padded_block_tables.tolist() == [[4, 2], [7, 0]]
    assert ctx.seq_lens_tensor.dtype == torch.int32 and ctx.seq_lens_tensor.tolist() == [20, 3]
    single = PagedAttentionContext(pool, SimpleNamespace(physical_block_ids=[5, 6]), 17)
    assert not single.is_batched and single.single_seq_len == 17
    assert single.block_table_tensor.tolist() == [5, 6]


def _cpu_runner():
    from engine.kernels.paged_attention_integration import KernelPagedManualDecode

    model = SimpleNamespace(config=SimpleNamespace(num_hidden_layers=1, num_key_value_heads=2,
                                                   head_dim=64, hidden_size=128,
                                                   num_attention_heads=2))
    return KernelPagedManualDecode(model, block_size=16, num_blocks=4, device="cpu")


def test_runner_refuses_writes_without_a_block_or_into_shared_blocks():
    """Host-side guards of decode_step (reference integration.py:580-592) run before any kernel."""
    from engine.memory.block_allocator import BlockTable

    runner = _cpu_runner()
    full = BlockTable(0, 16, [runner.allocator.allocate()], 16)  # block full, no next block
    with pytest.raises(AssertionError, match="no allocated block"):
        with torch.inference_mode():
            runner.decode_step([SimpleNamespace(seq_id=0, block_table=full, last_token_id=1)])
    b = runner.allocator.allocate()
    runner.allocator.fork(b)
    shared = BlockTable(1, 16, [b], 3)
    with pytest.raises(AssertionError, match="shared block"):
        with torch.inference_mode():
            runner.decode_step([SimpleNamespace(seq_id=1, block_table=shared, last_token_id=1)])
    assert shared.num_tokens == 3  # nothing was bumped
    with pytest.raises(ValueError):
        runner.prefill(SimpleNamespace(prompt_token_ids=None, prompt=None, block_table=shared))


def test_free_list_allocator_counts_references():
    from engine.memory.block_allocator import BlockTable, BlockAllocator

    a = BlockAllocator(3)
    ids = [a.allocate() for _ in range(3)]
    assert not a.can_allocate(1)
    with pytest.raises(MemoryError):
        a.allocate()
    a.fork(ids[0])
    t = BlockTable(0, 16, list(ids), 40)
    assert t.num_blocks_needed_for(40) == 3 and t.last_block_has_space()
    t.free(a)
    assert a.num_free_blocks == 2 and a.ref_counts == {ids[0]: 1}
    with pytest.raises(ValueError):
        a.free(ids[1])


def test_launch_tensors_must_share_one_device():
    """The kernels take raw device pointers: mixing devices is refused before any launch."""
    from engine.kernels import _native

    a, b = torch.zeros(2), torch.zeros(2, device="meta")
    _native.same_device(a, torch.ones(3))
    with pytest.raises(AssertionError, match="same device"):
        _native.same_device(a, b)


def test_workspace_is_never_allocated_during_graph_capture(monkeypatch):
    """A scratch buffer missing or too small while a graph is capturing raises instead of
    allocating (a fill recorded into the graph, memory from the capture's pool); one that is
    already large enough is handed out; a grown buffer keeps the old one alive."""
    from engine.kernels import _native

    dev = torch.device("cpu")  # the allocation itself never happens below
    key = (dev.index, 0x1234, _native.WS_DECODE)
    monkeypatch.setattr(_native, "_workspaces", {})
    monkeypatch.setattr(_native, "_retired", [])
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(_native.CaptureAllocationError, match="capturing"):
        _native.workspace(4096, dev, 0x1234)
    assert key not in _native._workspaces
    held = torch.zeros(8192, dtype=torch.uint8)
    _native._workspaces[key] = held
    assert _native.workspace(4096, dev, 0x1234) == held.data_ptr()
    with pytest.raises(_native.CaptureAllocationError):
        _native.workspace(16384, dev, 0x1234)
    assert _native._workspaces[key] is held
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    addr = _native.workspace(16384, dev, 0x1234)
    assert addr != held.data_ptr() and _native._retired == [held]
    assert _native._workspaces[key].numel() >= 1 << 20 and _native._workspaces[key].sum() == 0
    assert _native.workspace(0, dev, 0x1234) is None


def test_fused_layers_patch_only_when_asked():
    """Decode contexts bind the fused decoder layer (and the one-launch norm) on prepared
    layers only with fuse_layers; without it, and for prefill contexts, transformers' layer
    forwards stay; attention modules are always patched, and everything is restored."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from engine.kernels.paged_attention_integration import (
        patch_paged_attention, prepare_fused_layers)

    torch.manual_seed(0)
    model = Qwen2ForCausalLM(Qwen2Config(vocab_size=64, hidden_size=32, intermediate_size=64,
                                         num_hidden_layers=2, num_attention_heads=4,
                                         num_key_value_heads=2)).half()
    assert prepare_fused_layers(model) == 2
    layer = model.model.layers[0]
    decode = SimpleNamespace(is_decode=True)
    prefill = SimpleNamespace(is_decode=False, is_prefill=True)
    for ctx, fuse, fused in ((decode, True, True), (decode, False, False), (prefill, True, False)):
        with patch_paged_attention(model, ctx, fuse_layers=fuse):
            assert ("forward" in vars(layer)) == fused
            assert ("forward" in vars(layer.input_layernorm)) == fused
            assert "forward" in vars(layer.self_attn)
        assert "forward" not in vars(layer) and "forward" not in vars(layer.self_attn)
