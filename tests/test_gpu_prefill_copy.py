"""The HIP prefill block copy leaves the pool exactly as the reference's pad + index_copy_ does."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from engine.kernels.paged_attention_integration import paged_prefill_copy
from oracle.paged_attention_oracle import prefill_copy_reference

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.cpu().contiguous().view(torch.int16).numpy()


@pytest.mark.parametrize("hkv,d,bs,prompt,skip", [(2, 64, 16, 67, 0), (2, 64, 16, 64, 1),
                                                  (4, 128, 16, 5, 0), (3, 40, 8, 45, 2),
                                                  (2, 64, 16, 300, 3)])
def test_prefill_copy_matches_reference(cuda_device, hkv, d, bs, prompt, skip):
    g = torch.Generator().manual_seed(prompt * 7 + skip)
    nb_total = (prompt + bs - 1) // bs
    pool_blocks = nb_total * 3 + 2
    ids = torch.randperm(pool_blocks, generator=g)[:nb_total].tolist()
    pk = torch.randn(pool_blocks, bs, hkv, d, generator=g).half()
    pv = torch.randn(pool_blocks, bs, hkv, d, generator=g).half()
    # The prefill cache layout [1, Hkv, T, D] and the reference's permuted slice.
    keys = torch.randn(1, hkv, prompt, d, generator=g).half()
    values = torch.randn(1, hkv, prompt, d, generator=g).half()
    start = skip * bs
    ks = keys[0, :, start:prompt, :].permute(1, 0, 2)
    vs = values[0, :, start:prompt, :].permute(1, 0, 2)
    kd, vd = pk.to(cuda_device), pv.to(cuda_device)
    paged_prefill_copy(keys.to(cuda_device)[0, :, start:prompt, :].permute(1, 0, 2),
                       values.to(cuda_device)[0, :, start:prompt, :].permute(1, 0, 2), kd, vd,
                       torch.tensor(ids[skip:], dtype=torch.int32, device=cuda_device), prompt - start)
    rk, rv = pk.clone(), pv.clone()
    prefill_copy_reference(ks, vs, rk, rv, ids[skip:], prompt - start)
    assert np.array_equal(_bits(kd), _bits(rk)) and np.array_equal(_bits(vd), _bits(rv))


def test_fp32_source_is_cast_like_the_reference(cuda_device):
    g = torch.Generator().manual_seed(3)
    pk = torch.zeros(6, 16, 2, 64, dtype=torch.float16)
    pv = torch.zeros_like(pk)
    ks = torch.randn(20, 2, 64, generator=g)
    vs = torch.randn(20, 2, 64, generator=g)
    kd, vd = pk.to(cuda_device), pv.to(cuda_device)
    paged_prefill_copy(ks.to(cuda_device), vs.to(cuda_device), kd, vd,
                       torch.tensor([4, 1], dtype=torch.int32, device=cuda_device), 20)
    prefill_copy_reference(ks, vs, pk, pv, [4, 1], 20)
    assert np.array_equal(_bits(kd), _bits(pk)) and np.array_equal(_bits(vd), _bits(pv))


class FakePrefillModel:
    """Deterministic K/V = (position, position + 1); V = K + 100 (the reference's fixture model,
    tests/test_paged_attention_prefix_cache.py:10-57, here on the GPU in fp16)."""

    def __init__(self, device):
        self.config = SimpleNamespace(num_hidden_layers=1, num_key_value_heads=1, head_dim=64,
                                      hidden_size=64, num_attention_heads=1)
        self.device = device
        self.calls = []

    def __call__(self, input_ids, use_cache, attention_mask=None, position_ids=None,
                 past_key_values=None, logits_to_keep=0):
        self.calls.append({"input_ids": input_ids.clone(), "position_ids": position_ids,
                           "past_key_values": past_key_values, "logits_to_keep": logits_to_keep,
                           "attention_mask": attention_mask,
                           "inference_mode": torch.is_inference_mode_enabled()})
        n = input_ids.shape[1]
        pos = (position_ids[0] if position_ids is not None
               else torch.arange(n, device=input_ids.device)).float()
        key = torch.zeros(1, 1, n, 64, device=input_ids.device)
        key[0, 0, :, 0] = pos
        key[0, 0, :, 1] = pos + 1
        key = key.half()
        value = key + 100
        logits = torch.zeros((1, n, 5), dtype=torch.float32, device=input_ids.device)
        logits[:, :, 3] = 1
        if logits_to_keep:
            logits = logits[:, -logits_to_keep:, :]
        layer = SimpleNamespace(keys=key, values=value)
        if past_key_values is not None:
            lay = past_key_values.layers[0]
            lay.keys = torch.cat((lay.keys, key), dim=2)
            lay.values = torch.cat((lay.values, value), dim=2)
            return SimpleNamespace(logits=logits, past_key_values=past_key_values)
        return SimpleNamespace(logits=logits, past_key_values=SimpleNamespace(layers=[layer]))


def _runner(model, mode, device, debug=False):
    """The fixture model has no attention modules to patch, so "full" mode runs the
    reference's own DynamicCache path (paged_prefill=False), which these fixtures pin."""
    from engine.kernels.paged_attention_integration import KernelPagedManualDecode

    return KernelPagedManualDecode(model=model, block_size=2, num_blocks=2, device=str(device),
                                   dtype=torch.float16, prefix_mode=mode, paged_prefill=False,
                                   debug_prefix_cache=debug)


def test_prefill_keeps_hit_blocks_and_copies_only_owned_blocks(cuda_device, caplog):
    """Reference fixture :60-91: block 0 is a cache hit and must not be overwritten; with
    debug_prefix_cache the cached rows are compared with the fresh prefill and the reference's
    log line reports no difference (:91)."""
    import logging

    from engine.memory.block_allocator import BlockTable

    caplog.set_level(logging.INFO, logger="engine.kernels.paged_attention_integration")
    runner = _runner(FakePrefillModel(cuda_device), "share", cuda_device, debug=True)
    for t in runner.pool.k_cache + runner.pool.v_cache:
        t.zero_()
    hit_k = torch.zeros(2, 1, 64, dtype=torch.float16, device=cuda_device)
    hit_k[0, 0, :2] = torch.tensor([0, 1])
    hit_k[1, 0, :2] = torch.tensor([1, 2])
    runner.pool.k_cache[0][0] = hit_k
    runner.pool.v_cache[0][0] = hit_k + 100
    table = BlockTable(seq_id=0, block_size=2, physical_block_ids=[0, 1], num_tokens=4)
    seq = SimpleNamespace(prompt_token_ids=[10, 11, 12, 13], block_table=table, num_cached_tokens=2,
                          last_logits=None, last_logit_margin=None)
    assert runner.prefill(seq) == 3
    assert torch.equal(runner.pool.k_cache[0][0], hit_k)
    assert torch.equal(runner.pool.v_cache[0][0], hit_k + 100)
    k1 = runner.pool.k_cache[0][1].float().cpu()
    assert k1[:, 0, :2].tolist() == [[2, 3], [3, 4]]
    assert runner.pool.v_cache[0][1].float().cpu()[:, 0, :2].tolist() == [[102, 103], [103, 104]]
    assert seq.last_logit_margin == 1.0
    assert "layer=0 max_abs_difference=0 (cached_tokens=2)" in caplog.text


def test_debug_prefix_cache_reports_the_largest_difference(cuda_device, caplog):
    """A cached row that differs from the fresh prefill shows up as the logged maximum: the
    reference's per-token loop (integration.py:328-362) restated as one device reduction."""
    import logging

    from engine.memory.block_allocator import BlockTable

    caplog.set_level(logging.INFO, logger="engine.kernels.paged_attention_integration")
    runner = _runner(FakePrefillModel(cuda_device), "share", cuda_device, debug=True)
    for t in runner.pool.k_cache + runner.pool.v_cache:
        t.zero_()
    runner.pool.k_cache[0][0, :, 0, :2] = torch.tensor([[0, 1], [1, 2]], dtype=torch.float16)
    runner.pool.v_cache[0][0, :, 0, :] = 100
    runner.pool.v_cache[0][0, :, 0, :2] = torch.tensor([[100, 101], [101, 102]], dtype=torch.float16)
    runner.pool.k_cache[0][0, 1, 0, 5] = 0.75   # key row of token 1 off by 0.75
    runner.pool.v_cache[0][0, 0, 0, 9] = 100.25  # value row of token 0 off by 0.25
    table = BlockTable(seq_id=0, block_size=2, physical_block_ids=[0, 1], num_tokens=4)
    seq = SimpleNamespace(prompt_token_ids=[10, 11, 12, 13], block_table=table, num_cached_tokens=2,
                          last_logits=None, last_logit_margin=None)
    runner.prefill(seq)
    assert "layer=0 max_abs_difference=0.75 (cached_tokens=2)" in caplog.text


def test_full_prefill_uses_cached_prefix_and_only_forwards_suffix(cuda_device):
    """Reference fixture :94-125: "full" mode forwards only the suffix over the cached prefix."""
    from engine.memory.block_allocator import BlockTable

    model = FakePrefillModel(cuda_device)
    runner = _runner(model, "full", cuda_device)
    for t in runner.pool.k_cache + runner.pool.v_cache:
        t.zero_()
    runner.pool.k_cache[0][0, :, 0, :2] = torch.tensor([[0, 1], [1, 2]], dtype=torch.float16)
    runner.pool.v_cache[0][0, :, 0, :2] = torch.tensor([[100, 101], [101, 102]], dtype=torch.float16)
    table = BlockTable(seq_id=0, block_size=2, physical_block_ids=[0, 1], num_tokens=4)
    seq = SimpleNamespace(prompt_token_ids=[10, 11, 12, 13], block_table=table, num_cached_tokens=2,
                          last_logits=None, last_logit_margin=None)
    assert runner.prefill(seq) == 3
    call = model.calls[0]
    assert call["input_ids"].tolist() == [[12, 13]]
    assert call["position_ids"].tolist() == [[2, 3]]
    assert call["past_key_values"].layers[0].keys.shape == (1, 1, 4, 64)
    assert call["logits_to_keep"] == 1 and call["inference_mode"]
    assert runner.pool.k_cache[0][1].float().cpu()[:, 0, :2].tolist() == [[2, 3], [3, 4]]
    assert runner.pool.v_cache[0][1].float().cpu()[:, 0, :2].tolist() == [[102, 103], [103, 104]]


def test_full_prefill_with_zero_hit_uses_normal_full_prompt_path(cuda_device):
    """Reference fixture :129-151: no cached tokens in "full" mode forwards the whole prompt."""
    from engine.memory.block_allocator import BlockTable

    model = FakePrefillModel(cuda_device)
    runner = _runner(model, "full", cuda_device)
    table = BlockTable(seq_id=0, block_size=2, physical_block_ids=[0, 1], num_tokens=3)
    seq = SimpleNamespace(prompt_token_ids=[10, 11, 12], block_table=table, num_cached_tokens=0,
                          last_logits=None, last_logit_margin=None)
    runner.prefill(seq)
    assert model.calls[0]["input_ids"].tolist() == [[10, 11, 12]]
    assert model.calls[0]["past_key_values"] is None
    assert model.calls[0]["inference_mode"]


def test_full_prefill_handles_cached_prefix_and_single_remaining_token(cuda_device):
    """Reference fixture :154-182: one block cached, one prompt token left to forward."""
    from engine.memory.block_allocator import BlockTable

    model = FakePrefillModel(cuda_device)
    runner = _runner(model, "full", cuda_device)
    table = BlockTable(seq_id=0, block_size=2, physical_block_ids=[0, 1], num_tokens=3)
    runner.pool.k_cache[0][0, :, 0, :2] = torch.tensor([[0, 1], [1, 2]], dtype=torch.float16)
    runner.pool.v_cache[0][0, :, 0, :2] = torch.tensor([[100, 101], [101, 102]], dtype=torch.float16)
    seq = SimpleNamespace(prompt_token_ids=[10, 11, 12], block_table=table, num_cached_tokens=2,
                          last_logits=None, last_logit_margin=None)
    runner.prefill(seq)
    call = model.calls[0]
    assert call["input_ids"].tolist() == [[12]]
    assert call["position_ids"].tolist() == [[2]]
    assert torch.equal(call["attention_mask"].cpu(), torch.ones((1, 3), dtype=torch.long))
    assert call["past_key_values"].get_seq_length() == 3
    assert call["inference_mode"]
