"""The "full" prefix-cache prefill through the paged prefill kernel matches the reference path.

The reference's "full" mode (engine/kernels/paged_attention_integration.py:459-482)
copies the cached prefix blocks of every layer into a DynamicCache (:364-392)
and forwards the prompt suffix through transformers' attention, then copies
the suffix's K/V into the sequence's blocks. The runner here (paged_prefill,
the default) forwards the suffix with the paged prefill kernel reading the
prefix from the pool. Both run on the same random-init Qwen2 model and pool;
gates: last-position logits within 0.1 of the reference path's and of a plain
forward over the whole prompt (the per-step logits tolerance of the reference's
own tests, tests/test_kernel_qwen_integration.py:72-123), the same greedy token
unless the top-1/top-2 margin is below 0.05, layer-0 K/V rows bit-identical,
deeper layers' rows within 0.05, and the cached prefix blocks untouched.
"""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

pytestmark = pytest.mark.gpu

QWEN_HEADS = dict(vocab_size=512, hidden_size=896, intermediate_size=1024, num_hidden_layers=3,
                  num_attention_heads=14, num_key_value_heads=2, max_position_embeddings=4096,
                  rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=False)
SMALL = dict(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
             num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
             rope_theta=1e6, tie_word_embeddings=False)
LOGIT_TOL = 0.1
NEAR_TIE = 0.05
KV_TOL = 0.05


def make_model(kw, seed, device):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(seed)
    with torch.device(device):
        model = Qwen2ForCausalLM(Qwen2Config(**kw))
    return model.half().eval()


def make_runner(model, device, paged_prefill):
    from engine.kernels.paged_attention_integration import KernelPagedManualDecode

    return KernelPagedManualDecode(model=model, block_size=16, num_blocks=64, device=str(device),
                                   dtype=torch.float16, prefix_mode="full",
                                   paged_prefill=paged_prefill, use_graphs=False)


def seq(seq_id, tokens, ids, cached):
    from engine.memory.block_allocator import BlockTable

    bt = BlockTable(seq_id=seq_id, block_size=16, physical_block_ids=list(ids),
                    num_tokens=len(tokens))
    return SimpleNamespace(seq_id=seq_id, prompt_token_ids=list(tokens), block_table=bt,
                           num_cached_tokens=cached, last_logits=None, last_logit_margin=None)


def run_pair(runner, prompt_a, prompt_b, shared_blocks):
    """Prefill A (no cache), then B whose first shared_blocks blocks are A's."""
    alloc = runner.allocator
    nb_a = (len(prompt_a) + 15) // 16
    nb_b = (len(prompt_b) + 15) // 16
    ids_a = [alloc.allocate() for _ in range(nb_a)]
    a = seq(0, prompt_a, ids_a, 0)
    runner.prefill(a)
    ids_b = ([alloc.fork(i) for i in ids_a[:shared_blocks]]
             + [alloc.allocate() for _ in range(nb_b - shared_blocks)])
    b = seq(1, prompt_b, ids_b, shared_blocks * 16)
    shared = ids_a[:shared_blocks]
    prefix_before = [(k[shared].clone(), v[shared].clone())
                     for k, v in zip(runner.pool.k_cache, runner.pool.v_cache)]
    tok = runner.prefill(b)
    return tok, b, ids_b, prefix_before


@pytest.mark.parametrize("cfg,cached_blocks,suffix", [
    (QWEN_HEADS, 3, 37),   # head_dim 64, g = 7 (Qwen2.5-0.5B heads)
    (QWEN_HEADS, 1, 150),
    (SMALL, 2, 16),        # head_dim 32, g = 2; the suffix fills whole blocks
    (QWEN_HEADS, 2, 1),    # a single remaining prompt token after the cached blocks
])
def test_full_mode_paged_prefill_matches_reference_path(cuda_device, cfg, cached_blocks, suffix):
    model = make_model(cfg, 7, cuda_device)
    g = torch.Generator().manual_seed(cached_blocks * 100 + suffix)
    prompt_a = torch.randint(0, cfg["vocab_size"], (cached_blocks * 16 + 21,), generator=g).tolist()
    prompt_b = prompt_a[:cached_blocks * 16] + torch.randint(
        0, cfg["vocab_size"], (suffix,), generator=g).tolist()

    fast = make_runner(model, cuda_device, paged_prefill=True)
    ref = make_runner(model, cuda_device, paged_prefill=False)
    tok_f, b_f, ids_b, prefix_before = run_pair(fast, prompt_a, prompt_b, cached_blocks)
    tok_r, b_r, _, _ = run_pair(ref, prompt_a, prompt_b, cached_blocks)

    with torch.inference_mode():
        whole = model(input_ids=torch.tensor([prompt_b], device=cuda_device)).logits[0, -1].float()
    lf, lr = b_f.last_logits.float(), b_r.last_logits.float()
    err_ref = (lf - lr).abs().max().item()
    err_whole = (lf - whole).abs().max().item()
    print(f"[prefix-prefill] cached={cached_blocks * 16} suffix={suffix} "
          f"logit err vs reference path {err_ref:.3e}, vs whole-prompt forward {err_whole:.3e}",
          flush=True)
    assert err_ref <= LOGIT_TOL and err_whole <= LOGIT_TOL
    if b_r.last_logit_margin >= NEAR_TIE:
        assert tok_f == tok_r

    new_ids = ids_b[cached_blocks:]
    for layer in range(cfg["num_hidden_layers"]):
        kf, vf = fast.pool.k_cache[layer][new_ids], fast.pool.v_cache[layer][new_ids]
        kr, vr = ref.pool.k_cache[layer][new_ids], ref.pool.v_cache[layer][new_ids]
        if layer == 0:
            assert torch.equal(kf, kr) and torch.equal(vf, vr)
        else:
            assert (kf.float() - kr.float()).abs().max().item() <= KV_TOL
            assert (vf.float() - vr.float()).abs().max().item() <= KV_TOL
        pk, pv = prefix_before[layer]
        assert torch.equal(fast.pool.k_cache[layer][ids_b[:cached_blocks]], pk)
        assert torch.equal(fast.pool.v_cache[layer][ids_b[:cached_blocks]], pv)


def test_decode_after_paged_prefix_prefill(cuda_device):
    """Greedy decode steps continue from the paged prefill's pool contents like the reference's."""
    model = make_model(QWEN_HEADS, 11, cuda_device)
    g = torch.Generator().manual_seed(5)
    prompt_a = torch.randint(0, 512, (70,), generator=g).tolist()
    prompt_b = prompt_a[:64] + torch.randint(0, 512, (9,), generator=g).tolist()
    streams = []
    for paged in (True, False):
        runner = make_runner(model, cuda_device, paged_prefill=paged)
        tok, b, _, _ = run_pair(runner, prompt_a, prompt_b, 4)
        b.last_token_id = tok
        b.generated_ids = [tok]
        toks, margins = [tok], []
        for _ in range(6):
            if b.block_table.num_tokens % 16 == 0:
                b.block_table.physical_block_ids.append(runner.allocator.allocate())
            nxt = runner.decode_step([b])[0]
            b.last_token_id = nxt
            toks.append(nxt)
            margins.append(b.last_logit_margin)
        streams.append((toks, margins))
    (tf, _), (tr, mr) = streams
    for i, (x, y) in enumerate(zip(tf, tr)):
        if x != y:
            assert i > 0 and mr[i - 1] < NEAR_TIE, f"streams diverge at step {i}: {tf} vs {tr}"
            break
