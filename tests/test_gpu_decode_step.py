"""Decode steps through the paged HIP path match the model's own contiguous-cache path.

The oracle is the same random-init Qwen2 model run by transformers with its
DynamicCache (no paging, no HIP kernels). Gates, as stated for this path:
greedy streams equal except where the oracle's top-1/top-2 logit margin is
below 0.05 (an fp16 near-tie), and -- with the oracle's tokens fed to both
paths (teacher forcing) -- per-step logits within 0.1 of the oracle's
(the reference's own per-step logits tolerance, tests/test_kernel_qwen_integration.py:72-123).
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TINY = dict(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
            rope_theta=1e6, tie_word_embeddings=False)
QWEN05 = dict(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_hidden_layers=24,
              num_attention_heads=14, num_key_value_heads=2, max_position_embeddings=32768,
              rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=False)
NEAR_TIE = 0.05
LOGIT_TOL = 0.1


def make_model(kw, seed, device):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(seed)
    cfg = Qwen2Config(**kw)
    with torch.device(device):
        model = Qwen2ForCausalLM(cfg)
    return model.half().eval()


@torch.inference_mode()
def oracle_greedy(model, prompt, steps, forced=None):
    """Contiguous-cache greedy decode: tokens, logits [steps, vocab] (fp32, cpu), margins."""
    dev = next(model.parameters()).device
    out = model(input_ids=torch.tensor([prompt], device=dev), use_cache=True)
    pkv = out.past_key_values
    toks, logits_all, margins = [], [], []
    logits = out.logits[0, -1].float()
    for i in range(steps):
        top2 = torch.topk(logits, 2).values
        margins.append(float(top2[0] - top2[1]))
        logits_all.append(logits.cpu())
        tok = int(torch.argmax(logits)) if forced is None else forced[i]
        toks.append(int(torch.argmax(logits)))
        if i + 1 == steps:
            break
        out = model(input_ids=torch.tensor([[tok]], device=dev), past_key_values=pkv, use_cache=True)
        pkv = out.past_key_values
        logits = out.logits[0, -1].float()
    return toks, torch.stack(logits_all), margins


@torch.inference_mode()
def paged_greedy(runner, prompts, steps, forced=None):
    """Prefill each prompt, then batched decode steps; optional forced input tokens per sequence."""
    from engine.memory.block_pool import BlockTable

    bs = runner.block_size
    alloc = runner.allocator
    seqs = []
    for i, p in enumerate(prompts):
        bt = BlockTable(seq_id=i, block_size=bs)
        bt.physical_block_ids = [alloc.allocate() for _ in range((len(p) + bs - 1) // bs)]
        bt.num_tokens = len(p)
        seq = SimpleNamespace(seq_id=i, prompt_token_ids=list(p), block_table=bt, num_cached_tokens=0,
                              last_token_id=None, generated_ids=[], last_logits=None,
                              last_logit_margin=None)
        first = runner.prefill(seq)
        seq.generated_ids.append(first)
        seq.last_token_id = first if forced is None else forced[i][0]
        seqs.append(seq)
    logits = [[s.last_logits.float().cpu()] for s in seqs]
    for step in range(1, steps):
        for s in seqs:  # the scheduler's job: a new block at each block boundary
            if s.block_table.num_tokens // bs >= len(s.block_table.physical_block_ids):
                s.block_table.physical_block_ids.append(alloc.allocate())
        toks = runner.decode_step(seqs)
        for i, (s, t) in enumerate(zip(seqs, toks)):
            s.generated_ids.append(t)
            s.last_token_id = t if forced is None else forced[i][step]
            logits[i].append(s.last_logits.float().cpu())
    return [s.generated_ids for s in seqs], [torch.stack(l) for l in logits]


def _runner(model, device, need, bs, interleave):
    from engine.kernels.paged_attention_integration import KernelPagedManualDecode

    runner = KernelPagedManualDecode(model, block_size=bs, num_blocks=2 * need + 8, device=str(device))
    if interleave:
        # Every real block is followed by one taken for "another sequence", so a sequence's
        # physical blocks are never adjacent (reference tests/test_paged_manual_decode.py:114-174).
        take = runner.allocator.allocate

        def allocate():
            b = take()
            take()
            return b

        runner.allocator.allocate = allocate
    return runner


def _check(model, prompts, steps, device, bs=16, interleave=False):
    need = sum((len(p) + steps + bs - 1) // bs + 1 for p in prompts)
    runner = _runner(model, device, need, bs, interleave)
    toks, _ = paged_greedy(runner, prompts, steps)
    divergences = 0
    ref_tokens = []
    for p, got in zip(prompts, toks):
        want, _, margins = oracle_greedy(model, p, steps)
        ref_tokens.append(want)
        for i, (a, b) in enumerate(zip(got, want)):
            if a != b:
                divergences += 1
                assert margins[i] < NEAR_TIE, (f"stream diverged at step {i} with oracle margin "
                                               f"{margins[i]:.4f} >= {NEAR_TIE}")
                break
    # Teacher forcing: both paths consume the oracle's tokens; compare logits per step.
    runner2 = _runner(model, device, need, bs, interleave)
    _, paged_logits = paged_greedy(runner2, prompts, steps, forced=ref_tokens)
    worst = 0.0
    for p, want, got in zip(prompts, ref_tokens, paged_logits):
        _, ref_logits, _ = oracle_greedy(model, p, steps, forced=want)
        worst = max(worst, (got - ref_logits).abs().max().item())
    print(f"[decode-step] {len(prompts)} seqs x {steps} steps, block {bs}"
          f"{' interleaved' if interleave else ''}: {divergences} near-tie divergences, "
          f"teacher-forced max |logit diff| {worst:.4f}", flush=True)
    assert worst <= LOGIT_TOL
    return divergences


def test_tiny_model_greedy_and_teacher_forced(cuda_device):
    model = make_model(TINY, 0, cuda_device)
    rng = np.random.default_rng(1)
    prompts = [rng.integers(0, 512, size=n).tolist() for n in (1, 5, 16, 17, 40, 100)]
    _check(model, prompts, 40, cuda_device)


@pytest.mark.parametrize("bs,interleave", [(4, False), (4, True), (8, True)])
def test_small_blocks_and_interleaved_allocation(cuda_device, bs, interleave):
    """Reference tests/test_paged_manual_decode.py:78-174: with block size 4 a short prompt and its
    generation span many blocks (every layer crosses block boundaries), and physical blocks
    interleaved with another sequence's allocations are gathered through the table."""
    model = make_model(TINY, 6, cuda_device)
    rng = np.random.default_rng(6)
    prompts = [rng.integers(0, 512, size=n).tolist() for n in (5, 9, 23)]
    _check(model, prompts, 16, cuda_device, bs=bs, interleave=interleave)


def test_qwen05_architecture_greedy_and_teacher_forced(cuda_device):
    """Qwen2.5-0.5B shape, random init: 24 layers, 14/2 heads, head_dim 64."""
    model = make_model(QWEN05, 0, cuda_device)
    rng = np.random.default_rng(2)
    prompts = [rng.integers(0, 151936, size=int(n)).tolist() for n in rng.integers(64, 1025, size=6)]
    _check(model, prompts, 16, cuda_device)


def test_single_sequence_generate_matches_batched_path(cuda_device):
    from engine.kernels.paged_attention_integration import KernelPagedManualDecode

    model = make_model(TINY, 3, cuda_device)
    prompt = np.random.default_rng(3).integers(0, 512, size=37).tolist()
    runner = KernelPagedManualDecode(model, block_size=16, num_blocks=64, device=str(cuda_device))
    got = runner.generate(prompt, max_new_tokens=20)
    want, _, margins = oracle_greedy(model, prompt, 20)
    for i, (a, b) in enumerate(zip(got, want)):
        if a != b:
            assert margins[i] < NEAR_TIE
            break


def test_shared_write_block_is_refused(cuda_device):
    """A decode write into a block with ref_count > 1 raises (reference integration.py:587-592)."""
    from engine.kernels.paged_attention_integration import KernelPagedManualDecode
    from engine.memory.block_pool import BlockTable

    model = make_model(TINY, 4, cuda_device)
    runner = KernelPagedManualDecode(model, block_size=16, num_blocks=8, device=str(cuda_device))
    b = runner.allocator.allocate()
    runner.allocator.fork(b)
    seq = SimpleNamespace(seq_id=0, block_table=BlockTable(0, 16, [b], 5), last_token_id=1)
    with pytest.raises(AssertionError, match="shared block"):
        runner.decode_step([seq])


def test_graph_replays_match_eager_steps(cuda_device):
    """Graphed decode steps (the default) against eager steps of the same model, step by step.

    Two runners with identical pools decode the same prompts, one replaying
    captured graphs and one eager, interleaved so that eager work and host
    synchronisations sit between the replays; block boundaries are crossed and
    the batch is reordered midway (its tables are then rewritten). Every
    step's tokens must agree and its logits be within fp16 accumulation noise.
    """
    from engine.kernels.paged_attention_integration import KernelPagedManualDecode
    from engine.memory.block_pool import BlockTable

    model = make_model(TINY, 5, cuda_device)
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, 512, size=n).tolist() for n in (3, 15, 16, 31, 33, 70)]
    bs, steps = 16, 24
    runners = [KernelPagedManualDecode(model, block_size=bs, num_blocks=128, device=str(cuda_device),
                                       use_graphs=g) for g in (True, False)]
    batches = []
    for runner in runners:
        seqs = []
        for i, p in enumerate(prompts):
            bt = BlockTable(i, bs, [runner.allocator.allocate() for _ in range((len(p) + bs - 1) // bs)],
                            len(p))
            seq = SimpleNamespace(seq_id=i, prompt_token_ids=list(p), block_table=bt,
                                  num_cached_tokens=0, last_token_id=None, last_logits=None,
                                  last_logit_margin=None)
            seq.last_token_id = runner.prefill(seq)
            seqs.append(seq)
        batches.append(seqs)
    worst = 0.0
    for step in range(steps):
        if step == steps // 2:  # reorder the batch: every table row changes
            batches = [list(reversed(b)) for b in batches]
        outs = []
        for runner, seqs in zip(runners, batches):
            for s in seqs:
                if s.block_table.num_tokens // bs >= len(s.block_table.physical_block_ids):
                    s.block_table.physical_block_ids.append(runner.allocator.allocate())
            toks = runner.decode_step(seqs)
            torch.cuda.synchronize()
            outs.append((toks, torch.stack([s.last_logits.float() for s in seqs])))
            for s, t in zip(seqs, toks):
                s.last_token_id = t
        (tg, lg), (te, le) = outs
        assert tg == te, f"step {step}: graphed tokens {tg} != eager tokens {te}"
        worst = max(worst, (lg - le).abs().max().item())
    print(f"[graph] {len(prompts)} seqs x {steps} steps: max |graph - eager logits| {worst:.2e}",
          flush=True)
    assert worst <= 1e-2
    assert len(runners[0]._graphs) >= 1
