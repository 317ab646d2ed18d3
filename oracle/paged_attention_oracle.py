"""CPU oracle for paged decode attention and the per-step K/V write.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or, in
bench.py, as the timed CPU baseline) -- never as a product path. The product
path (vllm-inference-engine_amd/engine) runs HIP kernels only.

Each function restates the reference algorithm from its source, cited by
file:line in the reference repository:

  naive_reference_paged_attention  engine/kernels/paged_attention.py:30-83
  pad_block_tables_reference       engine/kernels/paged_attention.py:473-505
  kv_write_reference               engine/kernels/paged_attention_integration.py:148-161
  kv_write_scatter                 same semantics, vectorised (cross-check of the loop)
  prefill_copy_reference           engine/kernels/paged_attention_integration.py:278-326
  rope_fp16                        transformers apply_rotary_pos_emb (rotate_half form), as the
                                   reference calls it at paged_attention_integration.py:108-109
  prefix_prefill_attention         "full" prefix-cache mode: the uncached prompt suffix
                                   attends causally over the cached blocks plus itself
                                   (engine/kernels/paged_attention_integration.py:459-482,
                                   prefix gathered as :364-392)

Pinning (tests/test_oracle.py): the attention oracle is checked against closed
forms that do not share its code -- contiguous scaled-dot-product attention via
torch.nn.functional.scaled_dot_product_attention on K/V gathered by table,
the repeat_interleave GQA form the reference's own tests use
(tests/test_paged_attention_reference.py:136-158), an fp64 brute force with
explicit loops, and special cases (seq_len 1 returns v_0, identical keys return
the mean of V, a dominant score returns that token's V, block-permutation and
pool-slack invariance). tests/test_oracle_mutants.py plants plausible mistakes
in copies of the oracle and shows each is caught. The K/V write is pinned
bit-exactly by two independent statements (the reference's per-token loop and
a vectorised scatter) and by block-id-encoded patterns. pad_block_tables is
pinned by its specification (int32, zero padded, at least one column). The
prefill copy is pinned by the reference's own exact-content fixture
(tests/test_paged_attention_prefix_cache.py:60-125, restated on the GPU in
tests/test_gpu_prefill_copy.py) besides this restatement. rope_fp16 is pinned
bit for bit against transformers' own apply_rotary_pos_emb (5.15.0, the
version the reference pins in requirements.txt:3) on CPU fp16 tensors, and
by closed forms (position 0 is the identity; a quarter turn maps (x1, x2) to
(-x2, x1)). prefix_prefill_attention is pinned (tests/test_oracle_prefill.py)
against code it does not share: with one new token it equals
naive_reference_paged_attention; its rows equal the last rows of
torch's causal scaled_dot_product_attention (is_causal=True) over the whole
gathered sequence, which fixes the position offset and the mask boundary; an
fp64 brute force with explicit loops agrees on tiny sizes; and planted
mistakes (mask off by one, positions counted from the suffix start, kv head
h % Hkv) each fail one of these.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np
import torch


def naive_reference_paged_attention(
    q: torch.Tensor,              # [num_seqs, num_q_heads, head_dim]
    k_cache: torch.Tensor,        # [num_blocks, block_size, num_kv_heads, head_dim]
    v_cache: torch.Tensor,        # [num_blocks, block_size, num_kv_heads, head_dim]
    block_tables: Sequence[Sequence[int]],
    seq_lens: Sequence[int],
    scale: float,
    compute_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Gather K/V per sequence through its block table and run plain softmax attention.

    Follows engine/kernels/paged_attention.py:30-83: for each sequence take
    min(block_size, remaining) rows of each listed block in order (:58-66),
    concatenate (:68-69), map query head h to kv head h // group (:73-76),
    softmax((q k^T) * scale) v with einsums (:78-80); the output starts as
    zeros_like(q) (:51). Table entries past ceil(L / block_size) are ignored.

    compute_dtype=None evaluates in the inputs' dtype, exactly as the
    reference does (the literal fp16 path for fp16 inputs); torch.float32 or
    torch.float64 evaluates the same algorithm on upcast copies of the
    gathered rows and returns that dtype.
    """
    num_seqs, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[2]
    assert num_q_heads % num_kv_heads == 0, (
        f"num_q_heads ({num_q_heads}) must be divisible by num_kv_heads ({num_kv_heads})")
    group_size = num_q_heads // num_kv_heads
    out_dtype = compute_dtype or q.dtype
    outputs = torch.zeros(q.shape, dtype=out_dtype, device=q.device)
    block_size = k_cache.shape[1]
    kv_head_indices = torch.arange(num_q_heads, device=q.device) // group_size

    for s in range(num_seqs):
        seq_len = int(seq_lens[s])
        k_parts, v_parts = [], []
        remaining = seq_len
        for b in block_tables[s]:
            take = min(block_size, remaining)
            k_parts.append(k_cache[b, :take])
            v_parts.append(v_cache[b, :take])
            remaining -= take
            if remaining <= 0:
                break
        k = torch.cat(k_parts, dim=0)
        v = torch.cat(v_parts, dim=0)
        q_s = q[s]
        if compute_dtype is not None:
            k, v, q_s = k.to(compute_dtype), v.to(compute_dtype), q_s.to(compute_dtype)
        k_expanded = k[:, kv_head_indices, :]
        v_expanded = v[:, kv_head_indices, :]
        scores = torch.einsum("hd,shd->hs", q_s, k_expanded) * scale
        probs = torch.softmax(scores, dim=-1)
        outputs[s] = torch.einsum("hs,shd->hd", probs, v_expanded)
    return outputs


def pad_block_tables_reference(block_tables: Sequence) -> np.ndarray:
    """int32 [num_seqs, max(1, max_len)], zero padded (paged_attention.py:473-505)."""
    if len(block_tables) == 0:
        return np.zeros((0, 0), dtype=np.int32)
    rows = [list(bt.physical_block_ids) if hasattr(bt, "physical_block_ids") else list(bt)
            for bt in block_tables]
    width = max(1, max(len(r) for r in rows))
    out = np.zeros((len(rows), width), dtype=np.int32)
    for i, r in enumerate(rows):
        out[i, :len(r)] = r
    return out


def kv_write_reference(key, value, k_cache, v_cache, block_tables, seq_lens, block_size):
    """Per-sequence index_put loop, as engine/kernels/paged_attention_integration.py:148-161.

    key/value: [num_seqs, num_kv_heads, head_dim]; block_tables: lists of ids;
    seq_lens: ints counting the new token. Mutates k_cache/v_cache in place.
    """
    for b in range(key.shape[0]):
        cur_pos = int(seq_lens[b]) - 1
        phys_id = block_tables[b][cur_pos // block_size]
        offset = cur_pos % block_size
        k_cache[phys_id, offset] = key[b]
        v_cache[phys_id, offset] = value[b]


def kv_write_scatter(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                     block_tables: np.ndarray, seq_lens: np.ndarray) -> None:
    """Same write as kv_write_reference, stated as one vectorised numpy scatter.

    Operates on raw uint16 views so the comparison is on bits. Rows with
    seq_len <= 0 are skipped.
    """
    block_size = k_cache.shape[1]
    lens = np.asarray(seq_lens, dtype=np.int64)
    sel = np.nonzero(lens > 0)[0]
    pos = lens[sel] - 1
    ids = block_tables[sel, pos // block_size]
    k_cache[ids, pos % block_size] = key[sel]
    v_cache[ids, pos % block_size] = value[sel]


def prefill_copy_reference(k_src: torch.Tensor, v_src: torch.Tensor, k_cache: torch.Tensor,
                           v_cache: torch.Tensor, block_ids: Sequence[int], num_tokens: int) -> None:
    """Pad the token rows to whole blocks with zeros and index_copy_ them into the pool.

    As engine/kernels/paged_attention_integration.py:308-326: k_src/v_src are
    [tokens, num_kv_heads, head_dim] (tokens >= num_tokens, only the first
    num_tokens used), cast to the pool dtype, padded (:315-317), viewed as
    blocks (:319-320) and index_copy_'d at block_ids (:322-326).
    """
    bs = k_cache.shape[1]
    nb = len(block_ids)
    pad = nb * bs - num_tokens
    ks, vs = k_src[:num_tokens], v_src[:num_tokens]
    if pad > 0:
        ks = torch.nn.functional.pad(ks, (0, 0, 0, 0, 0, pad))
        vs = torch.nn.functional.pad(vs, (0, 0, 0, 0, 0, pad))
    idx = torch.tensor(list(block_ids), dtype=torch.long)
    k_cache.index_copy_(0, idx, ks.reshape(nb, bs, *ks.shape[1:]).to(k_cache.dtype))
    v_cache.index_copy_(0, idx, vs.reshape(nb, bs, *vs.shape[1:]).to(v_cache.dtype))


def rope_fp16(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotary embedding of fp16 rows as transformers computes it in fp16.

    x [..., D] with cos/sin broadcastable to it, all numpy float16. transformers'
    apply_rotary_pos_emb (the reference's RoPE, paged_attention_integration.py:108-109)
    evaluates (x * cos) + (rotate_half(x) * sin) with rotate_half(x) =
    cat(-x[..., D/2:], x[..., :D/2]), each op rounded to fp16; numpy's float16
    arithmetic rounds each op the same way.
    """
    assert x.dtype == np.float16 and cos.dtype == np.float16 and sin.dtype == np.float16
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return (x * cos) + (rot * sin)


def prefix_prefill_attention(
    q: torch.Tensor,              # [num_tokens, num_q_heads, head_dim], sequences packed in order
    k_cache: torch.Tensor,        # [num_blocks, block_size, num_kv_heads, head_dim]
    v_cache: torch.Tensor,
    block_tables: Sequence[Sequence[int]],
    seq_lens: Sequence[int],      # context length after the new tokens (cached + new)
    query_lens: Sequence[int],    # new tokens per sequence; their rows are consecutive in q
    scale: float,
    compute_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Causal attention of each sequence's new tokens over its whole paged context.

    The reference's "full" prefix-cache mode (paged_attention_integration.py:459-482)
    gathers the cached prefix blocks into a DynamicCache (:364-392) and forwards
    only the prompt suffix with position_ids cached..prompt_len-1 and an all-ones
    attention mask over the prompt; transformers' causal mask then lets the query
    at position p see keys 0..p (the prefix and the suffix up to itself). Here
    the suffix's own K/V are read from the pool like the prefix (they are
    written there before attention), so new token i of a sequence with context
    length L and n new tokens sits at position p = L - n + i and attends to
    pool rows 0..p. Rows are gathered as naive_reference_paged_attention
    gathers them (paged_attention.py:58-69); query head h reads kv head
    h // group (:73-76). Returns compute_dtype.
    """
    num_tokens, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[2]
    assert num_q_heads % num_kv_heads == 0
    group = num_q_heads // num_kv_heads
    bs = k_cache.shape[1]
    out = torch.zeros((num_tokens, num_q_heads, head_dim), dtype=compute_dtype)
    kv_head = torch.arange(num_q_heads) // group
    row = 0
    for s_idx, (L, n) in enumerate(zip(seq_lens, query_lens)):
        L, n = int(L), int(n)
        assert 0 <= n <= L
        if n == 0:
            continue
        nb = (L + bs - 1) // bs
        ids = torch.tensor(list(block_tables[s_idx])[:nb], dtype=torch.long)
        k = k_cache[ids].reshape(nb * bs, num_kv_heads, head_dim)[:L].to(compute_dtype)
        v = v_cache[ids].reshape(nb * bs, num_kv_heads, head_dim)[:L].to(compute_dtype)
        qs = q[row:row + n].to(compute_dtype)                    # [n, Hq, D]
        scores = torch.einsum("nhd,shd->hns", qs, k[:, kv_head]) * scale   # [Hq, n, L]
        pos = torch.arange(L - n, L).unsqueeze(1)                 # [n, 1]
        visible = torch.arange(L).unsqueeze(0) <= pos             # [n, L]
        scores = scores.masked_fill(~visible, float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        out[row:row + n] = torch.einsum("hns,shd->nhd", probs, v[:, kv_head])
        row += n
    return out
