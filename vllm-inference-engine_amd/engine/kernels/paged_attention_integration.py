"""Per-layer decode attention over the paged pool: K/V write + paged attention.

Mirrors the decode path of the reference module
engine/kernels/paged_attention_integration.py:
  * PagedAttentionContext (reference :29-62): per-step block tables and lengths;
  * paged_decode_attention_forward (reference :65-176): projections, RoPE, the
    new token's K/V written into its block, batched paged attention, o_proj;
  * patch_paged_attention (reference :179-208): binds that forward onto every
    attention module of a model for the duration of a decode step.

  * KernelPagedManualDecode (reference :211-731): prefill into the pool,
    batched decode steps, single-sequence greedy generation.
  * PagedPrefillContext / paged_prefill_attention_forward: the "full"
    prefix-cache prefill (reference :459-482) without the DynamicCache copy of
    the cached blocks (:364-392): each layer writes the suffix's K/V into its
    blocks and runs the paged prefill attention kernel over the pool.

The reference writes K/V with a Python loop of two index_put calls per sequence
and a device-to-host `.item()` per sequence per layer (:148-161). Here the
write is one HIP launch, paged_kv_write(), that computes every slot on the
device from the block tables and lengths, so a decode step's layers make no
host syncs. Prompt K/V go into the pool with one paged_prefill_copy launch per
layer (reference pad + index_copy_, :278-326).
"""
from __future__ import annotations

import itertools
import logging
import math
from collections import OrderedDict
from contextlib import contextmanager
from typing import Any, Callable, Dict, List, Optional, Tuple, Union

import numpy as np
import torch
import torch.nn as nn

from engine.kernels import _native
from engine.kernels.paged_attention import (
    _on_device,
    pad_block_tables,
    paged_attention_prefill,
)
from engine.memory.block_allocator import BlockAllocator, BlockTable, PhysicalBlockPool

logger = logging.getLogger(__name__)

__all__ = [
    "PagedAttentionContext",
    "paged_kv_write",
    "paged_rope_kv_write",
    "paged_rope_decode_attention",
    "paged_decode_kv_write_attention",
    "paged_prefill_copy",
    "paged_decode_attention_forward",
    "paged_prefill_attention_forward",
    "PagedPrefillContext",
    "patch_paged_attention",
    "prepare_fused_layers",
    "fused_decoder_layer_forward",
    "rms_norm",
    "silu_mul",
    "greedy_top2",
    "KernelPagedManualDecode",
]


def _as_rows(x: torch.Tensor) -> torch.Tensor:
    """[B, Hkv, 1, D] (the projection layout) or [B, Hkv, D] -> a [B, Hkv, D] view."""
    if x.dim() == 4:
        assert x.shape[2] == 1, f"expected one new token per sequence, got shape {tuple(x.shape)}"
        x = x.squeeze(2)
    assert x.dim() == 3, f"expected [num_seqs, num_kv_heads, head_dim], got {tuple(x.shape)}"
    return x


def paged_kv_write(
    key: torch.Tensor,           # [num_seqs, num_kv_heads, head_dim] or [.., 1, ..]; any strides
    value: torch.Tensor,         # same
    k_cache: torch.Tensor,       # [num_blocks, block_size, num_kv_heads, head_dim] fp16
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,  # [num_seqs, max_blocks_per_seq] int32 (or 1-D for one sequence)
    seq_lens: Union[torch.Tensor, int],  # [num_seqs] int32, or one host int for one sequence
) -> None:
    """Write each sequence's newest K/V row into its paged slot, bit for bit.

    Sequence b writes position L_b - 1 (L_b counts the new token, reference
    decode_step integration.py:593-596) into block block_tables[b][(L_b-1)//bs],
    row (L_b-1) % bs -- the slot the reference's loop computes at
    integration.py:150-160 (single sequence :122-132). Asynchronous on the
    current stream; no host synchronisation.
    """
    key = _as_rows(key)
    value = _as_rows(value)
    assert key.is_cuda and value.is_cuda and k_cache.is_cuda and v_cache.is_cuda
    _native.same_device(key, value, k_cache, v_cache, block_tables,
                        *([seq_lens] if isinstance(seq_lens, torch.Tensor) else []))
    assert key.dtype == torch.float16 and value.dtype == torch.float16
    assert k_cache.dtype == torch.float16 and v_cache.dtype == torch.float16
    assert block_tables.dtype == torch.int32 and block_tables.is_cuda
    assert k_cache.shape == v_cache.shape, "k_cache and v_cache must have the same shape"
    num_blocks, block_size, num_kv_heads, head_dim = k_cache.shape
    num_seqs = key.shape[0]
    assert key.shape == (num_seqs, num_kv_heads, head_dim), (
        f"key shape {tuple(key.shape)} does not match the pool ({num_kv_heads}, {head_dim})")
    assert value.shape == key.shape, f"value shape {tuple(value.shape)} != key shape {tuple(key.shape)}"
    if block_tables.dim() == 1:
        block_tables = block_tables.unsqueeze(0)
    assert block_tables.shape[0] == num_seqs
    if isinstance(seq_lens, torch.Tensor):
        assert seq_lens.is_cuda and seq_lens.dtype == torch.int32 and seq_lens.shape == (num_seqs,)
        lens_ptr, uniform = _native.ptr(seq_lens), 0
    else:
        assert num_seqs == 1, "a host integer length is only accepted for one sequence"
        lens_ptr, uniform = None, int(seq_lens)
    if num_seqs == 0:
        return
    lib = _native.load()
    dev = key.device
    with _on_device(dev):
        status = lib.pa_kv_write_f16(
            key.data_ptr(), _native.strides_of(key),
            value.data_ptr(), _native.strides_of(value),
            k_cache.data_ptr(), _native.strides_of(k_cache),
            v_cache.data_ptr(), _native.strides_of(v_cache),
            block_tables.data_ptr(), _native.strides_of(block_tables),
            lens_ptr, uniform,
            num_seqs, num_kv_heads, head_dim, block_size, num_blocks, block_tables.shape[1],
            _native.stream_handle(dev))
    _native.check(status, "pa_kv_write_f16")


def _rope_rows(t: torch.Tensor) -> torch.Tensor:
    """cos/sin as one row per sequence: [B, 1, D] (the model's rotary output) or [B, D]."""
    if t.dim() == 3:
        assert t.shape[1] == 1, f"expected one position per sequence, got shape {tuple(t.shape)}"
        t = t.squeeze(1)
    assert t.dim() == 2, f"expected [num_seqs, head_dim], got {tuple(t.shape)}"
    return t


def paged_rope_kv_write(
    query: torch.Tensor,         # [num_seqs, num_q_heads, (1,) head_dim] fp16, any strides
    key: torch.Tensor,           # [num_seqs, num_kv_heads, (1,) head_dim]
    value: torch.Tensor,         # same as key
    cos: torch.Tensor,           # [num_seqs, (1,) head_dim] fp16, the rotary table rows
    sin: torch.Tensor,
    k_cache: torch.Tensor,       # [num_blocks, block_size, num_kv_heads, head_dim] fp16
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,  # [num_seqs, max_blocks_per_seq] int32 (or 1-D for one sequence)
    seq_lens: Union[torch.Tensor, int],
) -> torch.Tensor:
    """Rotary embedding of the new token's q and k plus its K/V write, in one launch.

    Same results, bit for bit, as transformers' apply_rotary_pos_emb in fp16
    (called by the reference at integration.py:108-109) followed by
    paged_kv_write of the rotated key and the value (reference write loop
    :148-161): returns the rotated queries [num_seqs, num_q_heads, head_dim]
    (contiguous) and writes the rotated key and the value into each sequence's
    slot of position L_b - 1. Asynchronous; no host synchronisation.
    """
    query = _as_rows(query)
    key = _as_rows(key)
    value = _as_rows(value)
    cos = _rope_rows(cos)
    sin = _rope_rows(sin)
    for t in (query, key, value, cos, sin, k_cache, v_cache):
        assert t.is_cuda and t.dtype == torch.float16
    assert block_tables.dtype == torch.int32 and block_tables.is_cuda
    _native.same_device(query, key, value, cos, sin, k_cache, v_cache, block_tables,
                        *([seq_lens] if isinstance(seq_lens, torch.Tensor) else []))
    assert k_cache.shape == v_cache.shape, "k_cache and v_cache must have the same shape"
    num_blocks, block_size, num_kv_heads, head_dim = k_cache.shape
    num_seqs, num_q_heads = query.shape[0], query.shape[1]
    assert query.shape[2] == head_dim and head_dim % 2 == 0
    assert key.shape == (num_seqs, num_kv_heads, head_dim) and value.shape == key.shape
    assert cos.shape == (num_seqs, head_dim) and sin.shape == cos.shape
    if block_tables.dim() == 1:
        block_tables = block_tables.unsqueeze(0)
    assert block_tables.shape[0] == num_seqs
    if isinstance(seq_lens, torch.Tensor):
        assert seq_lens.is_cuda and seq_lens.dtype == torch.int32 and seq_lens.shape == (num_seqs,)
        lens_ptr, uniform = _native.ptr(seq_lens), 0
    else:
        assert num_seqs == 1, "a host integer length is only accepted for one sequence"
        lens_ptr, uniform = None, int(seq_lens)
    q_out = torch.empty((num_seqs, num_q_heads, head_dim), dtype=torch.float16, device=query.device)
    if num_seqs == 0:
        return q_out
    lib = _native.load()
    dev = query.device
    with _on_device(dev):
        status = lib.pa_rope_kv_write_f16(
            query.data_ptr(), _native.strides_of(query),
            key.data_ptr(), _native.strides_of(key),
            value.data_ptr(), _native.strides_of(value),
            cos.data_ptr(), _native.strides_of(cos),
            sin.data_ptr(), _native.strides_of(sin),
            q_out.data_ptr(), _native.strides_of(q_out),
            k_cache.data_ptr(), _native.strides_of(k_cache),
            v_cache.data_ptr(), _native.strides_of(v_cache),
            block_tables.data_ptr(), _native.strides_of(block_tables),
            lens_ptr, uniform,
            num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
            block_tables.shape[1], _native.stream_handle(dev))
    _native.check(status, "pa_rope_kv_write_f16")
    return q_out


_rope_ws_sizes: Dict[tuple, int] = {}


def paged_rope_decode_attention(
    query: torch.Tensor,         # [num_seqs, num_q_heads, (1,) head_dim] fp16, unrotated
    key: torch.Tensor,           # [num_seqs, num_kv_heads, (1,) head_dim], unrotated
    value: torch.Tensor,         # same as key
    cos: torch.Tensor,           # [num_seqs, (1,) head_dim] fp16, the rotary table rows
    sin: torch.Tensor,
    k_cache: torch.Tensor,       # [num_blocks, block_size, num_kv_heads, head_dim] fp16
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,  # [num_seqs, max_blocks_per_seq] int32
    seq_lens: torch.Tensor,      # [num_seqs] int32, lengths including the new token
    scale: float,
) -> torch.Tensor:
    """One decode step's attention block of a layer, in one call.

    The same bits as paged_rope_kv_write(query, key, value, cos, sin, k_cache,
    v_cache, block_tables, seq_lens) followed by paged_attention_decode_batched
    on the rotated queries -- the reference's apply_rotary_pos_emb
    (integration.py:108-109), K/V write loop (:148-161) and batched attention
    call (:164-171). Batches that take one workgroup per (sequence, kv-head
    group) pair run as one kernel launch; the others as those two launches.
    Returns [num_seqs, num_q_heads, head_dim]; asynchronous on the current stream.
    """
    query = _as_rows(query)
    key = _as_rows(key)
    value = _as_rows(value)
    cos = _rope_rows(cos)
    sin = _rope_rows(sin)
    for t in (query, key, value, cos, sin, k_cache, v_cache):
        assert t.is_cuda and t.dtype == torch.float16
    assert block_tables.dtype == torch.int32 and block_tables.is_cuda and block_tables.dim() == 2
    assert seq_lens.is_cuda and seq_lens.dtype == torch.int32
    _native.same_device(query, key, value, cos, sin, k_cache, v_cache, block_tables, seq_lens)
    assert k_cache.shape == v_cache.shape, "k_cache and v_cache must have the same shape"
    num_blocks, block_size, num_kv_heads, head_dim = k_cache.shape
    num_seqs, num_q_heads = query.shape[0], query.shape[1]
    assert query.shape[2] == head_dim and head_dim % 2 == 0
    assert num_q_heads % num_kv_heads == 0, (
        f"num_q_heads ({num_q_heads}) must be divisible by num_kv_heads ({num_kv_heads})")
    assert key.shape == (num_seqs, num_kv_heads, head_dim) and value.shape == key.shape
    assert cos.shape == (num_seqs, head_dim) and sin.shape == cos.shape
    assert block_tables.shape[0] == num_seqs and seq_lens.shape == (num_seqs,)
    out = torch.empty((num_seqs, num_q_heads, head_dim), dtype=torch.float16, device=query.device)
    if num_seqs == 0:
        return out
    assert block_tables.shape[1] > 0, "block_tables needs at least one column"
    lib = _native.load()
    dev = query.device
    max_blocks = block_tables.shape[1]
    ws_key = (dev.index, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks)
    stream = _native.stream_handle(dev)
    with _on_device(dev):
        ws_bytes = _rope_ws_sizes.get(ws_key)
        if ws_bytes is None:
            ws_bytes = _rope_ws_sizes[ws_key] = lib.pa_decode_rope_batched_workspace_bytes(
                *ws_key[1:])
        status = lib.pa_decode_rope_batched_f16(
            query.data_ptr(), _native.strides_of(query),
            key.data_ptr(), _native.strides_of(key),
            value.data_ptr(), _native.strides_of(value),
            cos.data_ptr(), _native.strides_of(cos),
            sin.data_ptr(), _native.strides_of(sin),
            k_cache.data_ptr(), _native.strides_of(k_cache),
            v_cache.data_ptr(), _native.strides_of(v_cache),
            block_tables.data_ptr(), _native.strides_of(block_tables),
            seq_lens.data_ptr(), out.data_ptr(), _native.strides_of(out),
            num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, max_blocks,
            float(scale), _native.workspace(ws_bytes, dev, stream, _native.WS_DECODE), ws_bytes,
            stream)
    _native.check(status, "pa_decode_rope_batched_f16")
    return out


def _rows16(x: torch.Tensor) -> torch.Tensor:
    """Rows with unit head_dim stride, 8-element aligned strides and a 16-byte aligned base."""
    ok = (x.stride(-1) == 1 and all(st % 8 == 0 for st in x.stride()[:-1])
          and x.data_ptr() % 16 == 0)
    return x if ok else x.contiguous()


def paged_decode_kv_write_attention(
    query: torch.Tensor,         # [num_seqs, num_q_heads, head_dim] (or [B, Hq, 1, D])
    key: torch.Tensor,           # [num_seqs, num_kv_heads, head_dim] (or [B, Hkv, 1, D])
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,  # [num_seqs, max_blocks] int32
    seq_lens: torch.Tensor,      # [num_seqs] int32, counting the new token
    scale: float,
) -> torch.Tensor:
    """The new token's K/V write followed by batched paged attention, in one launch.

    The reference's K/V write loop and the paged_attention_decode_batched call
    after it (integration.py:148-161, :164-171): key/value row b goes to
    position seq_lens[b] - 1 of sequence b, then every query attends over its
    seq_lens[b] tokens, the new one included. The same bits as paged_kv_write
    followed by paged_attention_decode_batched; one kernel launch where the
    batch takes one workgroup per (sequence, kv-head group) pair at head_dim
    64 or 128 with blocks of 16 or 32 tokens (the decode step's shapes), else
    those two launches.
    Returns [num_seqs, num_q_heads, head_dim]; asynchronous on the current stream.
    """
    query = _as_rows(query)
    key = _as_rows(key)
    value = _as_rows(value)
    for t in (query, key, value, k_cache, v_cache):
        assert t.is_cuda and t.dtype == torch.float16
    assert block_tables.dtype == torch.int32 and block_tables.is_cuda and block_tables.dim() == 2
    assert seq_lens.is_cuda and seq_lens.dtype == torch.int32
    _native.same_device(query, key, value, k_cache, v_cache, block_tables, seq_lens)
    assert k_cache.shape == v_cache.shape, "k_cache and v_cache must have the same shape"
    num_blocks, block_size, num_kv_heads, head_dim = k_cache.shape
    num_seqs, num_q_heads = query.shape[0], query.shape[1]
    assert query.shape[2] == head_dim, f"Head dimensions must match: {query.shape[2]} vs {head_dim}"
    assert num_q_heads % num_kv_heads == 0, (
        f"num_q_heads ({num_q_heads}) must be divisible by num_kv_heads ({num_kv_heads})")
    assert key.shape == (num_seqs, num_kv_heads, head_dim) and value.shape == key.shape
    assert block_tables.shape[0] == num_seqs and seq_lens.shape == (num_seqs,)
    out = torch.empty((num_seqs, num_q_heads, head_dim), dtype=torch.float16, device=query.device)
    if num_seqs == 0:
        return out
    assert block_tables.shape[1] > 0, "block_tables needs at least one column"
    query, key, value = _rows16(query), _rows16(key), _rows16(value)
    lib = _native.load()
    dev = query.device
    max_blocks = block_tables.shape[1]
    ws_key = (dev.index, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks)
    stream = _native.stream_handle(dev)
    with _on_device(dev):
        ws_bytes = _write_ws_sizes.get(ws_key)
        if ws_bytes is None:
            ws_bytes = _write_ws_sizes[ws_key] = lib.pa_decode_batched_workspace_bytes(
                *ws_key[1:])
        status = lib.pa_decode_kv_write_batched_f16(
            query.data_ptr(), _native.strides_of(query),
            key.data_ptr(), _native.strides_of(key),
            value.data_ptr(), _native.strides_of(value),
            k_cache.data_ptr(), _native.strides_of(k_cache),
            v_cache.data_ptr(), _native.strides_of(v_cache),
            block_tables.data_ptr(), _native.strides_of(block_tables),
            seq_lens.data_ptr(), out.data_ptr(), _native.strides_of(out),
            num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, max_blocks,
            float(scale), _native.workspace(ws_bytes, dev, stream, _native.WS_DECODE), ws_bytes,
            stream)
    _native.check(status, "pa_decode_kv_write_batched_f16")
    return out


_write_ws_sizes: dict = {}


class PagedAttentionContext:
    """Per-step metadata handed to the patched attention modules (reference integration.py:29-62).

    `pool` is any object with per-layer `k_cache`/`v_cache` lists and a
    `device` (the reference's PhysicalBlockPool). Block tables are BlockTable-like
    objects (`.physical_block_ids`) or plain lists.
    """

    def __init__(
        self,
        pool: Any,
        block_tables: Union[Any, List[Any]],
        seq_lens: Union[int, List[int], torch.Tensor],
        block_size: int = 16,
        is_decode: bool = True,
    ):
        self.pool = pool
        self.block_size = block_size
        self.is_decode = is_decode

        if hasattr(block_tables, "physical_block_ids"):
            self.is_batched = False
            self.single_block_table = block_tables
            self.single_seq_len = int(seq_lens)
            self.block_table_tensor = torch.tensor(
                list(block_tables.physical_block_ids), dtype=torch.int32, device=pool.device)
        else:
            self.is_batched = True
            self.block_table_list = block_tables
            self.padded_block_tables = pad_block_tables(block_tables, device=pool.device)
            if isinstance(seq_lens, torch.Tensor):
                self.seq_lens_tensor = seq_lens.to(device=pool.device, dtype=torch.int32)
            else:
                self.seq_lens_tensor = torch.tensor(seq_lens, dtype=torch.int32, device=pool.device)

    @classmethod
    def from_device(cls, pool: Any, block_tables: torch.Tensor, seq_lens: torch.Tensor,
                    block_size: int = 16) -> "PagedAttentionContext":
        """Batched context over tables and lengths already on the device (no host copies)."""
        ctx = cls.__new__(cls)
        ctx.pool = pool
        ctx.block_size = block_size
        ctx.is_decode = True
        ctx.is_batched = True
        ctx.block_table_list = None
        ctx.padded_block_tables = block_tables
        ctx.seq_lens_tensor = seq_lens
        return ctx


class PagedPrefillContext:
    """Metadata of one sequence's paged prefill: the prompt after `cached_tokens` cached tokens.

    The new tokens' K/V go to the sequence's blocks from cached_tokens // block_size
    on (whole blocks, rows past the prompt zeroed, as the reference's
    _copy_prefill_kv with skip_blocks writes them, integration.py:278-326); the
    attention reads the cached blocks and those new rows from the pool.
    """

    is_decode = False
    is_prefill = True

    def __init__(self, pool: Any, block_ids: List[int], cached_tokens: int, prompt_len: int,
                 block_size: int):
        assert cached_tokens % block_size == 0 and 0 <= cached_tokens < prompt_len
        nb = (prompt_len + block_size - 1) // block_size
        assert len(block_ids) >= nb, "block table shorter than the prompt"
        dev = pool.device
        self.pool = pool
        self.block_size = block_size
        self.num_new = prompt_len - cached_tokens
        self.block_tables = torch.tensor([list(block_ids[:nb])], dtype=torch.int32, device=dev)
        self.write_ids = torch.tensor(list(block_ids[cached_tokens // block_size:nb]),
                                      dtype=torch.int32, device=dev)
        self.seq_lens = torch.tensor([prompt_len], dtype=torch.int32, device=dev)
        self.query_start_loc = torch.tensor([0, self.num_new], dtype=torch.int32, device=dev)


def paged_decode_attention_forward(
    self: nn.Module,
    hidden_states: torch.Tensor,
    position_embeddings: Tuple[torch.Tensor, torch.Tensor],
    attention_mask: Optional[torch.Tensor] = None,
    past_key_values: Any = None,
    **kwargs: Any,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Drop-in Qwen2Attention.forward for one decode step (reference integration.py:65-176).

    q/k/v projections; then paged_rope_decode_attention: RoPE of q and k, the
    new K/V's write into the pool (bit-identical to transformers'
    apply_rotary_pos_emb followed by the reference's write loop) and batched
    paged attention over L_b tokens (the write precedes the read, as in the
    reference), in one launch where the batch allows; then o_proj.
    """
    ctx: Optional[PagedAttentionContext] = getattr(self, "_paged_attention_context", None)
    if ctx is not None and getattr(ctx, "is_prefill", False):
        return paged_prefill_attention_forward(self, hidden_states, position_embeddings,
                                               attention_mask, past_key_values, **kwargs)
    if ctx is None or not ctx.is_decode:
        orig_forward = getattr(self, "_orig_attention_forward", None)
        if orig_forward is not None:
            return orig_forward(
                hidden_states=hidden_states,
                position_embeddings=position_embeddings,
                attention_mask=attention_mask,
                past_key_values=past_key_values,
                **kwargs,
            )
        raise RuntimeError("No fallback forward method found on attention module.")

    layer_idx = self.layer_idx
    input_shape = hidden_states.shape[:-1]  # [batch, 1]
    hidden_shape = (*input_shape, -1, self.head_dim)

    query_states = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    key_states = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)

    cos, sin = position_embeddings

    scale = self.scaling if hasattr(self, "scaling") else 1.0 / math.sqrt(self.head_dim)
    pool = ctx.pool
    k_cache = pool.k_cache[layer_idx]
    v_cache = pool.v_cache[layer_idx]

    if not ctx.is_batched:
        bt_2d = ctx.block_table_tensor.unsqueeze(0)
        seq_lens_t = torch.tensor([ctx.single_seq_len], dtype=torch.int32, device=pool.device)
    else:
        bt_2d = ctx.padded_block_tables
        seq_lens_t = ctx.seq_lens_tensor

    # RoPE of q and k, the write of the new K/V into the pool, then attention
    # over L_b tokens (the write precedes the read, as in the reference).
    attn_output = paged_rope_decode_attention(query_states, key_states, value_states, cos, sin,
                                              k_cache, v_cache, bt_2d, seq_lens_t, scale)
    attn_output = attn_output.reshape(*input_shape, -1).contiguous()
    attn_output = self.o_proj(attn_output)
    return attn_output, None


def paged_prefill_attention_forward(
    self: nn.Module,
    hidden_states: torch.Tensor,
    position_embeddings: Tuple[torch.Tensor, torch.Tensor],
    attention_mask: Optional[torch.Tensor] = None,
    past_key_values: Any = None,
    **kwargs: Any,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Attention forward for a prompt suffix of one sequence over its cached prefix blocks.

    Replaces the reference's "full" prefix-cache prefill attention
    (integration.py:459-482), which copies the cached blocks of every layer
    into a DynamicCache (:364-392) and runs transformers' causal attention over
    prefix + suffix. Here: q/k/v projections; RoPE with transformers'
    apply_rotary_pos_emb (the reference's, :108-109); the suffix's K/V written
    into the sequence's own blocks with paged_prefill_copy; causal paged
    prefill attention over the pool; o_proj. The causal mask is the kernel's
    (new token i at position cached + i sees pool positions 0 .. cached + i),
    so `attention_mask` is not used.
    """
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    ctx: PagedPrefillContext = self._paged_attention_context
    input_shape = hidden_states.shape[:-1]  # [1, n]
    assert input_shape[0] == 1 and input_shape[1] == ctx.num_new
    hidden_shape = (*input_shape, -1, self.head_dim)
    query_states = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    key_states = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    cos, sin = position_embeddings
    query_states, key_states = apply_rotary_pos_emb(query_states, key_states, cos, sin)

    scale = self.scaling if hasattr(self, "scaling") else 1.0 / math.sqrt(self.head_dim)
    k_cache = ctx.pool.k_cache[self.layer_idx]
    v_cache = ctx.pool.v_cache[self.layer_idx]
    # [1, H, n, D] -> [n, H, D] views; the kernels take any token/head strides.
    paged_prefill_copy(key_states[0].transpose(0, 1), value_states[0].transpose(0, 1),
                       k_cache, v_cache, ctx.write_ids, ctx.num_new)
    attn = paged_attention_prefill(query_states[0].transpose(0, 1), k_cache, v_cache,
                                   ctx.block_tables, ctx.seq_lens, ctx.query_start_loc,
                                   ctx.num_new, scale)
    attn_output = attn.reshape(*input_shape, -1).contiguous()
    return self.o_proj(attn_output), None


# ---- fused layer pieces of the decode step --------------------------------------

def _rows(t: torch.Tensor) -> torch.Tensor:
    rows = t.reshape(-1, t.shape[-1])
    return rows if rows.stride(-1) == 1 else rows.contiguous()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             residual: Optional[torch.Tensor] = None):
    """transformers' Qwen2RMSNorm.forward in one launch (same roundings): fp16 rows [..., H].

    With `residual`, the norm is taken of fp16(x + residual) -- the decoder
    layer's residual add -- and (sum, normed) is returned.
    """
    assert x.is_cuda and x.dtype == torch.float16 and weight.dtype == torch.float16
    _native.same_device(x, weight, *([residual] if residual is not None else []))
    h = x.shape[-1]
    rows = _rows(x)
    out = torch.empty(rows.shape, dtype=torch.float16, device=x.device)
    res_ptr, res_stride, sum_ptr, sum_stride, total = 0, 0, 0, 0, None
    if residual is not None:
        assert residual.shape == x.shape and residual.dtype == torch.float16
        res = _rows(residual)
        total = torch.empty(rows.shape, dtype=torch.float16, device=x.device)
        res_ptr, res_stride = res.data_ptr(), res.stride(0)
        sum_ptr, sum_stride = total.data_ptr(), total.stride(0)
    lib = _native.load()
    with _on_device(x.device):
        status = lib.pa_rmsnorm_f16(rows.data_ptr(), rows.stride(0), res_ptr, res_stride, sum_ptr,
                                    sum_stride, weight.contiguous().data_ptr(), out.data_ptr(),
                                    out.stride(0), rows.shape[0], h, float(eps),
                                    _native.stream_handle(x.device))
    _native.check(status, "pa_rmsnorm_f16")
    if total is None:
        return out.view(x.shape)
    return total.view(x.shape), out.view(x.shape)


def greedy_top2(logits: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per row of fp16 logits [rows, vocab]: (argmax int64 [rows], top-2 values fp32 [rows, 2]).

    torch.argmax (first index of the maximum) and torch.topk(row, 2).values in one launch.
    """
    assert logits.is_cuda and logits.dtype == torch.float16 and logits.dim() == 2
    assert logits.stride(-1) == 1
    rows, vocab = logits.shape
    idx = torch.empty(rows, dtype=torch.int64, device=logits.device)
    top = torch.empty(rows, 2, dtype=torch.float32, device=logits.device)
    lib = _native.load()
    with _on_device(logits.device):
        status = lib.pa_top2_f16(logits.data_ptr(), logits.stride(0), rows, vocab, idx.data_ptr(),
                                 top.data_ptr(), _native.stream_handle(logits.device))
    _native.check(status, "pa_top2_f16")
    return idx, top


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up of a merged [rows, 2 * I] gate/up projection, in one launch."""
    assert gate_up.is_cuda and gate_up.dtype == torch.float16 and gate_up.dim() == 2
    assert gate_up.stride(-1) == 1 and gate_up.shape[1] % 2 == 0
    inter = gate_up.shape[1] // 2
    out = torch.empty(gate_up.shape[0], inter, dtype=torch.float16, device=gate_up.device)
    lib = _native.load()
    with _on_device(gate_up.device):
        status = lib.pa_silu_mul_f16(gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(),
                                     out.stride(0), gate_up.shape[0], inter,
                                     _native.stream_handle(gate_up.device))
    _native.check(status, "pa_silu_mul_f16")
    return out


def _is_decoder_layer(m: nn.Module) -> bool:
    attn, mlp = getattr(m, "self_attn", None), getattr(m, "mlp", None)
    return (attn is not None and mlp is not None
            and all(hasattr(attn, n) for n in ("q_proj", "k_proj", "v_proj", "o_proj"))
            and all(hasattr(mlp, n) for n in ("gate_proj", "up_proj", "down_proj"))
            and hasattr(m, "input_layernorm") and hasattr(m, "post_attention_layernorm"))


def prepare_fused_layers(model: nn.Module) -> int:
    """Concatenate each decoder layer's q/k/v and gate/up weights once, for the fused decode path.

    The merged copies live on the layer (`_pa_fused`); the model's own modules
    are left as they are. Returns the number of layers prepared. Inference
    only: the copies do not follow later changes of the weights.
    """
    n = 0
    if not isinstance(model, nn.Module):
        return n
    with torch.no_grad():
        for m in model.modules():
            if not _is_decoder_layer(m) or hasattr(m, "_pa_fused"):
                continue
            attn, mlp = m.self_attn, m.mlp
            if getattr(mlp, "act_fn", None) is not None and \
                    type(mlp.act_fn).__name__ not in ("SiLU", "SiLUActivation"):
                continue
            biases = [attn.q_proj.bias, attn.k_proj.bias, attn.v_proj.bias]
            qkv_b = torch.cat(biases) if all(b is not None for b in biases) else None
            if qkv_b is None and any(b is not None for b in biases):
                continue
            m._pa_fused = (
                torch.cat([attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight]).contiguous(),
                qkv_b,
                torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight]).contiguous(),
            )
            n += 1
    return n


def fused_decoder_layer_forward(
    self: nn.Module,
    hidden_states: torch.Tensor,
    attention_mask: Optional[torch.Tensor] = None,
    position_ids: Optional[torch.Tensor] = None,
    past_key_values: Any = None,
    use_cache: Optional[bool] = False,
    position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    **kwargs: Any,
) -> torch.Tensor:
    """One decoder layer of a decode step in nine launches instead of about thirty.

    The same computation as transformers' Qwen2DecoderLayer.forward with the
    paged attention forward patched in: RMSNorm (one kernel), the q/k/v
    projections as one GEMM over the concatenated weights, the fused RoPE +
    K/V write and the batched paged attention, o_proj, the residual add and
    RMSNorm in one kernel, gate and up as one GEMM, silu * up (one kernel),
    down_proj with the residual added by the GEMM into the residual sum's own
    buffer. Only decode steps (one token per sequence, paged decode context)
    take this path.
    """
    attn = self.self_attn
    ctx = getattr(attn, "_paged_attention_context", None)
    if (ctx is None or not ctx.is_decode or getattr(ctx, "is_prefill", False)
            or hidden_states.dim() != 3 or hidden_states.shape[1] != 1):
        return self._orig_layer_forward(hidden_states, attention_mask=attention_mask,
                                        position_ids=position_ids, past_key_values=past_key_values,
                                        use_cache=use_cache, position_embeddings=position_embeddings,
                                        **kwargs)
    qkv_w, qkv_b, gu_w = self._pa_fused
    b, _, hidden = hidden_states.shape
    x = hidden_states.reshape(b, hidden)
    hd = attn.head_dim
    nq = attn.q_proj.out_features // hd
    nkv = attn.k_proj.out_features // hd
    xn = rms_norm(x, self.input_layernorm.weight, self.input_layernorm.variance_epsilon)
    qkv = torch.nn.functional.linear(xn, qkv_w, qkv_b)
    q = qkv[:, :nq * hd].view(b, nq, hd)
    k = qkv[:, nq * hd:(nq + nkv) * hd].view(b, nkv, hd)
    v = qkv[:, (nq + nkv) * hd:].view(b, nkv, hd)
    cos, sin = position_embeddings
    scale = attn.scaling if hasattr(attn, "scaling") else 1.0 / math.sqrt(hd)
    k_cache = ctx.pool.k_cache[attn.layer_idx]
    v_cache = ctx.pool.v_cache[attn.layer_idx]
    if ctx.is_batched:
        bt_2d, lens = ctx.padded_block_tables, ctx.seq_lens_tensor
    else:
        bt_2d = ctx.block_table_tensor.unsqueeze(0)
        lens = torch.tensor([ctx.single_seq_len], dtype=torch.int32, device=ctx.pool.device)
    o = paged_rope_decode_attention(q, k, v, cos, sin, k_cache, v_cache, bt_2d, lens, scale)
    proj = torch.nn.functional.linear(o.reshape(b, nq * hd), attn.o_proj.weight, attn.o_proj.bias)
    h, hn = rms_norm(proj, self.post_attention_layernorm.weight,
                     self.post_attention_layernorm.variance_epsilon, residual=x)
    act = silu_mul(torch.nn.functional.linear(hn, gu_w))
    h.addmm_(act, self.mlp.down_proj.weight.t())  # h is this layer's own buffer
    return h.view(b, 1, hidden)


def _fused_rms_norm_forward(self: nn.Module, hidden_states: torch.Tensor) -> torch.Tensor:
    if hidden_states.dtype != torch.float16 or self.weight.dtype != torch.float16:
        return self._orig_norm_forward(hidden_states)
    return rms_norm(hidden_states, self.weight, self.variance_epsilon)


@contextmanager
def patch_paged_attention(model: nn.Module, context: PagedAttentionContext,
                          fuse_layers: bool = True):
    """Temporarily bind paged_decode_attention_forward on every attention module (reference :179-208).

    For a decode context with fuse_layers, decoder layers prepared by
    prepare_fused_layers() also get fused_decoder_layer_forward, and RMSNorm
    modules (those with `weight` and `variance_epsilon`) the one-launch norm,
    for the same duration; prefill contexts, and decode contexts without
    fuse_layers, keep transformers' layers and norms.
    """
    patched: List[Tuple[nn.Module, Callable, str]] = []
    decode = (fuse_layers and getattr(context, "is_decode", False)
              and not getattr(context, "is_prefill", False))
    for module in model.modules():
        if all(hasattr(module, n) for n in ("q_proj", "k_proj", "v_proj", "o_proj")):
            orig_fwd = module.forward
            module._orig_attention_forward = orig_fwd
            module._paged_attention_context = context
            module.forward = paged_decode_attention_forward.__get__(module, module.__class__)
            patched.append((module, orig_fwd, "attn"))
        elif decode and hasattr(module, "_pa_fused") and _is_decoder_layer(module):
            orig_fwd = module.forward
            module._orig_layer_forward = orig_fwd
            module.forward = fused_decoder_layer_forward.__get__(module, module.__class__)
            patched.append((module, orig_fwd, "layer"))
    if any(kind == "layer" for _, _, kind in patched):
        for module in model.modules():
            if hasattr(module, "variance_epsilon") and isinstance(getattr(module, "weight", None),
                                                                  torch.Tensor):
                orig_fwd = module.forward
                module._orig_norm_forward = orig_fwd
                module.forward = _fused_rms_norm_forward.__get__(module, module.__class__)
                patched.append((module, orig_fwd, "norm"))
    try:
        yield context
    finally:
        for module, orig_fwd, kind in patched:
            # A forward bound on the instance before patching is put back; otherwise the
            # class's forward shows through again (no instance attribute is left behind).
            if getattr(orig_fwd, "__self__", None) is module and \
                    getattr(orig_fwd, "__func__", None) is getattr(type(module).forward, "__func__",
                                                               type(module).forward):
                del module.forward
            else:
                module.forward = orig_fwd
            for attr in ("_orig_attention_forward", "_paged_attention_context",
                         "_orig_layer_forward", "_orig_norm_forward"):
                if hasattr(module, attr):
                    delattr(module, attr)


def paged_prefill_copy(
    key: torch.Tensor,        # [num_tokens, num_kv_heads, head_dim], any strides (fp16 or castable)
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_ids: torch.Tensor,  # 1-D int32 device tensor: destination block of each source block
    num_tokens: int,
) -> None:
    """Write a prompt slice's K/V into whole pool blocks, zero-padding the last block.

    Same pool contents as the reference's pad + index_copy_
    (integration.py:278-326): source block j goes to block_ids[j]; rows at or
    past num_tokens become zeros. Sources of another dtype are cast to fp16
    first, as the reference's `.to(self.dtype)` does.
    """
    assert k_cache.is_cuda and v_cache.is_cuda and block_ids.is_cuda
    _native.same_device(k_cache, v_cache, block_ids, key, value)
    assert k_cache.dtype == torch.float16 and v_cache.dtype == torch.float16
    assert block_ids.dtype == torch.int32 and block_ids.dim() == 1
    assert k_cache.shape == v_cache.shape
    num_blocks, block_size, num_kv_heads, head_dim = k_cache.shape
    if key.dtype != torch.float16:
        key = key.to(torch.float16)
    if value.dtype != torch.float16:
        value = value.to(torch.float16)
    assert key.shape[1:] == (num_kv_heads, head_dim) and value.shape == key.shape
    assert key.shape[0] >= num_tokens
    lib = _native.load()
    dev = k_cache.device
    with _on_device(dev):
        status = lib.pa_prefill_copy_f16(
            key.data_ptr(), _native.strides_of(key), value.data_ptr(), _native.strides_of(value),
            k_cache.data_ptr(), _native.strides_of(k_cache),
            v_cache.data_ptr(), _native.strides_of(v_cache),
            block_ids.data_ptr(), block_ids.shape[0], int(num_tokens),
            num_kv_heads, head_dim, block_size, num_blocks, _native.stream_handle(dev))
    _native.check(status, "pa_prefill_copy_f16")


def graph_batch_size(n: int) -> int:
    """Batch size of the captured graph that serves a step of n sequences.

    Steps replay a graph captured for the smallest bucket that holds the
    batch: 1, 2, 4, 8, then multiples of 16 up to 256, then multiples of 64.
    The rows past n are padding: length 0, which the K/V write skips and the
    attention kernel answers with a zero row, and their logits are dropped.
    Padding costs little (the projections are bound by their weights, not
    their rows), and a scheduler whose batch changes every step reuses a few
    graphs instead of capturing one per size.
    """
    assert n >= 1
    if n <= 8:
        return 1 << (n - 1).bit_length()
    if n <= 256:
        return -(-n // 16) * 16
    return -(-n // 64) * 64


class _DecodeGraph:
    """One decode step captured as a HIP graph for a batch-size bucket and table width.

    Static device buffers hold the step's inputs: token ids and lengths (one
    pinned host-to-device copy per step, unpacked inside the graph) and the
    zero-padded block tables (copied only when a row changed: a sequence
    gained a block or the batch was reordered). Rows past the step's batch are
    padding with length 0. The graph replays the whole model forward -- each
    layer's fused RoPE + K/V write and paged attention included -- so a step
    costs one replay instead of a few hundred kernel launches from Python.
    The greedy token and top-1/top-2 margin are computed after the replay,
    outside the graph: top-k and arg-max over a full vocabulary row use
    multi-block reductions whose scratch is cleared with memset operations,
    which are not captured into the graph. Every graph of a runner is
    captured on the runner's one capture stream into one shared memory pool:
    replays run one at a time on the current stream, and each graph's output
    buffer stays alive with it.
    """

    def __init__(self, runner: "KernelPagedManualDecode", batch: int, width: int):
        dev = runner.device
        self.batch, self.width = batch, width
        self.host_in = torch.zeros(2, batch, dtype=torch.long).pin_memory()  # ids, lengths
        self.dev_in = torch.zeros(2, batch, dtype=torch.long, device=dev)
        self.host_tables = torch.zeros(batch, width, dtype=torch.int32).pin_memory()
        self.tables = torch.zeros(batch, width, dtype=torch.int32, device=dev)
        self.mirror = np.full((batch, width), -1, dtype=np.int32)  # table contents on the device
        self.ids = torch.zeros(batch, 1, dtype=torch.long, device=dev)
        self.pos = torch.zeros(batch, 1, dtype=torch.long, device=dev)
        self.lens = torch.ones(batch, dtype=torch.int32, device=dev)
        self.ctx = PagedAttentionContext.from_device(runner.pool, self.tables, self.lens,
                                                     runner.block_size)
        self.runner = runner
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.logits: Optional[torch.Tensor] = None
        self.rows = 0

    def _body(self):
        self.ids.copy_(self.dev_in[0].view(-1, 1))
        self.lens.copy_(self.dev_in[1])
        self.pos.copy_((self.dev_in[1] - 1).clamp_min(0).view(-1, 1))  # padding rows: position 0
        model = self.runner.model
        with patch_paged_attention(model, self.ctx, fuse_layers=self.runner.fuse_layers):
            out = model(input_ids=self.ids, position_ids=self.pos, use_cache=False)
        return out.logits[:, -1, :]

    def load(self, tokens: List[int], lens: List[int], rows: List[List[int]]) -> None:
        """Stage this step's inputs (asynchronous copies on the current stream)."""
        n = len(tokens)
        assert n <= self.batch
        self.rows = n
        hin = self.host_in.numpy()
        hin[:, n:] = 0
        hin[0, :n] = tokens
        hin[1, :n] = lens
        self.dev_in.copy_(self.host_in, non_blocking=True)
        # One vectorised scatter of all rows (a Python loop over 128 rows of
        # numpy slice assignments costs about 0.1 ms per step).
        counts = np.zeros(self.batch, dtype=np.int64)
        counts[:n] = np.fromiter((len(r) for r in rows), dtype=np.int64, count=n)
        flat = np.fromiter(itertools.chain.from_iterable(rows), dtype=np.int32,
                           count=int(counts.sum()))
        table = np.zeros((self.batch, self.width), dtype=np.int32)
        table[np.arange(self.width) < counts[:, None]] = flat
        if not np.array_equal(table, self.mirror):
            self.host_tables.numpy()[:] = table
            self.tables.copy_(self.host_tables, non_blocking=True)
            self.mirror = table

    def run(self) -> torch.Tensor:
        """Replays the step (capturing it on first use); returns the batch's last-position logits."""
        if self.graph is None:
            runner = self.runner
            stream = runner._capture_stream()
            cur = torch.cuda.current_stream(runner.device)
            stream.wait_stream(cur)
            with torch.cuda.stream(stream):
                for _ in range(2):  # warm-up: libraries pick kernels, scratch is allocated
                    self._body()
            cur.wait_stream(stream)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, pool=runner._graph_pool, stream=stream):
                self.logits = self._body()
            runner.graph_captures += 1
        self.graph.replay()
        return self.logits[:self.rows]


def _seq_field(seq, name, default=None):
    if isinstance(seq, dict):
        return seq.get(name, default)
    return getattr(seq, name, default)


def _set_seq_field(seq, name, value):
    if isinstance(seq, dict):
        seq[name] = value
    elif hasattr(seq, name):
        setattr(seq, name, value)


class KernelPagedManualDecode:
    """Paged decode runner over the HIP kernels (reference integration.py:211-731).

    prefill(seq): Hugging Face forward over the prompt, then the owned K/V
    blocks are written into the pool with paged_prefill_copy (prefix modes
    "off", "share", "full" as in the reference). In "full" mode with a cached
    prefix (and paged_prefill, the default) only the suffix is forwarded, with
    paged_prefill_attention_forward patched in: its K/V go straight into the
    sequence's blocks and its attention reads the prefix from the pool. decode_step(seqs): one
    batched forward with paged_decode_attention_forward patched into every
    attention module, so each layer runs the fused RoPE + K/V write and the
    batched paged attention kernel. With use_graphs (the default) the forward
    is captured once per (batch-size bucket, table width) as a HIP graph over
    persistent device tables and lengths (graph_batch_size: the rows past the
    batch are zero-length padding), and each step replays it; at most
    max_graphs graphs are kept, sharing one capture stream and memory pool,
    so a batch that changes every step, as under continuous batching
    (reference engine/scheduler/continuous_batching.py:337-476), reuses a
    bounded set of graphs. The step
    makes one device-to-host transfer (tokens and top-1/top-2 margins
    together) instead of the reference's per-sequence logits copies
    (:643-651); `last_logits` stays on the device.
    """

    def __init__(
        self,
        model: nn.Module,
        tokenizer: Any = None,
        block_size: int = 16,
        num_blocks: Optional[int] = None,
        gpu_memory_utilization: float = 0.65,
        device: str = "cuda",
        dtype: torch.dtype = torch.float16,
        debug_prefix_cache: bool = False,
        prefix_mode: str = "off",
        use_graphs: bool = True,
        paged_prefill: bool = True,
        fuse_layers: bool = True,
        max_graphs: int = 32,
    ):
        if prefix_mode not in ("off", "share", "full"):
            raise ValueError(f"Unsupported prefix_mode {prefix_mode!r}; expected 'off', 'share', or 'full'.")
        self.model = model
        self.tokenizer = tokenizer
        self.block_size = block_size
        self.device = torch.device(device)
        self.dtype = dtype
        self.debug_prefix_cache = debug_prefix_cache
        self.prefix_mode = prefix_mode
        config = model.config
        self.num_layers = getattr(config, "num_hidden_layers", 24)
        self.num_kv_heads = getattr(config, "num_key_value_heads", 2)
        self.head_dim = getattr(config, "head_dim", None) or (
            config.hidden_size // config.num_attention_heads)
        if num_blocks is None:
            from engine.memory.block_allocator import compute_num_blocks
            num_blocks = max(1, compute_num_blocks(config, block_size, gpu_memory_utilization,
                                                   self.device, dtype))
        self.num_blocks = num_blocks
        self.pool = PhysicalBlockPool(num_blocks=num_blocks, block_size=block_size,
                                      num_layers=self.num_layers, num_kv_heads=self.num_kv_heads,
                                      head_dim=self.head_dim, dtype=dtype, device=self.device)
        self.allocator = BlockAllocator(num_blocks=num_blocks)
        self._grad_probed = False
        # Batched decode steps replay captured HIP graphs, one per (batch-size
        # bucket, table width rounded up to a multiple of 64 blocks), at most
        # max_graphs of them (least recently used dropped first), all captured
        # on one stream into one memory pool.
        self.use_graphs = use_graphs
        self.max_graphs = max(1, int(max_graphs))
        self._graphs: "OrderedDict[tuple, _DecodeGraph]" = OrderedDict()
        self._graph_stream: Optional[torch.cuda.Stream] = None
        self._graph_pool = None
        self.graph_captures = 0
        # "full" prefix mode: forward the suffix through the paged prefill
        # kernel over the pool (True) or, as the reference does, through
        # transformers' attention over a DynamicCache copy of the prefix.
        self.paged_prefill = paged_prefill
        # Decode steps run each decoder layer as fused_decoder_layer_forward
        # (merged q/k/v and gate/up GEMMs, one-launch RMSNorm and SwiGLU,
        # residual adds inside the GEMMs).
        self.fuse_layers = fuse_layers and dtype == torch.float16
        if self.fuse_layers:
            prepare_fused_layers(model)

    def _capture_stream(self) -> torch.cuda.Stream:
        if self._graph_stream is None:
            self._graph_stream = torch.cuda.Stream(self.device)
            self._graph_pool = torch.cuda.graph_pool_handle()
        return self._graph_stream

    def _decode_graph(self, n: int, width: int) -> _DecodeGraph:
        key = (graph_batch_size(n), width)
        graph = self._graphs.get(key)
        if graph is None:
            graph = self._graphs[key] = _DecodeGraph(self, *key)
            while len(self._graphs) > self.max_graphs:
                self._graphs.popitem(last=False)
        else:
            self._graphs.move_to_end(key)
        return graph

    # -- prefill -----------------------------------------------------------------
    def _copy_prefill_kv(self, pkv: Any, block_table: Any, prompt_len: int, skip_blocks: int = 0) -> None:
        """Write the owned prompt blocks of every layer (reference :278-326)."""
        start_token = skip_blocks * self.block_size
        if start_token >= prompt_len:
            return
        total_blocks = (prompt_len + self.block_size - 1) // self.block_size
        if total_blocks - skip_blocks <= 0:
            return
        ids = torch.tensor(block_table.physical_block_ids[skip_blocks:total_blocks],
                           dtype=torch.int32, device=self.device)
        for layer_idx in range(self.num_layers):
            if hasattr(pkv, "layers"):
                keys, values = pkv.layers[layer_idx].keys, pkv.layers[layer_idx].values
            else:
                keys, values = pkv[layer_idx][0], pkv[layer_idx][1]
            k_src = keys[0, :, start_token:prompt_len, :].permute(1, 0, 2)
            v_src = values[0, :, start_token:prompt_len, :].permute(1, 0, 2)
            paged_prefill_copy(k_src, v_src, self.pool.k_cache[layer_idx],
                               self.pool.v_cache[layer_idx], ids, prompt_len - start_token)

    def _compare_cached_prefill_kv(self, pkv: Any, block_table: Any, cached_tokens: int) -> None:
        """Log, per layer, how far the pool's cached prefix rows are from a fresh prefill's K/V.

        The reference's debug_prefix_cache diagnostic (integration.py:328-362,
        called at :490-491): the largest |fresh - stored| over the cached
        tokens' keys and values, compared in fp32 after casting the fresh rows
        to the pool dtype, logged as "Prefix-cache KV comparison layer=%d
        max_abs_difference=%g (cached_tokens=%d)". Here every layer's maximum
        is formed on the device and all of them come back in one transfer.
        """
        nb = cached_tokens // self.block_size
        ids = torch.tensor(block_table.physical_block_ids[:nb], dtype=torch.long, device=self.device)
        worst = []
        for layer_idx in range(self.num_layers):
            if hasattr(pkv, "layers"):
                keys, values = pkv.layers[layer_idx].keys, pkv.layers[layer_idx].values
            else:
                keys, values = pkv[layer_idx][0], pkv[layer_idx][1]
            diffs = []
            for fresh, pool in ((keys, self.pool.k_cache[layer_idx]),
                                (values, self.pool.v_cache[layer_idx])):
                # [1, Hkv, T, D] -> [cached, Hkv, D]; pool rows of the cached blocks, in order.
                f = fresh[0, :, :cached_tokens, :].permute(1, 0, 2).to(self.dtype).float()
                st = pool.index_select(0, ids).flatten(0, 1)[:cached_tokens].float()
                diffs.append((f - st).abs().amax())
            worst.append(torch.stack(diffs).amax())
        for layer_idx, diff in enumerate(torch.stack(worst).tolist()):
            logger.info("Prefix-cache KV comparison layer=%d max_abs_difference=%g "
                        "(cached_tokens=%d)", layer_idx, diff, cached_tokens)

    def _build_cached_prefix(self, block_table: Any, cached_tokens: int):
        """DynamicCache holding the cached prefix blocks (reference :364-392)."""
        from transformers.cache_utils import DynamicCache, DynamicLayer

        cache = DynamicCache()
        nb = cached_tokens // self.block_size
        ids = torch.tensor(block_table.physical_block_ids[:nb], dtype=torch.long, device=self.device)
        for layer_idx in range(self.num_layers):
            key = self.pool.k_cache[layer_idx].index_select(0, ids).flatten(0, 1)
            value = self.pool.v_cache[layer_idx].index_select(0, ids).flatten(0, 1)
            layer = DynamicLayer()
            layer.keys = key.permute(1, 0, 2).unsqueeze(0).contiguous()
            layer.values = value.permute(1, 0, 2).unsqueeze(0).contiguous()
            layer.is_initialized = True
            cache.layers.append(layer)
        return cache

    @torch.inference_mode()
    def prefill(self, seq: Any, allocator: Any = None) -> int:
        """Single-sequence prefill; the scheduler has allocated the blocks (reference :394-516)."""
        ids = _seq_field(seq, "prompt_token_ids")
        if ids:
            input_ids = torch.tensor([list(ids)], dtype=torch.long, device=self.device)
        else:
            prompt = _seq_field(seq, "prompt")
            if not prompt or self.tokenizer is None:
                raise ValueError(f"Unable to extract prompt or prompt_token_ids from sequence: {seq}")
            input_ids = self.tokenizer(prompt, return_tensors="pt").input_ids.to(self.device)
            _set_seq_field(seq, "prompt_token_ids", input_ids[0].tolist())
        prompt_len = input_ids.shape[1]
        block_table = _seq_field(seq, "block_table")
        if block_table is None:
            raise RuntimeError("prefill() requires seq.block_table to be pre-populated by the scheduler.")
        cached = _seq_field(seq, "num_cached_tokens", 0) or 0
        if cached < 0 or cached > prompt_len or cached % self.block_size:
            raise ValueError(f"num_cached_tokens={cached} must be a full-block prefix within "
                             f"prompt_len={prompt_len} (block_size={self.block_size}).")
        if cached // self.block_size > len(block_table.physical_block_ids):
            raise ValueError("num_cached_tokens exceeds the number of blocks in the sequence table.")
        positions = torch.arange(cached, prompt_len, device=self.device).unsqueeze(0)
        if self.prefix_mode == "full" and cached and self.paged_prefill and cached < prompt_len:
            # Each layer writes the suffix's K/V into the sequence's own blocks
            # and attends over the pool; nothing is left to copy afterwards.
            ctx = PagedPrefillContext(self.pool, list(block_table.physical_block_ids), cached,
                                      prompt_len, self.block_size)
            with patch_paged_attention(self.model, ctx):
                out = self.model(input_ids=input_ids[:, cached:], position_ids=positions,
                                 use_cache=False, logits_to_keep=1)
        else:
            if self.prefix_mode == "full" and cached:
                prefix = self._build_cached_prefix(block_table, cached)
                out = self.model(
                    input_ids=input_ids[:, cached:],
                    attention_mask=torch.ones((1, prompt_len), dtype=torch.long, device=self.device),
                    position_ids=positions, past_key_values=prefix, use_cache=True,
                    logits_to_keep=1)
            else:
                out = self.model(input_ids=input_ids, use_cache=True, logits_to_keep=1)
                if self.debug_prefix_cache and cached:
                    self._compare_cached_prefill_kv(out.past_key_values, block_table, cached)
            self._copy_prefill_kv(out.past_key_values, block_table, prompt_len,
                                  skip_blocks=cached // self.block_size)
        logits = out.logits[:, -1, :]
        top2 = torch.topk(logits[0], k=2).values.double()
        # float64 holds every token id exactly; one transfer for id and margin.
        tok_margin = torch.stack([torch.argmax(logits[0]).double(), top2[0] - top2[1]]).tolist()
        _set_seq_field(seq, "last_logits", logits[0].detach())
        _set_seq_field(seq, "last_logit_margin", float(tok_margin[1]))
        return int(tok_margin[0])

    # -- decode ------------------------------------------------------------------
    @torch.inference_mode()
    def decode_step(self, seqs: List[Any], allocator: Any = None) -> List[int]:
        """One batched decode step for the running sequences (reference :518-653)."""
        n = len(seqs)
        if n == 0:
            return []
        allocator = allocator or self.allocator
        if not self._grad_probed:
            self._grad_probed = True
            assert not torch.is_grad_enabled(), "decode_step must run under torch.inference_mode()"
        seq_lens: List[int] = []
        tables: List[Any] = []
        last_tokens: List[int] = []
        for seq in seqs:
            bt = _seq_field(seq, "block_table")
            if bt is None:
                raise ValueError("Sequence must provide a block_table attribute or dict key.")
            widx = bt.num_tokens // self.block_size
            if widx >= len(bt.physical_block_ids):
                raise AssertionError(f"Decode write for seq {_seq_field(seq, 'seq_id', '?')} has no "
                                     f"allocated block at logical index {widx}.")
            wid = bt.physical_block_ids[widx]
            if allocator.ref_counts.get(wid, 0) > 1:
                raise AssertionError(f"Decode write for seq {_seq_field(seq, 'seq_id', '?')} would "
                                     f"modify shared block {wid} with ref_count "
                                     f"{allocator.ref_counts[wid]}.")
            bt.num_tokens += 1
            seq_lens.append(bt.num_tokens)
            tables.append(bt)
            last = _seq_field(seq, "last_token_id")
            if last is None:
                gen = _seq_field(seq, "generated_ids")
                if not gen:
                    raise ValueError("Sequence must provide last_token_id or non-empty generated_ids.")
                last = gen[-1]
            last_tokens.append(int(last))
        if self.use_graphs:
            rows = [bt.physical_block_ids for bt in tables]
            width = max(64, -(-max(len(r) for r in rows) // 64) * 64)
            graph = self._decode_graph(n, width)
            graph.load(last_tokens, seq_lens, rows)
            logits = graph.run().clone()  # the graph's output buffer is reused by the next step
        else:
            input_ids = torch.tensor(last_tokens, dtype=torch.long, device=self.device).unsqueeze(1)
            position_ids = torch.tensor([[L - 1] for L in seq_lens], dtype=torch.long,
                                        device=self.device)
            ctx = PagedAttentionContext(self.pool, tables, seq_lens, self.block_size, True)
            with patch_paged_attention(self.model, ctx, fuse_layers=self.fuse_layers):
                out = self.model(input_ids=input_ids, position_ids=position_ids, use_cache=False)
            logits = out.logits[:, -1, :]
        if logits.dtype == torch.float16 and logits.stride(-1) == 1:
            # torch.argmax and torch.topk(k=2) in one launch (their three
            # multi-block reductions take about 0.17 ms at batch 128).
            idx, top = greedy_top2(logits)
            top2 = top.double()
            both = torch.stack([idx.double(), top2[:, 0] - top2[:, 1]])
        else:
            top2 = torch.topk(logits, k=2, dim=-1).values.double()
            both = torch.stack([torch.argmax(logits, dim=-1).double(), top2[:, 0] - top2[:, 1]])
        # float64 holds every token id exactly: tokens and margins in one transfer.
        toks, margins = both.tolist()
        for seq, row, margin in zip(seqs, logits.detach().unbind(0), margins):
            _set_seq_field(seq, "last_logits", row)
            _set_seq_field(seq, "last_logit_margin", float(margin))
        return [int(t) for t in toks]

    @torch.inference_mode()
    def generate(self, prompt: Any, max_new_tokens: int = 16, allocator: Any = None,
                 block_table: Any = None, return_logits_history: bool = False):
        """Single-sequence greedy generation through the paged decode path (reference :655-731).

        `prompt` is a string (needs a tokenizer) or a list of token ids.
        """
        alloc = allocator or self.allocator
        if isinstance(prompt, str):
            input_ids = self.tokenizer(prompt, return_tensors="pt").input_ids.to(self.device)
        else:
            input_ids = torch.tensor([list(prompt)], dtype=torch.long, device=self.device)
        prompt_len = input_ids.shape[1]
        if block_table is None:
            block_table = BlockTable(seq_id=0, block_size=self.block_size)
        while len(block_table.physical_block_ids) < (prompt_len + self.block_size - 1) // self.block_size:
            block_table.physical_block_ids.append(alloc.allocate())
        block_table.num_tokens = prompt_len
        out = self.model(input_ids=input_ids, use_cache=True)
        self._copy_prefill_kv(out.past_key_values, block_table, prompt_len)
        next_token = torch.argmax(out.logits[:, -1, :], dim=-1, keepdim=True)
        generated = [int(next_token.item())]
        history = [out.logits[:, -1, :]]
        seq_len = prompt_len
        for _ in range(1, max_new_tokens):
            seq_len += 1
            if not block_table.last_block_has_space():
                block_table.physical_block_ids.append(alloc.allocate())
            block_table.num_tokens += 1
            ctx = PagedAttentionContext(self.pool, [block_table], [seq_len], self.block_size, True)
            pos = torch.tensor([[seq_len - 1]], dtype=torch.long, device=self.device)
            with patch_paged_attention(self.model, ctx, fuse_layers=self.fuse_layers):
                step = self.model(input_ids=next_token, position_ids=pos, use_cache=False)
            logits = step.logits[:, -1, :]
            history.append(logits)
            next_token = torch.argmax(logits, dim=-1, keepdim=True)
            generated.append(int(next_token.item()))
        if return_logits_history:
            return generated, history
        return generated
