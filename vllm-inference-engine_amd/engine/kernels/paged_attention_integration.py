"""Per-layer decode attention over the paged pool: K/V write + paged attention.

Mirrors the decode path of the reference module
engine/kernels/paged_attention_integration.py:
  * PagedAttentionContext (reference :29-62): per-step block tables and lengths;
  * paged_decode_attention_forward (reference :65-176): projections, RoPE, the
    new token's K/V written into its block, batched paged attention, o_proj;
  * patch_paged_attention (reference :179-208): binds that forward onto every
    attention module of a model for the duration of a decode step.

The reference writes K/V with a Python loop of two index_put calls per sequence
and a device-to-host `.item()` per sequence per layer (:148-161). Here the
write is one HIP launch, paged_kv_write(), that computes every slot on the
device from the block tables and lengths, so a decode step has no host syncs.
"""
from __future__ import annotations

import math
from contextlib import contextmanager
from typing import Any, Callable, List, Optional, Tuple, Union

import torch
import torch.nn as nn

from . import _native
from .paged_attention import _on_device, pad_block_tables, paged_attention_decode_batched

__all__ = [
    "PagedAttentionContext",
    "paged_kv_write",
    "paged_decode_attention_forward",
    "patch_paged_attention",
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


def paged_decode_attention_forward(
    self: nn.Module,
    hidden_states: torch.Tensor,
    position_embeddings: Tuple[torch.Tensor, torch.Tensor],
    attention_mask: Optional[torch.Tensor] = None,
    past_key_values: Any = None,
    **kwargs: Any,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Drop-in Qwen2Attention.forward for one decode step (reference integration.py:65-176).

    q/k/v projections, RoPE, the new K/V written into the pool with one
    paged_kv_write launch, batched paged attention over L_b tokens (the write
    precedes the read, as in the reference), then o_proj.
    """
    ctx: Optional[PagedAttentionContext] = getattr(self, "_paged_attention_context", None)
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

    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    layer_idx = self.layer_idx
    input_shape = hidden_states.shape[:-1]  # [batch, 1]
    hidden_shape = (*input_shape, -1, self.head_dim)

    query_states = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    key_states = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)

    cos, sin = position_embeddings
    query_states, key_states = apply_rotary_pos_emb(query_states, key_states, cos, sin)

    scale = self.scaling if hasattr(self, "scaling") else 1.0 / math.sqrt(self.head_dim)
    pool = ctx.pool
    k_cache = pool.k_cache[layer_idx]
    v_cache = pool.v_cache[layer_idx]

    if not ctx.is_batched:
        bt = ctx.block_table_tensor
        seq_len = ctx.single_seq_len
        paged_kv_write(key_states, value_states, k_cache, v_cache, bt, seq_len)
        seq_lens_t = torch.tensor([seq_len], dtype=torch.int32, device=pool.device)
        bt_2d = bt.unsqueeze(0)
    else:
        bt_2d = ctx.padded_block_tables
        seq_lens_t = ctx.seq_lens_tensor
        paged_kv_write(key_states, value_states, k_cache, v_cache, bt_2d, seq_lens_t)

    attn_output = paged_attention_decode_batched(
        q=query_states.squeeze(2),
        k_cache=k_cache,
        v_cache=v_cache,
        block_tables=bt_2d,
        seq_lens=seq_lens_t,
        scale=scale,
    )
    attn_output = attn_output.reshape(*input_shape, -1).contiguous()
    attn_output = self.o_proj(attn_output)
    return attn_output, None


@contextmanager
def patch_paged_attention(model: nn.Module, context: PagedAttentionContext):
    """Temporarily bind paged_decode_attention_forward on every attention module (reference :179-208)."""
    attn_modules: List[Tuple[nn.Module, Callable]] = []
    for module in model.modules():
        if all(hasattr(module, n) for n in ("q_proj", "k_proj", "v_proj", "o_proj")):
            orig_fwd = module.forward
            module._orig_attention_forward = orig_fwd
            module._paged_attention_context = context
            module.forward = paged_decode_attention_forward.__get__(module, module.__class__)
            attn_modules.append((module, orig_fwd))
    try:
        yield context
    finally:
        for module, orig_fwd in attn_modules:
            module.forward = orig_fwd
            if hasattr(module, "_orig_attention_forward"):
                delattr(module, "_orig_attention_forward")
            if hasattr(module, "_paged_attention_context"):
                delattr(module, "_paged_attention_context")
