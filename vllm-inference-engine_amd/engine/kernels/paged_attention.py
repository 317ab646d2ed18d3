"""Paged decode attention on MI355X: the reference's Python operator API over HIP kernels.

Same entry points, argument meaning, asserts and return values as the
reference module engine/kernels/paged_attention.py; every compute call runs a
hand-written gfx950 kernel from libpa_gfx950.so (C ABI in
include/paged_attention.h). There is no CPU or Triton path: the kernels need
CUDA(HIP) tensors, exactly as the reference's Triton entry points assert.

Layouts (reference paged_attention.py:30-37, engine/memory/block_allocator.py:101):
  q        [num_seqs, num_q_heads, head_dim] fp16
  k_cache  [num_blocks, block_size, num_kv_heads, head_dim] fp16 (v_cache alike)
  block_tables [num_seqs, max_blocks_per_seq] int32, seq_lens [num_seqs] int32
Query head h reads kv head h // (num_q_heads // num_kv_heads).

Differences from the reference, all on inputs the reference leaves undefined:
  * seq_len 0 gives a zero output row (the Triton kernels divide 0 by 0);
  * sequence lengths beyond the table width are clamped to it and block ids
    outside the pool are clamped into it, so a malformed table cannot make the
    kernel read outside the pool.
"""
from __future__ import annotations

import math
from typing import Any, Sequence

import numpy as np
import torch

from . import _native

__all__ = [
    "paged_attention_decode",
    "paged_attention_decode_v1",
    "paged_attention_decode_v2",
    "paged_attention_decode_batched",
    "paged_attention_prefill",
    "pad_block_tables",
]


def _q_ready(q: torch.Tensor) -> torch.Tensor:
    """q with unit head_dim stride, 8-element aligned strides and a 16-byte aligned base."""
    ok = (q.stride(-1) == 1 and all(s % 8 == 0 for s in q.stride()[:-1])
          and q.data_ptr() % 16 == 0)
    return q if ok else q.contiguous()


_ws_sizes: dict[tuple, int] = {}


class _NoOp:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NOOP = _NoOp()


def _on_device(dev: torch.device):
    """Make dev the current HIP device for the launch (a no-op when it already is)."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return _NOOP
    return torch.cuda.device(dev)


def paged_attention_decode_batched(
    q: torch.Tensor,            # [num_seqs, num_q_heads, head_dim] (fp16, cuda)
    k_cache: torch.Tensor,      # [num_blocks, block_size, num_kv_heads, head_dim] (fp16, cuda)
    v_cache: torch.Tensor,      # [num_blocks, block_size, num_kv_heads, head_dim] (fp16, cuda)
    block_tables: torch.Tensor, # [num_seqs, max_blocks_per_seq] (int32, cuda)
    seq_lens: torch.Tensor,     # [num_seqs] (int32, cuda)
    scale: float,
) -> torch.Tensor:
    """Batched GQA paged decode attention (reference paged_attention.py:634-698).

    One persistent launch covers every sequence: the (sequence, kv-head group)
    pairs are split into equal contiguous ranges of 16-token tiles, one per
    compute unit, and a pair cut by a range boundary is merged by log-sum-exp
    inside the same launch. Asynchronous on the current stream, like the
    Triton launch it replaces; repeated calls return the same bits.
    """
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda
    assert block_tables.is_cuda and seq_lens.is_cuda
    _native.same_device(q, k_cache, v_cache, block_tables, seq_lens)
    assert q.dtype == torch.float16 and k_cache.dtype == torch.float16 and v_cache.dtype == torch.float16
    assert block_tables.dtype == torch.int32 and seq_lens.dtype == torch.int32

    num_seqs, num_q_heads, head_dim = q.shape
    num_blocks, block_size, num_kv_heads, head_dim_k = k_cache.shape
    assert head_dim == head_dim_k, f"Head dimensions must match: {head_dim} vs {head_dim_k}"
    assert num_q_heads % num_kv_heads == 0, (
        f"num_q_heads ({num_q_heads}) must be divisible by num_kv_heads ({num_kv_heads})"
    )
    assert block_tables.shape[0] == num_seqs
    assert seq_lens.shape[0] == num_seqs
    assert v_cache.shape == k_cache.shape, "k_cache and v_cache must have the same shape"
    assert block_tables.dim() == 2 and seq_lens.dim() == 1

    q = _q_ready(q)
    out = torch.empty_like(q)
    if num_seqs == 0:
        return out
    max_blocks = block_tables.shape[1]
    lib = _native.load()
    dev = q.device
    # The workspace size depends on the device's compute-unit count: keyed by
    # device and queried with that device current.
    key = (dev.index, num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks)
    stream = _native.stream_handle(dev)
    with _on_device(dev):
        ws_bytes = _ws_sizes.get(key)
        if ws_bytes is None:
            ws_bytes = _ws_sizes[key] = lib.pa_decode_batched_workspace_bytes(*key[1:])
        status = lib.pa_decode_batched_f16(
            q.data_ptr(), _native.strides_of(q),
            k_cache.data_ptr(), _native.strides_of(k_cache),
            v_cache.data_ptr(), _native.strides_of(v_cache),
            block_tables.data_ptr(), _native.strides_of(block_tables),
            seq_lens.data_ptr(),
            out.data_ptr(), _native.strides_of(out),
            num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, max_blocks,
            float(scale), _native.workspace(ws_bytes, dev, stream, _native.WS_DECODE), ws_bytes,
            stream)
    _native.check(status, "pa_decode_batched_f16")
    return out


def paged_attention_prefill(
    q: torch.Tensor,                # [num_tokens, num_q_heads, head_dim] (fp16, cuda)
    k_cache: torch.Tensor,          # [num_blocks, block_size, num_kv_heads, head_dim]
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,     # [num_seqs, max_blocks_per_seq] (int32, cuda)
    seq_lens: torch.Tensor,         # [num_seqs] (int32, cuda): context length after the new tokens
    query_start_loc: torch.Tensor,  # [num_seqs + 1] (int32, cuda): first q row of each sequence
    max_query_len: int,
    scale: float,
) -> torch.Tensor:
    """Causal attention of each sequence's new tokens over its paged context.

    The attention of the reference's "full" prefix-cache prefill
    (engine/kernels/paged_attention_integration.py:459-482): the uncached prompt
    suffix attends over the cached prefix blocks (:364-392) and itself. The
    new tokens' K/V must already be in the pool. Sequence b owns q rows
    query_start_loc[b] .. query_start_loc[b+1]-1; its new token i sits at
    position seq_lens[b] - n_b + i and sees pool positions 0 .. that position.
    max_query_len (a host int, at least every n_b) sizes the grid, so the
    call never reads device memory on the host. Asynchronous on the current
    stream. When the launch has too few column blocks to fill the GPU, long
    key ranges are split over several workgroups that merge through a
    per-stream scratch buffer (zero-filled once, like the decode one).
    """
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda
    assert block_tables.is_cuda and seq_lens.is_cuda and query_start_loc.is_cuda
    _native.same_device(q, k_cache, v_cache, block_tables, seq_lens, query_start_loc)
    assert q.dtype == torch.float16 and k_cache.dtype == torch.float16 and v_cache.dtype == torch.float16
    assert block_tables.dtype == torch.int32 and seq_lens.dtype == torch.int32
    assert query_start_loc.dtype == torch.int32
    num_tokens, num_q_heads, head_dim = q.shape
    num_blocks, block_size, num_kv_heads, head_dim_k = k_cache.shape
    assert head_dim == head_dim_k, f"Head dimensions must match: {head_dim} vs {head_dim_k}"
    assert num_q_heads % num_kv_heads == 0, (
        f"num_q_heads ({num_q_heads}) must be divisible by num_kv_heads ({num_kv_heads})"
    )
    num_seqs = seq_lens.shape[0]
    assert block_tables.dim() == 2 and block_tables.shape[0] == num_seqs
    assert query_start_loc.dim() == 1 and query_start_loc.shape[0] == num_seqs + 1
    assert v_cache.shape == k_cache.shape, "k_cache and v_cache must have the same shape"
    assert max_query_len >= 0

    q = _q_ready(q)
    out = torch.empty_like(q)
    if num_seqs == 0 or num_tokens == 0 or max_query_len == 0:
        return out
    lib = _native.load()
    dev = q.device
    max_blocks = block_tables.shape[1]
    key = ("prefill", num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks,
           int(max_query_len), dev.index)
    stream = _native.stream_handle(dev)
    with _on_device(dev):
        ws_bytes = _ws_sizes.get(key)
        if ws_bytes is None:
            ws_bytes = _ws_sizes[key] = lib.pa_prefill_attention_workspace_bytes(*key[1:8])
        status = lib.pa_prefill_attention_f16(
            q.data_ptr(), _native.strides_of(q),
            k_cache.data_ptr(), _native.strides_of(k_cache),
            v_cache.data_ptr(), _native.strides_of(v_cache),
            block_tables.data_ptr(), _native.strides_of(block_tables),
            seq_lens.data_ptr(), query_start_loc.data_ptr(), int(max_query_len),
            out.data_ptr(), _native.strides_of(out),
            num_seqs, num_tokens, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
            max_blocks, float(scale), _native.workspace(ws_bytes, dev, stream, _native.WS_PREFILL),
            ws_bytes, stream)
    _native.check(status, "pa_prefill_attention_f16")
    return out


def _single_seq_args(q, k_cache, v_cache, block_table, seq_len):
    assert q.is_cuda and k_cache.is_cuda and v_cache.is_cuda and block_table.is_cuda
    _native.same_device(q, k_cache, v_cache, block_table)
    assert q.dtype == torch.float16 and k_cache.dtype == torch.float16 and v_cache.dtype == torch.float16
    assert block_table.dtype == torch.int32

    num_q_heads, head_dim = q.shape
    num_blocks, block_size, num_kv_heads, head_dim_k = k_cache.shape
    assert head_dim == head_dim_k, f"Head dimensions must match: {head_dim} vs {head_dim_k}"
    assert num_q_heads % num_kv_heads == 0, (
        f"num_q_heads ({num_q_heads}) must be divisible by num_kv_heads ({num_kv_heads})"
    )
    num_blocks_for_seq = (seq_len + block_size - 1) // block_size
    assert block_table.shape[0] >= num_blocks_for_seq, (
        f"block_table size ({block_table.shape[0]}) smaller than needed ({num_blocks_for_seq})"
    )
    assert v_cache.shape == k_cache.shape, "k_cache and v_cache must have the same shape"
    assert block_table.dim() == 1
    return num_q_heads, head_dim, num_blocks, block_size, num_kv_heads


def _single_seq_call(fn_name, ws_name, q, k_cache, v_cache, block_table, seq_len, scale, ws_last,
                     ws_kind):
    seq_len = int(seq_len)
    num_q_heads, head_dim, num_blocks, block_size, num_kv_heads = _single_seq_args(
        q, k_cache, v_cache, block_table, seq_len)
    q = _q_ready(q)
    out = torch.empty_like(q)
    lib = _native.load()
    table_len = block_table.shape[0]
    if table_len == 0:
        # Only reachable with seq_len == 0: nothing to attend to.
        return out.zero_()
    dev = q.device
    stream = _native.stream_handle(dev)
    with _on_device(dev):
        ws_bytes = getattr(lib, ws_name)(num_q_heads, num_kv_heads, head_dim, block_size,
                                         ws_last(table_len, seq_len))
        status = getattr(lib, fn_name)(
            q.data_ptr(), _native.strides_of(q),
            k_cache.data_ptr(), _native.strides_of(k_cache),
            v_cache.data_ptr(), _native.strides_of(v_cache),
            block_table.data_ptr(), int(block_table.stride(0)), table_len, seq_len,
            out.data_ptr(), _native.strides_of(out),
            num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, float(scale),
            _native.workspace(ws_bytes, dev, stream, ws_kind), ws_bytes, stream)
    _native.check(status, fn_name)
    return out


def paged_attention_decode_v1(
    q: torch.Tensor,            # [num_q_heads, head_dim] (fp16, cuda)
    k_cache: torch.Tensor,      # [num_blocks, block_size, num_kv_heads, head_dim] (fp16, cuda)
    v_cache: torch.Tensor,      # [num_blocks, block_size, num_kv_heads, head_dim] (fp16, cuda)
    block_table: torch.Tensor,  # 1D int32 cuda tensor of physical block IDs
    seq_len: int,
    scale: float,
) -> torch.Tensor:
    """Single-sequence two-pass decode attention (reference paged_attention.py:254-305).

    Pass 1 computes every score and their maximum, a denominator pass sums the
    exponentials, pass 2 accumulates the normalised probabilities times V.
    Scores are kept in a workspace, so K is read once rather than three times.
    """
    return _single_seq_call("pa_decode_v1_f16", "pa_decode_v1_workspace_bytes",
                            q, k_cache, v_cache, block_table, seq_len, scale,
                            lambda table_len, n: n, _native.WS_SCORES)


def paged_attention_decode_v2(
    q: torch.Tensor,            # [num_q_heads, head_dim] (fp16, cuda)
    k_cache: torch.Tensor,      # [num_blocks, block_size, num_kv_heads, head_dim] (fp16, cuda)
    v_cache: torch.Tensor,      # [num_blocks, block_size, num_kv_heads, head_dim] (fp16, cuda)
    block_table: torch.Tensor,  # 1D int32 cuda tensor of physical block IDs
    seq_len: int,
    scale: float,
) -> torch.Tensor:
    """Single-sequence online-softmax decode attention (reference paged_attention.py:419-470)."""
    return _single_seq_call("pa_decode_v2_f16", "pa_decode_v2_workspace_bytes",
                            q, k_cache, v_cache, block_table, seq_len, scale,
                            lambda table_len, n: table_len, _native.WS_DECODE)


def pad_block_tables(
    block_tables: Sequence[Sequence[int]] | Sequence[Any],
    device: torch.device | str = "cuda",
) -> torch.Tensor:
    """List of block-id lists (or objects with .physical_block_ids) -> int32 [num_seqs, max(1, max_len)].

    Zero padded, like reference paged_attention.py:473-505; the padding is never
    dereferenced because the kernels stop at each sequence's length. The table
    is assembled on the host and copied to the device in one transfer.
    """
    num_seqs = len(block_tables)
    if num_seqs == 0:
        return torch.empty((0, 0), dtype=torch.int32, device=device)

    raw_lists: list[list[int]] = []
    for bt in block_tables:
        if hasattr(bt, "physical_block_ids"):
            raw_lists.append(list(bt.physical_block_ids))
        elif isinstance(bt, (list, tuple)):
            raw_lists.append(list(bt))
        else:
            raise TypeError(f"Unsupported block table type: {type(bt)}")

    max_len = max((len(l) for l in raw_lists), default=0)
    max_len = max(max_len, 1)
    host = np.zeros((num_seqs, max_len), dtype=np.int32)
    for i, row in enumerate(raw_lists):
        if row:
            host[i, :len(row)] = row
    return torch.from_numpy(host).to(device)


def paged_attention_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: list[list[int]],
    seq_lens: list[int],
    scale: float,
) -> torch.Tensor:
    """List-based decode entry point (reference paged_attention.py:86-99).

    The reference routes this name to its CPU oracle; here the lists are turned
    into device tensors and the batched HIP kernel runs.
    """
    assert q.is_cuda, "paged_attention_decode runs on the GPU only"
    tables = pad_block_tables(block_tables, device=q.device)
    lens = torch.tensor([int(n) for n in seq_lens], dtype=torch.int32, device=q.device)
    return paged_attention_decode_batched(q, k_cache, v_cache, tables, lens, scale)


def default_scale(head_dim: int) -> float:
    """1/sqrt(head_dim), the scale the reference integration falls back to (integration.py:114)."""
    return 1.0 / math.sqrt(head_dim)
