"""Seeded synthetic paged-decode workloads at the shapes the kernels are measured on.

Each generator returns a Workload: fp16 q and K/V pools, int32 block tables and
lengths on the requested device, the same tables/lengths as Python lists, and
the algorithmic byte count one attention call must move.

Values are drawn with a torch.Generator seeded per workload on the target
device, so the same seed gives the same bits on every run of the same device
type. Block tables are slices of a seeded permutation of the pool, so layouts
are shuffled and non-contiguous and last blocks are partial.

Shapes (all fp16, block_size 16 unless stated):
  qwen_layer      B 8, 14 q / 2 kv heads, head_dim 64, 512-block pool,
                  lengths U[1, 512]
  gqa_sweep       B 64, 28 q heads, head_dim 128, kv heads in {28, 14, 7, 4},
                  every length 2048, pool B*128 blocks + 10%
  softmax_stress  B 32, 14 q / 2 kv, head_dim 64, q,k ~ N(0, 8^2), v ~ N(0, 1),
                  lengths from {17, 33, 1023, 2049, 4097}
  long_context    B 256, 14 q / 2 kv, head_dim 64, lengths lognormal with median
                  4096 and sigma 0.5 clipped to [256, 32768]; groups of 8
                  sequences share their first min(64, (L-1)//16) blocks (same
                  physical ids); pool B * ceil(max_len / 16) blocks
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass
class Workload:
    name: str
    q: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # int32 [B, max_blocks]
    seq_lens: torch.Tensor      # int32 [B]
    tables: list                # list[list[int]]
    lens: list                  # list[int]
    scale: float
    unique_slots: int           # distinct (block, row) slots read by one call
    meta: dict = field(default_factory=dict)

    @property
    def num_seqs(self) -> int:
        return self.q.shape[0]

    def algorithmic_bytes(self, unique: bool = True) -> int:
        """K+V at the valid token slots + Q + O + block-table entries + lengths."""
        _, num_q_heads, head_dim = self.q.shape
        num_kv_heads = self.k_cache.shape[2]
        bs = self.k_cache.shape[1]
        slots = self.unique_slots if unique else sum(self.lens)
        kv = 2 * num_kv_heads * head_dim * 2 * slots
        qo = 2 * self.num_seqs * num_q_heads * head_dim * 2
        tables = 4 * sum((n + bs - 1) // bs for n in self.lens)
        return kv + qo + tables + 4 * self.num_seqs


def _randn(shape, gen, device, std=1.0):
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if std != 1.0:
        x.mul_(std)
    return x.to(torch.float16)


def _finish(name, q, k, v, tables, lens, scale, unique_slots, device, meta=None) -> Workload:
    width = max(1, max(len(t) for t in tables))
    host = np.zeros((len(tables), width), dtype=np.int32)
    for i, t in enumerate(tables):
        host[i, :len(t)] = t
    return Workload(
        name=name, q=q, k_cache=k, v_cache=v,
        block_tables=torch.from_numpy(host).to(device),
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=device),
        tables=[list(t) for t in tables], lens=list(lens), scale=scale,
        unique_slots=unique_slots, meta=meta or {})


def _distinct_tables(lens, num_blocks, bs, rng):
    perm = rng.permutation(num_blocks)
    tables, pos = [], 0
    for n in lens:
        nb = (n + bs - 1) // bs
        tables.append(perm[pos:pos + nb].tolist())
        pos += nb
    assert pos <= num_blocks, "pool too small for the requested lengths"
    return tables


def make_random(num_seqs, num_q_heads, num_kv_heads, head_dim, lens, block_size=16,
                num_blocks=None, seed=0, device="cpu", qk_std=1.0, name="random") -> Workload:
    """Generic shuffled-table workload (used by the tests for odd shapes)."""
    rng = np.random.default_rng(seed)
    need = sum((n + block_size - 1) // block_size for n in lens)
    if num_blocks is None:
        num_blocks = need * 2 + 5
    gen = torch.Generator(device=device).manual_seed(seed)
    q = _randn((num_seqs, num_q_heads, head_dim), gen, device, qk_std)
    shape = (num_blocks, block_size, num_kv_heads, head_dim)
    k = _randn(shape, gen, device, qk_std)
    v = _randn(shape, gen, device)
    tables = _distinct_tables(lens, num_blocks, block_size, rng)
    return _finish(name, q, k, v, tables, lens, head_dim ** -0.5, sum(lens), device)


def from_tables(tables, lens, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
                seed=0, device="cpu", name="tables") -> Workload:
    """Workload over given block tables (which may repeat blocks across sequences, as a
    prefix cache's shared prompts do): N(0, 1) q and pool, distinct slots counted once."""
    gen = torch.Generator(device=device).manual_seed(seed)
    q = _randn((len(tables), num_q_heads, head_dim), gen, device)
    shape = (num_blocks, block_size, num_kv_heads, head_dim)
    k = _randn(shape, gen, device)
    v = _randn(shape, gen, device)
    slots = {(t[i // block_size], i % block_size) for t, n in zip(tables, lens) for i in range(n)}
    return _finish(name, q, k, v, tables, lens, head_dim ** -0.5, len(slots), device)


def qwen_layer(device="cpu", seed=0) -> Workload:
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, 513, size=8).tolist()
    w = make_random(8, 14, 2, 64, lens, 16, num_blocks=512, seed=seed, device=device,
                    name="qwen_layer")
    return w


def gqa_sweep(num_kv_heads: int, device="cpu", seed=0) -> Workload:
    B, L = 64, 2048
    num_blocks = int(B * 128 * 1.1)
    return make_random(B, 28, num_kv_heads, 128, [L] * B, 16, num_blocks=num_blocks, seed=seed,
                       device=device, name=f"gqa_sweep_kv{num_kv_heads}")


def softmax_stress(device="cpu", seed=0) -> Workload:
    rng = np.random.default_rng(seed)
    lens = rng.choice([17, 33, 1023, 2049, 4097], size=32).tolist()
    need = sum((n + 15) // 16 for n in lens)
    return make_random(32, 14, 2, 64, lens, 16, num_blocks=need + 64, seed=seed, device=device,
                       qk_std=8.0, name="softmax_stress")


def long_context(device="cpu", seed=0, num_seqs=256, sigma=0.5, group=8,
                 prefix_blocks=64) -> Workload:
    """Batch 256 x ~4k contexts with shared prefixes (the headline decode workload)."""
    rng = np.random.default_rng(seed)
    z = rng.standard_normal(num_seqs)
    lens = np.clip(np.round(4096.0 * np.exp(sigma * z)), 256, 32768).astype(np.int64).tolist()
    bs = 16
    max_len = max(lens)
    num_blocks = num_seqs * ((max_len + bs - 1) // bs)
    perm = rng.permutation(num_blocks).tolist()
    pos = 0
    tables = []
    unique = 0
    for g0 in range(0, num_seqs, group):
        members = list(range(g0, min(g0 + group, num_seqs)))
        shared = [min(prefix_blocks, (lens[i] - 1) // bs) for i in members]
        prefix = perm[pos:pos + max(shared)]
        pos += max(shared)
        for i, s in zip(members, shared):
            nb = (lens[i] + bs - 1) // bs
            private = perm[pos:pos + nb - s]
            pos += nb - s
            tables.append(prefix[:s] + private)
            unique += lens[i] - s * bs
        unique += max(shared) * bs
    assert pos <= num_blocks
    gen = torch.Generator(device=device).manual_seed(seed)
    q = _randn((num_seqs, 14, 64), gen, device)
    shape = (num_blocks, bs, 2, 64)
    k = _randn(shape, gen, device)
    v = _randn(shape, gen, device)
    return _finish("long_context", q, k, v, tables, lens, 64 ** -0.5, unique, device,
                   meta={"sigma": sigma, "group": group, "prefix_blocks": prefix_blocks})


def decode_step_layer(num_seqs=128, device="cpu", seed=0) -> Workload:
    """One layer's attention call in the middle of the batch-128 decode step.

    Qwen2.5-0.5B heads (14 q / 2 kv, head_dim 64), block 16; lengths are the
    decode-step workload's prompts, U[64, 1024], plus 64 generated tokens.
    """
    rng = np.random.default_rng(seed)
    lens = (rng.integers(64, 1025, size=num_seqs) + 64).tolist()
    return make_random(num_seqs, 14, 2, 64, lens, 16, seed=seed, device=device,
                       name=f"decode_step_layer_b{num_seqs}")


# Qwen2.5-0.5B architecture: 24 layers, hidden 896, 14 q / 2 kv heads (head_dim
# 64), SwiGLU MLP 4864, RMSNorm eps 1e-6, RoPE theta 1e6, vocabulary 151936;
# the lm_head is not tied to the embeddings (transformers' Qwen2Config default).
QWEN25_05B = dict(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_hidden_layers=24,
                  num_attention_heads=14, num_key_value_heads=2, max_position_embeddings=32768,
                  rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=False)


def decode_model(device, seed=0, config=None):
    """Random-init (transformers' N(0, 0.02)) Qwen2 causal LM in fp16, eval mode."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(seed)
    with torch.device(device):
        model = Qwen2ForCausalLM(Qwen2Config(**(config or QWEN25_05B)))
    return model.half().eval()


def decode_prompts(seed=0, batch=128, vocab=QWEN25_05B["vocab_size"]) -> list:
    """The decode-step workload's prompts: lengths U[64, 1024], random token ids."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(64, 1025, size=batch)
    return [rng.integers(0, vocab, size=int(n)).tolist() for n in lens]


def gather_subset(w: Workload, seqs: list[int]) -> tuple:
    """Copy the blocks the given sequences read to the CPU with a compact table.

    Returns (q, k_cache, v_cache, tables, lens) on the CPU for an oracle check
    of a few sequences of a workload too large to copy whole.
    """
    ids = sorted({b for i in seqs for b in w.tables[i][:(w.lens[i] + w.k_cache.shape[1] - 1)
                                                      // w.k_cache.shape[1]]})
    remap = {b: j for j, b in enumerate(ids)}
    idx = torch.tensor(ids, dtype=torch.long, device=w.k_cache.device)
    k = w.k_cache.index_select(0, idx).cpu()
    v = w.v_cache.index_select(0, idx).cpu()
    bs = w.k_cache.shape[1]
    tables = [[remap[b] for b in w.tables[i][:(w.lens[i] + bs - 1) // bs]] for i in seqs]
    q = w.q[seqs].cpu()
    return q, k, v, tables, [w.lens[i] for i in seqs]


def lognormal_mean_len(sigma: float = 0.5) -> float:
    return 4096.0 * math.exp(sigma * sigma / 2)
