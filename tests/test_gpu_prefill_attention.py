"""Parity of the paged prefill attention kernel with the CPU oracle (needs an MI355X).

The kernel computes the attention of the reference's "full" prefix-cache
prefill (engine/kernels/paged_attention_integration.py:459-482): each
sequence's new tokens attend causally over its cached prefix blocks and
themselves, all read from the pool. Gate: max |kernel - oracle| <= 2e-3 with
the oracle (prefix_prefill_attention) in fp32 on the same fp16 inputs, as for
the decode kernels.
"""
from __future__ import annotations

import random

import pytest
import torch

from engine.kernels import _native
from engine.kernels.paged_attention import (
    paged_attention_decode_batched,
    paged_attention_prefill,
    pad_block_tables,
)
from oracle.paged_attention_oracle import prefix_prefill_attention

pytestmark = pytest.mark.gpu

TOL = 2e-3


def build(hq, hkv, d, bs, ctx_lens, q_lens, seed, device, slack=3):
    """Pool holding every position of each sequence (prefix and new tokens) in shuffled
    blocks of a random-filled pool; q rows of the new tokens packed sequence by sequence."""
    g = torch.Generator().manual_seed(seed)
    rnd = random.Random(seed)
    nlog = sum((n + bs - 1) // bs for n in ctx_lens)
    nphys = nlog * slack + 4
    kc = torch.randn(nphys, bs, hkv, d, generator=g).half()
    vc = torch.randn(nphys, bs, hkv, d, generator=g).half()
    ids = rnd.sample(range(nphys), nlog)
    tables, pos = [], 0
    for n in ctx_lens:
        nb = (n + bs - 1) // bs
        tables.append(ids[pos:pos + nb])
        pos += nb
    q = torch.randn(sum(q_lens), hq, d, generator=g).half()
    qsl = [0]
    for n in q_lens:
        qsl.append(qsl[-1] + n)
    return dict(
        q=q, kc=kc, vc=vc, tables=tables, lens=list(ctx_lens), qlens=list(q_lens),
        qd=q.to(device), kd=kc.to(device), vd=vc.to(device),
        btd=pad_block_tables(tables, device=device),
        lensd=torch.tensor(ctx_lens, dtype=torch.int32, device=device),
        qsld=torch.tensor(qsl, dtype=torch.int32, device=device))


def run(c, scale, q=None):
    return paged_attention_prefill(c["qd"] if q is None else q, c["kd"], c["vd"], c["btd"],
                                   c["lensd"], c["qsld"], max(c["qlens"]), scale)


def oracle(c, scale):
    return prefix_prefill_attention(c["q"], c["kc"], c["vc"], c["tables"], c["lens"], c["qlens"],
                                     scale, torch.float32)


def max_err(got, want):
    return (got.float().cpu() - want.float()).abs().max().item()


@pytest.mark.parametrize("hq,hkv,d,bs", [
    (14, 2, 64, 16),    # Qwen2.5-0.5B heads
    (28, 4, 128, 16),   # g = 7 at head_dim 128
    (8, 8, 128, 16),    # g = 1
    (32, 2, 32, 16),    # g = 16, head_dim 32
    (16, 2, 256, 16),   # head_dim 256
    (14, 2, 64, 8),     # blocks smaller than a 16-key sub-tile
    (14, 2, 64, 32),
    (6, 2, 64, 5),      # odd block size, g = 3
])
def test_matches_oracle(cuda_device, hq, hkv, d, bs):
    # Cached prefix + suffix, whole prompts (context == new tokens), single new tokens,
    # and a sequence with no new tokens, in one launch.
    ctx = [100, 17, 1000, 64, 33, 300]
    new = [36, 17, 200, 1, 0, 300]
    c = build(hq, hkv, d, bs, ctx, new, seed=hq * 1000 + d + bs, device=cuda_device)
    scale = d ** -0.5
    out = run(c, scale)
    err = max_err(out, oracle(c, scale))
    print(f"[prefill] hq={hq} hkv={hkv} d={d} bs={bs} max_err={err:.2e}", flush=True)
    assert err <= TOL


def test_long_context_long_suffix(cuda_device):
    c = build(14, 2, 64, 16, [4096, 2500], [512, 700], seed=11, device=cuda_device)
    out = run(c, 0.125)
    err = max_err(out, oracle(c, 0.125))
    print(f"[prefill] long max_err={err:.2e}", flush=True)
    assert err <= TOL


def test_one_new_token_matches_decode_kernel(cuda_device):
    c = build(14, 2, 64, 16, [1, 40, 513, 2048], [1, 1, 1, 1], seed=12, device=cuda_device)
    pre = run(c, 0.125)
    dec = paged_attention_decode_batched(c["qd"], c["kd"], c["vd"], c["btd"], c["lensd"], 0.125)
    assert max_err(pre, dec.cpu()) <= TOL
    assert max_err(pre, oracle(c, 0.125)) <= TOL


def test_strided_query_view(cuda_device):
    c = build(14, 2, 64, 16, [90, 200], [30, 64], seed=13, device=cuda_device)
    base = run(c, 0.125)
    big = torch.zeros(c["qd"].shape[0], 14, 2, 64, dtype=torch.float16, device=cuda_device)
    big[:, :, 1] = c["qd"]
    out = run(c, 0.125, q=big[:, :, 1])
    assert torch.equal(out, base)


def test_block_relocation_invariance(cuda_device):
    """The same K/V at other physical blocks (another pool order) gives the same bits."""
    c = build(14, 2, 64, 16, [150, 47], [50, 47], seed=14, device=cuda_device)
    base = run(c, 0.125)
    nb = c["kc"].shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(3))
    inv = torch.empty(nb, dtype=torch.long)
    inv[perm] = torch.arange(nb)
    k2, v2 = c["kd"][perm.to(cuda_device)], c["vd"][perm.to(cuda_device)]
    t2 = pad_block_tables([[int(inv[b]) for b in t] for t in c["tables"]], device=cuda_device)
    out = paged_attention_prefill(c["qd"], k2, v2, t2, c["lensd"], c["qsld"], 50, 0.125)
    assert torch.equal(out, base)


def test_repeatable_bits(cuda_device):
    c = build(14, 2, 64, 16, [1200, 300], [400, 300], seed=15, device=cuda_device)
    a = run(c, 0.125)
    for _ in range(3):
        assert torch.equal(run(c, 0.125), a)


def test_context_shorter_than_new_tokens(cuda_device):
    """Rows whose position would be negative are zeros; the others see positions 0..p."""
    c = build(14, 2, 64, 16, [3], [5], seed=16, device=cuda_device)
    out = run(c, 0.125).cpu()
    assert torch.count_nonzero(out[:2]) == 0
    sub = dict(c, q=c["q"][2:], qlens=[3])
    assert max_err(out[2:], oracle(sub, 0.125)) <= TOL


def test_query_rows_placed_by_query_start_loc(cuda_device):
    c = build(14, 2, 64, 16, [40], [8], seed=17, device=cuda_device)
    # 12 query rows, but the sequence owns rows 2..9 only.
    q = torch.zeros(12, 14, 64, dtype=torch.float16, device=cuda_device)
    q[2:10] = c["qd"]
    qsl = torch.tensor([2, 10], dtype=torch.int32, device=cuda_device)
    out = paged_attention_prefill(q, c["kd"], c["vd"], c["btd"], c["lensd"], qsl, 8, 0.125)
    assert max_err(out[2:10], oracle(c, 0.125)) <= TOL


def test_single_sequence_long_prefix_split(cuda_device):
    """One sequence (the reference prefills one at a time): its few column blocks are split
    along the keys over several workgroups, merged in the kernel."""
    c = build(14, 2, 64, 16, [8192], [1024], seed=18, device=cuda_device)
    out = run(c, 0.125)
    err = max_err(out, oracle(c, 0.125))
    print(f"[prefill] single long max_err={err:.2e}", flush=True)
    assert err <= TOL
    for _ in range(2):
        assert torch.equal(run(c, 0.125), out)


@pytest.mark.parametrize("d,bs,ragged", [(64, 16, False), (32, 16, False), (64, 32, True),
                                         (64, 8, True), (32, 32, True)])
def test_both_wavefront_forms(cuda_device, d, bs, ragged):
    """Up to head_dim 64 a block of 128 columns runs as four wavefronts of two column groups
    when the launch is not split and the new tokens are at most half the table's positions,
    else as eight wavefronts of one group. A larger max_query_len (still a valid bound) selects
    the second form for the same inputs; both match the oracle and each other. Block 16 takes
    the kernels specialised for it, the other sizes the general ones; ragged batches leave
    some column blocks empty and cut others short."""
    ctx = [1536, 1500, 1400, 1536, 1300, 1536, 1536, 1200] if ragged else [1536] * 8
    new = [512, 300, 512, 450, 512, 17, 512, 512] if ragged else [512] * 8
    c = build(14, 2, d, bs, ctx, new, seed=25 + d + bs, device=cuda_device)
    scale = d ** -0.5
    four = run(c, scale)  # 448 workgroups, no split, 2 x 512 <= 1536
    eight = paged_attention_prefill(c["qd"], c["kd"], c["vd"], c["btd"], c["lensd"], c["qsld"],
                                    1024, scale)  # 2 x 1024 > 1536: 896 workgroups, half empty
    want = oracle(c, scale)
    e4, e8 = max_err(four, want), max_err(eight, want)
    print(f"[prefill] d={d} bs={bs} ragged={ragged} four-wavefront max_err={e4:.2e} "
          f"eight-wavefront {e8:.2e}", flush=True)
    assert e4 <= TOL and e8 <= TOL
    assert (four.float() - eight.float()).abs().max().item() <= TOL
    assert torch.equal(run(c, scale), four)


def test_long_split_pieces_four_wavefronts(cuda_device):
    """At head_dim 64, key ranges split into pieces of 48 tiles or more run as four wavefronts
    of two column groups (192 column blocks split two ways, 48 tiles each); a larger
    max_query_len gives 384 blocks and no split. Both match the oracle and each other."""
    c = build(16, 8, 64, 16, [12288, 4000, 12000], [512, 512, 300], seed=31, device=cuda_device)
    split = run(c, 0.125)
    whole = paged_attention_prefill(c["qd"], c["kd"], c["vd"], c["btd"], c["lensd"], c["qsld"],
                                    1024, 0.125)
    want = oracle(c, 0.125)
    es, ew = max_err(split, want), max_err(whole, want)
    print(f"[prefill] long split pieces max_err={es:.2e}, unsplit {ew:.2e}", flush=True)
    assert es <= TOL and ew <= TOL
    assert (split.float() - whole.float()).abs().max().item() <= TOL
    for _ in range(2):
        assert torch.equal(run(c, 0.125), split)


def test_split_counters_return_to_zero(cuda_device):
    c = build(28, 4, 128, 16, [3000, 10], [700, 10], seed=19, device=cuda_device)
    run(c, 128 ** -0.5)
    torch.cuda.synchronize()
    stream = _native.stream_handle(cuda_device)
    ws = _native._workspaces.get((cuda_device.index, stream, _native.WS_PREFILL))
    assert ws is not None, "this launch should have split its key ranges"
    lib = _native.load()
    need = lib.pa_prefill_attention_workspace_bytes(2, 28, 4, 128, 16, c["btd"].shape[1], 700)
    assert need > 0
    # The fixed counter region at the start of the buffer (16384 ints) is all zero again.
    assert torch.count_nonzero(ws[:16384 * 4]) == 0
    assert max_err(run(c, 128 ** -0.5), oracle(c, 128 ** -0.5)) <= TOL


def test_launches_of_different_sizes_share_the_scratch(cuda_device):
    """Split launches of different sizes in a row reuse one scratch buffer: each finds its
    counters at zero, whatever the previous launch left in its records."""
    cases = [build(14, 2, 64, 16, [3000], [200], seed=22, device=cuda_device),
             build(28, 4, 128, 16, [5000, 900], [1000, 3], seed=23, device=cuda_device),
             build(14, 2, 64, 16, [2500, 2600], [64, 100], seed=24, device=cuda_device)]
    want = [oracle(c, 0.125) for c in cases]
    for _ in range(2):
        for c, w in zip(cases, want):
            assert max_err(run(c, 0.125), w) <= TOL


def test_prefill_and_decode_interleaved_on_one_stream(cuda_device):
    """Both kernels keep their own scratch; alternating them changes no result."""
    c = build(14, 2, 64, 16, [2000, 600], [300, 1], seed=20, device=cuda_device)
    d = build(14, 2, 64, 16, [4000, 37, 900], [1, 1, 1], seed=21, device=cuda_device)
    p0 = run(c, 0.125)
    d0 = paged_attention_decode_batched(d["qd"], d["kd"], d["vd"], d["btd"], d["lensd"], 0.125)
    for _ in range(3):
        assert torch.equal(run(c, 0.125), p0)
        assert torch.equal(paged_attention_decode_batched(d["qd"], d["kd"], d["vd"], d["btd"],
                                                          d["lensd"], 0.125), d0)
