"""Benchmark of the MI355X paged-decode hot path: K/V write + batched GQA paged attention.

One step = write every sequence's newest K/V row into its block, then one
batched paged-attention call over the whole batch (the per-layer work of a
decode step, reference engine/kernels/paged_attention_integration.py:148-171).

Default workload (the headline configuration): batch 256, 14 q / 2 kv heads,
head_dim 64, block 16, fp16, lengths lognormal (median 4096, sigma 0.5) clipped
to [256, 32768], groups of 8 sequences sharing their first 64 blocks. Inputs are
synthetic N(0, 1) data resident in HBM before timing starts. R copies of the
pool are rotated so that no step finds the previous step's data in the 256 MB
MALL (Infinity Cache).

Output: one JSON line. value = bytes of one step (the attention call's
algorithmic bytes: K/V at the distinct token slots read, Q, O, table entries,
lengths; and the K/V write's rows, lengths and table entries) / mean step time,
the K timed steps run back to back between two synchronisations with one HIP
event pair on the launch stream around them (a GPU busy-wait before the start
event lets the host queue the steps first, so the window holds device work
only). roofline.achieved = the attention call's algorithmic bytes / its mean
duration over K calls enqueued back to back (one event pair around them, the
same busy-wait before it). Beside them: per-call event timings (an event pair
around each call adds a few microseconds of marker processing), the median
of 60 such calls, the other measured shapes (one Qwen2.5-0.5B layer at batch
8, the GQA sweep, the softmax stress shape, one layer of the batch-128 decode
step), the paged prefill attention against
the MFMA peak, decode tokens/s of the Qwen2.5-0.5B-shaped model with and
without fused decoder layers, and the reference's CPU algorithm timed on this
host (the oracle's fp16 and fp32 attention over the headline batch, and two
decode steps of the whole model on the CPU).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT))
sys.path.insert(0, str(REPO_ROOT / "vllm-inference-engine_amd"))

HBM_PEAK_GBS = 8000.0
TRAFFIC_SUMMARY = REPO_ROOT / "profiles" / "long_context_traffic.md"
# GPU busy-wait (torch.cuda._sleep cycles, about 50 us on MI355X) enqueued before a timed call
# whose kernel is shorter than the host's enqueue cost (about 19 us per call): the call is then
# queued before the GPU reaches its start event, and the events bracket device time only.
LEAD_CYCLES = 100_000


def log(msg):
    """Progress line on stderr (the JSON result is the only line on stdout)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="long_context",
                   help="long_context | gqa_sweep_kv{28,14,7,4} | qwen_layer | softmax_stress | "
                        "decode_step_layer_b128")
    p.add_argument("--copies", type=int, default=4, help="rotated pool copies (cache defeat)")
    p.add_argument("--flush-mb", type=int, default=0,
                   help="write this many MB before each step's attention call (cache defeat "
                        "with one pool); inside ms_per_step, outside the per-call attention "
                        "events, from which value is then computed")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=8.0,
                   help="approximate CPU time budget of each oracle baseline variant")
    p.add_argument("--no-configs", action="store_true",
                   help="skip the timings of the other measured shapes")
    p.add_argument("--reference-grid", action="store_true",
                   help="latency of the batched kernel over the reference's published grid "
                        "(batch 1/4/16/32 x length 128/512/2048, cache flushed before each call) "
                        "and print it")
    p.add_argument("--decode-only", action="store_true",
                   help="run only the decode-step tokens/sec measurement (for kernel profiles of "
                        "the decode step) and print its result")
    p.add_argument("--no-decode", action="store_true",
                   help="skip the decode-step tokens/sec measurement")
    p.add_argument("--no-prefill", action="store_true",
                   help="skip the prefix-prefill attention measurement")
    p.add_argument("--profile-workloads", default="",
                   help="comma-separated workloads: run --profile-calls attention calls of each "
                        "(4 rotated pool copies) and exit, for rocprofv3 kernel statistics")
    p.add_argument("--profile-calls", type=int, default=40)
    p.add_argument("--library", default="",
                   help="file name of another build of the library in engine/kernels/ to load "
                        "instead of libpa_gfx950.so (A/B profiles)")
    p.add_argument("--decode-batch", type=int, default=128)
    p.add_argument("--decode-steps", type=int, default=128)
    return p.parse_args()


def decode_benchmark(dev, model, prompts, steps, fuse_layers=True, attention_share=True):
    """Greedy decode of a random-init Qwen2.5-0.5B-shaped model through the paged HIP path.

    len(prompts) sequences with prompt lengths U[64, 1024] of random token ids;
    each decode step runs the model with the fused RoPE + K/V write and the
    batched paged-attention kernel in all 24 layers, replayed as a captured
    graph; fuse_layers also runs each decoder layer's norms, projections and
    MLP through the fused layer forward. Prefill (transformers forward +
    prefill block copy) is timed separately; tokens/sec counts decode steps
    only. Returns (result, runner, seqs).
    """
    import torch

    from engine.kernels.paged_attention_integration import KernelPagedManualDecode
    from engine.memory.block_allocator import BlockTable
    from types import SimpleNamespace

    batch = len(prompts)
    bs = 16
    need = sum((len(p) + steps + 2 * bs) // bs for p in prompts)
    runner = KernelPagedManualDecode(model, block_size=bs, num_blocks=need, device=str(dev),
                                     fuse_layers=fuse_layers)
    alloc = runner.allocator
    seqs = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i, p in enumerate(prompts):
        bt = BlockTable(i, bs, [alloc.allocate() for _ in range((len(p) + bs - 1) // bs)], len(p))
        seq = SimpleNamespace(seq_id=i, prompt_token_ids=p, block_table=bt, num_cached_tokens=0,
                              last_token_id=None, last_logits=None, last_logit_margin=None)
        seq.last_token_id = runner.prefill(seq)
        seqs.append(seq)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0

    def one_step():
        for q in seqs:
            if q.block_table.num_tokens // bs >= len(q.block_table.physical_block_ids):
                q.block_table.physical_block_ids.append(alloc.allocate())
        for q, t in zip(seqs, runner.decode_step(seqs)):
            q.last_token_id = t

    warm = 2
    for _ in range(warm):
        one_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    torch.cuda.nvtx.range_push("decode_steps")  # marks the timed steps in profiler traces
    for _ in range(steps - warm):
        one_step()
    torch.cuda.synchronize()
    torch.cuda.nvtx.range_pop()
    dt = time.perf_counter() - t0
    timed = steps - warm
    res = {
        "tokens_per_s": round(batch * timed / dt, 1),
        "ms_per_step": round(1e3 * dt / timed, 3),
        "batch": batch,
        "decode_steps_timed": timed,
        "warmup_steps": warm,
        "prefill_s": round(prefill_s, 3),
        "fused_layers": runner.fuse_layers,
        "graphs_captured": runner.graph_captures,
        "model": "Qwen2.5-0.5B architecture, random init N(0, 0.02), fp16, untied lm_head",
        "prompt_lens": "U[64, 1024], random token ids",
    }
    if attention_share:
        attn_ms = attention_share_ms(dev, runner, seqs)
        res["attention_ms_per_step"] = round(attn_ms, 3)
        res["attention_share"] = round(attn_ms / (1e3 * dt / timed), 3)
    return res, runner, seqs


def cpu_decode_steps(model, seqs, block_size=16, steps=2):
    """The reference's decode step on the host CPU: time `steps` steps of the whole model.

    The reference runs its decode attention (integration.py:65-176) as the
    q/k/v projections, transformers' RoPE, a per-sequence index_put K/V write
    (:148-161) and the batched paged attention; on the CPU the attention is its
    PyTorch algorithm (paged_attention.py:30-83). Here every attention module
    of the same fp16 model, moved to the host, runs exactly that, with the
    oracle's restatements of the write loop and the attention, over a pool
    holding the decode run's block tables at its final lengths (pool values
    synthetic: one K and one V tensor shared by the layers, the timing does
    not depend on them). One untimed step first.
    """
    import torch
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    from oracle.paged_attention_oracle import kv_write_reference, naive_reference_paged_attention

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    model = model.to("cpu")
    cfg = model.config
    bs = block_size
    tables = [list(s.block_table.physical_block_ids) for s in seqs]
    lens = [s.block_table.num_tokens for s in seqs]
    nblocks = max(max(t) for t in tables) + 1
    g = torch.Generator().manual_seed(3)
    shape = (nblocks, bs, cfg.num_key_value_heads, cfg.hidden_size // cfg.num_attention_heads)
    kc = torch.randn(shape, generator=g).half()
    vc = torch.randn(shape, generator=g).half()

    def attention(self, hidden_states, position_embeddings, attention_mask=None,
                  past_key_values=None, **kwargs):
        b = hidden_states.shape[0]
        shp = (b, 1, -1, self.head_dim)
        q = self.q_proj(hidden_states).view(shp).transpose(1, 2)
        k = self.k_proj(hidden_states).view(shp).transpose(1, 2)
        v = self.v_proj(hidden_states).view(shp).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        kv_write_reference(k[:, :, 0], v[:, :, 0], kc, vc, tables, cur_lens, bs)
        o = naive_reference_paged_attention(q[:, :, 0], kc, vc, tables, cur_lens, self.scaling)
        return self.o_proj(o.reshape(b, 1, -1)), None

    mods = [m for m in model.modules()
            if all(hasattr(m, n) for n in ("q_proj", "k_proj", "v_proj", "o_proj"))]
    for m in mods:
        m.forward = attention.__get__(m, m.__class__)
    ids = torch.randint(0, model.config.vocab_size, (len(seqs), 1), generator=g)
    times = []
    try:
        with torch.inference_mode():
            for i in range(steps + 1):
                cur_lens = [n + 1 + i for n in lens]
                for t, n in zip(tables, cur_lens):
                    while len(t) * bs < n:  # a block for the new token, as the scheduler adds
                        t.append(t[-1])
                pos = torch.tensor([[n - 1] for n in cur_lens])
                t0 = time.perf_counter()
                logits = model(input_ids=ids, position_ids=pos, use_cache=False).logits
                ids = logits[:, -1].argmax(-1, keepdim=True)
                if i:
                    times.append(time.perf_counter() - t0)
    finally:
        for m in mods:
            del m.forward
    t = sum(times)
    return {
        "tokens_per_s": round(len(seqs) * steps / t, 2),
        "s_per_step": round(t / steps, 3),
        "steps_timed": steps,
        "cores": torch.get_num_threads(),
        "batch": len(seqs),
        "extrapolated_128_steps_s": round(128 * t / steps, 1),
        "sample": (f"{steps} decode steps (after 1 untimed) of the same fp16 model on the host, "
                   "each attention module running the reference's CPU algorithm (projections, "
                   "transformers RoPE, per-sequence index_put K/V write, per-sequence gather + "
                   "einsum + softmax); 128 steps extrapolated linearly"),
    }


MFMA_F16_PEAK_TFLOPS = 2500.0


def prefill_benchmark(dev, seed, B=8, cached=2048, new=512, iters=30, warmup=5):
    """Paged prefill attention of prompt suffixes over cached prefix blocks.

    B sequences, each `cached` cached tokens plus `new` new ones, Qwen2.5-0.5B
    heads (14 q / 2 kv, head_dim 64), block 16, shuffled physical blocks. The
    kernel is MFMA work: causal FLOPs = 4 * head_dim * q_heads * (keys seen,
    summed over the new tokens), priced against the dense fp16 MFMA peak.
    """
    import torch

    from engine.kernels.paged_attention import paged_attention_prefill

    hq, hkv, d, bs = 14, 2, 64, 16
    L = cached + new
    nb = (L + bs - 1) // bs
    g = torch.Generator(device=dev).manual_seed(seed + 11)
    pool = B * nb + 16
    kc = torch.randn(pool, bs, hkv, d, generator=g, device=dev).half()
    vc = torch.randn(pool, bs, hkv, d, generator=g, device=dev).half()
    perm = torch.randperm(pool, generator=g, device=dev)[:B * nb].to(torch.int32)
    bt = perm.view(B, nb).contiguous()
    lens = torch.full((B,), L, dtype=torch.int32, device=dev)
    qsl = (torch.arange(B + 1, device=dev) * new).to(torch.int32)
    q = torch.randn(B * new, hq, d, generator=g, device=dev).half()
    for _ in range(warmup):
        paged_attention_prefill(q, kc, vc, bt, lens, qsl, new, d ** -0.5)
    torch.cuda.synchronize()
    # The kernel rate: one event pair around `iters` calls enqueued back to back behind a GPU
    # busy-wait (the statistic of the decode figures); an event pair around each call adds the
    # events' own processing, kept beside it.
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(window_lead_cycles(iters))
    a.record()
    for _ in range(iters):
        paged_attention_prefill(q, kc, vc, bt, lens, qsl, new, d ** -0.5)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / iters * 1e3
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(iters)]
    for a, b in ev:
        a.record()
        paged_attention_prefill(q, kc, vc, bt, lens, qsl, new, d ** -0.5)
        b.record()
    torch.cuda.synchronize()
    us_events = statistics.fmean(a.elapsed_time(b) for a, b in ev) * 1e3
    keys_seen = B * sum(cached + i + 1 for i in range(new))
    flops = 4.0 * d * hq * keys_seen
    tflops = flops / (us * 1e-6) / 1e12
    return {
        "config": {"workload": "prefix_prefill", "num_seqs": B, "cached_tokens": cached,
                   "new_tokens": new, "num_q_heads": hq, "num_kv_heads": hkv, "head_dim": d,
                   "block_size": bs},
        "attention_us_mean": round(us, 2),
        "attention_us_mean_per_call_events": round(us_events, 2),
        "flops": flops,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)},
    }


def attention_share_ms(dev, runner, seqs, iters=20):
    """The decode step's paged-attention work timed on its own: per layer one RoPE + K/V
    write + batched attention call (paged_rope_decode_attention, as the decode step makes
    it) at the batch's final lengths, times the layers.

    Synthetic q/k/v/cos/sin of the step's shapes; layer 0's pool is written (after the
    timed steps, so nothing measured reads it).
    """
    import torch

    from engine.kernels.paged_attention import pad_block_tables
    from engine.kernels.paged_attention_integration import paged_rope_decode_attention
    from engine.workloads import QWEN25_05B as QWEN05

    b = len(seqs)
    hq, hkv, d = QWEN05["num_attention_heads"], QWEN05["num_key_value_heads"], runner.head_dim
    tables = pad_block_tables([s.block_table.physical_block_ids for s in seqs], device=dev)
    lens = torch.tensor([s.block_table.num_tokens for s in seqs], dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn(b, hq, d, generator=g, device=dev).half()
    k = torch.randn(b, hkv, d, generator=g, device=dev).half()
    v = torch.randn(b, hkv, d, generator=g, device=dev).half()
    cos = torch.rand(b, d, generator=g, device=dev).half()
    sin = torch.rand(b, d, generator=g, device=dev).half()
    kc, vc = runner.pool.k_cache[0], runner.pool.v_cache[0]

    def layer():
        return paged_rope_decode_attention(q, k, v, cos, sin, kc, vc, tables, lens, d ** -0.5)

    for _ in range(3):
        layer()
    torch.cuda.synchronize()
    a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # The GPU waits while the host queues every call, as in the decode step's graph replay:
    # the events then time the calls' device work, not the host's enqueue cost.
    torch.cuda._sleep(LEAD_CYCLES * iters)
    a.record()
    for _ in range(iters):
        layer()
    e.record()
    torch.cuda.synchronize()
    return a.elapsed_time(e) / iters * QWEN05["num_hidden_layers"]


def make_workload(name, device, seed):
    from engine import workloads

    if name == "long_context":
        return workloads.long_context(device=device, seed=seed)
    if name.startswith("gqa_sweep_kv"):
        return workloads.gqa_sweep(int(name[len("gqa_sweep_kv"):]), device=device, seed=seed)
    if name == "qwen_layer":
        return workloads.qwen_layer(device=device, seed=seed)
    if name == "softmax_stress":
        return workloads.softmax_stress(device=device, seed=seed)
    if name == "decode_step_layer_b128":
        return workloads.decode_step_layer(128, device, seed)
    raise SystemExit(f"unknown workload {name}")


def source_digest():
    """sha256 over the library's sources (csrc/*, include/*), names and contents, sorted."""
    h = hashlib.sha256()
    files = sorted((REPO_ROOT / "vllm-inference-engine_amd" / "csrc").glob("*")) + \
        sorted((REPO_ROOT / "include").glob("*.h"))
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()


def read_traffic():
    """(HBM bytes per launch, sources digest) from the committed rocprofv3 --pmc summary."""
    if not TRAFFIC_SUMMARY.exists():
        return None, None
    nbytes = digest = None
    for line in TRAFFIC_SUMMARY.read_text().splitlines():
        key, _, val = line.partition(":")
        if key == "traffic_bytes_per_launch":
            try:
                nbytes = int(float(val.strip()))
            except ValueError:
                nbytes = None
        elif key == "kernel_sources_sha256":
            digest = val.strip()
    return nbytes, digest


def copy_ceiling(dev, nbytes=2 << 30, iters=10):
    """Plain device copy bandwidth (read + write bytes), the box's practical bandwidth line."""
    import torch

    x = torch.empty(nbytes // 2, dtype=torch.float16, device=dev).normal_()
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        y.copy_(x)
    b.record()
    torch.cuda.synchronize()
    t = a.elapsed_time(b) * 1e-3 / iters
    del x, y
    torch.cuda.empty_cache()
    return round(2 * nbytes / t / 1e9, 1)


PROBE_LIB = REPO_ROOT / "vllm-inference-engine_amd" / "probes" / "libbw_probe_gfx950.so"


def read_ceilings(dev, stream_bytes=1 << 30, pool_blocks=600_000, gather_blocks=150_000,
                  block_bytes=4096, iters=20):
    """Practical HBM read ceilings of this box, measured in the same run as the kernel.

    read_stream_gbps: a 1 GiB buffer read once per launch with the decode kernel's load
    instruction (16-byte non-temporal buffer loads, each wavefront instruction covering 1 KB,
    16 KB in flight per wavefront). gather_4kb_gbps: 150,000 random 4 KB blocks of a 2.4 GB
    pool (the headline pool's block size and about its distinct block count) read per launch,
    four blocks in flight per wavefront, four disjoint block lists rotated so that no launch
    finds the previous one's blocks in the 256 MB MALL. Both: the best of a few grid sizes,
    `iters` launches back to back between one HIP event pair behind a GPU busy-wait.
    """
    import ctypes

    import torch

    lib = ctypes.CDLL(str(PROBE_LIB))
    lib.bwp_read_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_void_p]
    lib.bwp_gather_blocks.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    stream = torch.cuda.current_stream(dev).cuda_stream
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count

    def window(launch):
        for _ in range(3):
            launch(0)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(window_lead_cycles(iters))
        a.record()
        for i in range(iters):
            launch(i)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e-3 / iters

    out = {}
    buf = torch.empty(stream_bytes, dtype=torch.uint8, device=dev).random_(0, 255)
    nread = stream_bytes // (16 << 10) * (16 << 10)
    best = 0.0
    for grid in (cus, 2 * cus, 4 * cus):
        def launch(i, grid=grid):
            rc = lib.bwp_read_stream(buf.data_ptr(), stream_bytes, sink.data_ptr(), grid, stream)
            assert rc == 0, f"bwp_read_stream failed ({rc})"
        best = max(best, nread / window(launch) / 1e9)
    out["read_stream_gbps"] = round(best, 1)
    del buf
    torch.cuda.empty_cache()
    pool = torch.empty(pool_blocks * block_bytes, dtype=torch.uint8, device=dev).random_(0, 255)
    gen = torch.Generator(device="cpu").manual_seed(123)
    perm = torch.randperm(pool_blocks, generator=gen)[:4 * gather_blocks].to(torch.int32)
    lists = perm.view(4, gather_blocks).to(dev)
    best = 0.0
    for grid in (cus, 2 * cus):
        def launch(i, grid=grid):
            rc = lib.bwp_gather_blocks(pool.data_ptr(), pool_blocks, block_bytes,
                                       lists[i % 4].data_ptr(), gather_blocks, sink.data_ptr(),
                                       grid, stream)
            assert rc == 0, f"bwp_gather_blocks failed ({rc})"
        best = max(best, gather_blocks * block_bytes / window(launch) / 1e9)
    out["gather_4kb_gbps"] = round(best, 1)
    del pool, lists
    torch.cuda.empty_cache()
    return out


def cpu_attention_passes(w, budget_s, compute_dtype=None):
    """The oracle's attention (the reference's CPU PyTorch algorithm) over the workload's
    sequences, in whole passes over the batch until about budget_s of oracle time (or part of
    one pass when a single pass exceeds it). Returns (seconds, sequences done, whole passes,
    bytes on the per-sequence basis, unique bytes of the whole passes and their seconds)."""
    from engine import workloads
    from oracle.paged_attention_oracle import naive_reference_paged_attention

    bs = w.k_cache.shape[1]
    hkv, d = w.k_cache.shape[2], w.k_cache.shape[3]
    hq = w.q.shape[1]
    subsets = [workloads.gather_subset(w, [i]) for i in range(w.num_seqs)]
    t_total, logical, passes, done, t_whole = 0.0, 0, 0, 0, 0.0
    while t_total < budget_s and passes < 100:
        for q, k, v, tables, lens in subsets:
            t0 = time.perf_counter()
            naive_reference_paged_attention(q, k, v, tables, lens, w.scale,
                                            compute_dtype=compute_dtype)
            t_total += time.perf_counter() - t0
            n = lens[0]
            logical += 2 * hkv * d * 2 * n + 2 * hq * d * 2 + 4 * ((n + bs - 1) // bs) + 4
            if passes == 0:
                done += 1
            if passes == 0 and t_total >= budget_s and done < w.num_seqs:
                break
        else:
            passes += 1
            t_whole = t_total
            continue
        break
    return t_total, done, passes, logical, passes * w.algorithmic_bytes(unique=True), t_whole


def cpu_baseline(w, budget_s):
    """The reference's CPU path on the headline batch: the oracle's literal fp16 attention
    (value) and the same algorithm on fp32-upcast rows, each on this host's cores."""
    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    out = {}
    for name, dtype in (("fp16", None), ("fp32", torch.float32)):
        t, done, passes, logical, unique, t_whole = cpu_attention_passes(w, budget_s, dtype)
        out[name] = {
            "gbps_unique": round(unique / t_whole / 1e9, 4) if passes else None,
            "gbps_per_sequence": round(logical / t / 1e9, 4),
            "seconds": round(t, 1), "passes": passes, "sequences_first_pass": done,
        }
    lit = out["fp16"]
    value = lit["gbps_unique"] if lit["gbps_unique"] is not None else lit["gbps_per_sequence"]
    return {
        "value": value,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle literal fp16 path (per-sequence gather + einsum + softmax) over the "
                   f"whole headline batch ({w.num_seqs} sequences, {sum(w.lens)} tokens), "
                   f"{lit['passes']} whole pass(es) in {lit['seconds']} s; value counts the "
                   "GPU attention call's algorithmic bytes (shared prefix slots once) per "
                   "whole pass"),
        "fp16": lit,
        "fp32_upcast": out["fp32"],
    }


def reference_grid(dev, flush_mb=512):
    """The reference's batched-kernel benchmark grid, measured the same way.

    scripts/benchmark_l2_flushed_sdpa_fair.py:56-128 of the reference: 14 q / 2
    kv heads, head_dim 64, block 16, equal lengths S, block ids shuffled over a
    pool of B * ceil(S / 16) + 128 blocks (seed 42 + 100 B + S), 15 untimed
    calls, then 35 calls each preceded by a buffer write that evicts the caches
    (512 MB here, above the MI355X's 256 MB MALL), median of the events around
    each call; bytes B*S*Hkv*D*2*2 + B*Hq*D*2*2.
    """
    import random

    import torch

    from engine.kernels.paged_attention import paged_attention_decode_batched, pad_block_tables

    hq, hkv, d, bs = 14, 2, 64, 16
    flush = torch.empty(flush_mb << 20, dtype=torch.uint8, device=dev)
    out = []
    for b in (1, 4, 16, 32):
        for s_len in (128, 512, 2048):
            q = torch.randn(b, hq, d, dtype=torch.float16, device=dev)
            mb = (s_len + bs - 1) // bs
            total = b * mb + 128
            ids = list(range(total))
            random.seed(42 + b * 100 + s_len)
            random.shuffle(ids)
            tables = [ids[i * mb:(i + 1) * mb] for i in range(b)]
            kc = torch.randn(total, bs, hkv, d, dtype=torch.float16, device=dev)
            vc = torch.randn(total, bs, hkv, d, dtype=torch.float16, device=dev)
            bt = pad_block_tables(tables, device=dev)
            sl = torch.full((b,), s_len, dtype=torch.int32, device=dev)
            call = lambda: paged_attention_decode_batched(q, kc, vc, bt, sl, d ** -0.5)
            for _ in range(15):
                call()
            torch.cuda.synchronize()
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(35)]
            for e0, e1 in ev:
                flush.zero_()
                e0.record()
                call()
                e1.record()
            torch.cuda.synchronize()
            ms = statistics.median(e0.elapsed_time(e1) for e0, e1 in ev)
            nbytes = b * s_len * hkv * d * 2 * 2 + b * hq * d * 2 * 2
            out.append({"batch": b, "seq_len": s_len, "us": round(ms * 1e3, 2),
                        "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1)})
    return out


def clone_workload(w):
    from engine.workloads import Workload

    return Workload(name=w.name, q=w.q.clone(), k_cache=w.k_cache.clone(),
                    v_cache=w.v_cache.clone(), block_tables=w.block_tables.clone(),
                    seq_lens=w.seq_lens.clone(), tables=w.tables, lens=w.lens, scale=w.scale,
                    unique_slots=w.unique_slots, meta=w.meta)


def window_lead_cycles(n):
    """GPU busy-wait (torch.cuda._sleep cycles) before a timed window of n calls: about 100 us
    per call (at most 10 ms), more than the host needs to enqueue one."""
    return 2 * LEAD_CYCLES * min(max(n, 1), 100)


def window_calls(copies, calls, warmup=5):
    """Mean duration (ms) of `calls` attention calls enqueued back to back over the rotated
    pool copies, timed by one HIP event pair on the launch stream around all of them."""
    import torch

    from engine.kernels.paged_attention import paged_attention_decode_batched

    def call(w):
        return paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables,
                                              w.seq_lens, w.scale)

    for i in range(warmup):
        call(copies[i % len(copies)])
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(window_lead_cycles(calls))  # queue the calls before the GPU reaches them
    a.record()
    for i in range(calls):
        call(copies[i % len(copies)])
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / calls


def window_write_calls(copies, calls, warmup=5):
    """As window_calls, for the decode layer's write and attention together: each call writes
    every sequence's new K/V row and attends (paged_decode_kv_write_attention; one launch on
    the one-workgroup-per-pair schedule, the K/V write launch plus the attention launch
    otherwise). The rows land in the rotated copies' pools at each sequence's last position."""
    import torch

    from engine.kernels.paged_attention_integration import paged_decode_kv_write_attention

    w0 = copies[0]
    g = torch.Generator(device=w0.q.device).manual_seed(17)
    shape = (w0.num_seqs, w0.k_cache.shape[2], w0.k_cache.shape[3])
    nk = torch.randn(shape, generator=g, device=w0.q.device).half()
    nv = torch.randn(shape, generator=g, device=w0.q.device).half()

    def call(w):
        return paged_decode_kv_write_attention(w.q, nk, nv, w.k_cache, w.v_cache,
                                               w.block_tables, w.seq_lens, w.scale)

    for i in range(warmup):
        call(copies[i % len(copies)])
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(window_lead_cycles(calls))
    a.record()
    for i in range(calls):
        call(copies[i % len(copies)])
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / calls


def time_calls(copies, calls, warmup=5, lead_cycles=0, host_us=None):
    """HIP-event durations (ms) of `calls` attention calls rotating over the pool copies.

    With `lead_cycles`, each call follows a GPU busy-wait outside its events. `host_us`, a
    list, receives the host time of each call (enqueue only, nothing waits for the GPU).
    """
    import torch

    from engine.kernels.paged_attention import paged_attention_decode_batched

    def call(w):
        return paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables,
                                              w.seq_lens, w.scale)

    for i in range(warmup):
        call(copies[i % len(copies)])
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(calls)]
    for i, (a, b) in enumerate(ev):
        w = copies[i % len(copies)]
        if lead_cycles:
            torch.cuda._sleep(lead_cycles)
        t0 = time.perf_counter()
        a.record()
        call(w)
        b.record()
        if host_us is not None:
            host_us.append((time.perf_counter() - t0) * 1e6)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def config_timings(dev, seed, copies=4, calls=50):
    """The other measured shapes, each over rotated pool copies.

    `us_mean` (and gbps, pct_of_hbm_peak) is the headline's statistic: `calls` calls enqueued
    back to back between one HIP event pair, behind a GPU busy-wait that lets the host queue
    them first, so the window holds device time only. `kv_write_attention_us_mean`: the same
    for the decode layer's K/V write and attention as one call. Beside them, per-call event pairs (each
    call behind its own busy-wait; the pair adds a few microseconds of marker processing):
    `us_mean_per_call_events`, `us_median_per_call_events`; the host's time per call
    (`host_enqueue_us_median`), and the same calls issued back to back without the lead
    (`us_mean_back_to_back`, host-bound where a kernel is shorter than the host's enqueue).
    """
    import torch

    from engine import workloads

    shapes = [("qwen_layer", lambda: workloads.qwen_layer(device=dev, seed=seed)),
              ("softmax_stress", lambda: workloads.softmax_stress(device=dev, seed=seed)),
              ("decode_step_layer_b128", lambda: workloads.decode_step_layer(128, dev, seed))]
    shapes += [(f"gqa_sweep_kv{h}", lambda h=h: workloads.gqa_sweep(h, device=dev, seed=seed))
               for h in (28, 14, 7, 4)]
    out = {}
    for name, make in shapes:
        ws = [make()]
        ws += [clone_workload(ws[0]) for _ in range(copies - 1)]
        host = []
        win = window_calls(ws, calls)
        fused = window_write_calls(ws, calls)
        ms = time_calls(ws, calls, lead_cycles=LEAD_CYCLES, host_us=host)
        nbytes = ws[0].algorithmic_bytes(unique=True)
        mean, med = statistics.fmean(ms), statistics.median(ms)
        out[name] = {"num_seqs": ws[0].num_seqs, "num_q_heads": ws[0].q.shape[1],
                     "num_kv_heads": ws[0].k_cache.shape[2], "head_dim": ws[0].k_cache.shape[3],
                     "total_tokens": sum(ws[0].lens), "algorithmic_bytes": nbytes,
                     "us_mean": round(win * 1e3, 2),
                     "gbps": round(nbytes / (win * 1e-3) / 1e9, 1),
                     "pct_of_hbm_peak": round(100 * nbytes / (win * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                     "kv_write_attention_us_mean": round(fused * 1e3, 2),
                     "us_mean_per_call_events": round(mean * 1e3, 2),
                     "us_median_per_call_events": round(med * 1e3, 2),
                     "calls": calls, "pool_copies_rotated": copies,
                     "host_enqueue_us_median": round(statistics.median(host), 1),
                     "us_mean_back_to_back": round(statistics.fmean(time_calls(ws, calls)) * 1e3, 2)}
        del ws
        torch.cuda.empty_cache()
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU only; --gpus must be 1 (the path would shard by "
                          "sequence or by kv head, each GPU running this kernel on its share)"}))
        raise SystemExit(2)
    import torch

    from engine import workloads
    from engine.kernels.paged_attention import paged_attention_decode_batched
    from engine.kernels.paged_attention_integration import (paged_decode_kv_write_attention,
                                                           paged_kv_write)

    dev = torch.device("cuda", 0)
    if args.library:
        from engine.kernels import _native
        _native.LIB_PATH = _native.LIB_PATH.with_name(args.library)
    if args.profile_workloads:
        for name in args.profile_workloads.split(","):
            base = make_workload(name, dev, args.seed)
            ws = [base] + [clone_workload(base) for _ in range(3)]
            for i in range(args.profile_calls):
                w = ws[i % 4]
                paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables,
                                               w.seq_lens, w.scale)
            torch.cuda.synchronize()
            log(f"profiled {name}: {args.profile_calls} calls")
            del ws, base
            torch.cuda.empty_cache()
        return
    if args.reference_grid:
        print(json.dumps({"reference_grid": reference_grid(dev)}), flush=True)
        return
    if args.decode_only:
        model = workloads.decode_model(dev, args.seed)
        prompts = workloads.decode_prompts(args.seed, args.decode_batch)
        dec, _, _ = decode_benchmark(dev, model, prompts, args.decode_steps)
        print(json.dumps({"decode_tokens_per_s": dec["tokens_per_s"], "decode": dec}), flush=True)
        return
    base = make_workload(args.workload, dev, args.seed)
    copies = [base] + [clone_workload(base) for _ in range(1, max(1, args.copies))]
    g = torch.Generator(device=dev).manual_seed(args.seed + 7)
    hkv, d = base.k_cache.shape[2], base.k_cache.shape[3]
    new_k = torch.randn(base.num_seqs, hkv, d, generator=g, device=dev).half()
    new_v = torch.randn(base.num_seqs, hkv, d, generator=g, device=dev).half()

    flush = (torch.empty(args.flush_mb << 20, dtype=torch.uint8, device=dev)
             if args.flush_mb > 0 else None)

    def step(i, ev=None):
        """One decode layer's work: every sequence's new K/V row written to its slot, then
        the batched attention. Without `ev`, as the decode step makes it
        (paged_decode_kv_write_attention: the write launch also derives the attention
        launch's schedule plan); with `ev`, as two calls with an event pair around the
        attention call alone."""
        w = copies[i % len(copies)]
        if flush is not None:
            flush.fill_(i & 0xFF)
        if ev is None:
            return paged_decode_kv_write_attention(w.q, new_k, new_v, w.k_cache, w.v_cache,
                                                   w.block_tables, w.seq_lens, w.scale)
        paged_kv_write(new_k, new_v, w.k_cache, w.v_cache, w.block_tables, w.seq_lens)
        ev[0].record()
        out = paged_attention_decode_batched(w.q, w.k_cache, w.v_cache, w.block_tables,
                                             w.seq_lens, w.scale)
        ev[1].record()
        return out

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # Timed region: K whole steps (K/V write + attention) back to back, bracketed by
    # synchronisations and one HIP event pair on the launch stream. No event sits between
    # the steps: an event pair around each call adds 3-5 us of marker processing to a
    # ~97 us kernel (rocprofv3 kernel durations against per-call events).
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    # A GPU busy-wait ahead of the start event lets the host queue the steps before the GPU
    # reaches them: the window then holds the steps' device work and no host launch gaps (in
    # a fresh process the host's first ~100 enqueues can fall behind a ~100 us step).
    torch.cuda._sleep(window_lead_cycles(args.steps))
    t_start.record()
    for i in range(args.steps):
        step(args.warmup + i)
    t_end.record()
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    step_ms = total_ms / args.steps
    # The dominant kernel's average launch duration: the same number of attention calls
    # back to back over the rotated copies, one event pair around them.
    attn_window_ms = window_calls(copies, args.steps)
    # Per-call event pairs (the previous statistic), then the median of 60 such calls.
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    for i in range(args.steps):
        step(args.warmup + args.steps + i, events[i])
    torch.cuda.synchronize()
    attn_ms = [a.elapsed_time(b) for a, b in events]
    attn_mean = statistics.fmean(attn_ms)
    attn_med = statistics.median(attn_ms)
    med60 = statistics.median(time_calls(copies, 60, warmup=0))

    alg_bytes = base.algorithmic_bytes(unique=True)
    logical_bytes = base.algorithmic_bytes(unique=False)
    # The step's K/V write: the new rows read and written, one length and one table entry
    # read per sequence.
    write_bytes = 2 * 2 * new_k.numel() * new_k.element_size() + 8 * base.num_seqs
    if flush is None:
        value = (alg_bytes + write_bytes) / (step_ms * 1e-3) / 1e9
    else:  # the step then also holds the flush writes: attention bytes per attention call
        value = alg_bytes / (attn_mean * 1e-3) / 1e9
    achieved = alg_bytes / (attn_window_ms * 1e-3) / 1e9
    traffic, traffic_digest = (read_traffic() if args.workload == "long_context"
                               else (None, None))
    digest = source_digest()

    result = {
        "metric": "paged-decode attention HBM GB/s (% of peak) + decode tokens/sec, 1 MI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 storage, f32 accumulate",
        "data": "synthetic N(0,1), random block tables, seeded",
        "config": {
            "workload": base.name,
            "num_seqs": base.num_seqs,
            "num_q_heads": base.q.shape[1],
            "num_kv_heads": hkv,
            "head_dim": d,
            "block_size": base.k_cache.shape[1],
            "total_tokens": sum(base.lens),
            "max_len": max(base.lens),
            "pool_copies_rotated": len(copies),
            "flush_mb_per_step": args.flush_mb,
            **base.meta,
        },
        "step_bytes": alg_bytes + write_bytes,
        "attention_ms_window": round(attn_window_ms, 5),
        "attention_ms_mean_per_call_events": round(attn_mean, 5),
        "attention_ms_median_per_call_events": round(attn_med, 5),
        "gbps_per_call_events": round(alg_bytes / (attn_mean * 1e-3) / 1e9, 2),
        "attention_ms_median_of_60": round(med60, 5),
        "gbps_median_of_60": round(alg_bytes / (med60 * 1e-3) / 1e9, 2),
        "algorithmic_bytes": alg_bytes,
        "logical_bytes": logical_bytes,
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            # FETCH_SIZE + WRITE_SIZE per launch from the committed rocprofv3 summary, used only
            # when it was measured on these very sources.
            "traffic": traffic if traffic_digest == digest else None,
        },
        "traffic_profile": {"bytes": traffic, "sources_sha256": traffic_digest,
                            "matches_current_sources": traffic_digest == digest},
        "sources_sha256": digest,
        "decode_tokens_per_s": None,
    }
    log(f"headline: {step_ms * 1e3:.1f} us per step, {value:.0f} GB/s; attention "
        f"{attn_window_ms * 1e3:.1f} us per call back to back ({achieved:.0f} GB/s), "
        f"{attn_mean * 1e3:.1f} us between per-call events")
    result["copy_ceiling_gbps"] = copy_ceiling(dev)
    ceil = read_ceilings(dev)
    result["read_ceiling_gbps"] = ceil["read_stream_gbps"]
    result["gather_ceiling_gbps"] = ceil["gather_4kb_gbps"]
    result["roofline"]["frac_of_gather_ceiling"] = round(achieved / ceil["gather_4kb_gbps"], 4)
    log(f"ceilings: copy {result['copy_ceiling_gbps']} GB/s, read {ceil['read_stream_gbps']} "
        f"GB/s, 4 KB gather {ceil['gather_4kb_gbps']} GB/s")
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(base, args.cpu_seconds)
        log(f"cpu baseline: {result['cpu_baseline']['value']} GB/s")
    del copies, base
    torch.cuda.empty_cache()
    if not args.no_configs:
        result["configs"] = config_timings(dev, args.seed)
        log("config timings done")
    if not args.no_prefill:
        # A batch of prompt suffixes, and one long prompt the way the reference
        # prefills (one sequence at a time; its key ranges are split).
        result["prefix_prefill"] = prefill_benchmark(dev, args.seed)
        result["prefix_prefill_single"] = prefill_benchmark(dev, args.seed, B=1, cached=8192,
                                                            new=1024)
        log("prefill attention done")
    if not args.no_decode:
        model = workloads.decode_model(dev, args.seed)
        prompts = workloads.decode_prompts(args.seed, args.decode_batch)
        dec, runner, seqs = decode_benchmark(dev, model, prompts, args.decode_steps)
        log(f"decode: {dec['tokens_per_s']} tokens/s")
        del runner
        torch.cuda.empty_cache()
        unfused, _, _ = decode_benchmark(dev, model, prompts, args.decode_steps,
                                         fuse_layers=False, attention_share=False)
        log(f"decode without fused layers: {unfused['tokens_per_s']} tokens/s")
        dec["unfused_layers"] = {k: unfused[k] for k in ("tokens_per_s", "ms_per_step",
                                                         "graphs_captured")}
        result["decode_tokens_per_s"] = dec["tokens_per_s"]
        result["decode"] = dec
        if not args.no_cpu_baseline:
            result["cpu_baseline"]["decode_step"] = cpu_decode_steps(model, seqs)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
