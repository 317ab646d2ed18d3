"""The C-ABI library loads, exports every symbol the header declares, and validates
arguments on the host before any GPU work (no GPU needed)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch  # noqa: F401  (loaded before the HIP library, as the bindings do)

from engine.kernels import _native

HEADER = Path(__file__).resolve().parent.parent / "include" / "paged_attention.h"


def _declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"PA_API\s+[\w\s\*]+?\b(pa_\w+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = _declared_symbols()
    for n in ["pa_decode_batched_f16", "pa_decode_v1_f16", "pa_decode_v2_f16", "pa_kv_write_f16",
              "pa_prefill_copy_f16", "pa_rope_kv_write_f16", "pa_prefill_attention_f16",
              "pa_last_error", "pa_abi_version"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    missing = [n for n in _declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"symbols declared in the header but not exported: {missing}"
    assert set(_declared_symbols()) == set(_native.SIGNATURES), "bindings and header disagree"


def test_abi_version():
    assert _native.load().pa_abi_version() == _native.ABI_VERSION


def _device_cus():
    """Compute units the library plans for: the current device's, 256 without a GPU."""
    if torch.cuda.is_available():
        return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    return 256


def test_workspace_sizes():
    lib = _native.load()
    cus = _device_cus()
    rec = (32 + 16 * 64) * 4
    # The head of every decode workspace: per-pair arrival counters, then the schedule plan a
    # K/V write launch leaves for the attention launch after it (2 x 1024 + 64 ints).
    counters = 65536 * 4 + (2 * 1024 + 64) * 4

    def streamk(seqs, kv_heads, grid, pair_heads, share):
        # Two record slots per workgroup of the grid; a slot holds one record per kv head of
        # a pair, or, where prefix items may be built (head_dim <= 64, block 16 or 32, 64 or
        # more sequences), one per column block of a prefix item (4). Prefix items add a
        # suffix and a prefix record per (sequence, kv head).
        slot = max(pair_heads, 4) if share else pair_heads
        return counters + grid * 2 * slot * rec + (2 * seqs * kv_heads * rec if share else 0)

    # Stream-K (<= 1024 sequences): the grid is one workgroup per CU, or the tile count
    # when that is smaller (8 sequences x 2 kv heads x 32 tiles = 512 here).
    assert lib.pa_decode_batched_workspace_bytes(8, 14, 2, 64, 16, 32) == \
        streamk(8, 2, min(cus, 512), 1, False)
    assert lib.pa_decode_batched_workspace_bytes(64, 14, 2, 64, 16, 32) == \
        streamk(64, 2, min(cus, 4096), 1, True)
    assert lib.pa_decode_batched_workspace_bytes(256, 14, 2, 64, 16, 2048) == \
        streamk(256, 2, cus, 2 if 256 * 2 > cus else 1, True)
    rec128 = (32 + 16 * 128) * 4
    assert lib.pa_decode_batched_workspace_bytes(64, 28, 7, 128, 16, 128) == \
        counters + cus * 2 * rec128
    # Block size 8 never shares prefixes.
    assert lib.pa_decode_batched_workspace_bytes(64, 14, 2, 64, 8, 64) == \
        streamk(64, 2, min(cus, 4096), 1, False)
    # One sequence (the single-sequence entry points) has nothing to share.
    assert lib.pa_decode_batched_workspace_bytes(1, 14, 2, 64, 16, 2048) == \
        streamk(1, 2, min(cus, 256), 1, False)
    # Fixed-split path beyond 1024 sequences: 2048-block rows -> 64 splits of 512 tokens,
    # placed after the counter region so one buffer serves both paths.
    assert lib.pa_decode_batched_workspace_bytes(2000, 14, 2, 64, 16, 2048) == counters + 2000 * 2 * 64 * rec
    assert lib.pa_decode_batched_workspace_bytes(2000, 14, 2, 64, 16, 32) == 0
    # kv heads per pair: one while sequences x kv heads stay within the current device's CU
    # count (256 when no GPU is visible, as on an MI355X), two above it
    half = cus // 2
    assert lib.pa_decode_batched_workspace_bytes(half, 14, 2, 64, 16, 2048) == \
        streamk(half, 2, cus, 1, True)
    assert lib.pa_decode_batched_workspace_bytes(half + 1, 14, 2, 64, 16, 2048) == \
        streamk(half + 1, 2, cus, 2, True)
    assert lib.pa_decode_v1_workspace_bytes(14, 2, 64, 16, 67) == 2 * 16 * 80 * 4
    assert lib.pa_decode_batched_workspace_bytes(8, 14, 2, 48, 16, 2048) == 0  # unsupported dim
    # Prefill: one sequence, 512 new tokens of 2560. Two column groups per wavefront would give
    # 7 x 512 / 128 = 28 column blocks x 2 kv heads = 56 workgroups, fewer than 64, so one group:
    # 56 column blocks of 64 columns x 2 kv heads = 112 workgroups, fewer than 3/4 of 2 x 256
    # slots: 20 key tiles of 128 split in 4 pieces of 5; the fixed counter region (16384 ints),
    # then 112 x 4 records of 64 columns x (64 + 2) floats.
    assert lib.pa_prefill_attention_workspace_bytes(1, 14, 2, 64, 16, 160, 512) == \
        16384 * 4 + 112 * 4 * 64 * 66 * 4
    # 1024 new tokens of 9216: 56 column blocks of 128 x 2 = 112 workgroups keep two groups;
    # 72 key tiles in 4 pieces of 18.
    assert lib.pa_prefill_attention_workspace_bytes(1, 14, 2, 64, 16, 576, 1024) == \
        16384 * 4 + 112 * 4 * 128 * 66 * 4
    # 64 sequences give 3584 workgroups: no split, no workspace.
    assert lib.pa_prefill_attention_workspace_bytes(64, 14, 2, 64, 16, 160, 512) == 0
    # Short contexts (at most 4 key tiles) are never split.
    assert lib.pa_prefill_attention_workspace_bytes(1, 14, 2, 64, 16, 32, 16) == 0


def _strides(*vals):
    return _native.i64_array(vals)


def _decode_call(lib, head_dim=64, nq=14, nkv=2, q=16, k=16, v=16, out=16, ws=0, max_blocks=4096,
                 kstr=(2048, 128, 64, 1)):
    return lib.pa_decode_batched_f16(
        q, _strides(896, 64, 1), k, _strides(*kstr), v, _strides(*kstr),
        16, _strides(max_blocks, 1), 16, out, _strides(896, 64, 1),
        4, nq, nkv, head_dim, 16, 100, max_blocks, 0.125, ws, 0, None)


def test_argument_errors_are_reported_before_launch():
    lib = _native.load()
    assert _decode_call(lib, head_dim=48) == _native.PA_ERR_UNSUPPORTED
    assert b"head_dim 48" in lib.pa_last_error()
    assert _decode_call(lib, nq=15, nkv=2) == _native.PA_ERR_ARG
    assert b"divisible" in lib.pa_last_error()
    assert _decode_call(lib, nq=34, nkv=2) == _native.PA_ERR_UNSUPPORTED
    assert _decode_call(lib, q=0) == _native.PA_ERR_ARG
    assert _decode_call(lib, k=8) == _native.PA_ERR_ARG  # misaligned pool pointer
    assert _decode_call(lib, kstr=(2048, 128, 64, 2)) == _native.PA_ERR_ARG
    assert _decode_call(lib) == _native.PA_ERR_WORKSPACE  # 4096-block rows need split-K scratch
    assert b"workspace" in lib.pa_last_error()


def test_kv_write_argument_errors():
    lib = _native.load()
    rc = lib.pa_kv_write_f16(0, _strides(128, 64, 1), 16, _strides(128, 64, 1), 16,
                             _strides(2048, 128, 64, 1), 16, _strides(2048, 128, 64, 1), 16,
                             _strides(4, 1), 16, 0, 4, 2, 64, 16, 100, 4, None)
    assert rc == _native.PA_ERR_ARG
    assert b"null" in lib.pa_last_error()


def _prefill_call(lib, head_dim=64, nq=14, nkv=2, q=16, qstart=16, qstr=(896, 64, 1), maxq=8,
                  ntok=32, scale=0.125):
    kstr = (2048, 128, 64, 1)
    return lib.pa_prefill_attention_f16(
        q, _strides(*qstr), 16, _strides(*kstr), 16, _strides(*kstr), 16, _strides(64, 1), 16,
        qstart, maxq, 16, _strides(896, 64, 1), 4, ntok, nq, nkv, head_dim, 16, 100, 64, scale,
        None, 0, None)


def test_prefill_argument_errors():
    lib = _native.load()
    assert _prefill_call(lib, head_dim=48) == _native.PA_ERR_UNSUPPORTED
    assert _prefill_call(lib, nq=15) == _native.PA_ERR_ARG
    assert _prefill_call(lib, qstart=0) == _native.PA_ERR_ARG
    assert b"null" in lib.pa_last_error()
    assert _prefill_call(lib, qstr=(900, 64, 1)) == _native.PA_ERR_ARG  # token stride not 8-aligned
    assert _prefill_call(lib, maxq=-1) == _native.PA_ERR_ARG
    assert _prefill_call(lib, scale=0.0) == _native.PA_ERR_ARG
    assert _prefill_call(lib, scale=-0.125) == _native.PA_ERR_ARG
    assert b"scale" in lib.pa_last_error()
    # Nothing to compute: no launch, no pointer is touched.
    assert _prefill_call(lib, q=0, qstart=0, maxq=0) == _native.PA_OK
    assert _prefill_call(lib, q=0, qstart=0, ntok=0) == _native.PA_OK


def test_error_text_is_thread_local():
    import threading

    lib = _native.load()
    assert _decode_call(lib, head_dim=48) == _native.PA_ERR_UNSUPPORTED
    seen = {}

    def other():
        seen["msg"] = lib.pa_last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == b""
    assert b"head_dim" in lib.pa_last_error()


def test_noalloc_entry_refuses_what_its_scratch_cannot_hold():
    """The no-allocation entry point checks its limits on the host, before any launch."""
    lib = _native.load()
    args = (16, _strides(896, 64, 1), 16, _strides(2048, 128, 64, 1), 16,
            _strides(2048, 128, 64, 1), 16, _strides(64, 1), 16, 16, _strides(896, 64, 1))
    rc = lib.pa_decode_batched_noalloc_f16(*args, 1100, 14, 2, 64, 16, 100, 64, 0.125, None)
    assert rc == _native.PA_ERR_UNSUPPORTED
    assert b"no-allocation" in lib.pa_last_error() and b"1024" in lib.pa_last_error()
    assert lib.pa_decode_batched_noalloc_f16(*args, 4, 14, 2, 48, 16, 100, 64, 0.125, None) == \
        _native.PA_ERR_UNSUPPORTED  # head_dim outside the built set, as for the workspace entry



def test_rope_decode_refuses_an_empty_table_before_launch():
    """The fused RoPE + K/V write + attention entry checks the table width and the
    output strides on the host, as pa_decode_batched_f16 does, for both of its forms."""
    lib = _native.load()
    rows = _strides(896, 64, 1)
    kv_rows = _strides(128, 64, 1)
    cs = _strides(64, 1)
    pool = _strides(2048, 128, 64, 1)

    def call(max_blocks, out_str=(896, 64, 1)):
        return lib.pa_decode_rope_batched_f16(
            16, rows, 16, kv_rows, 16, kv_rows, 16, cs, 16, cs, 16, pool, 16, pool,
            16, _strides(max(max_blocks, 1), 1), 16, 16, _strides(*out_str),
            4, 14, 2, 64, 16, 100, max_blocks, 0.125, 16, 1 << 30, None)

    assert call(0) == _native.PA_ERR_ARG
    assert b"at least one column" in lib.pa_last_error()
    assert call(-3) == _native.PA_ERR_ARG
    assert call(4, out_str=(896, 64, 2)) == _native.PA_ERR_ARG
    assert b"out" in lib.pa_last_error()


def test_bandwidth_probe_library_exports_its_header():
    """The benchmark's read-ceiling probes (include/bw_probe.h) load and check their
    arguments on the host before any launch."""
    import ctypes

    hdr = HEADER.with_name("bw_probe.h").read_text()
    names = sorted(set(re.findall(r"BWP_API\s+int\s+(bwp_\w+)\s*\(", hdr)))
    assert names == ["bwp_gather_blocks", "bwp_read_stream"]
    lib = ctypes.CDLL(str(Path(_native.__file__).resolve().parents[2] / "probes" /
                          "libbw_probe_gfx950.so"))
    for n in names:
        assert hasattr(lib, n)
    lib.bwp_read_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_void_p]
    lib.bwp_gather_blocks.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_int, ctypes.c_void_p]
    assert lib.bwp_read_stream(None, 1 << 20, 16, 256, None) == 1
    assert lib.bwp_read_stream(24, 1 << 20, 16, 256, None) == 1  # misaligned buffer
    assert lib.bwp_gather_blocks(16, 100, 8192, 16, 10, 16, 256, None) == 1  # block > 4 KB
    assert lib.bwp_gather_blocks(16, 100, 1000, 16, 10, 16, 256, None) == 1  # not whole KB


def test_schedule_query_names_each_path():
    """pa_decode_batched_schedule reports the path a shape takes, with no launch (the CU
    count is the current device's, 256 without a GPU as on an MI355X)."""
    cus = _device_cus()
    # One Qwen2.5-0.5B layer at batch 8: 16 short pairs, one workgroup each, no sharing.
    s = _native.decode_schedule(8, 14, 2, 64, 16, 32)
    assert s == {"path": "pair_per_workgroup", "kv_heads_per_pair": 1, "workgroups": 16,
                 "shared_prefixes": False}
    # Batch 256 of long sequences: stream-K ranges, two kv heads per pair, one workgroup per
    # CU, prefix sharing searched.
    s = _native.decode_schedule(256, 14, 2, 64, 16, 2048)
    assert s == {"path": "stream_k", "kv_heads_per_pair": 2 if 512 > cus else 1,
                 "workgroups": cus, "shared_prefixes": True}
    # Block size 8 never shares; more than 1024 sequences take the fixed splits.
    assert not _native.decode_schedule(256, 14, 2, 64, 8, 4096)["shared_prefixes"]
    assert _native.decode_schedule(1100, 14, 2, 64, 16, 64)["path"] == "fixed_split"
    lib = _native.load()
    info = (ctypes.c_int * 4)()
    assert lib.pa_decode_batched_schedule(8, 14, 2, 48, 16, 32, info) == _native.PA_ERR_ARG
