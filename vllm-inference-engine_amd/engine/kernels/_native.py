"""ctypes binding of libpa_gfx950.so, the gfx950 paged-attention library.

The C ABI is declared in include/paged_attention.h. torch is imported before
the library is opened: torch ships the HIP runtime as libamdhip64.so with the
SONAME libamdhip64.so.7, and the library's own dependency on that SONAME then
binds to the copy torch already loaded, so both share one runtime.

There is no fallback: when the library is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library, see above)

LIB_NAME = "libpa_gfx950.so"
LIB_PATH = Path(__file__).with_name(LIB_NAME)
ABI_VERSION = 14

PA_OK = 0
PA_ERR_ARG = 1
PA_ERR_UNSUPPORTED = 2
PA_ERR_WORKSPACE = 3
PA_ERR_HIP = 4

_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); every symbol include/paged_attention.h declares.
SIGNATURES: dict[str, tuple] = {
    "pa_abi_version": (_i32, []),
    "pa_last_error": (ctypes.c_char_p, []),
    "pa_decode_batched_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp, _i64p,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz, _vp]),
    "pa_decode_batched_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "pa_decode_kv_write_batched_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp, _i64p,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz, _vp]),
    "pa_decode_batched_schedule": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32,
                                          ctypes.POINTER(ctypes.c_int)]),
    "pa_decode_v2_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64, _i32, _i32, _vp, _i64p,
        _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz, _vp]),
    "pa_decode_v2_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "pa_decode_v1_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64, _i32, _i32, _vp, _i64p,
        _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz, _vp]),
    "pa_decode_v1_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "pa_kv_write_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "pa_prefill_copy_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i32, _i32,
        _i32, _i32, _i32, _i32, _vp]),
    "pa_rope_kv_write_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i32,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "pa_prefill_attention_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp, _i32, _vp, _i64p,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz, _vp]),
    "pa_prefill_attention_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "pa_rmsnorm_f16": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _f32,
                               _vp]),
    "pa_top2_f16": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp, _vp]),
    "pa_silu_mul_f16": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _vp]),
    "pa_decode_rope_batched_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        _vp, _i64p, _vp, _vp, _i64p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz,
        _vp]),
    "pa_decode_rope_batched_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "pa_decode_batched_noalloc_f16": (_i32, [
        _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp, _i64p,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp]),
}

_lib = None
_lock = threading.Lock()


class NativeLibraryError(RuntimeError):
    """The gfx950 library is missing, stale, or reported a failure."""


def load() -> ctypes.CDLL:
    """Open the library once and declare every exported signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryError(
                    f"{LIB_PATH} is not built; run `python vllm-inference-engine_amd/build.py` "
                    "(there is no non-HIP fallback)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            ver = lib.pa_abi_version()
            if ver != ABI_VERSION:
                raise NativeLibraryError(
                    f"{LIB_PATH} has ABI {ver}, the bindings expect {ABI_VERSION}; rebuild it")
            _lib = lib
    return _lib


def i64_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (ctypes.c_int64 * len(vals))(*vals)


_arrays: dict[tuple, ctypes.Array] = {}


def strides_of(t: torch.Tensor) -> ctypes.Array:
    """The tensor's element strides as a ctypes int64 array (cached per stride tuple)."""
    key = t.stride()
    arr = _arrays.get(key)
    if arr is None:
        if len(_arrays) > 4096:
            _arrays.clear()
        arr = _arrays[key] = i64_array(key)
    return arr


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


# torch's raw accessor of the current stream (what current_stream(d).cuda_stream
# returns, without building a Stream object: about 0.2 us a call instead of 1.8).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The HIP stream the caller's current torch stream on `device` wraps."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


_workspaces: dict[tuple, torch.Tensor] = {}

# Workspace kinds. "decode" serves pa_decode_batched_f16 and pa_decode_v2_f16:
# its first bytes are the stream-K pair counters, which must be zero when a
# buffer is first used and which every call leaves zero, so the buffer is
# zero-filled on allocation and never lent to anything else. "scores" serves
# pa_decode_v1_f16 (score rows, no zero requirement).
WS_DECODE = "decode"
WS_SCORES = "scores"
# "prefill" serves pa_prefill_attention_f16: its counters follow the same
# zero-between-calls contract as the decode ones, with another layout.
WS_PREFILL = "prefill"


# Buffers replaced by larger ones. A HIP graph captured with an older buffer's
# address keeps writing there on every replay, so a replaced buffer is never
# handed back to the allocator.
_retired: list[torch.Tensor] = []


class CaptureAllocationError(NativeLibraryError):
    """A scratch buffer would have to be allocated while a HIP graph is being captured."""


def workspace(nbytes: int, device: torch.device, stream: int, kind: str = WS_DECODE) -> int | None:
    """Device address of a scratch buffer of at least nbytes for this (device, stream, kind).

    The buffer is kept and reused by later calls on the same stream; work on
    one stream is ordered, so a call never overwrites scratch a previous call
    on that stream still reads. Calls on different streams get different
    buffers. Memory comes from torch's caching allocator; a new buffer starts
    zero-filled (the decode kernels' counters rely on it). A buffer that grows
    is replaced by one of at least twice its size and the old one is kept
    alive, since graphs captured with it still address it.

    Allocating (and zero-filling) while the current stream is capturing a
    HIP graph would record a fill into the graph and tie the buffer to the
    capture's memory pool, so it raises CaptureAllocationError instead: run
    the captured work once eagerly first, which sizes the buffer.
    """
    if nbytes == 0:
        return None
    key = (device.index, stream, kind)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise CaptureAllocationError(
                f"{kind} workspace of {nbytes} bytes for stream {stream:#x} is not allocated yet "
                "and the stream is capturing a graph; run the step once before capturing it")
        size = max(nbytes, 1 << 20, 0 if buf is None else 2 * buf.numel())
        if buf is not None:
            _retired.append(buf)
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = buf
    return buf.data_ptr()


def same_device(*tensors: torch.Tensor) -> None:
    """Every tensor of a launch lives on one GPU (the kernels take raw device pointers)."""
    dev = tensors[0].device
    assert all(t.device == dev for t in tensors), (
        "all tensors must be on the same device: " + ", ".join(str(t.device) for t in tensors))


def check(status: int, what: str) -> None:
    if status != PA_OK:
        msg = load().pa_last_error().decode(errors="replace")
        raise NativeLibraryError(f"{what} failed (status {status}): {msg}")


def decode_schedule(num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                    block_size: int, max_blocks: int) -> dict:
    """The kernel path pa_decode_batched_f16 takes for these sizes (host only, no launch)."""
    info = (ctypes.c_int * 4)()
    check(load().pa_decode_batched_schedule(num_seqs, num_q_heads, num_kv_heads, head_dim,
                                            block_size, max_blocks, info),
          "pa_decode_batched_schedule")
    path = {0: "stream_k", 1: "pair_per_workgroup", 2: "fixed_split"}[info[0]]
    return {"path": path, "kv_heads_per_pair": info[1], "workgroups": info[2],
            "shared_prefixes": bool(info[3])}
