"""Split-KV forward for short query blocks against a long KV cache.

Host side of the flash-decoding path (reference gqa_kernels/gqa_split.py:153-194):
the fp32 partials live in one workspace allocated here with torch
(caller-owned memory: the HIP library never allocates).  By default two C-ABI
launches run the first pass and then the log-sum-exp combine, the reference's
structure; ``fused=True`` runs a single launch in which the last workgroup of
each kv head combines.
"""
from __future__ import annotations

import math
import threading
import warnings

import torch

from . import _lib

__all__ = ["split_kv_forward", "decode_forward", "workspace_bytes", "stream_handle"]

# Zeroed int32 counters for the fused combine, one buffer per (device,
# stream): the kernel leaves them zero, so a buffer is reused by every call on
# its stream (calls on one stream never overlap).
_counters: dict = {}
_counters_lock = threading.Lock()

# fp32 split workspaces, one per (device, stream), grown on demand: a call's
# partials are dead once its combine has run, and calls on one stream run in
# order, so every call on that stream can reuse one buffer.  (The caching
# allocator would hand out the same memory anyway; keeping it saves the
# allocation on every decode step.)
_workspaces: dict = {}
# Buffers replaced by a larger one.  A CUDA/HIP graph captured while a buffer
# was current keeps its raw address and writes to it on every replay, so a
# superseded buffer is never released: it stays here for the life of the
# process.  Each replacement at least doubles the size, so everything kept is
# less than the current buffer again.
_retired: list = []


# The current stream's raw handle: one C call, where torch.cuda.current_stream()
# builds a Stream object (~2 µs per decode step on the host).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """hipStream_t (as an int) of the current stream on `device`."""
    if _raw_stream is None:
        return torch.cuda.current_stream(device).cuda_stream
    return _raw_stream(torch.cuda.current_device() if device.index is None else device.index)


def _workspace_buffer(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device.index, stream)
    with _counters_lock:
        buf = _workspaces.get(key)
        if buf is None or buf.numel() * 4 < nbytes:
            n = max(-(-nbytes // 4), 1 << 16)
            if buf is not None:
                _retired.append(buf)  # a captured graph may still write to it
                n = max(n, 2 * buf.numel())
            buf = torch.empty(n, dtype=torch.float32, device=device)
            _workspaces[key] = buf
        return buf


# Counter buffers of calls made while a graph was being captured: each such
# call gets its own (replays of two graphs may run concurrently on different
# streams, so they must not count in one shared buffer), and keeps it for the
# life of the process, as the graph replays into it.
_captured: list = []


def _counter_buffer(device: torch.device, stream: int, n: int) -> torch.Tensor:
    if torch.cuda.is_current_stream_capturing():
        # Zeroed by a fill kernel recorded in the graph (not a memset node),
        # so every replay also starts from zero counters.
        buf = torch.zeros(max(n, 1), dtype=torch.int32, device=device)
        with _counters_lock:
            _captured.append(buf)
        return buf
    key = (device.index, stream)
    with _counters_lock:
        buf = _counters.get(key)
        if buf is None or buf.numel() < n:
            m = max(n, 1024)
            if buf is not None:
                _retired.append(buf)  # a captured graph may still count in it
                m = max(m, 2 * buf.numel())
            buf = torch.zeros(m, dtype=torch.int32, device=device)
            _counters[key] = buf
        return buf

LOG2E = math.log2(math.e)
# The fused combine stages (valid rows of a 32-row block) x splits values in
# LDS; above this bound the two-launch form is used.
FUSED_MAX_ROW_SPLITS = 4096
# ... and addresses the partial accumulators with 32-bit byte offsets.
FUSED_MAX_ACC_BYTES = 0xFFFFFFF0

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}


def workspace_bytes(batch: int, num_heads: int, seq_q: int, head_dim: int, splits: int) -> int:
    """fp32 workspace size: acc (B,Hq,Sq,S,D) then m and l (B,Hq,Sq,S)."""
    return batch * num_heads * seq_q * splits * (head_dim + 2) * 4


_SCALE_LOG2 = {64: 64 ** -0.5 * LOG2E, 128: 128 ** -0.5 * LOG2E}


# The torch-tensor binding of the decode call, once loaded, or the reason it
# could not be (then every decode step takes the ctypes entry point).
_host_failed: list = []


def _decode_host():
    """The _gqa_host.so module, or None when it cannot be loaded (missing,
    stale, or built against another torch or library ABI): a warning is
    given once and decode_forward calls gqa_split_launch through ctypes —
    the same C entry point, with more host time per step."""
    if _lib._host is not None:
        return _lib._host
    if _host_failed:
        return None
    try:
        return _lib.load_host()
    except (RuntimeError, ImportError, OSError) as e:
        _host_failed.append(repr(e))
        warnings.warn(f"gqa_kernels: torch-tensor decode binding unavailable ({e}); "
                      "decode steps call gqa_split_launch through ctypes", RuntimeWarning, stacklevel=3)
        return None


def _split_launch_ctypes(q, k, v, ws, splits, causal, scale_log2, return_lse, stream):
    """gqa_split_launch through ctypes into a fresh o (and lse)."""
    lib = _lib.load()
    batch, num_heads, seq_q, head_dim = q.shape
    _, num_kv_heads, seq_kv, _ = k.shape
    o = torch.empty_like(q)
    lse = torch.empty(batch, num_heads, seq_q, dtype=torch.float32, device=q.device) if return_lse else None
    _lib.check(lib.gqa_split_launch(
        q.data_ptr(), _lib.strides(q), k.data_ptr(), _lib.strides(k), v.data_ptr(), _lib.strides(v),
        o.data_ptr(), _lib.strides(o), None if lse is None else lse.data_ptr(), ws.data_ptr(), splits,
        batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, scale_log2, int(bool(causal)),
        _DTYPES[q.dtype], stream))
    return o if lse is None else (o, lse)


def decode_forward(q, k, v, causal, splits, return_lse, dev):
    """The two-launch split-KV forward as gqa_flash_attn takes it: kernel-ready
    q, k, v on device index `dev` (the current device), the stream's cached
    workspace.  Computes exactly what split_kv_forward(q, k, v, causal,
    splits, return_lse=return_lse) does, with the host work of a decode step
    kept to one pass over the arguments (every value read once)."""
    batch, num_heads, seq_q, head_dim = q.shape
    stream = _raw_stream(dev) if _raw_stream is not None else torch.cuda.current_stream(dev).cuda_stream
    need = batch * num_heads * seq_q * splits * (head_dim + 2) * 4
    ws = _workspaces.get((dev, stream))
    if ws is None or ws.numel() * 4 < need:
        ws = _workspace_buffer(q.device, stream, need)
    # gqa_split_launch through the torch-tensor binding (_gqa_host.so): the
    # argument marshalling of a decode step in C++ rather than ctypes.
    host = _lib._host if _lib._host is not None else _decode_host()
    if host is None:
        return _split_launch_ctypes(q, k, v, ws, splits, causal, _SCALE_LOG2[head_dim], return_lse, stream)
    return host.split_decode(q, k, v, ws, splits, bool(causal), _SCALE_LOG2[head_dim], _DTYPES[q.dtype],
                             bool(return_lse))


def split_kv_forward(q, k, v, causal, splits, workspace=None, fused=False, return_lse=False):
    """Split-KV forward: first pass over `splits` chunks of the keys, then the
    log-sum-exp combine (a second launch, or fused into the first pass with
    ``fused=True``; the two-launch form measured faster on MI355X because the
    fused combine of the last workgroup sits on the critical path).

    ``return_lse`` also returns the natural-log LSE per query row, fp32
    (B, Hq, Sq), computed by the combine; the result is then ``(o, lse)``.

    ``workspace`` may be a caller-provided fp32 CUDA tensor with at least
    ``workspace_bytes(...) / 4`` elements; otherwise the stream's cached
    workspace is used (grown when too small).
    """
    lib = _lib.load()
    batch, num_heads, seq_q, head_dim = q.shape
    _, num_kv_heads, seq_kv, _ = k.shape
    scale_log2 = (head_dim ** -0.5) * LOG2E
    dtype = _DTYPES[q.dtype]

    need = workspace_bytes(batch, num_heads, seq_q, head_dim, splits)
    stream = stream_handle(q.device)
    if workspace is None:
        workspace = _workspace_buffer(q.device, stream, need)
    else:
        assert workspace.dtype == torch.float32 and workspace.device == q.device
        assert workspace.numel() * 4 >= need, "workspace too small"
    o = torch.empty_like(q)
    lse = torch.empty(batch, num_heads, seq_q, dtype=torch.float32, device=q.device) if return_lse else None

    group = num_heads // num_kv_heads
    if (fused and min(32, group * seq_q) * splits <= FUSED_MAX_ROW_SPLITS
            and batch * num_heads * seq_q * splits * head_dim * 4 <= FUSED_MAX_ACC_BYTES):
        n = lib.gqa_split_counters_count(batch, num_heads, num_kv_heads, seq_q)
        counters = _counter_buffer(q.device, stream, n)
        qkvo = (q.data_ptr(), _lib.strides(q), k.data_ptr(), _lib.strides(k),
                v.data_ptr(), _lib.strides(v), o.data_ptr(), _lib.strides(o))
        rest = (workspace.data_ptr(), counters.data_ptr(), splits,
                batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim,
                scale_log2, int(bool(causal)), dtype, stream)
        if lse is None:
            _lib.check(lib.gqa_split_fused_launch(*qkvo, *rest))
            return o
        _lib.check(lib.gqa_split_fused_lse_launch(*qkvo, lse.data_ptr(), *rest))
        return o, lse
    # First pass and combine through one C call (gqa_split_launch: the two
    # launches of gqa_split.py:168-193, one ctypes transition).
    _lib.check(
        lib.gqa_split_launch(
            q.data_ptr(), _lib.strides(q),
            k.data_ptr(), _lib.strides(k),
            v.data_ptr(), _lib.strides(v),
            o.data_ptr(), _lib.strides(o), None if lse is None else lse.data_ptr(),
            workspace.data_ptr(), splits,
            batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim,
            scale_log2, int(bool(causal)), dtype, stream,
        )
    )
    return o if lse is None else (o, lse)
