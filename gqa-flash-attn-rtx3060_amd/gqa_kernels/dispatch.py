"""Public entrypoint: choose single-pass vs split-KV path per workload.

MI355X rewrite of reference gqa_kernels/dispatch.py:14-62.  Same signature,
same asserts and the same bottom-right causal semantics; the route is sized
for the device's compute-unit count (256 on MI355X) instead of the fixed
``SM_COUNT = 28`` of the RTX 3060 version, and both routes launch hand-written
HIP kernels through the C ABI of libgqa_hip.so.
"""
from __future__ import annotations

import contextlib
import functools
import math
from dataclasses import dataclass

import torch

from . import _lib
from .gqa_split import split_kv_forward

__all__ = ["gqa_flash_attn", "Route", "choose_route"]

LOG2E = math.log2(math.e)

# Packed query rows of one single-pass workgroup, and of one split-KV row block.
FWD_ROWS = 256
SPLIT_ROWS = 32
# The split-KV path is taken for at most this many packed rows per kv head.
SPLIT_MAX_ROWS = 64
# Shortest key cache worth splitting (the reference's threshold, dispatch.py:37).
SPLIT_MIN_KV = 1024
# Keys per split-KV tile; a chunk is never shorter than this many tiles.
SPLIT_TILE = 128
SPLIT_MIN_TILES = 2
# Target workgroups per compute unit for the split-KV first pass (the kernel
# runs two per CU at once; one round of workgroups measured fastest).
SPLIT_WG_PER_CU = 2

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}


@dataclass(frozen=True)
class Route:
    kind: str  # "single" or "split"
    splits: int = 1
    workgroups: int = 0


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def choose_route(batch: int, num_heads: int, num_kv_heads: int, seq_q: int, seq_kv: int,
                 cu_count: int) -> Route:
    """Pick the kernel path for one call (pure function of the shapes).

    Counterpart of reference dispatch.py:35-45.  A query block of at most
    SPLIT_MAX_ROWS packed rows per kv head (e.g. decode: group * seq_q = 4)
    against a cache of at least SPLIT_MIN_KV keys streams K/V with the
    split-KV kernels; the split count is the power of two that brings the
    first pass to SPLIT_WG_PER_CU workgroups per compute unit, while every
    chunk keeps at least SPLIT_MIN_TILES tiles of SPLIT_TILE keys.  Anything
    else (prefill, chunked prefill) runs the single-pass kernel.
    """
    group = num_heads // num_kv_heads
    rows = group * seq_q
    single_wgs = _cdiv(seq_q, max(1, FWD_ROWS // group)) * num_kv_heads * batch
    if rows <= SPLIT_MAX_ROWS and seq_kv >= SPLIT_MIN_KV:
        base = _cdiv(rows, SPLIT_ROWS) * num_kv_heads * batch
        target = SPLIT_WG_PER_CU * cu_count
        splits = 1
        while (base * splits < target and splits < _lib.GQA_MAX_SPLITS
               and _cdiv(seq_kv, splits * 2) >= SPLIT_MIN_TILES * SPLIT_TILE):
            splits *= 2
        return Route("split", splits, base * splits)
    return Route("single", 1, single_wgs)


_route_cached = functools.lru_cache(maxsize=4096)(choose_route)


@functools.lru_cache(maxsize=None)
def _cu_count(device_index: int) -> int:
    n = _lib.load().gqa_device_cu_count(device_index)
    if n <= 0:
        raise RuntimeError(f"gqa_device_cu_count({device_index}) failed: {n}")
    return n


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """The kernels need a unit last-dim stride and 16-byte aligned rows."""
    es = t.element_size()
    ok = (t.stride(3) == 1 and t.data_ptr() % 16 == 0
          and all((s * es) % 16 == 0 for s in t.stride()[:3]))
    return t if ok else t.contiguous()


def gqa_flash_attn(q, k, v, causal=True, *, return_lse=False):
    """GQA flash attention.

    Args:
        q: (batch, num_heads,    seq_q,  head_dim)  — fp16 or bf16
        k: (batch, num_kv_heads, seq_kv, head_dim)
        v: (batch, num_kv_heads, seq_kv, head_dim)
        causal: if True, q position i (in K coordinates: i + seq_kv - seq_q)
                attends to K positions [0, q_pos]. Works for prefill
                (seq_q == seq_kv) and decode / chunked-prefill (seq_q < seq_kv).

        return_lse: (keyword-only extension, not in the reference) also return
                the natural-log log-sum-exp of the scaled scores of every
                query row, fp32 (batch, num_heads, seq_q); -inf for a row
                with no visible key.  Two attention outputs over disjoint key
                ranges merge exactly with it (context-parallel / ring
                attention, prefix-cache composition).

    Returns:
        (batch, num_heads, seq_q, head_dim), same dtype as q; with
        return_lse=True the pair (o, lse).
    """
    batch, num_heads, seq_q, head_dim = q.shape
    _, num_kv_heads, seq_kv, _ = k.shape
    assert num_heads % num_kv_heads == 0, "num_heads must be divisible by num_kv_heads"
    assert head_dim in (64, 128), f"unsupported head_dim {head_dim}"
    assert q.is_cuda and k.is_cuda and v.is_cuda
    assert q.dtype in _DTYPES, f"unsupported dtype {q.dtype}"
    assert k.dtype == q.dtype and v.dtype == q.dtype, "q, k, v must share one dtype"
    assert tuple(v.shape) == tuple(k.shape), "k and v must have the same shape"
    assert k.shape[0] == batch and k.shape[3] == head_dim, "k/v batch or head_dim differ from q"
    assert q.device == k.device == v.device, "q, k, v must be on one device"

    q_in = q
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    dev = q.device.index if q.device.index is not None else torch.cuda.current_device()
    route = _route_cached(batch, num_heads, num_kv_heads, seq_q, seq_kv, _cu_count(dev))

    # Launch on q's device (a no-op context when it is already current).
    with torch.cuda.device(dev) if dev != torch.cuda.current_device() else contextlib.nullcontext():
        if route.kind == "split":
            return split_kv_forward(q, k, v, causal, route.splits, return_lse=return_lse)

        lib = _lib.load()
        o = torch.empty_like(q_in)  # as dispatch.py:47; contiguous if unusable
        if _kernel_ready(o) is not o:
            o = torch.empty_like(q_in, memory_format=torch.contiguous_format)
        scale_log2 = (head_dim ** -0.5) * LOG2E
        stream = torch.cuda.current_stream(q.device).cuda_stream
        common = (batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim,
                  scale_log2, int(bool(causal)), _DTYPES[q.dtype], stream)
        qkvo = (q.data_ptr(), _lib.strides(q), k.data_ptr(), _lib.strides(k),
                v.data_ptr(), _lib.strides(v), o.data_ptr(), _lib.strides(o))
        if not return_lse:
            _lib.check(lib.gqa_fwd_launch(*qkvo, *common))
            return o
        lse = torch.empty(batch, num_heads, seq_q, dtype=torch.float32, device=q.device)
        _lib.check(lib.gqa_fwd_lse_launch(*qkvo, lse.data_ptr(), *common))
        return o, lse
