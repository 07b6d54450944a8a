"""Paged KV cache: attention over a block table, cache writes, prefix sharing.

The reference lists a persistent prefix KV cache and a vLLM-shaped interface
as the next step after its kernel (reference README.md:140-146: "Caching the
K/V for the static prefix and computing attention only over the new tokens";
"wrapping it in a vLLM-shaped Attention interface is mostly glue code"; "none
of the above is in this repo").  This module is that step on MI355X:

* ``paged_attention`` — the kernels of ``gqa_flash_attn`` reading K/V
  through a block table, with a length per sequence and the bottom-right
  causal alignment applied per sequence: for short query blocks (decode,
  speculative verification) the split-KV pass (libgqa_hip.so
  ``gqa_paged_split_first_launch`` + ``gqa_split_reduce[_lse]_launch``), for
  longer ones (chunked prefill against a cached prefix) the single-pass
  kernel loading each tile from its block(s)
  (``gqa_paged_fwd_launch``, blocks of >= 512 / head_dim keys).
* ``write_kv`` — store new tokens' K/V at their cache slots
  (``gqa_paged_cache_write_launch``).
* ``PagedKVCache`` — host-side block allocator with reference-counted blocks:
  a shared prefix (system prompt, memory block) is stored once and every
  sequence forked from it attends to it without recomputing its K/V; a
  partly filled shared block is copied before a sequence writes into it.
* ``GQAPagedAttention`` / ``PagedAttentionMetadata`` — a vLLM-shaped layer:
  ``forward(query, key, value, kv_cache, attn_metadata)`` on flattened
  token-major tensors, cache ``(2, num_blocks, block_size, Hkv, D)``.

Cache layout: ``k_cache``/``v_cache`` are ``(num_blocks, block_size, Hkv, D)``
(block_size a power of two); key j of sequence b is slot ``j % block_size``
of block ``block_table[b, j // block_size]``.  A slot index is
``block * block_size + offset``.
"""
from __future__ import annotations

import functools
import math
import threading
from dataclasses import dataclass
from typing import Dict, Hashable, List, Optional, Sequence

import torch

from . import _lib
from .dispatch import (FWD_ROWS, SPLIT_MIN_KV, _fwd_block_tiles, choose_fwd_split, choose_kv_chunks,
                       fwd_split_makespan)
from .gqa_split import _counter_buffer, _decode_host, _workspace_buffer, stream_handle, workspace_bytes

__all__ = [
    "paged_attention",
    "write_kv",
    "paged_chunk",
    "paged_splits",
    "paged_kv_chunks",
    "paged_single_plan",
    "PagedKVCache",
    "PagedAttentionMetadata",
    "GQAPagedAttention",
]

LOG2E = math.log2(math.e)
_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}

# Split sizing: a power of two split count that brings the first pass to a
# number of workgroups per compute unit, every chunk keeping at least two
# 128-key tiles.  Workgroups per CU: two for the register-staged first pass
# (head_dim 64 over more than 16 rows, pages of 1-2 keys, or 4 at head_dim
# 64); for the LDS-DMA first pass (head_dim 128 with pages of >= 4 keys, and
# head_dim 64 with at most 16 rows and pages of >= 8 keys) one, or four for
# a single-token step of a batch of sequences over pages whose heads of a
# key are interleaved (token-major, slot stride != head_dim).  Measured on MI355X (bf16, Hq = 32, Hkv = 8,
# random block order, us): head-major 64-key pages, one token, 131072 keys
# 32 / 64 splits 83.3 / 85.0, B = 4 x 32768 8 / 16 splits 81.0 / 84.6,
# B = 16 x 8192 2 / 4 80.8 / 83.0, 16 tokens at 32768 keys 32 / 64 32.7 /
# 39.2; token-major 16-key pages, one token, 131072 keys 32 / 64 87.8 /
# 89.1, B = 4 x 32768 8 / 16 / 32 splits 90.3 / 88.3 / 86.4, B = 16 x 8192
# 2 / 4 / 8 90.3 / 92.2 / 88.9; several tokens, B = 2 x 32768 16 tokens
# 16 / 32 / 64 splits 56.6 / 58.4 / 71.3, B = 8 x 8192 4 tokens 4 / 8 / 16
# 49.8 / 50.6 / 51.1.  Head_dim 64, one token, fill / 2x / 4x the fill
# count: head-major 64-key pages 131072 keys 44.7 / 45.8 / 46.5, B = 16 x
# 8192 44.7 / 46.1 / 47.2; token-major 16-key pages 131072 keys 51.0 / 52.3
# / 52.8, B = 4 x 32768 53.5 / 48.6 / 48.9, B = 16 x 8192 54.0 / 56.2 /
# 49.5.
# Batches of several sequences: the counts above assume every sequence is
# max_seq_len keys long; with unequal lengths the longest sequences' few
# long chunks set the run time, so such a batch is cut into at least
# _BATCH_MIN_SPLITS chunks per sequence while chunks keep _MIN_CHUNK keys
# and the first pass stays within _BATCH_MAX_WG_PER_CU workgroups per CU.
# Measured (16-key pages, one token, us, the count chosen before -> after):
# lengths random in 100-8000, B = 32: token-major 4 -> 8 splits 113.3 ->
# 107.3, head-major 1 -> 8 120.2 -> 108.2; 500-16000, B = 16: head-major
# 2 -> 8 121.0 -> 109.6 (token-major already 8); 1000-30000, B = 8:
# head-major 4 -> 8 113.4 -> 101.2; 100-4000, B = 64: token-major 2 -> 4
# 122.8 -> 120.0, head-major 1 -> 4 113.5 -> 116.7 (8 splits: 119.9, so the
# workgroup cap); eight such batches 929 -> 887 us in all.  Uniform lengths
# pay: B = 32 x 4096 head-major 82.8 -> 88.5, B = 8 x 16384 82.9 -> 84.9
# (four uniform batches 345 -> 353 us).
_BATCH_MIN_SPLITS = 8
_BATCH_MAX_WG_PER_CU = 8
_SPLIT_ROWS = 32
_SPLIT_WG_PER_CU = 2
_LDS_WG_PER_CU = 1
_LDS_WG_PER_CU_INTERLEAVED = 4
_MIN_CHUNK = 256
_SPLIT_MAX_ROWS = 64  # packed rows per kv head up to which the split-KV pass is used
_SPLIT_MAX_ROWS_WIDE = 128  # ... at head_dim 128 with pages of >= 4 keys (128-row workgroups)
_DEC16_ROWS = 16  # packed rows up to which head_dim 64 runs the LDS-DMA first pass

_cu_lock = threading.Lock()
_cu_counts: dict = {}


def _cu_count(device_index: int) -> int:
    with _cu_lock:
        n = _cu_counts.get(device_index)
        if n is None:
            n = _lib.load().gqa_device_cu_count(device_index)
            if n <= 0:
                raise RuntimeError(f"gqa_device_cu_count({device_index}) failed: {n}")
            _cu_counts[device_index] = n
        return n


def paged_chunk(max_seq_len: int, splits: int) -> int:
    """Keys per split chunk of the paged first pass: ceil(max_seq_len /
    splits) rounded up to a multiple of 64 (as gqa_paged_split_first_launch
    computes it)."""
    return (-(-max_seq_len // splits) + 63) & ~63


@functools.lru_cache(maxsize=4096)
def paged_splits(batch: int, num_heads: int, num_kv_heads: int, seq_q: int, max_seq_len: int,
                 cu_count: int, block_size: int = 64, head_dim: int = 128,
                 heads_interleaved: bool = False) -> int:
    """Split count for a paged call: the power of two that brings the first
    pass to its target workgroups per compute unit (for the LDS-DMA first
    pass — head_dim 128 with pages of >= 4 keys, head_dim 64 with at most 16
    packed rows and pages of >= 8 keys — one, or four for a single-token
    step of a batch over pages whose heads are interleaved; else two) while every chunk keeps at
    least 256 keys (pure function of the shapes and of ``heads_interleaved``:
    the cache's slot stride differs from head_dim); a batch of several
    sequences, whose lengths may differ, gets at least 8 chunks per sequence
    within 8 workgroups per CU.  With pages under 64 keys a chunk spans
    at most GQA_PAGED_CHUNK_PAGES pages (the slice of the block table a
    workgroup stages in LDS), which can ask for more splits."""
    group = num_heads // num_kv_heads
    rows = group * seq_q
    # Rows per first-pass workgroup: up to four 32-row blocks at head_dim 128
    # with pages of >= 4 keys (the LDS-DMA first pass), else one.
    lds_pass = ((head_dim == 128 and block_size >= 4)
                or (head_dim == 64 and block_size >= 8 and rows <= _DEC16_ROWS))
    rpw = _SPLIT_ROWS
    if lds_pass and rows > _SPLIT_ROWS:
        rpw = 2 * _SPLIT_ROWS if rows <= 2 * _SPLIT_ROWS else 4 * _SPLIT_ROWS
    base = -(-rows // rpw) * num_kv_heads * batch
    if lds_pass:
        wide = heads_interleaved and batch > 1 and seq_q == 1
        per_cu = _LDS_WG_PER_CU_INTERLEAVED if wide else _LDS_WG_PER_CU
    else:
        per_cu = _SPLIT_WG_PER_CU
    target = per_cu * cu_count
    splits = 1
    while (base * splits < target and splits < _lib.GQA_MAX_SPLITS
           and -(-max_seq_len // (splits * 2)) >= _MIN_CHUNK):
        splits *= 2
    if batch > 1:
        while (splits < _BATCH_MIN_SPLITS and base * splits * 2 <= _BATCH_MAX_WG_PER_CU * cu_count
               and -(-max_seq_len // (splits * 2)) >= _MIN_CHUNK):
            splits *= 2
    if block_size < 64:
        def too_many_pages(s):
            return paged_chunk(max_seq_len, s) // block_size > _lib.GQA_PAGED_CHUNK_PAGES
        while too_many_pages(splits) and splits < _lib.GQA_MAX_SPLITS:
            splits *= 2
        if too_many_pages(splits):
            raise ValueError(
                f"paged split-KV: max_seq_len {max_seq_len} over {block_size}-key blocks needs chunks of at "
                f"most {_lib.GQA_PAGED_CHUNK_PAGES} blocks, more than {_lib.GQA_MAX_SPLITS} splits give; "
                f"use blocks of >= 64 keys or a shorter max_seq_len")
    return splits


_ROUTE_IDS = {"split": 0, "single": 1, "chunks": 2}


def _paged_host():
    """The torch-tensor bindings (_gqa_host.so paged_forward / cache_write),
    or None when they cannot be loaded: paged_attention and write_kv then
    call the same C entry points through ctypes, with more host time per
    call."""
    host = _lib._host if _lib._host is not None else _decode_host()
    return host if host is not None and hasattr(host, "paged_forward") else None


def _rows_ready(t: torch.Tensor) -> bool:
    """Unit last-dim stride and 16-byte aligned rows (what the kernels load):
    the pointer and every other stride in bytes a multiple of 16, tested at
    once on their bitwise or."""
    st = t.stride()
    if st[-1] != 1:
        return False
    bits = 0
    for x in st[:-1]:
        bits |= x
    return (t.data_ptr() | bits * t.element_size()) % 16 == 0


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor) -> int:
    assert k_cache.dim() == 4 and tuple(k_cache.shape) == tuple(v_cache.shape), \
        "k_cache / v_cache must be (num_blocks, block_size, num_kv_heads, head_dim)"
    assert k_cache.dtype == v_cache.dtype and k_cache.device == v_cache.device
    block_size = k_cache.shape[1]
    assert 1 <= block_size <= _lib.GQA_MAX_BLOCK_SIZE and block_size & (block_size - 1) == 0, \
        "block_size must be a power of two"
    assert _rows_ready(k_cache) and _rows_ready(v_cache), "cache rows must be contiguous and 16-byte aligned"
    return block_size


def single_pass_min_block(head_dim: int) -> int:
    """Smallest block_size the single-pass paged kernel takes: the 512 /
    head_dim rows one of its LDS-DMA instructions loads must lie in one
    block."""
    return 512 // head_dim


def paged_route(num_heads: int, num_kv_heads: int, seq_q: int, block_size: int, head_dim: int = 128) -> str:
    """"split" (split-KV first pass + combine) for short query blocks, as the
    contiguous decode route; "single" (the single-pass kernel loading each
    tile from its blocks) for longer ones when blocks hold at least
    single_pass_min_block(head_dim) keys."""
    max_rows = _SPLIT_MAX_ROWS_WIDE if head_dim == 128 and block_size >= 4 else _SPLIT_MAX_ROWS
    if (num_heads // num_kv_heads) * seq_q <= max_rows or block_size < single_pass_min_block(head_dim):
        return "split"
    return "single"


@functools.lru_cache(maxsize=4096)
def paged_single_plan(batch: int, num_heads: int, num_kv_heads: int, seq_q: int, max_seq_len: int,
                      cu_count: int, causal: bool = True, head_dim: int = 128):
    """(key chunks, split blocks) for the paged single pass, at most one of
    them non-zero.

    The paged single pass runs one workgroup per query block.  Under causal
    masking the last blocks of a sequence see the most keys and set the run
    time when there are few workgroups per CU; running the heaviest ones as
    two key halves (gqa_paged_fwd_split_launch) shortens that chain
    (dispatch.choose_fwd_split).  With fewer blocks than compute units
    against long sequences (a chunk of new tokens over a long cached prefix,
    few sequences) most CUs idle, and splitting every block's key range
    (gqa_paged_fwd_chunks_launch) fills them at the cost of the fp32
    partials and the combine launch (dispatch.choose_kv_chunks, against the
    split single pass, from SPLIT_MIN_KV keys on: the length from which the
    reference splits the key axis at all).  The models are those of the
    contiguous route for a kernel of one workgroup per item.  Cached: every
    layer of a model step asks with the same arguments."""
    n_split = choose_fwd_split(batch, num_heads, num_kv_heads, seq_q, max_seq_len, cu_count, causal, head_dim,
                               persistent=False)
    block_m = max(1, FWD_ROWS // (num_heads // num_kv_heads))
    n_mblk = -(-seq_q // block_m)
    if n_mblk * num_kv_heads * batch < cu_count and seq_q > 0 and max_seq_len >= SPLIT_MIN_KV:
        tiles = _fwd_block_tiles(n_mblk, block_m, seq_q, max_seq_len, causal)
        base = fwd_split_makespan(tiles, n_split, num_kv_heads * batch, cu_count, causal, persistent=False)
        kc = choose_kv_chunks(batch, num_heads, num_kv_heads, seq_q, max_seq_len, cu_count, causal, head_dim, base,
                              persistent=False)
        if kc:
            return kc, 0
    return 0, n_split


def paged_kv_chunks(batch: int, num_heads: int, num_kv_heads: int, seq_q: int, max_seq_len: int,
                    cu_count: int, causal: bool = True, head_dim: int = 128) -> int:
    """Key chunks per query block for the paged single pass (0: none; see
    paged_single_plan)."""
    return paged_single_plan(batch, num_heads, num_kv_heads, seq_q, max_seq_len, cu_count, causal, head_dim)[0]


def paged_attention(q, k_cache, v_cache, block_table, seq_lens, causal=True, *,
                    max_seq_len: Optional[int] = None, scale: Optional[float] = None,
                    splits: Optional[int] = None, return_lse: bool = False,
                    out: Optional[torch.Tensor] = None, route: Optional[str] = None,
                    query_start: Optional[torch.Tensor] = None, query_lens: Optional[torch.Tensor] = None,
                    max_query_len: Optional[int] = None):
    """GQA attention of q over K/V held in a paged cache.

    Args:
        q: (batch, num_heads, seq_q, head_dim), fp16 or bf16 (any strides with
            a contiguous, 16-byte aligned last dimension).
        k_cache, v_cache: (num_blocks, block_size, num_kv_heads, head_dim),
            q's dtype; block_size a power of two.
        block_table: int32 (batch, max_blocks_per_seq); row b lists the
            blocks of sequence b in key order (entries past the sequence's
            length are not read).
        seq_lens: int32 (batch,) — keys of each sequence, including the
            seq_q new tokens (whose K/V must already be in the cache).
        causal: query row i of sequence b attends keys
            [0, i + seq_lens[b] - seq_q] (bottom-right alignment, as
            gqa_flash_attn with seq_kv = seq_lens[b]).
        max_seq_len: an upper bound of seq_lens (sizes the split chunks;
            keys past it are not read).  Default: the table's capacity,
            max_blocks_per_seq * block_size, which needs no device read.
        scale: score scale (default head_dim ** -0.5, the reference's).
        splits: split count of the split route (default: ``paged_splits``),
            key chunks per query block of the "chunks" route (default:
            ``paged_kv_chunks``, at least 2), or query blocks run as two key
            halves on the "single" route (default: none when "single" is
            forced, ``paged_single_plan``'s count when routed).
        return_lse: also return the natural-log LSE per row, fp32
            (batch, num_heads, seq_q).
        out: optional (batch, num_heads, seq_q, head_dim) tensor of q's dtype
            (any strides with 16-byte aligned rows) to write o into.
        route: "split", "single" or "chunks" to force a kernel (default:
            paged_route, and "chunks" in place of "single" when
            paged_kv_chunks finds few query blocks against long sequences;
            "single" and "chunks" need block_size >= 512 / head_dim).
        query_start, query_lens, max_query_len: variable query lengths.  q
            is then token-major (num_tokens, num_heads, head_dim); sequence
            b's queries are tokens query_start[b] .. + query_lens[b] - 1
            (int32 device tensors of batch entries), max_query_len (a host
            int) bounds query_lens; causal alignment per sequence uses its own
            query length; o (and out) are (num_tokens, num_heads, head_dim),
            lse (num_tokens, num_heads).

    Returns:
        o (batch, num_heads, seq_q, head_dim), or (o, lse).
    """
    varlen = query_start is not None
    qdev = q.device
    if varlen:
        assert query_lens is not None and max_query_len is not None, "varlen needs query_lens and max_query_len"
        assert q.dim() == 3, "varlen q is (num_tokens, num_heads, head_dim)"
        num_tokens, num_heads, head_dim = q.shape
        batch, seq_q = seq_lens.shape[0], int(max_query_len)
        assert query_start.dtype == torch.int32 and query_lens.dtype == torch.int32
        assert tuple(query_start.shape) == (batch,) and tuple(query_lens.shape) == (batch,)
        assert query_start.device == qdev and query_lens.device == qdev
        query_start, query_lens = query_start.contiguous(), query_lens.contiguous()
    else:
        batch, num_heads, seq_q, head_dim = q.shape
    block_size = _check_cache(k_cache, v_cache)
    num_kv_heads = k_cache.shape[2]
    assert num_heads % num_kv_heads == 0, "num_heads must be divisible by num_kv_heads"
    assert head_dim in (64, 128), f"unsupported head_dim {head_dim}"
    assert k_cache.shape[3] == head_dim, "cache head_dim differs from q"
    assert q.dtype in _DTYPES and k_cache.dtype == q.dtype, "q and the caches must share one fp16/bf16 dtype"
    assert q.is_cuda and k_cache.device == qdev
    assert block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == batch
    assert seq_lens.dtype == torch.int32 and tuple(seq_lens.shape) == (batch,)
    assert block_table.device == qdev and seq_lens.device == qdev
    if block_table.stride(1) != 1 or (batch > 1 and block_table.stride(0) < block_table.shape[1]):
        block_table = block_table.contiguous()
    seq_lens = seq_lens.contiguous()
    if not _rows_ready(q):
        q = q.contiguous()
    if varlen:
        # one 16-byte aligned token row per head
        assert q.stride(2) == 1 and (q.stride(1) * q.element_size()) % 16 == 0

    table_stride = block_table.stride(0) if batch > 1 else block_table.shape[1]
    capacity = block_table.shape[1] * block_size
    if max_seq_len is None:
        max_seq_len = capacity
    assert 0 <= max_seq_len <= capacity, "max_seq_len exceeds the block table's capacity"
    dev = qdev.index if qdev.index is not None else torch.cuda.current_device()
    splits_given = splits is not None
    if splits is None:
        interleaved = k_cache.stride(1) != head_dim or v_cache.stride(1) != head_dim
        splits = paged_splits(batch, num_heads, num_kv_heads, seq_q, max_seq_len, _cu_count(dev), block_size,
                              head_dim, interleaved)
    if scale is None:
        scale = head_dim ** -0.5

    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=qdev)
    else:
        assert tuple(out.shape) == tuple(q.shape) and out.dtype == q.dtype and out.device == qdev
        assert _rows_ready(out), "out rows must be contiguous and 16-byte aligned"
    lse_shape = (q.shape[0], num_heads) if varlen else (batch, num_heads, seq_q)

    lib = _lib.load()
    dtype = _DTYPES[q.dtype]
    stream = stream_handle(qdev)
    kv_chunks = fwd_split = 0
    if route is None:
        route = paged_route(num_heads, num_kv_heads, seq_q, block_size, head_dim)
        if route == "single":
            kv_chunks, fwd_split = paged_single_plan(batch, num_heads, num_kv_heads, seq_q, max_seq_len,
                                                     _cu_count(dev), bool(causal), head_dim)
            route = "chunks" if kv_chunks else route
    elif route == "single":
        fwd_split = splits if splits_given else 0
    elif route == "chunks":
        kv_chunks = splits if splits_given else max(2, paged_kv_chunks(
            batch, num_heads, num_kv_heads, seq_q, max_seq_len, _cu_count(dev), causal, head_dim))
    assert route in ("split", "single", "chunks")
    assert route == "split" or block_size >= single_pass_min_block(head_dim)
    lse = torch.empty(lse_shape, dtype=torch.float32, device=qdev) if return_lse else None
    counters = None
    if route == "single":
        # Split query blocks: their halves' fp32 state and the stream's
        # zeroed merge counters (left zero by the kernel).
        n_parts = fwd_split
        workspace = None if not fwd_split else _workspace_buffer(
            qdev, stream, lib.gqa_fwd_split_workspace_bytes(batch, num_kv_heads, head_dim, fwd_split))
        if fwd_split:
            counters = _counter_buffer(qdev, stream, lib.gqa_fwd_split_counters_count(batch, num_kv_heads, fwd_split))
    else:
        n_parts = kv_chunks if route == "chunks" else splits
        workspace = _workspace_buffer(qdev, stream, workspace_bytes(batch, num_heads, seq_q, head_dim, n_parts))
    host = _paged_host()
    if host is not None:
        host.paged_forward(_ROUTE_IDS[route], q, k_cache, v_cache, block_table, table_stride, seq_lens,
                           query_start if varlen else None, query_lens if varlen else None, max_seq_len, out, lse,
                           workspace, counters, n_parts, batch, seq_q, scale * LOG2E, bool(causal), dtype)
        return out if lse is None else (out, lse)
    # Token-major q / o as the kernels address them: (unused, head, token, d).
    qst = _lib._i64x4(0, q.stride(1), q.stride(0), 1) if varlen else _lib.strides(q)
    ost = _lib._i64x4(0, out.stride(1), out.stride(0), 1) if varlen else _lib.strides(out)
    qs_p = query_start.data_ptr() if varlen else None
    ql_p = query_lens.data_ptr() if varlen else None
    lse_p = None if lse is None else lse.data_ptr()
    if route == "chunks":
        _lib.check(lib.gqa_paged_fwd_chunks_launch(
            q.data_ptr(), qst, k_cache.data_ptr(), _lib.strides(k_cache),
            v_cache.data_ptr(), _lib.strides(v_cache), block_table.data_ptr(), table_stride,
            seq_lens.data_ptr(), qs_p, ql_p, block_size, max_seq_len, out.data_ptr(), ost,
            lse_p, workspace.data_ptr(), kv_chunks, batch, num_heads, num_kv_heads, seq_q, head_dim,
            scale * LOG2E, int(bool(causal)), dtype, stream))
        return out if lse is None else (out, lse)
    if route == "single" and fwd_split:
        _lib.check(lib.gqa_paged_fwd_split_launch(
            q.data_ptr(), qst, k_cache.data_ptr(), _lib.strides(k_cache),
            v_cache.data_ptr(), _lib.strides(v_cache), block_table.data_ptr(), table_stride,
            seq_lens.data_ptr(), qs_p, ql_p, block_size, max_seq_len, out.data_ptr(), ost,
            lse_p, workspace.data_ptr(), counters.data_ptr(), fwd_split, batch, num_heads, num_kv_heads, seq_q,
            head_dim, scale * LOG2E, int(bool(causal)), dtype, stream))
        return out if lse is None else (out, lse)
    if route == "single":
        _lib.check(lib.gqa_paged_fwd_launch(
            q.data_ptr(), qst, k_cache.data_ptr(), _lib.strides(k_cache),
            v_cache.data_ptr(), _lib.strides(v_cache), block_table.data_ptr(), table_stride,
            seq_lens.data_ptr(), qs_p, ql_p, block_size, max_seq_len, out.data_ptr(), ost,
            lse_p, batch, num_heads, num_kv_heads, seq_q, head_dim,
            scale * LOG2E, int(bool(causal)), dtype, stream))
        return out if lse is None else (out, lse)
    _lib.check(lib.gqa_paged_split_first_launch(
        q.data_ptr(), qst, k_cache.data_ptr(), _lib.strides(k_cache),
        v_cache.data_ptr(), _lib.strides(v_cache), block_table.data_ptr(), table_stride,
        seq_lens.data_ptr(), qs_p, ql_p, block_size, max_seq_len, workspace.data_ptr(), splits,
        batch, num_heads, num_kv_heads, seq_q, head_dim, scale * LOG2E, int(bool(causal)), dtype, stream))
    if varlen:
        _lib.check(lib.gqa_split_reduce_varlen_launch(workspace.data_ptr(), splits, out.data_ptr(), ost, lse_p,
                                                      qs_p, ql_p, batch, num_heads, seq_q, head_dim, dtype, stream))
    elif lse is None:
        _lib.check(lib.gqa_split_reduce_launch(workspace.data_ptr(), splits, out.data_ptr(), ost,
                                               batch, num_heads, seq_q, head_dim, dtype, stream))
    else:
        _lib.check(lib.gqa_split_reduce_lse_launch(workspace.data_ptr(), splits, out.data_ptr(), ost,
                                                   lse_p, batch, num_heads, seq_q, head_dim, dtype, stream))
    return out if lse is None else (out, lse)


def write_kv(key, value, k_cache, v_cache, slot_mapping):
    """Store K/V of new tokens at their cache slots (in place).

    key, value: (num_tokens, num_kv_heads, head_dim) in the caches' dtype;
    slot_mapping: int64 (num_tokens,), slot = block * block_size + offset,
    negative = skip (padding).  Every non-negative slot must lie inside the
    caches.
    """
    block_size = _check_cache(k_cache, v_cache)
    num_tokens, num_kv_heads, head_dim = key.shape
    assert tuple(value.shape) == tuple(key.shape)
    assert k_cache.shape[2] == num_kv_heads and k_cache.shape[3] == head_dim
    assert key.dtype == k_cache.dtype == value.dtype and key.dtype in _DTYPES
    assert slot_mapping.dtype == torch.int64 and tuple(slot_mapping.shape) == (num_tokens,)
    assert key.device == value.device == k_cache.device == slot_mapping.device and key.is_cuda
    slot_mapping = slot_mapping.contiguous()
    key = key if _rows_ready(key) else key.contiguous()
    value = value if _rows_ready(value) else value.contiguous()
    host = _paged_host()
    if host is not None:
        host.cache_write(key, value, k_cache, v_cache, slot_mapping, _DTYPES[key.dtype])
        return
    lib = _lib.load()
    stream = stream_handle(key.device)
    _lib.check(lib.gqa_paged_cache_write_launch(
        key.data_ptr(), _lib.strides3(key), value.data_ptr(), _lib.strides3(value),
        k_cache.data_ptr(), _lib.strides(k_cache), v_cache.data_ptr(), _lib.strides(v_cache),
        slot_mapping.data_ptr(), num_tokens, num_kv_heads, head_dim, block_size, _DTYPES[key.dtype], stream))


# ---------------------------------------------------------------------------
# Block allocator with prefix sharing
# ---------------------------------------------------------------------------
class _Seq:
    __slots__ = ("blocks", "length")

    def __init__(self, blocks: List[int], length: int):
        self.blocks = blocks
        self.length = length


class PagedKVCache:
    """K/V of many sequences in one pair of paged caches.

    Blocks are reference counted: ``fork`` gives a new sequence the blocks of
    an existing one (a persistent prefix is computed and stored once), and a
    partly filled block that more than one sequence holds is copied before
    one of them appends to it, so forks never see each other's new tokens.

    The K/V tensors are ``kv[0]`` and ``kv[1]`` of one
    ``(2, num_blocks, block_size, num_kv_heads, head_dim)`` tensor (indexing
    order), the shape a vLLM attention backend receives as ``kv_cache``.
    ``layout`` is the storage order inside a block: "HND" (default; heads
    outer, so each head's rows of a block are consecutive and the split-KV
    kernel streams them with the same access pattern as contiguous K/V,
    about 8% faster on MI355X at 131072 keys) or "NHD" (slots outer, vLLM's
    FlashAttention layout).  Both are strided views the kernels take as they
    are.
    """

    def __init__(self, num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
                 dtype=torch.bfloat16, device="cuda", layout: str = "HND"):
        assert num_blocks > 0 and block_size > 0 and block_size & (block_size - 1) == 0
        assert layout in ("HND", "NHD"), layout
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.layout = layout
        if layout == "HND":
            self.kv = torch.zeros(2, num_blocks, num_kv_heads, block_size, head_dim, dtype=dtype,
                                  device=device).transpose(2, 3)
        else:
            self.kv = torch.zeros(2, num_blocks, block_size, num_kv_heads, head_dim, dtype=dtype, device=device)
        self._free: List[int] = list(range(num_blocks - 1, -1, -1))
        self._refs: List[int] = [0] * num_blocks
        self._seqs: Dict[Hashable, _Seq] = {}

    # -- views ---------------------------------------------------------------
    @property
    def k_cache(self) -> torch.Tensor:
        return self.kv[0]

    @property
    def v_cache(self) -> torch.Tensor:
        return self.kv[1]

    def num_free_blocks(self) -> int:
        return len(self._free)

    def seq_len(self, seq_id) -> int:
        return self._seqs[seq_id].length

    def blocks(self, seq_id) -> List[int]:
        return list(self._seqs[seq_id].blocks)

    # -- sequence lifetime ---------------------------------------------------
    def add_sequence(self, seq_id) -> None:
        assert seq_id not in self._seqs, f"sequence {seq_id!r} exists"
        self._seqs[seq_id] = _Seq([], 0)

    def fork(self, src_id, dst_id) -> None:
        """New sequence dst_id sharing every block (and the length) of src_id."""
        assert dst_id not in self._seqs, f"sequence {dst_id!r} exists"
        src = self._seqs[src_id]
        for b in src.blocks:
            self._refs[b] += 1
        self._seqs[dst_id] = _Seq(list(src.blocks), src.length)

    def free(self, seq_id) -> None:
        for b in self._seqs.pop(seq_id).blocks:
            self._refs[b] -= 1
            if self._refs[b] == 0:
                self._free.append(b)

    def _alloc(self) -> int:
        if not self._free:
            raise RuntimeError("paged KV cache out of blocks")
        b = self._free.pop()
        self._refs[b] = 1
        return b

    # -- writing -------------------------------------------------------------
    def reserve(self, seq_id, n: int) -> List[int]:
        """Slots for the next n tokens of seq_id (allocating blocks, copying a
        shared partly filled last block first); the length grows by n."""
        s = self._seqs[seq_id]
        bs = self.block_size
        if n <= 0:
            return []
        cow = s.length % bs != 0 and self._refs[s.blocks[-1]] > 1
        need = -(-(s.length + n) // bs) - len(s.blocks)
        if need + cow > len(self._free):
            raise RuntimeError("paged KV cache out of blocks")
        if cow:
            old = s.blocks[-1]
            new = self._alloc()
            self.kv[:, new].copy_(self.kv[:, old])
            self._refs[old] -= 1
            s.blocks[-1] = new
        for _ in range(need):
            s.blocks.append(self._alloc())
        slots = [s.blocks[j // bs] * bs + j % bs for j in range(s.length, s.length + n)]
        s.length += n
        return slots

    def append(self, seq_ids: Sequence, key: torch.Tensor, value: torch.Tensor,
               num_new: Optional[Sequence[int]] = None) -> torch.Tensor:
        """Append K/V of new tokens, sequence-major: the first num_new[0]
        rows of key/value (num_tokens, num_kv_heads, head_dim) belong to
        seq_ids[0], and so on (default: an equal share each).  Returns the
        int64 slot mapping written."""
        if num_new is None:
            assert key.shape[0] % len(seq_ids) == 0
            num_new = [key.shape[0] // len(seq_ids)] * len(seq_ids)
        assert sum(num_new) == key.shape[0]
        slots: List[int] = []
        for sid, n in zip(seq_ids, num_new):
            slots += self.reserve(sid, n)
        slot_mapping = torch.tensor(slots, dtype=torch.int64).to(self.kv.device)
        write_kv(key, value, self.k_cache, self.v_cache, slot_mapping)
        return slot_mapping

    # -- attention -----------------------------------------------------------
    def block_table(self, seq_ids: Sequence) -> torch.Tensor:
        """int32 (len(seq_ids), max blocks) on the cache's device; unused
        entries are 0 (never read)."""
        rows = [self._seqs[s].blocks for s in seq_ids]
        width = max(1, max(len(r) for r in rows))
        table = torch.zeros(len(rows), width, dtype=torch.int32)
        for i, r in enumerate(rows):
            if r:
                table[i, :len(r)] = torch.tensor(r, dtype=torch.int32)
        return table.to(self.kv.device)

    def seq_lens(self, seq_ids: Sequence) -> torch.Tensor:
        return torch.tensor([self._seqs[s].length for s in seq_ids], dtype=torch.int32).to(self.kv.device)

    def attend(self, q: torch.Tensor, seq_ids: Sequence, causal: bool = True, *, return_lse: bool = False):
        """paged_attention of q (len(seq_ids), num_heads, seq_q, head_dim)
        over these sequences (their new tokens already appended)."""
        max_len = max(self._seqs[s].length for s in seq_ids)
        return paged_attention(q, self.k_cache, self.v_cache, self.block_table(seq_ids), self.seq_lens(seq_ids),
                               causal, max_seq_len=max_len, return_lse=return_lse)


# ---------------------------------------------------------------------------
# vLLM-shaped layer
# ---------------------------------------------------------------------------
@dataclass
class PagedAttentionMetadata:
    """Per-step batch description, in the names vLLM's attention metadata uses.

    slot_mapping: int64 (num_tokens,) cache slot of every new token (-1: pad).
    block_tables: int32 (num_seqs, max_blocks_per_seq).
    seq_lens: int32 (num_seqs,) keys per sequence, new tokens included.
    query_len: new tokens per sequence when they are all equal (1 for
        decode, k for speculative verification, the chunk for chunked prefill).
    query_lens: new tokens of each sequence (host ints) for a mixed batch
        (prefill chunks and decode steps together); overrides query_len.
    max_seq_len: an upper bound of seq_lens (default: the tables' capacity).
    """
    slot_mapping: torch.Tensor
    block_tables: torch.Tensor
    seq_lens: torch.Tensor
    query_len: int = 1
    max_seq_len: Optional[int] = None
    query_lens: Optional[Sequence[int]] = None


class GQAPagedAttention(torch.nn.Module):
    """Attention layer with the call shape of a vLLM attention backend.

    ``forward(query, key, value, kv_cache, attn_metadata)``:
      query (num_tokens, num_heads * head_size), key/value
      (num_tokens, num_kv_heads * head_size) or None (nothing to store),
      kv_cache (2, num_blocks, block_size, num_kv_heads, head_size).
    Tokens are sequence-major: ``attn_metadata.query_len`` per sequence, or
    ``attn_metadata.query_lens[b]`` for sequence b of a mixed batch.  The new
    K/V are stored at ``slot_mapping`` first, then every query attends its
    sequence's cache (causal, bottom-right aligned).  A mixed batch runs as
    up to two launches over token-major q/o views, one for the sequences
    whose query block suits the split-KV pass (decode-like) and one for the
    rest (prefill chunks).  Returns (num_tokens, num_heads * head_size),
    written in place when ``output`` is given.
    """

    def __init__(self, num_heads: int, head_size: int, scale: Optional[float] = None,
                 num_kv_heads: Optional[int] = None, causal: bool = True):
        super().__init__()
        self.num_heads = num_heads
        self.head_size = head_size
        self.num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        assert num_heads % self.num_kv_heads == 0, "num_heads must be divisible by num_kv_heads"
        assert head_size in (64, 128), f"unsupported head_size {head_size}"
        self.scale = head_size ** -0.5 if scale is None else float(scale)
        self.causal = causal

    def forward(self, query, key, value, kv_cache, attn_metadata: PagedAttentionMetadata, output=None):
        md = attn_metadata
        num_tokens = query.shape[0]
        H, Hkv, D = self.num_heads, self.num_kv_heads, self.head_size
        batch = md.block_tables.shape[0]
        assert kv_cache.dim() == 5 and kv_cache.shape[0] == 2 and kv_cache.shape[3] == Hkv and kv_cache.shape[4] == D
        k_cache, v_cache = kv_cache[0], kv_cache[1]
        if md.query_lens is None:
            assert num_tokens == batch * md.query_len, "num_tokens must equal num_seqs * query_len"
        else:
            assert len(md.query_lens) == batch and sum(md.query_lens) == num_tokens
        if key is not None:
            write_kv(key.view(num_tokens, Hkv, D), value.view(num_tokens, Hkv, D), k_cache, v_cache,
                     md.slot_mapping)
        if output is None:
            output = torch.empty(num_tokens, H * D, dtype=query.dtype, device=query.device)
        if md.query_lens is None:
            sq = md.query_len
            q4 = query.view(batch, sq, H, D).permute(0, 2, 1, 3)
            o4 = output.view(batch, sq, H, D).permute(0, 2, 1, 3)
            paged_attention(q4, k_cache, v_cache, md.block_tables, md.seq_lens, self.causal,
                            max_seq_len=md.max_seq_len, scale=self.scale, out=o4)
            return output
        # Mixed batch: token-major views, one launch per kernel route over
        # that route's sequences only (a launch spreads its sequences' work
        # items over the XCDs in contiguous ranges, so sequences without
        # rows in it would leave XCDs idle).  A route's sequences that are
        # adjacent in the batch (prefills and decode steps grouped, as
        # serving engines order them) take views of the block table and
        # lengths; otherwise their rows are gathered on the device.  The
        # indices, query starts and lengths of every launch go to the
        # device in one asynchronous copy from pinned memory.
        q3, o3 = query.view(num_tokens, H, D), output.view(num_tokens, H, D)
        block_size = k_cache.shape[1]
        routes = [paged_route(H, Hkv, ql, block_size, D) if ql > 0 else None for ql in md.query_lens]
        starts, t = [], 0
        for ql in md.query_lens:
            starts.append(t)
            t += ql
        groups = [(kind, [b for b, r in enumerate(routes) if r == kind]) for kind in ("split", "single")]
        groups = [(kind, idx) for kind, idx in groups if idx]
        host = []
        for _, idx in groups:
            host += idx + [starts[b] for b in idx] + [md.query_lens[b] for b in idx]
        meta = torch.tensor(host, dtype=torch.int32, pin_memory=True).to(query.device, non_blocking=True)
        max_seq_len = md.max_seq_len if md.max_seq_len is not None else md.block_tables.shape[1] * block_size
        off = 0
        for kind, idx in groups:
            n = len(idx)
            sel, qs, ql = meta[off:off + n], meta[off + n:off + 2 * n], meta[off + 2 * n:off + 3 * n]
            off += 3 * n
            if idx[-1] - idx[0] + 1 == n:
                tables, lens = md.block_tables[idx[0]:idx[-1] + 1], md.seq_lens[idx[0]:idx[-1] + 1]
            else:
                tables, lens = md.block_tables.index_select(0, sel), md.seq_lens.index_select(0, sel)
            max_q = max(md.query_lens[b] for b in idx)
            route, splits = kind, None
            if kind == "single":
                dev = query.device.index if query.device.index is not None else torch.cuda.current_device()
                kc, ns = paged_single_plan(n, H, Hkv, max_q, max_seq_len, _cu_count(dev), bool(self.causal), D)
                route, splits = ("chunks", kc) if kc else ("single", ns)
            paged_attention(q3, k_cache, v_cache, tables, lens, self.causal, max_seq_len=max_seq_len,
                            scale=self.scale, out=o3, route=route, splits=splits, query_start=qs,
                            query_lens=ql, max_query_len=max_q)
        return output
