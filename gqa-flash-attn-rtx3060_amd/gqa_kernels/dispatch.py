"""Public entrypoint: choose single-pass vs split-KV path per workload.

MI355X rewrite of reference gqa_kernels/dispatch.py:14-62.  Same signature,
same asserts and the same bottom-right causal semantics; the route is sized
for the device's compute-unit count (256 on MI355X) instead of the fixed
``SM_COUNT = 28`` of the RTX 3060 version, and both routes launch hand-written
HIP kernels through the C ABI of libgqa_hip.so.
"""
from __future__ import annotations

import bisect
import functools
import math
from dataclasses import dataclass

import torch

from . import _lib
from .gqa_split import _counter_buffer, _workspace_buffer, decode_forward, stream_handle

__all__ = ["gqa_flash_attn", "Route", "choose_route"]

LOG2E = math.log2(math.e)

# Packed query rows of one single-pass workgroup, and of one split-KV row block.
FWD_ROWS = 256
SPLIT_ROWS = 32
# At head_dim 128 one split-KV workgroup takes two row blocks when a kv head
# has more than one (each K/V chunk is then streamed once per 64 rows).
SPLIT_WIDE_ROWS = 64
# ... and all of them up to four (65-128 rows).
SPLIT_WIDER_ROWS = 128
# The split-KV path is taken for at most this many packed rows per kv head
# (at head_dim 128: SPLIT_WIDER_ROWS).
SPLIT_MAX_ROWS = 64
# At head_dim 128 (the decode first pass, gqa_decode_kernel) the split
# count first fills the compute units with one workgroup each (chunks of at
# least SPLIT_TILE keys), then doubles toward SPLIT_WG_PER_CU workgroups per
# CU only while chunks keep at least this many keys: a workgroup's first
# tiles and Q take 2-3 us to land, which short chunks do not amortise.
# Measured on MI355X (bf16, rotating K/V sets), one token at G = 4 (the
# 16-row first pass): 8192 keys 32 splits 11.5 us / 64 splits 11.8, 16384
# keys 16.0 / 16.7, 32768 keys 25.6 / 27.3, 65536 keys 44.0-44.3 / 45.1-45.3,
# 131072 keys 83.5-84.8 / 82.4-82.8 (so 64 only there); 16 tokens at 32768
# keys 35.7 / 41.5; 32 tokens at 32768 keys (128-row workgroups) 256
# workgroups 41 us, 512 51 us.  64-row workgroups (33-64 packed rows) need
# chunks of twice this: 16 tokens at 131072 keys 32 splits 92.2 us / 64
# 96.2 (8 tokens, 32-row workgroups: 87.7 / 88.7; 32 tokens, 128-row
# workgroups: 112.0 / 107.2).
SPLIT_WIDER_MIN_CHUNK = 2048
# Shortest key cache worth splitting (the reference's threshold, dispatch.py:37).
SPLIT_MIN_KV = 1024
# Keys per split-KV tile; a chunk is never shorter than this many tiles
# (one: at 4K-8K keys, 128-key chunks over twice the workgroups measured
# 5-8 % faster than 256-key chunks).
SPLIT_TILE = 128
SPLIT_MIN_TILES = 1
# Target workgroups per compute unit for the split-KV first pass (the kernel
# runs two per CU at once; one round of workgroups measured fastest).
SPLIT_WG_PER_CU = 2
# Packed rows per kv head up to which head_dim 64 also runs the 16-row
# LDS-DMA first pass (in 128-key steps), and with it the head_dim-128 split
# count with the doubling threshold counted in steps (SPLIT_WIDER_MIN_CHUNK
# keys of 64-key steps = twice as many keys of 128-key steps).  Measured on
# MI355X (bf16, one token unless noted, G = 4, rotating K/V sets, us):
# 32768 keys 32 splits 16.7 / 64 18.1 (register-staged pass: 20.1 at 64),
# 131072 keys 32 45.0 / 64 46.2 (47.9 at 64), B = 4 x 32768 8 45.1 / 16
# 46.5, 4 tokens at 131072 keys 32 45.7 / 64 47.1, B = 16 x 8192 2 45.7 / 4
# 46.5, 8192 keys 16 11.2 / 32 11.6.
DEC16_ROWS = 16
# Single pass with key-range split of the heaviest causal query blocks: only
# considered while there are fewer than this many workgroups per CU, and
# taken when the modelled run time drops by at least FWD_SPLIT_GAIN.
FWD_SPLIT_MAX_WG_PER_CU = 2
FWD_SPLIT_GAIN = 0.05
# Per-work-item overhead of the single-pass kernel (first loads in flight,
# output, and for split blocks the exchange of the fp32 partial state), in
# 64-key tile steps, for the run-time model.  Calibrated on MI355X against
# measured split counts of causal prefill at 1024 and 2048 tokens (best
# measured: 8 of 16 blocks, -18 %; 8 of 32, -10 %; none at 4096).
FWD_ITEM_OVERHEAD = 8
# Added to each half of a split block in the persistent kernel's model:
# the exchange of its fp32 partial state (fitted to measured split counts
# at 512-3072 tokens, B = 1-5; the one-workgroup-per-item form at head_dim
# 64 measured best without it).
FWD_MERGE_OVERHEAD = 1
FWD_TILE = 64
# The persistent single pass claims work dynamically only with at least this
# many items per workgroup (kFwdDynMinItemsPerWg, gqa_params.hpp); below it
# every workgroup takes a fixed list (gqa_fwd.hip item_at: XCD x's
# contiguous item range dealt to its workgroups round by round in snake
# order), which the run-time model then follows.
FWD_DYN_MIN_ITEMS_PER_WG = 8
# Key chunks (single pass over kv_splits key ranges per query block, then
# the split-KV combine): considered when there are fewer query blocks than
# compute units.  Per-item overhead (first loads, partial store) in tile
# steps; a tile step of the single pass takes ~1.65 us on MI355X, the
# combine launch ~3 us plus its read of the fp32 partials at ~5 TB/s.
CHUNK_ITEM_OVERHEAD = 12
CHUNK_MIN_TILES = 4
TILE_STEP_US = 1.65
COMBINE_LAUNCH_US = 3.0
COMBINE_BYTES_PER_US = 5.0e6
# Passes over the fp32 partials charged to the key-chunk route: written by
# the first pass, read back by the combine (fitted: 1.5).
CHUNK_PARTIAL_PASSES = 1.5

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}


@dataclass(frozen=True)
class Route:
    kind: str  # "single", "split" or "chunks" (splits: key chunks per query block)
    splits: int = 1
    workgroups: int = 0
    fwd_split: int = 0  # single pass: query blocks per (b, kv head) run as two key halves


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def _fwd_block_tiles(n_mblk: int, block_m: int, seq_q: int, seq_kv: int, causal: bool):
    """Key tiles of each single-pass query block (gqa_fwd.hip's key range)."""
    out = []
    for pid in range(n_mblk):
        kv_end = seq_kv
        if causal:
            pos_hi = min((pid + 1) * block_m, seq_q) - 1
            kv_end = min(seq_kv, pos_hi + (seq_kv - seq_q) + 1)
        out.append(_cdiv(max(kv_end, 0), FWD_TILE))
    return out


def fwd_split_makespan(tiles, n_split: int, n_bh: int, cu_count: int, causal: bool = True,
                       persistent: bool = True) -> float:
    """Modelled run time (tile steps) of the single pass with the n_split
    heaviest blocks split: work items in the kernel's order (per (b, kv
    head): upper halves of the split blocks, then every block heavy-first
    with split blocks as their lower halves), scheduled as _list_makespan
    describes (`persistent`: the head_dim-128 kernel over contiguous K/V)."""
    n = len(tiles)
    order = list(range(n - 1, -1, -1)) if causal else list(range(n))
    mo = FWD_MERGE_OVERHEAD if persistent else 0
    items = [tiles[n - 1 - i] - tiles[n - 1 - i] // 2 + mo for i in range(n_split)]
    for pid in order:
        items.append(tiles[pid] // 2 + mo if pid >= n - n_split else tiles[pid])
    runs = []
    for c in items:
        _push_run(runs, c + FWD_ITEM_OVERHEAD, 1)
    return _list_makespan(runs, n_bh, cu_count, persistent)


def _push_run(runs, cost, count: int) -> None:
    if count <= 0:
        return
    if runs and runs[-1][0] == cost:
        runs[-1][1] += count
    else:
        runs.append([cost, count])


def _slice_runs(runs, period: int, lo: int, cnt: int):
    """Runs of items [lo, lo + cnt) of `runs` (one period) repeated end to end."""
    out, i, off = [], 0, lo % period
    while off >= runs[i][1]:
        off -= runs[i][1]
        i += 1
    while cnt > 0:
        take = min(runs[i][1] - off, cnt)
        _push_run(out, runs[i][0], take)
        cnt -= take
        off, i = 0, (i + 1) % len(runs)
    return out


def _greedy_runs(runs, n: int) -> float:
    """Makespan of n CUs each taking the next item when free (the least
    loaded CU takes it), items in order.  A run of items of one cost c on
    loads within c of each other is dealt round-robin in load order (each
    item lands on the least loaded CU and leaves it the most loaded), so it
    is applied as whole rounds plus the remainder on the least loaded CUs."""
    loads = [0.0] * n  # ascending
    for c, k in runs:
        while k:
            if loads[-1] - loads[0] <= c:
                full, rem = divmod(k, n)
                if full:
                    loads = [x + full * c for x in loads]
                if rem:
                    loads = loads[rem:] + [x + c for x in loads[:rem]]
                break
            bisect.insort(loads, loads.pop(0) + c)
            k -= 1
    return loads[-1]


def _list_makespan(runs, n_rep: int, cu_count: int, persistent: bool = False) -> float:
    """Run time (tile steps) of the items of one (b, kv head), given as runs
    [cost, count] in the kernel's item order, repeated for n_rep (b, kv head)
    pairs: each XCD (cu_count / 8 CUs) takes its contiguous share of the
    whole list.  The persistent kernel with fewer than
    FWD_DYN_MIN_ITEMS_PER_WG items per workgroup deals fixed lists:
    workgroup `slot` of XCD x takes items slot, 2 S - 1 - slot, 2 S + slot,
    ... of the XCD's share (S workgroups on the XCD: gqa_fwd.hip item_at).
    Otherwise (the dynamic schedule, or one workgroup per item) each CU
    takes the next item when free.  XCD shares with the same start within
    the period and the same length are scheduled once (with 8 kv heads
    every XCD's share is the same list)."""
    period = sum(k for _, k in runs)
    total = period * n_rep
    if total == 0:
        return 0.0
    n_wg = min(total, cu_count)
    q, r = divmod(total, 8)
    static = persistent and total < FWD_DYN_MIN_ITEMS_PER_WG * n_wg
    flat = [c for c, k in runs for _ in range(k)] if static else None
    per_xcd = max(1, cu_count // 8)
    seen = {}
    worst = 0.0
    for x in range(8):
        lo, cnt = x * q + min(x, r), q + (1 if x < r else 0)
        slots = (n_wg - x + 7) >> 3
        key = (lo % period, cnt, slots if static else 0)
        if key in seen or cnt == 0:
            continue
        if static:
            # Rows of `slots` items, odd rows reversed (right-aligned when
            # short): workgroup `slot` sums column `slot`.
            share = (flat * (-(-(lo % period + cnt) // period)))[lo % period:lo % period + cnt]
            rows = []
            for j, i in enumerate(range(0, cnt, slots)):
                row = share[i:i + slots]
                pad = [0] * (slots - len(row))
                rows.append(pad + row[::-1] if j & 1 else row + pad)
            t_x = float(max(map(sum, zip(*rows))))
        else:
            t_x = _greedy_runs(_slice_runs(runs, period, lo, cnt), per_xcd)
        seen[key] = t_x
        worst = max(worst, t_x)
    return worst


def chunks_makespan(tiles, kv_splits: int, n_bh: int, cu_count: int, rows: int, head_dim: int,
                    causal: bool = True, persistent: bool = None) -> float:
    """Modelled run time (tile steps) of the single pass over key chunks:
    items (b, kv head) x chunk x query block (heavy first under causal),
    chunk c covering tiles [c * ct, (c + 1) * ct) of its block's range, plus
    the combine (launch and its read of rows x kv_splits partials).
    `persistent` (default: head_dim 128): the persistent kernel over
    contiguous K/V; paged caches run one workgroup per item."""
    n = len(tiles)
    ct = max(1, -(-max(tiles) // kv_splits))
    order = list(range(n - 1, -1, -1)) if causal else list(range(n))
    # Chunks below every block's end are full (ct tiles), chunks past every
    # block's end are empty; only the ones between differ per block.
    n_full = min(kv_splits, min(tiles) // ct)
    n_busy = min(kv_splits, -(-max(tiles) // ct))
    runs = []
    _push_run(runs, ct + CHUNK_ITEM_OVERHEAD, n_full * n)
    for c in range(n_full, n_busy):
        for m in order:
            _push_run(runs, min(ct, max(tiles[m] - c * ct, 0)) + CHUNK_ITEM_OVERHEAD, 1)
    _push_run(runs, CHUNK_ITEM_OVERHEAD, (kv_splits - n_busy) * n)
    if persistent is None:
        persistent = head_dim == 128
    first = _list_makespan(runs, n_bh, cu_count, persistent)
    # The fp32 partials are written by the first pass and read back by the
    # combine launch, each at about COMBINE_BYTES_PER_US.
    combine_us = COMBINE_LAUNCH_US + CHUNK_PARTIAL_PASSES * rows * kv_splits * (head_dim + 2) * 4 / COMBINE_BYTES_PER_US
    return first + combine_us / TILE_STEP_US


def choose_kv_chunks(batch: int, num_heads: int, num_kv_heads: int, seq_q: int, seq_kv: int,
                     cu_count: int, causal: bool, head_dim: int = 128, base: float = None,
                     persistent: bool = None) -> int:
    """Key chunks per query block for the single pass (0: none).

    With fewer query blocks than compute units (chunked prefill or a long
    verify step against a long cache) most CUs would idle; splitting every
    block's key range into kv_splits chunks (a power of two, each at least
    CHUNK_MIN_TILES tiles) fills them, at the cost of the fp32 partials and
    the combine launch.  Taken when the model beats the single pass (`base`:
    its modelled time) by FWD_SPLIT_GAIN.  `persistent` as chunks_makespan
    (False for paged caches)."""
    group = num_heads // num_kv_heads
    block_m = max(1, FWD_ROWS // group)
    n_mblk = _cdiv(seq_q, block_m)
    n_bh = batch * num_kv_heads
    if n_mblk * n_bh >= cu_count or seq_q == 0:
        return 0
    tiles = _fwd_block_tiles(n_mblk, block_m, seq_q, seq_kv, causal)
    if persistent is None:
        persistent = head_dim == 128
    if base is None:
        base = fwd_split_makespan(tiles, 0, n_bh, cu_count, causal, persistent=persistent)
    rows = batch * num_heads * seq_q
    best, best_s = base, 0
    s = 2
    while s <= _lib.GQA_MAX_SPLITS and -(-max(tiles) // s) >= CHUNK_MIN_TILES:
        t = chunks_makespan(tiles, s, n_bh, cu_count, rows, head_dim, causal, persistent)
        if t < best:
            best, best_s = t, s
        s *= 2
    return best_s if best <= (1.0 - FWD_SPLIT_GAIN) * base else 0


def choose_fwd_split(batch: int, num_heads: int, num_kv_heads: int, seq_q: int, seq_kv: int,
                     cu_count: int, causal: bool, head_dim: int = 128, persistent: bool = None) -> int:
    """Query blocks per (b, kv head) to run as two key halves (0: none).

    Only causal blocks differ in length; when there are few workgroups per
    CU the longest block sets the run time, and splitting the heaviest ones
    shortens it (fwd_split_makespan picks the count).  `persistent`
    (default: head_dim 128) as fwd_split_makespan; False for paged caches."""
    group = num_heads // num_kv_heads
    block_m = max(1, FWD_ROWS // group)
    n_mblk = _cdiv(seq_q, block_m)
    n_bh = batch * num_kv_heads
    if not causal or n_mblk < 2 or n_mblk * n_bh >= FWD_SPLIT_MAX_WG_PER_CU * cu_count:
        return 0
    tiles = _fwd_block_tiles(n_mblk, block_m, seq_q, seq_kv, causal)
    if persistent is None:
        persistent = head_dim == 128
    base = fwd_split_makespan(tiles, 0, n_bh, cu_count, persistent=persistent)
    best, best_ns = base, 0
    for f in (0.25, 0.375, 0.5, 0.625, 0.75, 1.0):
        ns = max(1, min(n_mblk, round(n_mblk * f)))
        t = fwd_split_makespan(tiles, ns, n_bh, cu_count, persistent=persistent)
        if t < best:
            best, best_ns = t, ns
    return best_ns if best <= (1.0 - FWD_SPLIT_GAIN) * base else 0


def split_rows_per_workgroup(rows: int, head_dim: int = 128) -> int:
    """Packed rows one split-KV workgroup covers (the first pass's row
    blocks: 32, or at head_dim 128 two or four of them)."""
    if head_dim != 128 or rows <= SPLIT_ROWS:
        return SPLIT_ROWS
    return SPLIT_WIDE_ROWS if rows <= SPLIT_WIDE_ROWS else SPLIT_WIDER_ROWS


def split_max_rows(head_dim: int = 128) -> int:
    """Packed rows per kv head up to which the split-KV path is taken."""
    return SPLIT_WIDER_ROWS if head_dim == 128 else SPLIT_MAX_ROWS


def split_count(base: int, seq_kv: int, cu_count: int, rows_per_wg: int, head_dim: int = 128,
                rows16: bool = False) -> int:
    """Split count of the split-KV path for `base` workgroups per split
    (head_dim 128, and head_dim 64 when the 16-row first pass runs
    (`rows16`: at most DEC16_ROWS packed rows): fill the CUs, then a second
    workgroup per CU only for chunks of SPLIT_WIDER_MIN_CHUNK keys (twice
    that for 64-row workgroups); head_dim
    64 over more rows: two workgroups per CU with chunks of SPLIT_MIN_TILES
    tiles)."""
    target = SPLIT_WG_PER_CU * cu_count
    splits = 1
    if head_dim == 128 or rows_per_wg > SPLIT_WIDE_ROWS or rows16:
        wider_min = SPLIT_WIDER_MIN_CHUNK * (2 if head_dim == 64 or rows_per_wg == SPLIT_WIDE_ROWS else 1)
        while (base * splits < cu_count and splits < _lib.GQA_MAX_SPLITS
               and _cdiv(seq_kv, splits * 2) >= SPLIT_MIN_TILES * SPLIT_TILE):
            splits *= 2
        while (base * splits < target and splits < _lib.GQA_MAX_SPLITS
               and _cdiv(seq_kv, splits * 2) >= wider_min):
            splits *= 2
        return splits
    while (base * splits < target and splits < _lib.GQA_MAX_SPLITS
           and _cdiv(seq_kv, splits * 2) >= SPLIT_MIN_TILES * SPLIT_TILE):
        splits *= 2
    return splits


def choose_route(batch: int, num_heads: int, num_kv_heads: int, seq_q: int, seq_kv: int,
                 cu_count: int, causal: bool = True, head_dim: int = 128) -> Route:
    """Pick the kernel path for one call (pure function of the shapes).

    Counterpart of reference dispatch.py:35-45.  A query block of at most
    split_max_rows(head_dim) packed rows per kv head (decode: group * seq_q = 4)
    against a cache of at least SPLIT_MIN_KV keys streams K/V with the
    split-KV kernels; the split count is a power of two: at head_dim 128
    the one that fills the compute units, doubled toward SPLIT_WG_PER_CU
    workgroups per CU while chunks keep SPLIT_WIDER_MIN_CHUNK keys; at
    head_dim 64 the one that brings the first pass to SPLIT_WG_PER_CU
    workgroups per CU, every chunk keeping at least SPLIT_MIN_TILES tiles of
    SPLIT_TILE keys (split_count).  Anything
    else (prefill, chunked prefill) runs the single-pass kernel: with a key
    split of its heaviest causal blocks (choose_fwd_split), or, when there
    are fewer query blocks than compute units, as key chunks combined by the
    split-KV combine (choose_kv_chunks, route kind "chunks") when the model
    says that is faster.
    """
    group = num_heads // num_kv_heads
    rows = group * seq_q
    single_wgs = _cdiv(seq_q, max(1, FWD_ROWS // group)) * num_kv_heads * batch
    if rows <= split_max_rows(head_dim) and seq_kv >= SPLIT_MIN_KV:
        rpw = split_rows_per_workgroup(rows, head_dim)
        base = _cdiv(rows, rpw) * num_kv_heads * batch
        splits = split_count(base, seq_kv, cu_count, rpw, head_dim, rows16=rows <= DEC16_ROWS)
        return Route("split", splits, base * splits)
    ns = choose_fwd_split(batch, num_heads, num_kv_heads, seq_q, seq_kv, cu_count, causal, head_dim)
    # Key chunks, against the better of the plain and the block-split single pass.
    # (Only from SPLIT_MIN_KV keys on, the length from which the reference
    # splits the key axis at all.)
    n_mblk = _cdiv(seq_q, max(1, FWD_ROWS // group))
    if n_mblk * num_kv_heads * batch < cu_count and seq_q > 0 and seq_kv >= SPLIT_MIN_KV:
        tiles = _fwd_block_tiles(n_mblk, max(1, FWD_ROWS // group), seq_q, seq_kv, causal)
        base = fwd_split_makespan(tiles, ns, num_kv_heads * batch, cu_count, causal, persistent=head_dim == 128)
        kc = choose_kv_chunks(batch, num_heads, num_kv_heads, seq_q, seq_kv, cu_count, causal, head_dim, base)
        if kc:
            return Route("chunks", kc, single_wgs * kc)
    return Route("single", 1, single_wgs + ns * num_kv_heads * batch, ns)


_route_cached = functools.lru_cache(maxsize=4096)(choose_route)


@functools.lru_cache(maxsize=None)
def _cu_count(device_index: int) -> int:
    n = _lib.load().gqa_device_cu_count(device_index)
    if n <= 0:
        raise RuntimeError(f"gqa_device_cu_count({device_index}) failed: {n}")
    return n


def _is_kernel_ready(t: torch.Tensor) -> bool:
    """The kernels need a unit last-dim stride and 16-byte aligned rows."""
    st = t.stride()
    # 16-byte alignment of the pointer and of every stride in bytes, in one
    # test (a multiple of 16 has its low four bits clear).
    return st[3] == 1 and (t.data_ptr() | ((st[0] | st[1] | st[2]) * t.element_size())) % 16 == 0


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """t itself, or a fresh contiguous copy when the kernels cannot read it."""
    return t if _is_kernel_ready(t) else t.clone(memory_format=torch.contiguous_format)


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
    assert v.shape == k.shape, "k and v must have the same shape"
    assert k.shape[0] == batch and k.shape[3] == head_dim, "k/v batch or head_dim differ from q"
    dev = q.get_device()  # device index (an int: no torch.device objects on this path)
    assert k.get_device() == dev and v.get_device() == dev, "q, k, v must be on one device"

    route = _route_cached(batch, num_heads, num_kv_heads, seq_q, seq_kv, _cu_count(dev), bool(causal), head_dim)
    if dev == torch.cuda.current_device():
        return _launch(route, q, k, v, causal, return_lse, dev)
    with torch.cuda.device(dev):  # launch on q's device
        return _launch(route, q, k, v, causal, return_lse, dev)


def _launch(route, q_in, k, v, causal, return_lse, dev):
    # One test for the usual case (all three kernel-ready; 2-byte elements:
    # the dtype is asserted), the per-tensor copies otherwise.
    qs, ks, vs = q_in.stride(), k.stride(), v.stride()
    if (qs[3] == 1 and ks[3] == 1 and vs[3] == 1
            and ((q_in.data_ptr() | k.data_ptr() | v.data_ptr()
                  | 2 * (qs[0] | qs[1] | qs[2] | ks[0] | ks[1] | ks[2] | vs[0] | vs[1] | vs[2])) & 15) == 0):
        q = q_in
    else:
        q, k, v = _kernel_ready(q_in), _kernel_ready(k), _kernel_ready(v)
    if route.kind == "split":
        return decode_forward(q, k, v, causal, route.splits, return_lse, dev)
    o = torch.empty_like(q_in)  # as dispatch.py:47; contiguous if unusable
    if not _is_kernel_ready(o):
        o = torch.empty_like(q_in, memory_format=torch.contiguous_format)
    if route.kind == "chunks":
        return chunks_forward(q, k, v, o, causal, route.splits, return_lse)
    return single_pass_forward(q, k, v, o, causal, route.fwd_split, return_lse)


def single_pass_forward(q, k, v, o, causal, fwd_split=0, return_lse=False):
    """Launch the single-pass kernel on kernel-ready q, k, v and output o
    through gqa_fwd_split_launch: with fwd_split > 0 the heaviest query
    blocks run as two key halves, and the work items are scheduled across
    the XCDs dynamically (workspace and counters are the stream's cached
    buffers)."""
    lib = _lib.load()
    batch, num_heads, seq_q, head_dim = q.shape
    _, num_kv_heads, seq_kv, _ = k.shape
    scale_log2 = (head_dim ** -0.5) * LOG2E
    stream = stream_handle(q.device)
    common = (batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim,
              scale_log2, int(bool(causal)), _DTYPES[q.dtype], stream)
    qkvo = (q.data_ptr(), _lib.strides(q), k.data_ptr(), _lib.strides(k),
            v.data_ptr(), _lib.strides(v), o.data_ptr(), _lib.strides(o))
    lse = torch.empty(batch, num_heads, seq_q, dtype=torch.float32, device=q.device) if return_lse else None
    # The stream's zeroed counters: split blocks' merge counters and the
    # dynamic schedule's queues (both left zero by the kernel).
    cnt = _counter_buffer(q.device, stream, lib.gqa_fwd_split_counters_count(batch, num_kv_heads, fwd_split))
    ws = None
    if fwd_split > 0:
        ws = _workspace_buffer(q.device, stream,
                               lib.gqa_fwd_split_workspace_bytes(batch, num_kv_heads, head_dim, fwd_split))
    _lib.check(lib.gqa_fwd_split_launch(*qkvo, None if lse is None else lse.data_ptr(),
                                        None if ws is None else ws.data_ptr(), cnt.data_ptr(), fwd_split, *common))
    return o if lse is None else (o, lse)


def chunks_forward(q, k, v, o, causal, kv_splits, return_lse=False):
    """Launch the single pass over key chunks on kernel-ready q, k, v and
    output o through gqa_fwd_chunks_launch: every query block runs as
    kv_splits work items over consecutive key ranges, each writing fp32
    partials into the stream's cached split workspace, which the split-KV
    combine reduces into o (and lse)."""
    lib = _lib.load()
    batch, num_heads, seq_q, head_dim = q.shape
    _, num_kv_heads, seq_kv, _ = k.shape
    stream = stream_handle(q.device)
    ws = _workspace_buffer(q.device, stream,
                           lib.gqa_split_workspace_bytes(batch, num_heads, seq_q, head_dim, kv_splits))
    cnt = _counter_buffer(q.device, stream, lib.gqa_fwd_split_counters_count(batch, num_kv_heads, 0))
    lse = torch.empty(batch, num_heads, seq_q, dtype=torch.float32, device=q.device) if return_lse else None
    _lib.check(lib.gqa_fwd_chunks_launch(
        q.data_ptr(), _lib.strides(q), k.data_ptr(), _lib.strides(k), v.data_ptr(), _lib.strides(v),
        o.data_ptr(), _lib.strides(o), None if lse is None else lse.data_ptr(), ws.data_ptr(), cnt.data_ptr(),
        kv_splits, batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, (head_dim ** -0.5) * LOG2E,
        int(bool(causal)), _DTYPES[q.dtype], stream))
    return o if lse is None else (o, lse)
