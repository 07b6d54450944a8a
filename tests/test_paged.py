"""Paged KV cache, CPU side: the oracle's gather against an independent
scatter, the C-ABI validation of the paged entry points (no kernel runs:
every call here is rejected before any HIP call, or is an empty no-op), the
split sizing, and the host block allocator (prefix sharing, copy on write,
reference counts) on CPU tensors."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle.gqa_oracle import gqa_lse, gqa_reference, paged_gather, paged_reference


# ---------------------------------------------------------------------------
# Oracle pins
# ---------------------------------------------------------------------------
def _scatter_loops(k, v, lens, block_size, num_blocks, rng):
    """Write contiguous per-sequence K/V (B, Hkv, L, D) into a paged cache by
    scalar loops, at a random block assignment; returns cache + table."""
    B, Hkv, L, D = k.shape
    kc = np.full((num_blocks, block_size, Hkv, D), np.nan)
    vc = np.full((num_blocks, block_size, Hkv, D), np.nan)
    free = list(rng.permutation(num_blocks))
    width = max(-(-n // block_size) for n in lens)
    table = np.zeros((B, width), dtype=np.int32)
    for b in range(B):
        for i in range(-(-lens[b] // block_size)):
            table[b, i] = free.pop()
        for j in range(lens[b]):
            for h in range(Hkv):
                kc[table[b, j // block_size], j % block_size, h] = k[b, h, j]
                vc[table[b, j // block_size], j % block_size, h] = v[b, h, j]
    return kc, vc, table


@pytest.mark.parametrize("block_size", [1, 4, 16])
def test_paged_gather_inverts_scatter(block_size):
    rng = np.random.default_rng(3)
    B, Hkv, L, D = 3, 2, 37, 8
    k = rng.standard_normal((B, Hkv, L, D))
    v = rng.standard_normal((B, Hkv, L, D))
    lens = [37, 1, 20]
    kc, vc, table = _scatter_loops(k, v, lens, block_size, 64, rng)
    got = paged_gather(kc, vc, table, lens)
    for b in range(B):
        assert np.array_equal(got[b][0][0], k[b, :, :lens[b]])
        assert np.array_equal(got[b][1][0], v[b, :, :lens[b]])
    # planted mistake: a gather that skips the block table (block j // bs)
    j = np.arange(lens[0])
    assert not np.array_equal(kc[j // block_size, j % block_size].transpose(1, 0, 2), k[0])


def test_paged_reference_is_per_sequence_attention():
    rng = np.random.default_rng(4)
    B, Hq, Hkv, Sq, L, D = 3, 8, 2, 3, 50, 16
    q = rng.standard_normal((B, Hq, Sq, D))
    k = rng.standard_normal((B, Hkv, L, D))
    v = rng.standard_normal((B, Hkv, L, D))
    lens = [50, 2, 33]  # sequence 1 is shorter than Sq: its first row sees no key
    kc, vc, table = _scatter_loops(k, v, lens, 8, 40, rng)
    for causal in (True, False):
        o, lse = paged_reference(q, kc, vc, table, lens, causal)
        for b in range(B):
            ref = gqa_reference(q[b:b + 1], k[b:b + 1, :, :lens[b]], v[b:b + 1, :, :lens[b]], causal,
                                dtype=np.float64)
            np.testing.assert_array_equal(o[b:b + 1], ref)
            np.testing.assert_array_equal(lse[b:b + 1], gqa_lse(q[b:b + 1], k[b:b + 1, :, :lens[b]],
                                                                 v[b:b + 1, :, :lens[b]], causal))
        # per-sequence bottom-right alignment: row 0 of sequence 1 (2 keys, 3 queries) sees nothing
        if causal:
            assert np.isnan(o[1, :, 0]).all() and np.isneginf(lse[1, :, 0]).all()
            assert np.isfinite(o[1, :, 1:]).all()


# ---------------------------------------------------------------------------
# C-ABI validation
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def lib():
    from gqa_kernels import _lib
    return _lib.load()


_S4 = (ctypes.c_int64 * 4)(8 * 128 * 128, 128 * 128, 128, 1)
_C4 = (ctypes.c_int64 * 4)(64 * 8 * 128, 8 * 128, 128, 1)  # (blocks, 64 slots, 8 heads, 128)
_FAKE = ctypes.c_void_p(1 << 20)


def _paged(lib, **kw):
    a = dict(q=_FAKE, qs=_S4, k=_FAKE, ks=_C4, v=_FAKE, vs=_C4, table=_FAKE, tstride=16,
             lens=_FAKE, qstart=None, qlen=None, bs=64, max_len=1024, ws=_FAKE, splits=8, B=2, Hq=32, Hkv=8,
             Sq=1, D=128, scale=0.1275, causal=1, dtype=0)
    a.update(kw)
    return lib.gqa_paged_split_first_launch(
        a["q"], a["qs"], a["k"], a["ks"], a["v"], a["vs"], a["table"], a["tstride"], a["lens"], a["qstart"],
        a["qlen"], a["bs"], a["max_len"], a["ws"], a["splits"], a["B"], a["Hq"], a["Hkv"], a["Sq"], a["D"],
        a["scale"], a["causal"], a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(bs=48), -8), (dict(bs=0), -8), (dict(bs=1 << 17), -8),   # block size
    (dict(tstride=15), -8),                                        # 15 * 64 < 1024 keys
    (dict(splits=0), -5), (dict(splits=2048), -5),
    (dict(lens=None), -7), (dict(table=None), -7), (dict(ws=None), -7),
    (dict(lens=ctypes.c_void_p((1 << 20) + 2)), -4),
    (dict(table=ctypes.c_void_p((1 << 20) + 2)), -4),
    (dict(ws=ctypes.c_void_p((1 << 20) + 4)), -4),
    (dict(ks=(ctypes.c_int64 * 4)(64 * 8 * 128, 8 * 128, 128, 2)), -4),
    (dict(D=96), -2), (dict(dtype=5), -3), (dict(Hq=30), -1), (dict(max_len=-1), -1),
    (dict(qstart=_FAKE), -7), (dict(qlen=_FAKE), -7),                # variable lengths need both
    (dict(qstart=_FAKE, qlen=ctypes.c_void_p((1 << 20) + 2)), -4),
    # pages under 64 keys: one chunk spans at most 2048 of them
    (dict(bs=1, tstride=4096, max_len=4096, splits=1), -5),
    (dict(bs=16, tstride=4096, max_len=65536, splits=1), -5),
    (dict(bs=32, tstride=4096, max_len=131072, splits=1), -5),
])
def test_paged_first_validation(lib, kw, code):
    assert _paged(lib, **kw) == code


def test_paged_first_empty_is_noop(lib):
    assert _paged(lib, B=0, q=None, k=None, v=None, table=None, lens=None, ws=None) == 0
    assert _paged(lib, Sq=0, q=None, k=None, v=None, table=None, lens=None, ws=None) == 0


def _write(lib, **kw):
    i3 = ctypes.c_int64 * 3
    a = dict(k=_FAKE, ks=i3(8 * 128, 128, 1), v=_FAKE, vs=i3(8 * 128, 128, 1), kc=_FAKE, kcs=_C4, vc=_FAKE,
             vcs=_C4, slots=_FAKE, n=4, Hkv=8, D=128, bs=64, dtype=0)
    a.update(kw)
    return lib.gqa_paged_cache_write_launch(a["k"], a["ks"], a["v"], a["vs"], a["kc"], a["kcs"], a["vc"],
                                            a["vcs"], a["slots"], a["n"], a["Hkv"], a["D"], a["bs"],
                                            a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(bs=6), -8), (dict(bs=0), -8),
    (dict(D=80), -2), (dict(dtype=2), -3), (dict(n=-1), -1), (dict(Hkv=0), -1),
    (dict(slots=None), -7), (dict(k=None), -7), (dict(kc=None), -7),
    (dict(slots=ctypes.c_void_p((1 << 20) + 4)), -4),
    (dict(ks=(ctypes.c_int64 * 3)(8 * 128, 128, 2)), -4),
    (dict(vs=(ctypes.c_int64 * 3)(8 * 128, 100, 1)), -4),
    (dict(v=ctypes.c_void_p((1 << 20) + 8)), -4),
])
def test_cache_write_validation(lib, kw, code):
    assert _write(lib, **kw) == code


def test_cache_write_empty_is_noop(lib):
    assert _write(lib, n=0, k=None, v=None, slots=None) == 0


def _pfwd(lib, **kw):
    a = dict(q=_FAKE, qs=_S4, k=_FAKE, ks=_C4, v=_FAKE, vs=_C4, table=_FAKE, tstride=16, lens=_FAKE,
             qstart=None, qlen=None, bs=64, max_len=1024, o=_FAKE, os=_S4, lse=None, B=2, Hq=32, Hkv=8, Sq=128,
             D=128, scale=0.1275, causal=1, dtype=0)
    a.update(kw)
    return lib.gqa_paged_fwd_launch(a["q"], a["qs"], a["k"], a["ks"], a["v"], a["vs"], a["table"], a["tstride"],
                                    a["lens"], a["qstart"], a["qlen"], a["bs"], a["max_len"], a["o"], a["os"],
                                    a["lse"], a["B"], a["Hq"], a["Hkv"], a["Sq"], a["D"], a["scale"], a["causal"],
                                    a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(bs=2), -8), (dict(bs=96), -8), (dict(bs=1 << 17), -8),    # blocks of >= 512 / D keys, power of two
    (dict(bs=4, D=64, tstride=256), -8),                            # D = 64: 8 rows per instruction
    (dict(tstride=15), -8),
    (dict(lens=None), -7), (dict(table=None), -7), (dict(o=None), -7),
    (dict(lens=ctypes.c_void_p((1 << 20) + 2)), -4),
    (dict(lse=ctypes.c_void_p((1 << 20) + 2)), -4),
    (dict(os=(ctypes.c_int64 * 4)(8 * 128 * 128, 128 * 128, 128, 3)), -4),
    (dict(D=96), -2), (dict(dtype=9), -3), (dict(Hq=12), -1), (dict(Hq=512, Hkv=1), -6),
    (dict(qstart=_FAKE), -7), (dict(qlen=_FAKE), -7),
    (dict(qstart=ctypes.c_void_p((1 << 20) + 1), qlen=_FAKE), -4),
])
def test_paged_fwd_validation(lib, kw, code):
    assert _pfwd(lib, **kw) == code


def test_paged_fwd_empty_is_noop(lib):
    assert _pfwd(lib, B=0, q=None, k=None, v=None, table=None, lens=None, o=None) == 0
    assert _pfwd(lib, Sq=0, q=None, k=None, v=None, table=None, lens=None, o=None) == 0


def _pchunks(lib, ws=_FAKE, splits=8, **kw):
    a = dict(q=_FAKE, qs=_S4, k=_FAKE, ks=_C4, v=_FAKE, vs=_C4, table=_FAKE, tstride=16, lens=_FAKE,
             qstart=None, qlen=None, bs=64, max_len=1024, o=_FAKE, os=_S4, lse=None, B=2, Hq=32, Hkv=8, Sq=128,
             D=128, scale=0.1275, causal=1, dtype=0)
    a.update(kw)
    return lib.gqa_paged_fwd_chunks_launch(a["q"], a["qs"], a["k"], a["ks"], a["v"], a["vs"], a["table"],
                                           a["tstride"], a["lens"], a["qstart"], a["qlen"], a["bs"], a["max_len"],
                                           a["o"], a["os"], a["lse"], ws, splits, a["B"], a["Hq"], a["Hkv"],
                                           a["Sq"], a["D"], a["scale"], a["causal"], a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(splits=0), -5), (dict(splits=1025), -5),                   # kv_splits in [1, GQA_MAX_SPLITS]
    (dict(ws=None), -7), (dict(ws=ctypes.c_void_p((1 << 20) + 8)), -4),  # workspace: non-NULL, 16-byte aligned
    (dict(bs=2), -8), (dict(lens=None), -7), (dict(D=96), -2),       # as gqa_paged_fwd_launch
])
def test_paged_chunks_validation(lib, kw, code):
    assert _pchunks(lib, **kw) == code


def test_paged_chunks_empty_is_noop(lib):
    assert _pchunks(lib, B=0, q=None, k=None, v=None, table=None, lens=None, o=None, ws=None) == 0


def _psplit(lib, ws=_FAKE, cnt=_FAKE, n_split=1, **kw):
    a = dict(q=_FAKE, qs=_S4, k=_FAKE, ks=_C4, v=_FAKE, vs=_C4, table=_FAKE, tstride=16, lens=_FAKE,
             qstart=None, qlen=None, bs=64, max_len=1024, o=_FAKE, os=_S4, lse=None, B=2, Hq=32, Hkv=8, Sq=128,
             D=128, scale=0.1275, causal=1, dtype=0)
    a.update(kw)
    return lib.gqa_paged_fwd_split_launch(a["q"], a["qs"], a["k"], a["ks"], a["v"], a["vs"], a["table"],
                                          a["tstride"], a["lens"], a["qstart"], a["qlen"], a["bs"], a["max_len"],
                                          a["o"], a["os"], a["lse"], ws, cnt, n_split, a["B"], a["Hq"], a["Hkv"],
                                          a["Sq"], a["D"], a["scale"], a["causal"], a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    # 128 queries at G = 4 are two 64-query blocks: n_split in [0, 2]
    (dict(n_split=3), -5), (dict(n_split=-1), -5),
    (dict(ws=None), -7), (dict(cnt=None), -7),                        # split state and counters: non-NULL
    (dict(ws=ctypes.c_void_p((1 << 20) + 8)), -4),                    # workspace 16-byte aligned
    (dict(cnt=ctypes.c_void_p((1 << 20) + 2)), -4),                   # counters 4-byte aligned
    (dict(bs=2), -8), (dict(lens=None), -7), (dict(D=96), -2),        # as gqa_paged_fwd_launch
])
def test_paged_fwd_split_validation(lib, kw, code):
    assert _psplit(lib, **kw) == code


def test_paged_fwd_split_empty_is_noop(lib):
    assert _psplit(lib, B=0, q=None, k=None, v=None, table=None, lens=None, o=None, ws=None, cnt=None) == 0


def test_reduce_varlen_validation(lib):
    r = lib.gqa_split_reduce_varlen_launch
    assert r(_FAKE, 8, _FAKE, _S4, None, None, None, 2, 32, 16, 128, 0, None) == -7
    assert r(_FAKE, 8, _FAKE, _S4, None, _FAKE, None, 2, 32, 16, 128, 0, None) == -7
    assert r(_FAKE, 8, _FAKE, _S4, ctypes.c_void_p((1 << 20) + 2), _FAKE, _FAKE, 2, 32, 16, 128, 0, None) == -4
    assert r(_FAKE, 0, _FAKE, _S4, None, _FAKE, _FAKE, 2, 32, 16, 128, 0, None) == -5
    assert r(None, 8, None, _S4, None, None, None, 0, 32, 16, 128, 0, None) == 0  # empty batch


def test_paged_route():
    from gqa_kernels.paged import paged_route
    assert paged_route(32, 8, 1, 16) == "split"      # decode
    assert paged_route(32, 8, 16, 64) == "split"     # 64 packed rows
    assert paged_route(32, 8, 32, 64) == "split"     # 128 packed rows: four blocks per workgroup at D = 128
    assert paged_route(32, 8, 33, 64) == "single"
    assert paged_route(32, 8, 17, 64, 64) == "single"  # D = 64: 64 packed rows at most
    assert paged_route(32, 8, 512, 16) == "single"   # 16-key blocks: one descriptor per 4-row instruction
    assert paged_route(32, 8, 512, 4) == "single"
    assert paged_route(32, 8, 512, 2) == "split"     # below one instruction's rows at D = 128
    assert paged_route(32, 8, 512, 4, 64) == "split"  # D = 64: 8 rows per instruction
    assert paged_route(32, 8, 512, 8, 64) == "single"
    assert paged_route(64, 8, 17, 128) == "single"


def test_strerror_block(lib):
    assert b"block_size" in lib.gqa_strerror(-8)


# ---------------------------------------------------------------------------
# Split sizing
# ---------------------------------------------------------------------------
def test_paged_splits():
    from gqa_kernels.paged import paged_splits
    # one 32-row block per kv head: 8 workgroups per split; the LDS-DMA first
    # pass (head_dim 128, pages of >= 4 keys) fills the 256 CUs once
    assert paged_splits(1, 32, 8, 1, 131072, 256) == 32
    assert paged_splits(1, 32, 8, 1, 131072, 256, heads_interleaved=True) == 32
    # a single-token step of a batch over token-major pages (heads
    # interleaved): four per CU; several tokens: one
    assert paged_splits(4, 32, 8, 1, 32768, 256) == 8
    assert paged_splits(4, 32, 8, 1, 32768, 256, heads_interleaved=True) == 32
    assert paged_splits(4, 32, 8, 4, 32768, 256, heads_interleaved=True) == 8
    # head_dim 64 with at most 16 rows and pages of >= 8 keys: the LDS-DMA
    # pass as well
    assert paged_splits(1, 32, 8, 1, 131072, 256, head_dim=64) == 32
    assert paged_splits(16, 32, 8, 1, 8192, 256, block_size=16, head_dim=64, heads_interleaved=True) == 8
    # the register-staged first pass (head_dim 64 over more rows or pages of
    # 4 keys, pages of 1-2 keys at head_dim 128): two per CU
    assert paged_splits(1, 32, 8, 8, 131072, 256, head_dim=64) == 64
    assert paged_splits(1, 32, 8, 1, 131072, 256, block_size=4, head_dim=64) == 64
    assert paged_splits(1, 32, 8, 1, 131072, 256, block_size=2) == 64
    # a batch of several sequences (lengths may differ): at least 8 chunks
    # per sequence within 8 workgroups per CU
    assert paged_splits(64, 32, 8, 1, 4096, 256) == 4
    assert paged_splits(8, 32, 8, 1, 30000, 256) == 8
    assert paged_splits(32, 32, 8, 1, 8000, 256) == 8
    assert paged_splits(32, 32, 8, 1, 1000, 256) == 2  # chunks keep 256 keys
    assert paged_splits(1, 32, 8, 1, 300, 256) == 1
    for L in (256, 1000, 5000, 1 << 20):
        for B in (1, 3, 16):
            s = paged_splits(B, 32, 8, 1, L, 256)
            assert s & (s - 1) == 0
            assert s == 1 or -(-L // s) >= 256


def test_paged_splits_small_pages():
    from gqa_kernels import _lib
    from gqa_kernels.paged import paged_chunk, paged_splits
    assert paged_chunk(4096, 2) == 2048 and paged_chunk(300, 1) == 320 and paged_chunk(40000, 2) == 20032
    # 512 workgroups from the batch alone: 4 splits (8 workgroups per CU),
    # more when a chunk would span more than 2048 pages
    assert paged_splits(512, 8, 1, 1, 4096, 256) == 4
    assert paged_splits(512, 8, 1, 1, 4096, 256, block_size=64) == 4
    assert paged_splits(512, 8, 1, 1, 40000, 256, block_size=1) == 32
    assert paged_splits(512, 8, 1, 1, 1 << 20, 256, block_size=16) == 32
    for bs in (1, 2, 4, 8, 16, 32):
        for L in (1, 300, 2048, 2049, 70000, 1 << 20):
            for B in (1, 64, 512):
                s = paged_splits(B, 32, 8, 1, L, 256, block_size=bs)
                assert s & (s - 1) == 0 and s <= _lib.GQA_MAX_SPLITS
                assert paged_chunk(L, s) // bs <= _lib.GQA_PAGED_CHUNK_PAGES
    # GQA_MAX_SPLITS chunks of at most 2048 one-key pages cover 2^21 keys:
    # beyond that no split count fits, and the error says why.
    assert paged_splits(1, 32, 8, 1, 1 << 21, 256, block_size=1) == _lib.GQA_MAX_SPLITS
    with pytest.raises(ValueError, match="2048 blocks"):
        paged_splits(1, 32, 8, 1, (1 << 21) + 64, 256, block_size=1)


# ---------------------------------------------------------------------------
# Block allocator (CPU tensors: no kernel involved)
# ---------------------------------------------------------------------------
def _cache(num_blocks=8, bs=4):
    from gqa_kernels.paged import PagedKVCache
    return PagedKVCache(num_blocks, bs, 2, 64, dtype=torch.float32, device="cpu")


def test_reserve_allocates_blocks_and_slots():
    c = _cache()
    c.add_sequence("a")
    s1 = c.reserve("a", 6)
    assert c.seq_len("a") == 6 and len(c.blocks("a")) == 2
    b0, b1 = c.blocks("a")
    assert s1 == [b0 * 4 + j for j in range(4)] + [b1 * 4, b1 * 4 + 1]
    s2 = c.reserve("a", 3)
    b2 = c.blocks("a")[2]
    assert s2 == [b1 * 4 + 2, b1 * 4 + 3, b2 * 4]
    assert c.num_free_blocks() == 5
    assert c.reserve("a", 0) == [] and c.seq_len("a") == 9


def test_fork_shares_blocks_and_copies_partial_block_on_write():
    c = _cache()
    c.add_sequence("p")
    slots = c.reserve("p", 6)  # one full block + 2 slots of a second
    for i, s in enumerate(slots):
        c.kv[:, s // 4, s % 4] = float(i + 1)
    c.fork("p", "x")
    c.fork("p", "y")
    assert c.blocks("x") == c.blocks("p") and c.num_free_blocks() == 6
    sx = c.reserve("x", 1)
    # x's partly filled last block was copied; its full block is still shared
    assert c.blocks("x")[0] == c.blocks("p")[0] and c.blocks("x")[1] != c.blocks("p")[1]
    nb = c.blocks("x")[1]
    assert sx == [nb * 4 + 2]
    assert torch.equal(c.kv[:, nb, :2], c.kv[:, c.blocks("p")[1], :2])
    c.kv[:, nb, 2] = 99.0
    assert (c.kv[:, c.blocks("p")[1], 2] == 0).all()  # the prefix block is untouched
    # y still shares p's partial block until it writes
    assert c.blocks("y") == c.blocks("p")


def test_free_returns_blocks_at_last_reference():
    c = _cache()
    c.add_sequence("p")
    c.reserve("p", 8)  # two full blocks
    c.fork("p", "x")
    c.reserve("x", 1)  # full blocks are shared as they are: one new block
    assert c.num_free_blocks() == 5
    c.free("p")
    assert c.num_free_blocks() == 5  # x still holds the prefix blocks
    c.free("x")
    assert c.num_free_blocks() == 8


def test_out_of_blocks_raises_without_changes():
    c = _cache(num_blocks=3)
    c.add_sequence("a")
    c.reserve("a", 10)
    c.fork("a", "b")
    with pytest.raises(RuntimeError, match="out of blocks"):
        c.reserve("b", 3)  # copy of the shared partial block + 1 more block > 0 free
    assert c.seq_len("b") == 10 and c.blocks("b") == c.blocks("a") and c.num_free_blocks() == 0


def test_block_table_and_seq_lens():
    c = _cache()
    for s, n in (("a", 5), ("b", 1), ("c", 0)):
        c.add_sequence(s)
        c.reserve(s, n)
    t = c.block_table(["a", "b", "c"])
    assert t.dtype == torch.int32 and tuple(t.shape) == (3, 2)
    assert t[0].tolist() == c.blocks("a") and t[1, 0] == c.blocks("b")[0] and t[2].tolist() == [0, 0]
    assert c.seq_lens(["a", "b", "c"]).tolist() == [5, 1, 0]


@pytest.mark.parametrize("layout", ["HND", "NHD"])
def test_cache_layouts_index_alike(layout):
    from gqa_kernels.paged import PagedKVCache
    c = PagedKVCache(4, 8, 2, 64, dtype=torch.float32, device="cpu", layout=layout)
    assert tuple(c.kv.shape) == (2, 4, 8, 2, 64) and tuple(c.k_cache.shape) == (4, 8, 2, 64)
    # head-major storage: one head's slots of a block are consecutive rows
    assert c.k_cache.stride(1) == (64 if layout == "HND" else 128)
    c.add_sequence(0)
    c.reserve(0, 10)
    c.kv[0, c.blocks(0)[1], 1, 1] = 5.0  # key 9, head 1
    c.fork(0, 1)
    c.reserve(1, 1)  # copy of the shared partial block
    assert (c.k_cache[c.blocks(1)[1], 1, 1] == 5.0).all()


def test_layer_arguments():
    from gqa_kernels.paged import GQAPagedAttention
    layer = GQAPagedAttention(32, 128, num_kv_heads=8)
    assert layer.scale == 128 ** -0.5 and layer.num_kv_heads == 8
    with pytest.raises(AssertionError):
        GQAPagedAttention(32, 96, num_kv_heads=8)
    with pytest.raises(AssertionError):
        GQAPagedAttention(30, 128, num_kv_heads=8)
