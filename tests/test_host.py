"""Host-side logic and the C ABI, without a GPU (CPU only).

* the library loads and exports every entry point declared in
  include/gqa_attn.h, with the ctypes signatures matching the header;
* argument validation in the C launchers (error codes are returned before any
  HIP call, so they are testable here);
* the dispatch rule (single-pass vs split-KV, split count for 256 CUs);
* the Python asserts of reference gqa_kernels/dispatch.py:30-33.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "gqa_attn.h"


def _declared():
    """(name, n_params) of every function declared in the public header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b([a-z_0-9]+)\s*\(([^;{]*?)\)\s*;", text):
        name, params = m.group(1), m.group(2).strip()
        if not name.startswith("gqa_"):
            continue
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    from gqa_kernels import _lib
    return _lib.load()


def test_header_declares_expected_entry_points():
    names = set(_declared())
    assert {"gqa_fwd_launch", "gqa_split_first_launch", "gqa_split_reduce_launch",
            "gqa_split_workspace_bytes", "gqa_device_cu_count", "gqa_strerror",
            "gqa_abi_version"} <= names


def test_library_exports_every_declared_symbol(lib):
    from gqa_kernels import _lib
    for name, nparams in _declared().items():
        assert hasattr(lib, name), f"libgqa_hip.so lacks {name}"
        assert name in _lib.SIGNATURES, f"no ctypes signature for {name}"
        assert len(_lib.SIGNATURES[name][1]) == nparams, name


def test_abi_version_and_strerror(lib):
    from gqa_kernels import _lib
    assert lib.gqa_abi_version() == _lib.ABI_VERSION
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -99):
        msg = lib.gqa_strerror(code)
        assert isinstance(msg, bytes) and msg
    assert b"head_dim" in lib.gqa_strerror(-2)


def test_host_binding_loads(lib):
    """The torch-tensor binding of the decode and paged calls (_gqa_host.so)
    loads, links against the same library ABI and exposes split_decode,
    paged_forward and cache_write (no GPU work: the binding is exercised by
    the GPU decode and paged tests)."""
    from gqa_kernels import _lib
    host = _lib.load_host()
    assert host.ABI_VERSION == lib.gqa_abi_version() == _lib.ABI_VERSION
    assert callable(host.split_decode)
    assert callable(host.paged_forward) and callable(host.cache_write)
    assert _lib.load_host() is host


def test_decode_falls_back_to_ctypes_without_host_binding(monkeypatch):
    """A decode step whose torch-tensor binding cannot be loaded (missing,
    stale, or built against another torch) still runs: decode_forward warns
    once and calls gqa_split_launch through ctypes with the same arguments
    (the C call is replaced by a recorder here: no GPU)."""
    from gqa_kernels import _lib, gqa_split

    calls = []

    class _Stub:
        def gqa_split_launch(self, *args):
            calls.append(args)
            return 0

    def _no_host():
        raise ImportError("undefined symbol: _ZN3c10 (built against another torch)")

    monkeypatch.setattr(_lib, "_host", None)
    monkeypatch.setattr(_lib, "load_host", _no_host)
    monkeypatch.setattr(_lib, "load", lambda: _Stub())
    monkeypatch.setattr(gqa_split, "_host_failed", [])
    monkeypatch.setattr(gqa_split, "_workspaces", {})
    monkeypatch.setattr(gqa_split, "_raw_stream", lambda dev: 1234)
    q = torch.zeros(1, 32, 1, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 8, 4096, 128, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    with pytest.warns(RuntimeWarning, match="ctypes"):
        o = gqa_split.decode_forward(q, k, v, True, 16, False, 0)
    assert o.shape == q.shape and o.dtype == q.dtype
    o2, lse = gqa_split.decode_forward(q, k, v, True, 16, True, 0)  # no second warning needed
    assert lse.shape == (1, 32, 1) and lse.dtype == torch.float32
    assert len(calls) == 2
    a = calls[0]
    # q, o pointers; splits; B, Hq, Hkv, Sq, Skv, D; scale; causal; dtype; stream
    assert a[0] == q.data_ptr() and a[6] == o.data_ptr() and a[8] is None
    assert a[10:17] == (16, 1, 32, 8, 1, 4096, 128)
    assert abs(a[17] - 128 ** -0.5 * 1.4426950408889634) < 1e-7
    assert a[18:] == (1, _lib.DTYPE_BF16, 1234)
    assert calls[1][8] == lse.data_ptr()
    assert len(gqa_split._host_failed) == 1


def test_workspace_bytes(lib):
    from gqa_kernels.gqa_split import workspace_bytes
    for args in ((1, 32, 1, 128, 128), (16, 64, 4, 128, 8), (2, 8, 3, 64, 7)):
        assert lib.gqa_split_workspace_bytes(*args) == workspace_bytes(*args)
        B, H, S, D, SP = args
        assert workspace_bytes(*args) == B * H * S * SP * (D + 2) * 4
    assert lib.gqa_split_workspace_bytes(0, 32, 1, 128, 8) == 0


_S4 = (ctypes.c_int64 * 4)(8 * 128 * 128, 128 * 128, 128, 1)
_BAD = (ctypes.c_int64 * 4)(8 * 128 * 128, 128 * 128, 128, 2)
_FAKE = ctypes.c_void_p(1 << 20)  # aligned, never dereferenced: validation fails first


@pytest.mark.parametrize("args,code", [
    (dict(Hq=32, Hkv=6), -1),       # heads not divisible
    (dict(D=96), -2),               # head_dim
    (dict(dtype=7), -3),            # dtype
    (dict(stride=_BAD), -4),        # last-dim stride
    (dict(Hq=512, Hkv=1), -6),      # group larger than one packed tile
    (dict(Sq=-1), -1),
])
def test_fwd_launch_validation(lib, args, code):
    p = dict(Hq=32, Hkv=8, D=128, dtype=0, stride=_S4, Sq=128)
    p.update(args)
    st = p["stride"]
    rc = lib.gqa_fwd_launch(_FAKE, st, _FAKE, _S4, _FAKE, _S4, _FAKE, _S4,
                            1, p["Hq"], p["Hkv"], p["Sq"], 128, p["D"], 0.1275, 1, p["dtype"], None)
    assert rc == code


def test_fwd_launch_rejects_rows_beyond_32bit_offsets(lib):
    # The single-pass kernel addresses one head's K/V rows with 32-bit byte
    # offsets up to two 64-key tiles past the end: (seq_kv + 192) * row
    # stride * 2 must stay below 2^31.
    # Rows of 2^21 bytes: seq_kv + 192 must stay below 1024, so 832 keys are
    # the first rejected length.  (Only rejected calls: a call that passes
    # validation would launch on these fake pointers.)
    ss = 1 << 20
    big = (ctypes.c_int64 * 4)(8 * 1024 * ss, 1024 * ss, ss, 1)
    args = lambda kst, vst, skv: (_FAKE, _S4, _FAKE, kst, _FAKE, vst, _FAKE, _S4,
                                  1, 32, 8, 128, skv, 128, 0.1275, 1, 0, None)
    assert lib.gqa_fwd_launch(*args(big, big, 832)) == -4
    assert lib.gqa_fwd_launch(*args(big, big, 1 << 20)) == -4
    assert lib.gqa_fwd_launch(*args(_S4, big, 832)) == -4  # V alone too long
    assert lib.gqa_fwd_launch(*args(big, _S4, 832)) == -4  # K alone too long


def test_empty_launches_are_noops(lib):
    # batch 0 / seq_q 0: nothing to do, no HIP call, success.
    assert lib.gqa_fwd_launch(None, _S4, None, _S4, None, _S4, None, _S4,
                              0, 32, 8, 16, 16, 128, 0.1, 1, 0, None) == 0
    assert lib.gqa_fwd_launch(None, _S4, None, _S4, None, _S4, None, _S4,
                              1, 32, 8, 0, 16, 128, 0.1, 1, 0, None) == 0


def test_fused_launch_validation(lib):
    f = lib.gqa_split_fused_launch
    args = lambda ws, cnt, splits: (_FAKE, _S4, _FAKE, _S4, _FAKE, _S4, _FAKE, _S4, ws, cnt, splits,
                                    1, 32, 8, 1, 4096, 128, 0.1, 1, 0, None)
    assert f(*args(_FAKE, None, 8)) == -7
    assert f(*args(None, _FAKE, 8)) == -7
    assert f(*args(_FAKE, _FAKE, 0)) == -5
    assert f(*args(_FAKE, ctypes.c_void_p((1 << 20) + 2), 8)) == -4
    # the fused combine stages min(32, G*seq_q) * splits values: 16 rows x 512 > 4096
    big = (_FAKE, _S4, _FAKE, _S4, _FAKE, _S4, _FAKE, _S4, _FAKE, _FAKE, 512,
           1, 32, 8, 4, 4096, 128, 0.1, 1, 0, None)
    assert f(*big) == -5
    assert lib.gqa_split_counters_count(1, 32, 8, 1) == 8
    assert lib.gqa_split_counters_count(16, 64, 8, 4) == 128
    assert lib.gqa_split_counters_count(2, 32, 8, 16) == 2 * 8 * 2
    assert lib.gqa_split_counters_count(1, 30, 8, 1) == 0


def test_split_launch_validation(lib):
    f = lib.gqa_split_first_launch
    assert f(_FAKE, _S4, _FAKE, _S4, _FAKE, _S4, _FAKE, 0, 1, 32, 8, 1, 4096, 128, 0.1, 1, 0, None) == -5
    assert f(_FAKE, _S4, _FAKE, _S4, _FAKE, _S4, _FAKE, 2048, 1, 32, 8, 1, 4096, 128, 0.1, 1, 0, None) == -5
    assert f(_FAKE, _S4, _FAKE, _S4, _FAKE, _S4, None, 8, 1, 32, 8, 1, 4096, 128, 0.1, 1, 0, None) == -7
    misaligned = ctypes.c_void_p((1 << 20) + 4)
    assert f(_FAKE, _S4, _FAKE, _S4, _FAKE, _S4, misaligned, 8, 1, 32, 8, 1, 4096, 128, 0.1, 1, 0,
             None) == -4
    r = lib.gqa_split_reduce_launch
    assert r(_FAKE, 8, _FAKE, _S4, 1, 32, 1, 80, 0, None) == -2
    assert r(_FAKE, 0, _FAKE, _S4, 1, 32, 1, 128, 0, None) == -5
    assert r(_FAKE, 8, _FAKE, _BAD, 1, 32, 1, 128, 0, None) == -4


def test_chunks_launch_validation(lib):
    f = lib.gqa_fwd_chunks_launch
    args = lambda ws, cnt, splits, lse=None, B=1, Sq=128: (
        _FAKE, _S4, _FAKE, _S4, _FAKE, _S4, _FAKE, _S4, lse, ws, cnt, splits,
        B, 32, 8, Sq, 4096, 128, 0.1, 1, 0, None)
    assert f(*args(_FAKE, None, 0)) == -5
    assert f(*args(_FAKE, None, 2048)) == -5
    assert f(*args(None, None, 8)) == -7
    assert f(*args(ctypes.c_void_p((1 << 20) + 4), None, 8)) == -4    # workspace alignment
    assert f(*args(_FAKE, ctypes.c_void_p((1 << 20) + 2), 8)) == -4   # counters alignment
    assert f(*args(_FAKE, None, 8, lse=ctypes.c_void_p((1 << 20) + 2))) == -4
    assert f(*args(None, None, 8, B=0)) == 0   # nothing to do
    assert f(*args(None, None, 8, Sq=0)) == 0
    bad = (_FAKE, _BAD, _FAKE, _S4, _FAKE, _S4, _FAKE, _S4, None, _FAKE, None, 8,
           1, 32, 8, 128, 4096, 128, 0.1, 1, 0, None)
    assert f(*bad) == -4


# ---------------------------------------------------------------------------
# Dispatch rule
# ---------------------------------------------------------------------------
def test_route_baseline_configs():
    from gqa_kernels.dispatch import choose_route
    cu = 256
    # prefill: single pass, 256 packed rows (64 positions x 4 heads) per workgroup
    r = choose_route(1, 32, 8, 16384, 16384, cu)
    assert r.kind == "single" and r.workgroups == 256 * 8
    # decode 131072: split to 2 workgroups per CU
    r = choose_route(1, 32, 8, 1, 131072, cu)
    assert r.kind == "split" and r.splits == 64 and r.workgroups == 512
    # decode 8192 / 32768 / 65536: one workgroup per CU (a second one only
    # for chunks of at least 2048 keys)
    r = choose_route(1, 32, 8, 1, 8192, cu)
    assert r.kind == "split" and r.splits == 32 and r.workgroups == 256
    r = choose_route(1, 32, 8, 1, 32768, cu)
    assert r.kind == "split" and r.splits == 32 and r.workgroups == 256
    r = choose_route(1, 32, 8, 1, 65536, cu)
    assert r.kind == "split" and r.splits == 32 and r.workgroups == 256
    # head_dim 64, one token (the 16-row first pass): the head_dim-128 count
    r = choose_route(1, 32, 8, 1, 8192, cu, True, 64)
    assert r.kind == "split" and r.splits == 32
    assert choose_route(1, 32, 8, 1, 131072, cu, True, 64).splits == 32  # doubling from 4096-key chunks
    # head_dim 64 over more than 16 rows (the register-staged first pass):
    # two per CU with 128-key chunks
    r = choose_route(1, 32, 8, 8, 8192, cu, True, 64)
    assert r.kind == "split" and r.splits == 64
    # decode 4096: limited by the minimum chunk (one 128-key tile)
    r = choose_route(1, 32, 8, 1, 4096, cu)
    assert r.kind == "split" and r.splits == 32
    # 70B multi-token decode: 32 packed rows per kv head, 128 (b, kv head) pairs
    r = choose_route(16, 64, 8, 4, 32768, cu)
    assert r.kind == "split" and r.splits == 4 and r.workgroups == 512
    # chunked prefill: single pass
    assert choose_route(4, 32, 8, 512, 8192, cu).kind == "single"
    # reference decode cases below the split threshold stay single-pass
    assert choose_route(1, 32, 8, 1, 512, cu).kind == "single"


def test_route_wide_row_blocks():
    # 33-64 packed rows per kv head (verify steps of 9-16 tokens at G = 4):
    # at head_dim 128 one workgroup covers both 32-row blocks, so the split
    # count is sized for half as many workgroups per split as at head_dim 64.
    from gqa_kernels.dispatch import choose_route, split_rows_per_workgroup
    from gqa_kernels.paged import paged_splits
    cu = 256
    assert split_rows_per_workgroup(32) == 32 and split_rows_per_workgroup(33) == 64
    assert split_rows_per_workgroup(64, 64) == 32
    for sq in (9, 16):
        # 64-row workgroups: the second doubling needs 4096-key chunks
        # (16 tokens at 131072 keys: 32 splits 92.2 us, 64 splits 96.2)
        r = choose_route(1, 32, 8, sq, 131072, cu)
        assert r.kind == "split" and r.splits == 32 and r.workgroups == 256
        assert choose_route(1, 32, 8, sq, 262144, cu).splits == 64
        # 32768 keys: the CUs filled once
        assert choose_route(1, 32, 8, sq, 32768, cu).splits == 32
        r64 = choose_route(1, 32, 8, sq, 131072, cu, True, 64)
        assert r64.kind == "split" and r64.splits == 32 and r64.workgroups == 512
    assert choose_route(1, 32, 8, 8, 131072, cu).workgroups == 512
    # 65-128 rows: four 32-row blocks per workgroup; the split count fills
    # the CUs, then doubles only while chunks keep 2048 keys
    r = choose_route(1, 32, 8, 17, 131072, cu)
    assert r.kind == "split" and r.splits == 64 and r.workgroups == 512
    assert choose_route(1, 32, 8, 32, 32768, cu).splits == 32
    assert choose_route(4, 32, 8, 32, 32768, cu).splits == 16
    assert split_rows_per_workgroup(65) == 128 and split_rows_per_workgroup(128) == 128
    assert choose_route(1, 32, 8, 33, 131072, cu).kind == "chunks"  # past the split path: key chunks
    assert choose_route(1, 32, 8, 17, 131072, cu, True, 64).kind == "chunks"  # head_dim 64: 64 rows at most
    assert paged_splits(1, 32, 8, 32, 32768, cu) == 32
    assert paged_splits(1, 32, 8, 16, 131072, cu) == 32
    assert paged_splits(1, 32, 8, 16, 131072, cu, block_size=16) == 32
    assert paged_splits(1, 32, 8, 16, 131072, cu, head_dim=64) == 32


def test_route_key_chunks():
    # Fewer query blocks than compute units against a long cache: the
    # single pass over key chunks (one item per block and chunk) when the
    # model beats the plain single pass; never for the BASELINE prefill
    # shapes, below the reference's 1024-key split threshold, or with a
    # compute unit per block already.
    from gqa_kernels.dispatch import (CHUNK_MIN_TILES, _fwd_block_tiles, choose_kv_chunks, choose_route,
                                      chunks_makespan, fwd_split_makespan)
    cu = 256
    r = choose_route(1, 32, 8, 128, 131072, cu)
    assert r.kind == "chunks" and r.splits == 16 and r.workgroups == 256
    r = choose_route(1, 32, 8, 512, 32768, cu)
    assert r.kind == "chunks" and r.splits == 4
    for S in (2048, 4096, 8192, 16384):
        assert choose_route(1, 32, 8, S, S, cu).kind == "single"
    assert choose_route(4, 32, 8, 512, 8192, cu).kind == "single"   # 256 blocks
    assert choose_route(1, 32, 8, 200, 900, cu).kind == "single"    # below 1024 keys
    assert choose_route(1, 32, 8, 2048, 131072, cu).kind == "single"
    # the model: chunk counts are powers of two with >= CHUNK_MIN_TILES tiles
    tiles = _fwd_block_tiles(2, 64, 128, 131072, True)
    base = fwd_split_makespan(tiles, 0, 8, cu)
    kc = choose_kv_chunks(1, 32, 8, 128, 131072, cu, True)
    assert kc & (kc - 1) == 0 and -(-max(tiles) // kc) >= CHUNK_MIN_TILES
    assert chunks_makespan(tiles, kc, 8, cu, 32 * 128, 128) < 0.1 * base


def test_fwd_split_choice():
    from gqa_kernels.dispatch import _fwd_block_tiles, choose_fwd_split, choose_route, fwd_split_makespan
    cu = 256
    # few causal blocks per CU: the heaviest blocks are split
    for S in (512, 1024, 2048):
        r = choose_route(1, 32, 8, S, S, cu, True)
        n_mblk = S // 64
        assert r.kind == "single" and 0 < r.fwd_split <= n_mblk
        assert r.workgroups == (n_mblk + r.fwd_split) * 8
        tiles = _fwd_block_tiles(n_mblk, 64, S, S, True)
        assert fwd_split_makespan(tiles, r.fwd_split, 8, cu) <= 0.95 * fwd_split_makespan(tiles, 0, 8, cu)
    # enough blocks per CU, non-causal, chunked (uniform blocks): no split
    assert choose_route(1, 32, 8, 16384, 16384, cu, True).fwd_split == 0
    assert choose_route(1, 32, 8, 2048, 2048, cu, False).fwd_split == 0
    assert choose_fwd_split(4, 32, 8, 512, 8192, cu, True) == 0
    # causal block tiles: block m of a square prefill sees m + 1 tiles
    assert _fwd_block_tiles(4, 64, 256, 256, True) == [1, 2, 3, 4]
    assert _fwd_block_tiles(2, 64, 128, 1000, True) == [15, 16]
    assert _fwd_block_tiles(2, 64, 128, 1000, False) == [16, 16]


def test_fwd_split_static_schedule_model():
    """With fewer than FWD_DYN_MIN_ITEMS_PER_WG items per workgroup the
    persistent single pass deals each workgroup a fixed item list
    (gqa_fwd.hip item_at); the run-time model's makespan is the heaviest of
    those lists, re-derived here per workgroup id as the kernel does
    (XCD = id % 8, slot = id / 8, snake rounds over the XCD's range)."""
    import random
    from gqa_kernels.dispatch import (FWD_DYN_MIN_ITEMS_PER_WG, FWD_ITEM_OVERHEAD, FWD_MERGE_OVERHEAD,
                                      _fwd_block_tiles, fwd_split_makespan)
    rng = random.Random(5)
    for _ in range(40):
        n_mblk = rng.randint(2, 40)
        n_bh = rng.randint(1, 12)
        cu = rng.choice([16, 24, 64, 256])
        ns = rng.randint(0, n_mblk)
        tiles = _fwd_block_tiles(n_mblk, 64, 64 * n_mblk, 64 * n_mblk, True)
        items = [tiles[n_mblk - 1 - i] - tiles[n_mblk - 1 - i] // 2 + FWD_MERGE_OVERHEAD for i in range(ns)]
        items += [tiles[m] // 2 + FWD_MERGE_OVERHEAD if m >= n_mblk - ns else tiles[m]
                  for m in range(n_mblk - 1, -1, -1)]
        total = len(items) * n_bh
        n_wg = min(total, cu)
        if total >= FWD_DYN_MIN_ITEMS_PER_WG * n_wg:
            continue
        q, r = divmod(total, 8)
        worst = 0
        for wg in range(n_wg):
            x, slot = wg % 8, wg // 8
            S = (n_wg - x + 7) // 8
            lo, n = x * q + min(x, r), q + (1 if x < r else 0)
            t, k = 0, 0
            while True:
                e = k * S + (S - 1 - slot if k % 2 else slot)
                if e >= n:
                    break
                t += items[(lo + e) % len(items)] + FWD_ITEM_OVERHEAD
                k += 1
            worst = max(worst, t)
        assert fwd_split_makespan(tiles, ns, n_bh, cu) == worst


def test_chunks_greedy_schedule_model():
    """The key-chunk model for one workgroup per item (paged caches) or the
    dynamic schedule: items per (b, kv head) chunk-major, blocks heavy-first
    within a chunk, each of min(ct, tiles left) + CHUNK_ITEM_OVERHEAD steps;
    each XCD's CUs take its contiguous share of the whole list, the next
    item going to the least loaded CU.  The model schedules runs of equal
    items in bulk; here every item is placed one at a time on a heap."""
    import heapq
    import random
    from gqa_kernels.dispatch import (CHUNK_ITEM_OVERHEAD, COMBINE_BYTES_PER_US, COMBINE_LAUNCH_US,
                                      CHUNK_PARTIAL_PASSES, TILE_STEP_US, _fwd_block_tiles, chunks_makespan)
    rng = random.Random(9)
    for _ in range(200):
        block_m = rng.choice([16, 32, 64])
        seq_q = rng.randint(1, 12 * block_m)
        seq_kv = seq_q + rng.choice([0, rng.randint(1, 300), rng.randint(1000, 40000)])
        causal = rng.random() < 0.7
        tiles = _fwd_block_tiles(-(-seq_q // block_m), block_m, seq_q, seq_kv, causal)
        ks = rng.choice([2, 4, 8, 32, 128])
        n_bh = rng.randint(1, 20)
        cu = rng.choice([16, 64, 256])
        ct = max(1, -(-max(tiles) // ks))
        order = range(len(tiles) - 1, -1, -1) if causal else range(len(tiles))
        items = [min(ct, max(tiles[m] - c * ct, 0)) + CHUNK_ITEM_OVERHEAD for c in range(ks) for m in order] * n_bh
        q, r = divmod(len(items), 8)
        worst = 0
        for x in range(8):
            lo = x * q + min(x, r)
            heap = [0] * max(1, cu // 8)
            for w in range(lo, lo + q + (1 if x < r else 0)):
                heapq.heapreplace(heap, heap[0] + items[w])
            worst = max(worst, max(heap))
        rows = 7 * seq_q
        combine = COMBINE_LAUNCH_US + CHUNK_PARTIAL_PASSES * rows * ks * 130 * 4 / COMBINE_BYTES_PER_US
        got = chunks_makespan(tiles, ks, n_bh, cu, rows, 128, causal, persistent=False)
        assert got == pytest.approx(worst + combine / TILE_STEP_US, rel=1e-12, abs=1e-9)


def test_fwd_split_measured_choices():
    # Causal prefill on one MI355X (us, the route taken vs the alternative):
    # G = 4, B = 2 x 1536 tokens 56.0 unsplit -> 49.3 with 6 blocks split;
    # B = 4 x 768 40.5 -> 35.1 with 4; B = 5 x 512 unsplit 27.9 vs 35.3
    # with 4 split.
    from gqa_kernels.dispatch import choose_route
    assert choose_route(2, 32, 8, 1536, 1536, 256, True).fwd_split > 0
    assert choose_route(4, 32, 8, 768, 768, 256, True).fwd_split > 0
    assert choose_route(5, 32, 8, 512, 512, 256, True).fwd_split == 0
    # Short chunks against short caches (the fp32 partials of key chunks
    # cost more than the chunks save): 512 new tokens over 2048 keys, key
    # chunks 43.0 us vs the single pass with every block split 32.1 (head
    # dim 64: 45.3 vs 25.9); 128 x 2048 at B = 4 42.0 vs 33.8.
    for D in (128, 64):
        r = choose_route(1, 32, 8, 512, 2048, 256, True, D)
        assert r.kind == "single" and r.fwd_split == 8
    assert choose_route(4, 32, 8, 128, 2048, 256, True).kind == "single"
    # Few query blocks against long caches keep the key chunks: 128 x 131072
    # 238 us in 16 chunks vs 1068 single; 64 x 8192 29.1 in 16 vs 81.2.
    assert choose_route(1, 32, 8, 128, 131072, 256, True).kind == "chunks"
    assert choose_route(1, 32, 8, 64, 8192, 256, True).kind == "chunks"
    # Two kv heads of 1024 tokens: the split single pass, 23.2 us (17.9 at
    # head_dim 64) vs key chunks 29.6 (26.7).
    for D in (128, 64):
        assert choose_route(1, 8, 2, 1024, 1024, 256, True, D).kind == "single"


def test_fwd_split_launch_validation(lib):
    f = lib.gqa_fwd_split_launch
    args = lambda lse, ws, cnt, ns: (_FAKE, _S4, _FAKE, _S4, _FAKE, _S4, _FAKE, _S4, lse, ws, cnt, ns,
                                     1, 32, 8, 1024, 1024, 128, 0.1275, 1, 0, None)
    assert f(*args(None, _FAKE, _FAKE, 17)) == -5   # 1024 / 64 = 16 query blocks
    assert f(*args(None, _FAKE, _FAKE, -1)) == -5
    assert f(*args(None, None, _FAKE, 4)) == -7
    assert f(*args(None, _FAKE, None, 4)) == -7
    assert f(*args(None, ctypes.c_void_p((1 << 20) + 8), _FAKE, 4)) == -4
    assert f(*args(None, _FAKE, ctypes.c_void_p((1 << 20) + 2), 4)) == -4
    assert f(*args(ctypes.c_void_p((1 << 20) + 2), _FAKE, _FAKE, 4)) == -4
    assert lib.gqa_fwd_split_workspace_bytes(2, 8, 128, 5) == 2 * 8 * 5 * 2 * 512 * (64 + 2) * 4
    assert lib.gqa_fwd_split_workspace_bytes(1, 8, 64, 3) == 8 * 3 * 2 * 512 * (32 + 2) * 4
    assert lib.gqa_fwd_split_workspace_bytes(1, 8, 96, 3) == 0
    # split blocks' counters, then the 32 scheduling counters
    assert lib.gqa_fwd_split_counters_count(2, 8, 5) == 80 + 32
    assert lib.gqa_fwd_split_counters_count(2, 8, 0) == 32
    assert lib.gqa_fwd_split_counters_count(2, 8, -1) == 0


def test_route_properties():
    from gqa_kernels.dispatch import SPLIT_MIN_TILES, SPLIT_TILE, choose_route
    for skv in (1024, 1500, 4096, 65536, 1 << 20):
        for b in (1, 2, 8, 64):
            for cu in (80, 256):
                r = choose_route(b, 32, 8, 1, skv, cu)
                assert r.kind == "split"
                assert r.splits & (r.splits - 1) == 0  # power of two
                assert r.splits == 1 or -(-skv // r.splits) >= SPLIT_MIN_TILES * SPLIT_TILE
                # never more splits than needed for the per-CU target
                from gqa_kernels.dispatch import SPLIT_WG_PER_CU, SPLIT_WIDER_MIN_CHUNK
                assert r.splits == 1 or (r.workgroups // 2) < SPLIT_WG_PER_CU * cu
                # a doubling past one workgroup per CU only with chunks of
                # >= SPLIT_WIDER_MIN_CHUNK keys (no doubling at one split)
                assert (r.splits == 1 or r.workgroups // 2 < cu
                        or -(-skv // r.splits) >= SPLIT_WIDER_MIN_CHUNK)


# ---------------------------------------------------------------------------
# Python asserts (reference dispatch.py:30-33), tripped on CPU tensors
# ---------------------------------------------------------------------------
def test_asserts_on_cpu():
    from gqa_kernels import gqa_flash_attn
    q = torch.zeros(1, 32, 4, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 8, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="divisible"):
        gqa_flash_attn(q, torch.zeros(1, 6, 4, 128, dtype=torch.bfloat16),
                       torch.zeros(1, 6, 4, 128, dtype=torch.bfloat16))
    with pytest.raises(AssertionError, match="head_dim"):
        gqa_flash_attn(q[..., :96], k[..., :96], k[..., :96])
    with pytest.raises(AssertionError):
        gqa_flash_attn(q, k, k)  # CPU tensors: is_cuda assert


def test_package_exports():
    import gqa_kernels
    assert gqa_kernels.__all__ == ["gqa_flash_attn"]
    assert gqa_kernels.__version__ == "0.1.0"


# ---------------------------------------------------------------------------
# Layouts the kernels accept as they are, and copies of the others
# ---------------------------------------------------------------------------
def test_kernel_ready_layouts():
    from gqa_kernels.dispatch import _is_kernel_ready, _kernel_ready
    base = torch.zeros(2, 8, 64, 128, dtype=torch.bfloat16)
    assert _is_kernel_ready(base) and _kernel_ready(base) is base
    # (B, S, H, D) storage viewed as (B, H, S, D): strides of 16-byte rows
    bshd = torch.zeros(2, 64, 8, 128, dtype=torch.bfloat16).transpose(1, 2)
    assert _is_kernel_ready(bshd) and _kernel_ready(bshd) is bshd
    cases = [
        torch.zeros(2, 8, 128, 64, dtype=torch.bfloat16).transpose(2, 3),  # last-dim stride 64
        torch.zeros(2 * 8 * 64 * 128 + 1, dtype=torch.bfloat16)[1:].view(2, 8, 64, 128),  # 2-byte offset
        base.as_strided((2, 8, 1, 128), (8 * 64 * 128, 64 * 128, 3, 1)),  # odd stride on a size-1 dim
        torch.zeros(2, 8, 64, 132, dtype=torch.bfloat16)[..., :128],  # 264-byte rows
    ]
    for t in cases:
        assert not _is_kernel_ready(t)
        c = _kernel_ready(t)
        assert c is not t and _is_kernel_ready(c) and torch.equal(c, t)
