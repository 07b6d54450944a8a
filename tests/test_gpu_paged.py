"""GPU parity of the paged KV-cache path (paged_attention, write_kv,
PagedKVCache, GQAPagedAttention) against the CPU oracle's paged_reference
(per-sequence gqa_reference over the gathered K/V), at the bf16/fp16 gates of
the contiguous path; the cache write is checked bit-exactly."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BASELINE_TOL, assert_close, to_np
from oracle.gqa_oracle import paged_reference

pytestmark = pytest.mark.gpu

DEV = "cuda"
LSE_TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _paged_inputs(B, Hq, Hkv, Sq, lens, D, block_size, dtype, seed, spare_blocks=5, width_pad=2, hnd=False):
    """Random q and a paged cache holding `lens[b]` keys per sequence at a
    shuffled block assignment (unused blocks and table entries hold junk that
    must never be read: NaN in the cache, 0 in the table).  hnd: the caches
    are (num_blocks, block_size, Hkv, D) views of (num_blocks, Hkv,
    block_size, D) storage."""
    g = torch.Generator().manual_seed(seed)
    per = [-(-n // block_size) for n in lens]
    nblk = sum(per) + spare_blocks
    kc = torch.full((nblk, block_size, Hkv, D), float("nan"))
    vc = torch.full((nblk, block_size, Hkv, D), float("nan"))
    perm = torch.randperm(nblk, generator=g).tolist()
    table = torch.zeros(B, max(per) + width_pad, dtype=torch.int32)
    for b, n in enumerate(lens):
        blocks = [perm.pop() for _ in range(per[b])]
        table[b, :len(blocks)] = torch.tensor(blocks, dtype=torch.int32)
        if n:
            k = torch.randn(n, Hkv, D, generator=g)
            v = torch.randn(n, Hkv, D, generator=g)
            j = torch.arange(n)
            kc[table[b, j // block_size].long(), j % block_size] = k
            vc[table[b, j // block_size].long(), j % block_size] = v
    q = torch.randn(B, Hq, Sq, D, generator=g)
    q, kc, vc = (t.to(dtype) for t in (q, kc, vc))
    if hnd:
        kc = kc.transpose(1, 2).contiguous().transpose(1, 2)
        vc = vc.transpose(1, 2).contiguous().transpose(1, 2)
    seq_lens = torch.tensor(lens, dtype=torch.int32)
    return q, kc, vc, table, seq_lens


def _check(o, lse, q, kc, vc, table, seq_lens, causal, dtype):
    ref_o, ref_lse = paged_reference(to_np(q), to_np(kc), to_np(vc), table.numpy(), seq_lens.numpy(), causal)
    got = to_np(o)
    # A sequence without keys: zero rows (tests/reference.py:33-34 over an
    # empty key axis), exactly.
    assert np.all(got[seq_lens.numpy() == 0] == 0) and np.all(ref_o[seq_lens.numpy() == 0] == 0)
    nan = np.isnan(ref_o)
    assert np.array_equal(np.isnan(got), nan), "fully masked rows differ"
    assert_close(got[~nan], ref_o[~nan], BASELINE_TOL[dtype], "paged")
    if lse is not None:
        got_l = to_np(lse).astype(np.float64)
        fin = np.isfinite(ref_lse)
        assert np.array_equal(np.isneginf(got_l), ~fin)
        assert np.abs(got_l[fin] - ref_lse[fin]).max() <= LSE_TOL


@pytest.mark.parametrize("B,Hq,Hkv,Sq,lens,D,bs,dtype,causal", [
    (4, 32, 8, 1, [1, 77, 300, 1024], 128, 16, torch.bfloat16, True),     # small pages, ragged
    (4, 32, 8, 1, [2000, 64, 129, 700], 128, 64, torch.bfloat16, True),   # 64-key pages
    (2, 32, 8, 1, [5000, 3001], 128, 128, torch.float16, True),           # 128-key pages, fp16
    (3, 64, 8, 4, [4096, 10, 555], 128, 32, torch.bfloat16, True),        # G=8, 4-token verify
    (2, 32, 8, 3, [2, 900], 64, 8, torch.float16, True),                  # seq shorter than Sq: masked rows
    (2, 32, 4, 16, [1500, 260], 64, 256, torch.bfloat16, False),          # chunk, non-causal, big pages
    (1, 16, 16, 1, [333], 128, 1, torch.bfloat16, True),                  # MHA, one-slot pages
    (3, 32, 8, 1, [0, 500, 64], 128, 16, torch.bfloat16, True),           # a sequence without keys: zeros
    (2, 32, 8, 16, [3000, 700], 128, 16, torch.bfloat16, True),           # 64 rows: one wide row block
    (3, 32, 8, 9, [1300, 64, 5], 128, 64, torch.float16, True),           # 36 rows, a sequence shorter than Sq
    (2, 32, 8, 32, [2500, 40], 128, 16, torch.bfloat16, True),            # 128 rows: four blocks per workgroup
])
def test_paged_attention_matches_oracle(B, Hq, Hkv, Sq, lens, D, bs, dtype, causal):
    from gqa_kernels.paged import paged_attention
    q, kc, vc, table, seq_lens = _paged_inputs(B, Hq, Hkv, Sq, lens, D, bs, dtype, seed=sum(lens))
    print(f"paged B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} lens={lens} D={D} bs={bs} {dtype}", flush=True)
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), causal)
    o, lse = paged_attention(*args, max_seq_len=max(lens), return_lse=True)
    o2 = paged_attention(*args)  # default bound: the table's capacity (more, empty splits)
    torch.cuda.synchronize()
    _check(o, lse, q, kc, vc, table, seq_lens, causal, dtype)
    _check(o2, None, q, kc, vc, table, seq_lens, causal, dtype)


@pytest.mark.parametrize("B,Hq,Hkv,Sq,lens,D,bs,dtype,causal,hnd", [
    (2, 32, 8, 100, [3000, 150], 128, 64, torch.bfloat16, True, False),      # chunk over a prefix
    (1, 32, 8, 512, [8192], 128, 128, torch.bfloat16, True, True),           # 512-token chunk, HND
    (3, 64, 8, 40, [1000, 41, 2500], 128, 256, torch.bfloat16, True, False),  # G = 8, sequence == chunk
    (2, 32, 8, 200, [150, 1000], 128, 64, torch.bfloat16, True, True),       # shorter than the chunk: masked rows
    (2, 16, 4, 70, [700, 333], 64, 64, torch.float16, False, False),         # D = 64, fp16, non-causal
    # pages under 64 keys: one descriptor per LDS-DMA instruction (4 rows at
    # D = 128, 8 at D = 64); ragged lengths end inside an instruction's rows
    (2, 32, 8, 100, [3001, 150], 128, 16, torch.bfloat16, True, False),      # vLLM's 16-key blocks, NHD
    (1, 32, 8, 300, [2047], 128, 16, torch.bfloat16, True, True),            # 16-key blocks, HND
    (2, 32, 8, 90, [1030, 91], 128, 4, torch.bfloat16, True, False),         # smallest block at D = 128
    (2, 32, 8, 90, [999, 400], 128, 32, torch.float16, False, True),         # 32-key blocks, fp16
    (2, 16, 4, 70, [701, 333], 64, 8, torch.float16, True, False),           # smallest block at D = 64
    (1, 16, 2, 120, [1500], 64, 16, torch.bfloat16, False, True),            # D = 64, 16-key HND
    (2, 16, 2, 120, [1500, 433], 64, 16, torch.bfloat16, True, False),       # D = 64, 16-key NHD
    (2, 16, 4, 80, [900, 2000], 64, 32, torch.float16, True, False),         # D = 64, 32-key NHD
    (2, 32, 8, 100, [0, 700], 128, 64, torch.bfloat16, True, False),         # a sequence without keys: zeros
])
def test_paged_single_pass_matches_oracle(B, Hq, Hkv, Sq, lens, D, bs, dtype, causal, hnd):
    """Query blocks above the split-KV size take the single-pass kernel with
    each tile loaded from its block(s)."""
    from gqa_kernels.paged import paged_attention, paged_route
    assert paged_route(Hq, Hkv, Sq, bs, D) == "single"
    q, kc, vc, table, seq_lens = _paged_inputs(B, Hq, Hkv, Sq, lens, D, bs, dtype, seed=sum(lens) + 1, hnd=hnd)
    print(f"paged single B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} lens={lens} D={D} bs={bs} {dtype} hnd={hnd}", flush=True)
    kd, vd = kc.to(DEV), vc.to(DEV)
    if hnd:
        kd, vd = (t.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for t in (kc, vc))
    args = (q.to(DEV), kd, vd, table.to(DEV), seq_lens.to(DEV), causal)
    o, lse = paged_attention(*args, max_seq_len=max(lens), return_lse=True, route="single")
    o_split = paged_attention(*args, max_seq_len=max(lens), route="split")
    o_default = paged_attention(*args, max_seq_len=max(lens))  # single, or key chunks (paged_kv_chunks)
    torch.cuda.synchronize()
    _check(o, lse, q, kc, vc, table, seq_lens, causal, dtype)
    _check(o_split, None, q, kc, vc, table, seq_lens, causal, dtype)
    _check(o_default, None, q, kc, vc, table, seq_lens, causal, dtype)


@pytest.mark.parametrize("pad", [32, 16])
def test_paged_single_pass_padded_rows(pad):
    """Caches whose slot stride is head_dim + pad elements (one kv head):
    at D = 64 a row stride of 192 bytes (a multiple of 64, not of 128) keeps
    the 16-32-key form, whose K offsets come from an XOR of bit 5; 160 bytes
    takes the per-instruction form."""
    from gqa_kernels.paged import paged_attention, paged_route
    B, Hq, Hkv, Sq, lens, D, bs = 2, 8, 1, 100, [777, 1500], 64, 16
    assert paged_route(Hq, Hkv, Sq, bs, D) == "single"
    q, kc, vc, table, seq_lens = _paged_inputs(B, Hq, Hkv, Sq, lens, D, bs, torch.bfloat16, seed=pad)
    print(f"paged single padded rows D={D} bs={bs} pad={pad}", flush=True)

    def padded(t):
        store = torch.full(t.shape[:-1] + (D + pad,), float("nan"), dtype=t.dtype, device=DEV)
        store[..., :D] = t.to(DEV)
        return store[..., :D]
    kd, vd = padded(kc), padded(vc)
    assert kd.stride(1) == D + pad
    o, lse = paged_attention(q.to(DEV), kd, vd, table.to(DEV), seq_lens.to(DEV), True, max_seq_len=max(lens),
                             return_lse=True)
    torch.cuda.synchronize()
    _check(o, lse, q, kc, vc, table, seq_lens, True, torch.bfloat16)


@pytest.mark.parametrize("D,bs", [(128, 128), (128, 16), (128, 4), (64, 8), (64, 16)])
def test_paged_single_pass_equals_contiguous_prefill_chunk(D, bs):
    """The chunked-prefill BASELINE shape (B=4, 512 new tokens over 8192 keys)
    from a shuffled block cache vs the contiguous single pass: bit-identical
    for blocks of whole tiles (128) and for blocks under a tile, where every
    LDS-DMA instruction gets its own descriptor (16, and 4 / 8: the fewest
    rows one instruction loads at D = 128 / 64)."""
    from gqa_kernels import gqa_flash_attn
    from gqa_kernels.paged import paged_attention
    B, Hq, Hkv, Sq, L = 4, 32, 8, 512, 8192
    print(f"paged == contiguous D={D} bs={bs}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(21)
    q = torch.randn(B, Hq, Sq, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, Hkv, L, D, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, Hkv, L, D, generator=g, device=DEV).to(torch.bfloat16)
    nper = L // bs
    perm = torch.randperm(B * nper, generator=g, device=DEV)
    kc = torch.empty(B * nper, bs, Hkv, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.empty_like(kc)
    kc[perm] = k.permute(0, 2, 1, 3).reshape(B * nper, bs, Hkv, D)
    vc[perm] = v.permute(0, 2, 1, 3).reshape(B * nper, bs, Hkv, D)
    table = perm.to(torch.int32).view(B, nper)
    lens = torch.full((B,), L, dtype=torch.int32, device=DEV)
    o_p = paged_attention(q, kc, vc, table, lens, True)
    o_c = gqa_flash_attn(q, k, v, causal=True)
    torch.cuda.synchronize()
    # same kernel, same tiles in the same order: identical results
    assert torch.equal(o_p, o_c)


@pytest.mark.parametrize("bs,causal", [(16, True), (128, True), (64, False)])
def test_paged_attention_head_major_cache(bs, causal):
    """Caches stored (num_blocks, Hkv, block_size, D): each head's rows of a
    block are consecutive (the layout the split kernel streams fastest)."""
    from gqa_kernels.paged import paged_attention
    q, kc, vc, table, seq_lens = _paged_inputs(3, 32, 8, 2, [4000, 130, 1111], 128, bs, torch.bfloat16,
                                               seed=bs, hnd=True)
    assert kc.stride(1) == 128
    kd, vd = (t.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for t in (kc, vc))
    o, lse = paged_attention(q.to(DEV), kd, vd, table.to(DEV), seq_lens.to(DEV), causal, max_seq_len=4000,
                             return_lse=True)
    torch.cuda.synchronize()
    _check(o, lse, q, kc, vc, table, seq_lens, causal, torch.bfloat16)


@pytest.mark.parametrize("splits", [1, 3, 16])
def test_paged_split_counts(splits):
    from gqa_kernels.paged import paged_attention
    q, kc, vc, table, seq_lens = _paged_inputs(2, 32, 8, 1, [3000, 1200], 128, 64, torch.bfloat16, seed=7)
    o = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True,
                        max_seq_len=3000, splits=splits)
    torch.cuda.synchronize()
    _check(o, None, q, kc, vc, table, seq_lens, True, torch.bfloat16)


@pytest.mark.parametrize("bs,max_len,splits", [(1, 4096, 2), (1, 4096, None), (16, 40000, 2), (4, 8000, 1)])
def test_paged_small_pages_table_slice(bs, max_len, splits):
    """Pages under 64 keys: each workgroup stages its chunk's block-table
    slice in LDS; (1, 4096, 2) and (16, 40000, 2) put 2048 and 1252 pages
    in a chunk (2048 is the most a chunk may span), None is the host's own
    split choice."""
    from gqa_kernels.paged import paged_attention
    q, kc, vc, table, seq_lens = _paged_inputs(2, 32, 8, 1, [max_len, max_len // 2 + 3], 128, bs,
                                               torch.bfloat16, seed=11)
    o, lse = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True,
                             max_seq_len=max_len, splits=splits, return_lse=True)
    torch.cuda.synchronize()
    _check(o, lse, q, kc, vc, table, seq_lens, True, torch.bfloat16)


@pytest.mark.parametrize("bs,max_len", [(1, 4096), (16, 40000)])
def test_paged_small_pages_rejects_oversized_chunks(bs, max_len):
    """One split over more than 2048 pages is refused before any launch."""
    from gqa_kernels import _lib
    from gqa_kernels.paged import paged_attention
    q, kc, vc, table, seq_lens = _paged_inputs(1, 32, 8, 1, [max_len], 128, bs, torch.bfloat16, seed=12)
    with pytest.raises(_lib.GQAError, match="-5"):
        paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True,
                        max_seq_len=max_len, splits=1)


def test_paged_equals_contiguous_at_decode_scale():
    """131072 keys in 128-key pages (shuffled) vs the contiguous split-KV
    route on the same K/V: same math, different chunking."""
    from gqa_kernels import gqa_flash_attn
    from gqa_kernels.paged import paged_attention
    Hq, Hkv, L, D, bs = 32, 8, 131072, 128, 128
    g = torch.Generator(device=DEV).manual_seed(11)
    k = torch.randn(1, Hkv, L, D, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, Hkv, L, D, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(1, Hq, 1, D, generator=g, device=DEV).to(torch.bfloat16)
    nblk = L // bs
    perm = torch.randperm(nblk, generator=g, device=DEV)
    kc = torch.empty(nblk, bs, Hkv, D, dtype=torch.bfloat16, device=DEV)
    vc = torch.empty_like(kc)
    kc[perm] = k[0].permute(1, 0, 2).reshape(nblk, bs, Hkv, D)
    vc[perm] = v[0].permute(1, 0, 2).reshape(nblk, bs, Hkv, D)
    table = perm.to(torch.int32)[None]
    o_p = paged_attention(q, kc, vc, table, torch.tensor([L], dtype=torch.int32, device=DEV), True)
    o_c = gqa_flash_attn(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert_close(o_p, o_c, BASELINE_TOL[torch.bfloat16], "paged vs contiguous")


@pytest.mark.parametrize("D,dtype", [(128, torch.bfloat16), (64, torch.float16)])
def test_write_kv_is_exact(D, dtype):
    from gqa_kernels.paged import write_kv
    nblk, bs, Hkv, T = 20, 16, 8, 57
    g = torch.Generator().manual_seed(2)
    kc = torch.randn(nblk, bs, Hkv, D, generator=g).to(dtype)
    vc = torch.randn(nblk, bs, Hkv, D, generator=g).to(dtype)
    key = torch.randn(T, Hkv, D, generator=g).to(dtype)
    val = torch.randn(T, Hkv, D, generator=g).to(dtype)
    slots = torch.randperm(nblk * bs, generator=g)[:T]
    slots[::7] = -1  # padding tokens are skipped
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    # key/value as strided views of a wider (T, 2*Hkv*D) projection output
    kv = torch.cat([key.reshape(T, -1), val.reshape(T, -1)], dim=1).to(DEV)
    write_kv(kv[:, :Hkv * D].view(T, Hkv, D), kv[:, Hkv * D:].view(T, Hkv, D), kc_d, vc_d, slots.to(DEV))
    torch.cuda.synchronize()
    keep = slots >= 0
    kc[slots[keep] // bs, slots[keep] % bs] = key[keep]
    vc[slots[keep] // bs, slots[keep] % bs] = val[keep]
    assert torch.equal(kc_d.cpu(), kc) and torch.equal(vc_d.cpu(), vc)


def test_prefix_cache_shared_across_sequences():
    """A 1000-token prefix stored once; three forks append their own turns
    (a chunk, then decode steps) and attend over prefix + own tokens."""
    from gqa_kernels.paged import PagedKVCache
    Hq, Hkv, D, bs = 32, 8, 128, 64
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(9)
    cache = PagedKVCache(200, bs, Hkv, D, dtype=dt, device=DEV)
    kp = torch.randn(1000, Hkv, D, generator=g).to(dt)
    vp = torch.randn(1000, Hkv, D, generator=g).to(dt)
    cache.add_sequence("prefix")
    cache.append(["prefix"], kp.to(DEV), vp.to(DEV))
    used = cache.num_blocks - cache.num_free_blocks()
    keys = {s: [kp] for s in "abc"}
    vals = {s: [vp] for s in "abc"}
    for s in "abc":
        cache.fork("prefix", s)
    # turn: 24-token chunk per fork (batched), then 3 decode steps
    for step, n in enumerate([24, 1, 1, 1]):
        kn = torch.randn(3 * n, Hkv, D, generator=g).to(dt)
        vn = torch.randn(3 * n, Hkv, D, generator=g).to(dt)
        q = torch.randn(3, Hq, n, D, generator=g).to(dt)
        cache.append(list("abc"), kn.to(DEV), vn.to(DEV))
        for i, s in enumerate("abc"):
            keys[s].append(kn[i * n:(i + 1) * n])
            vals[s].append(vn[i * n:(i + 1) * n])
        o, lse = cache.attend(q.to(DEV), list("abc"), return_lse=True)
        torch.cuda.synchronize()
        # oracle: contiguous prefix + own tokens per sequence, as a 1-block-per-key table
        for i, s in enumerate("abc"):
            k_all = torch.cat(keys[s])
            v_all = torch.cat(vals[s])
            L = k_all.shape[0]
            ref_o, ref_l = paged_reference(to_np(q[i:i + 1]), to_np(k_all[:, None]), to_np(v_all[:, None]),
                                           np.arange(L)[None], np.array([L]), True)
            assert_close(to_np(o[i:i + 1]), ref_o, BASELINE_TOL[dt], f"fork {s} step {step}")
            assert np.abs(to_np(lse[i:i + 1]) - ref_l).max() <= LSE_TOL
    # the prefix's 15 full blocks are stored once; its partial 16th was copied per fork
    assert cache.blocks("a")[:15] == cache.blocks("prefix")[:15] == cache.blocks("b")[:15]
    assert len({cache.blocks(s)[15] for s in ("prefix", "a", "b", "c")}) == 4
    # plus one copied block and one new block per fork
    assert cache.num_blocks - cache.num_free_blocks() == used + 6


@pytest.mark.parametrize("layout", ["HND", "NHD"])
def test_vllm_shaped_layer_decode_and_chunk(layout):
    from gqa_kernels.paged import GQAPagedAttention, PagedAttentionMetadata, PagedKVCache
    Hq, Hkv, D, bs = 32, 8, 128, 16
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(13)
    cache = PagedKVCache(400, bs, Hkv, D, dtype=dt, device=DEV, layout=layout)
    layer = GQAPagedAttention(Hq, D, scale=0.05, num_kv_heads=Hkv)
    hist = {}
    lens0 = [700, 33, 1500]
    for s, n in enumerate(lens0):
        cache.add_sequence(s)
        k = torch.randn(n, Hkv, D, generator=g).to(dt)
        v = torch.randn(n, Hkv, D, generator=g).to(dt)
        cache.append([s], k.to(DEV), v.to(DEV))
        hist[s] = (k, v)
    for sq in (1, 5):
        B = 3
        query = torch.randn(B * sq, Hq * D, generator=g).to(dt)
        key = torch.randn(B * sq, Hkv * D, generator=g).to(dt)
        value = torch.randn(B * sq, Hkv * D, generator=g).to(dt)
        slots = torch.tensor(sum((cache.reserve(s, sq) for s in range(B)), []), dtype=torch.int64)
        md = PagedAttentionMetadata(slot_mapping=slots.to(DEV), block_tables=cache.block_table(range(B)),
                                    seq_lens=cache.seq_lens(range(B)), query_len=sq)
        out = layer(query.to(DEV), key.to(DEV), value.to(DEV), cache.kv, md)
        torch.cuda.synchronize()
        assert tuple(out.shape) == (B * sq, Hq * D)
        for s in range(B):
            k, v = hist[s]
            k = torch.cat([k, key[s * sq:(s + 1) * sq].view(sq, Hkv, D)])
            v = torch.cat([v, value[s * sq:(s + 1) * sq].view(sq, Hkv, D)])
            hist[s] = (k, v)
            L = k.shape[0]
            # scale 0.05 = D^-0.5 applied to q * (0.05 * sqrt(D))
            q4 = to_np(query[s * sq:(s + 1) * sq].view(sq, Hq, D).permute(1, 0, 2)[None]).astype(np.float64)
            q4 = q4 * (0.05 * D ** 0.5)
            ref_o, _ = paged_reference(q4, to_np(k[:, None]), to_np(v[:, None]), np.arange(L)[None],
                                       np.array([L]), True)
            got = to_np(out[s * sq:(s + 1) * sq].view(sq, Hq, D).permute(1, 0, 2)[None])
            assert_close(got, ref_o, BASELINE_TOL[dt], f"layer seq {s} sq {sq}")


def _varlen_inputs(Hq, Hkv, D, lens, qlens, bs, dtype, seed):
    """Paged cache as _paged_inputs and a token-major q of sum(qlens) rows."""
    _, kc, vc, table, seq_lens = _paged_inputs(len(lens), Hq, Hkv, 1, lens, D, bs, dtype, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    q = torch.randn(sum(qlens), Hq, D, generator=g).to(dtype)
    starts = [sum(qlens[:b]) for b in range(len(qlens))]
    return q, kc, vc, table, seq_lens, starts


def _check_varlen(o, lse, q, kc, vc, table, seq_lens, starts, qlens, causal, dtype):
    for b, (s0, n) in enumerate(zip(starts, qlens)):
        if n == 0:
            continue
        qb = q[s0:s0 + n].permute(1, 0, 2)[None]  # (1, Hq, n, D)
        ob = o[s0:s0 + n].permute(1, 0, 2)[None]
        lb = None if lse is None else lse[s0:s0 + n].t()[None]
        _check(ob, lb, qb, kc, vc, table[b:b + 1], seq_lens[b:b + 1], causal, dtype)


@pytest.mark.parametrize("route,bs,causal", [("single", 64, True), ("split", 64, True), ("split", 16, True),
                                             ("single", 128, False), ("single", 16, True), ("single", 4, False)])
def test_paged_variable_query_lengths(route, bs, causal):
    from gqa_kernels.paged import paged_attention
    Hq, Hkv, D = 32, 8, 128
    lens = [900, 40, 2000, 130, 7]
    qlens = [1, 37, 5, 130, 7]  # a decode step, chunks, a whole short sequence
    dt = torch.bfloat16
    q, kc, vc, table, seq_lens, starts = _varlen_inputs(Hq, Hkv, D, lens, qlens, bs, dt, seed=31 + bs)
    print(f"varlen route={route} bs={bs} causal={causal}", flush=True)
    qs = torch.tensor(starts, dtype=torch.int32, device=DEV)
    ql = torch.tensor(qlens, dtype=torch.int32, device=DEV)
    o, lse = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), causal,
                             max_seq_len=max(lens), return_lse=True, route=route, query_start=qs, query_lens=ql,
                             max_query_len=max(qlens))
    torch.cuda.synchronize()
    assert tuple(o.shape) == tuple(q.shape) and tuple(lse.shape) == (q.shape[0], Hq)
    _check_varlen(o.cpu(), lse.cpu(), q, kc, vc, table, seq_lens, starts, qlens, causal, dt)


@pytest.mark.parametrize("bs,case", [(64, "interleaved"), (16, "interleaved"), (16, "long_prefix"),
                                     (32, "adjacent")])
def test_vllm_shaped_layer_mixed_batch(bs, case):
    """Prefill chunks and decode steps in one call: the layer runs one launch
    per kernel route over token-major views and that route's sequences —
    views of the block table when they are adjacent in the batch, rows
    gathered on the device otherwise (16-key blocks: both routes on blocks
    under one 64-key tile).  With a chunk over a long prefix the prefill
    launch takes the key chunks."""
    from gqa_kernels.dispatch import _cu_count
    from gqa_kernels.paged import (GQAPagedAttention, PagedAttentionMetadata, PagedKVCache, paged_kv_chunks,
                                   paged_route)
    Hq, Hkv, D = 32, 8, 128
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(17)
    long_prefix = case == "long_prefix"
    hist_lens, qlens = {
        "interleaved": ([1200, 0, 3000, 55], [1, 200, 1, 30]),  # decode, a whole prompt, decode, a chunk
        "long_prefix": ([16000, 700, 0, 2], [128, 1, 0, 1]),  # a chunk, decode, an idle slot, decode
        "adjacent": ([500, 2500, 40, 900], [64, 100, 1, 1]),  # two chunks, then two decode steps
    }[case]
    cache = PagedKVCache((sum(hist_lens) + sum(qlens)) // bs + 64, bs, Hkv, D, dtype=dt, device=DEV)
    layer = GQAPagedAttention(Hq, D, num_kv_heads=Hkv)
    hist = {}
    for s, n in enumerate(hist_lens):  # a sequence of 0 keys starts empty (a fresh prompt)
        cache.add_sequence(s)
        k = torch.randn(n, Hkv, D, generator=g).to(dt)
        v = torch.randn(n, Hkv, D, generator=g).to(dt)
        if n:
            cache.append([s], k.to(DEV), v.to(DEV))
        hist[s] = (k, v)
    T = sum(qlens)
    query = torch.randn(T, Hq * D, generator=g).to(dt)
    key = torch.randn(T, Hkv * D, generator=g).to(dt)
    value = torch.randn(T, Hkv * D, generator=g).to(dt)
    slots = torch.tensor(sum((cache.reserve(s, n) for s, n in enumerate(qlens)), []), dtype=torch.int64)
    md = PagedAttentionMetadata(slot_mapping=slots.to(DEV), block_tables=cache.block_table(range(4)),
                                seq_lens=cache.seq_lens(range(4)), query_lens=qlens)
    routes = [paged_route(Hq, Hkv, n, bs) if n else None for n in qlens]
    if case == "adjacent":
        assert routes == ["single", "single", "split", "split"]
    if long_prefix:
        capacity = md.block_tables.shape[1] * bs
        assert paged_kv_chunks(1, Hq, Hkv, 128, capacity, _cu_count(0), True, D) > 0
    print(f"mixed batch bs={bs} hist={hist_lens} qlens={qlens}", flush=True)
    out = layer(query.to(DEV), key.to(DEV), value.to(DEV), cache.kv, md)
    torch.cuda.synchronize()
    t0 = 0
    for s, n in enumerate(qlens):
        if n == 0:
            continue
        k, v = hist[s]
        k = torch.cat([k, key[t0:t0 + n].view(n, Hkv, D)])
        v = torch.cat([v, value[t0:t0 + n].view(n, Hkv, D)])
        L = k.shape[0]
        q4 = to_np(query[t0:t0 + n].view(n, Hq, D).permute(1, 0, 2)[None])
        ref_o, _ = paged_reference(q4, to_np(k[:, None]), to_np(v[:, None]), np.arange(L)[None], np.array([L]), True)
        got = to_np(out[t0:t0 + n].view(n, Hq, D).permute(1, 0, 2)[None])
        assert_close(got, ref_o, BASELINE_TOL[dt], f"mixed batch seq {s}")
        t0 += n


@pytest.mark.parametrize("route,varlen", [("split", False), ("single", False), ("chunks", False),
                                          ("split", True), ("single", True), ("chunks", True)])
def test_paged_binding_matches_ctypes(route, varlen, monkeypatch):
    """The torch-tensor binding (_gqa_host.so paged_forward) is what runs,
    and it gives the same bits as the ctypes calls of the same C entry
    points (the fallback when the binding cannot be loaded)."""
    from gqa_kernels import paged
    assert paged._paged_host() is not None, "the paged torch-tensor binding did not load"
    Hq, Hkv, D, bs = 32, 8, 128, 16
    lens = [3000, 700, 1500]
    splits = 4 if route != "single" else None
    if varlen:
        qlens = [1, 37, 5] if route == "split" else [64, 37, 130]
        q, kc, vc, table, seq_lens, starts = _varlen_inputs(Hq, Hkv, D, lens, qlens, bs, torch.bfloat16, seed=41)
        extra = dict(query_start=torch.tensor(starts, dtype=torch.int32, device=DEV),
                     query_lens=torch.tensor(qlens, dtype=torch.int32, device=DEV), max_query_len=max(qlens))
    else:
        sq = 1 if route == "split" else 64
        q, kc, vc, table, seq_lens = _paged_inputs(3, Hq, Hkv, sq, lens, D, bs, torch.bfloat16, seed=41)
        extra = {}
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True)
    print(f"binding vs ctypes route={route} varlen={varlen}", flush=True)

    def call():
        return paged.paged_attention(*args, max_seq_len=max(lens), return_lse=True, route=route, splits=splits,
                                     **extra)

    o1, l1 = call()
    monkeypatch.setattr(paged, "_paged_host", lambda: None)
    o2, l2 = call()
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_cache_write_binding_matches_ctypes(monkeypatch):
    from gqa_kernels import paged
    assert paged._paged_host() is not None
    g = torch.Generator().manual_seed(2)
    kc = torch.zeros(64, 16, 8, 128, dtype=torch.bfloat16, device=DEV)
    key = torch.randn(40, 8, 128, generator=g).to(torch.bfloat16).to(DEV)
    value = torch.randn(40, 8, 128, generator=g).to(torch.bfloat16).to(DEV)
    slots = torch.randperm(64 * 16, generator=g)[:40]
    slots[3] = -1  # padding
    slots = slots.to(DEV)
    k1, v1 = kc.clone(), kc.clone()
    paged.write_kv(key, value, k1, v1, slots)
    monkeypatch.setattr(paged, "_paged_host", lambda: None)
    k2, v2 = kc.clone(), kc.clone()
    paged.write_kv(key, value, k2, v2, slots)
    torch.cuda.synchronize()
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    keep = slots.cpu() >= 0
    s = slots.cpu()[keep]
    assert torch.equal(k1.view(-1, 8, 128)[s.to(DEV)], key[keep.to(DEV)])
