"""Paged single pass over key chunks (gqa_paged_fwd_chunks_launch through
gqa_kernels.paged.paged_attention, route "chunks"): few query blocks
against long sequences, the shape of a chunk of new tokens appended to a
long cached prefix.  Checked against the CPU oracle's paged_reference
(tests/reference.py:16-34 restated over a block table) on ragged lengths,
both in-block layouts, page sizes from 4 to 256 keys, fp16/bf16, head_dim
64/128, causal and not, variable query lengths, rows that see no key (NaN)
and a sequence without keys (zeros); and bit for bit against the contiguous
key-chunk route on the same keys."""
from __future__ import annotations

import pytest
import torch

from helpers import make_inputs
from test_gpu_paged import _check, _check_varlen, _paged_inputs, _varlen_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


@pytest.mark.parametrize("B,Hq,Hkv,Sq,lens,D,bs,dtype,causal,hnd,chunks", [
    (1, 32, 8, 256, [9000], 128, 16, torch.bfloat16, True, False, 8),        # 16-key NHD pages
    (2, 32, 8, 130, [5000, 700], 128, 64, torch.float16, True, True, 4),     # HND, a short sequence
    (3, 32, 4, 64, [3000, 0, 1500], 64, 32, torch.bfloat16, True, False, 4),  # D = 64, a sequence without keys
    (1, 16, 4, 100, [4000], 128, 128, torch.bfloat16, False, False, 16),     # non-causal
    (1, 32, 8, 96, [2500], 128, 4, torch.bfloat16, True, False, 8),          # smallest pages at D = 128
    (1, 64, 8, 40, [6000], 128, 16, torch.bfloat16, True, True, 16),         # G = 8, HND
    (2, 32, 8, 100, [60, 3000], 128, 16, torch.bfloat16, True, False, 4),    # fewer keys than queries: NaN rows
    (1, 16, 2, 200, [7000], 64, 8, torch.float16, True, True, 32),           # D = 64, 8-key HND pages
    (1, 32, 8, 64, [2049], 128, 256, torch.bfloat16, True, False, 2),        # ragged end inside a tile
])
def test_paged_chunks_match_oracle(B, Hq, Hkv, Sq, lens, D, bs, dtype, causal, hnd, chunks):
    from gqa_kernels.paged import paged_attention
    q, kc, vc, table, seq_lens = _paged_inputs(B, Hq, Hkv, Sq, lens, D, bs, dtype, seed=sum(lens) + 3, hnd=hnd)
    print(f"paged chunks B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} lens={lens} D={D} bs={bs} {dtype} causal={causal} "
          f"hnd={hnd} chunks={chunks}", flush=True)
    kd, vd = kc.to(DEV), vc.to(DEV)
    if hnd:
        kd, vd = (t.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for t in (kc, vc))
    args = (q.to(DEV), kd, vd, table.to(DEV), seq_lens.to(DEV), causal)
    o, lse = paged_attention(*args, max_seq_len=max(lens), return_lse=True, route="chunks", splits=chunks)
    torch.cuda.synchronize()
    _check(o, lse, q, kc, vc, table, seq_lens, causal, dtype)


@pytest.mark.parametrize("bs,causal", [(64, True), (16, True), (128, False)])
def test_paged_chunks_variable_query_lengths(bs, causal):
    from gqa_kernels.paged import paged_attention
    Hq, Hkv, D = 32, 8, 128
    lens = [5000, 40, 2000, 130]
    qlens = [100, 37, 5, 130]
    dt = torch.bfloat16
    q, kc, vc, table, seq_lens, starts = _varlen_inputs(Hq, Hkv, D, lens, qlens, bs, dt, seed=71 + bs)
    print(f"paged chunks varlen bs={bs} causal={causal}", flush=True)
    qs = torch.tensor(starts, dtype=torch.int32, device=DEV)
    ql = torch.tensor(qlens, dtype=torch.int32, device=DEV)
    o, lse = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), causal,
                             max_seq_len=max(lens), return_lse=True, route="chunks", splits=8, query_start=qs,
                             query_lens=ql, max_query_len=max(qlens))
    torch.cuda.synchronize()
    _check_varlen(o.cpu(), lse.cpu(), q, kc, vc, table, seq_lens, starts, qlens, causal, dt)


@pytest.mark.parametrize("D,bs", [(128, 64), (128, 16), (64, 32)])
def test_paged_chunks_equal_contiguous_chunks(D, bs):
    # The same keys in a contiguous cache and in shuffled pages: the paged
    # key chunks compute exactly what the contiguous key-chunk route does.
    from gqa_kernels.dispatch import chunks_forward
    from gqa_kernels.paged import paged_attention
    B, Hq, Hkv, Sq, Skv, S = 1, 32, 8, 128, 8192, 8
    q, k, v = make_inputs(B, Hq, Hkv, Sq, Skv, D, seed=5, device=DEV)
    g = torch.Generator().manual_seed(9)
    nblk = Skv // bs
    perm = torch.randperm(nblk, generator=g)
    kc = torch.empty(nblk, bs, Hkv, D, dtype=k.dtype, device=DEV)
    vc = torch.empty_like(kc)
    kc[perm] = k[0].transpose(0, 1).reshape(nblk, bs, Hkv, D)
    vc[perm] = v[0].transpose(0, 1).reshape(nblk, bs, Hkv, D)
    table = perm.to(torch.int32).reshape(1, nblk).to(DEV)
    lens = torch.tensor([Skv], dtype=torch.int32, device=DEV)
    print(f"paged chunks == contiguous chunks D={D} bs={bs}", flush=True)
    o_p = paged_attention(q, kc, vc, table, lens, True, max_seq_len=Skv, route="chunks", splits=S)
    o_c = chunks_forward(q, k, v, torch.empty_like(q), True, S)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_c)


def test_paged_default_route_takes_chunks_for_long_prefixes():
    from gqa_kernels.paged import paged_kv_chunks, paged_route
    assert paged_route(32, 8, 256, 16) == "single"
    assert paged_kv_chunks(1, 32, 8, 256, 32768, 256, True, 128) > 0
    assert paged_kv_chunks(4, 32, 8, 512, 8192, 256, True, 128) == 0


def test_paged_forced_chunks_default_count():
    # route="chunks" without splits takes the chunk model's count (at least
    # 2): the same result, bit for bit, as that count passed explicitly.
    from gqa_kernels.dispatch import _cu_count
    from gqa_kernels.paged import paged_attention, paged_kv_chunks
    B, Hq, Hkv, Sq, D, bs = 1, 32, 8, 64, 128, 16
    lens = [9000]
    q, kc, vc, table, seq_lens = _paged_inputs(B, Hq, Hkv, Sq, lens, D, bs, torch.bfloat16, seed=3)
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True)
    n = max(2, paged_kv_chunks(B, Hq, Hkv, Sq, max(lens), _cu_count(0), True, D))
    print(f"forced chunks default count {n}", flush=True)
    o_default = paged_attention(*args, max_seq_len=max(lens), route="chunks")
    o_explicit = paged_attention(*args, max_seq_len=max(lens), route="chunks", splits=n)
    o_other = paged_attention(*args, max_seq_len=max(lens), route="chunks", splits=2 * n)
    torch.cuda.synchronize()
    assert torch.equal(o_default, o_explicit)
    assert not torch.equal(o_default, o_other)
    _check(o_default, None, q, kc, vc, table, seq_lens, True, torch.bfloat16)
