"""The public path under HIP graph capture (torch.cuda.CUDAGraph): decode
steps (split-KV, two launches), the fused combine, prefill with and without
the key split, paged decode, the paged single pass with split blocks and
over key chunks, and the vLLM-shaped layer's decode step with its K/V write
are captured once and replayed several times, with eager work and synchronisations between replays; every replay
must equal the eager result bit for bit (the kernels are deterministic and
the captured launches see the same inputs)."""
from __future__ import annotations

import pytest
import torch

from helpers import make_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _capture(fn):
    # Warm-up on a side stream first: the cached workspaces and counters are
    # created (and zeroed) outside the capture.
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _replays(g, out, expect, n=4):
    for i in range(n):
        # eager work between replays (allocations, a reduction, a sync)
        junk = torch.randn(1 << 16, device=DEV).sum()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        outs = out if isinstance(out, tuple) else (out,)
        exps = expect if isinstance(expect, tuple) else (expect,)
        for a, b in zip(outs, exps):
            assert torch.equal(a, b), f"replay {i} differs from the eager result"
        del junk


@pytest.mark.parametrize("case", ["decode", "decode_lse", "prefill", "prefill_split", "chunked"])
def test_public_path_in_graph(case):
    from gqa_kernels import gqa_flash_attn
    shapes = {"decode": (1, 32, 8, 1, 16384), "decode_lse": (2, 32, 8, 1, 5000),
              "prefill": (1, 32, 8, 4096, 4096), "prefill_split": (1, 32, 8, 1024, 1024),
              "chunked": (2, 32, 8, 256, 3000)}
    B, Hq, Hkv, Sq, Skv = shapes[case]
    q, k, v = make_inputs(B, Hq, Hkv, Sq, Skv, 128, torch.bfloat16, seed=len(case), device=DEV)
    lse = case == "decode_lse"
    print(f"graph {case}", flush=True)
    fn = lambda: gqa_flash_attn(q, k, v, causal=True, return_lse=lse)
    expect = fn()
    torch.cuda.synchronize()
    expect = tuple(t.clone() for t in expect) if lse else expect.clone()
    g, out = _capture(fn)
    _replays(g, out, expect)


def test_graph_workspace_outlives_growth():
    """A decode graph keeps the raw address of the split workspace it was
    captured with.  A later, larger call on the same stream (a 1024-token
    prefill with the key split) replaces the stream's cached workspace; the
    replaced buffer must stay allocated, or the decode replays would write
    their partials into memory handed to other tensors.  Both calls warm up
    eagerly on the capture stream (so the first workspace comes from the
    general pool), the captures share one memory pool (vLLM's pattern), and
    tensors allocated afterwards at the first workspace's size must keep
    their contents across replays."""
    from gqa_kernels import gqa_flash_attn, gqa_split
    from gqa_kernels.dispatch import _cu_count, choose_route
    qd, kd, vd = make_inputs(1, 32, 8, 1, 16384, 128, torch.bfloat16, seed=31, device=DEV)
    qp, kp, vp = make_inputs(1, 32, 8, 1024, 1024, 128, torch.bfloat16, seed=32, device=DEV)
    assert choose_route(1, 32, 8, 1024, 1024, _cu_count(0)).fwd_split > 0
    dec = lambda: gqa_flash_attn(qd, kd, vd, causal=True)
    pre = lambda: gqa_flash_attn(qp, kp, vp, causal=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        exp_d = dec().clone()
    torch.cuda.synchronize()
    key = (torch.device(DEV).index or 0, s.cuda_stream)
    ws_dec = gqa_split._workspaces[key]
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1, stream=s):
        out_d = dec()
    with torch.cuda.stream(s):
        exp_p = pre().clone()  # grows the stream's workspace
    torch.cuda.synchronize()
    assert gqa_split._workspaces[key].data_ptr() != ws_dec.data_ptr()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s, pool=g1.pool()):
        out_p = pre()
    n = ws_dec.numel()
    del ws_dec
    fills = [torch.full((n,), float(i + 1), device=DEV) for i in range(6)]
    torch.cuda.synchronize()
    for i in range(3):
        g1.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_d, exp_d), f"decode replay {i} differs from eager"
        for j, f in enumerate(fills):
            assert bool((f == j + 1).all()), f"decode replay {i} wrote into a fresh tensor"
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_p, exp_p), f"prefill replay {i} differs from eager"


def test_fused_split_in_graph():
    from gqa_kernels.gqa_split import split_kv_forward
    q, k, v = make_inputs(1, 32, 8, 1, 8192, 128, torch.bfloat16, seed=3, device=DEV)
    fn = lambda: split_kv_forward(q, k, v, True, 32, fused=True)
    expect = fn().clone()
    g, out = _capture(fn)
    _replays(g, out, expect)


def test_paged_decode_in_graph():
    from gqa_kernels.paged import PagedKVCache
    g0 = torch.Generator().manual_seed(5)
    cache = PagedKVCache(256, 64, 8, 128, dtype=torch.bfloat16, device=DEV)
    for s, n in enumerate((3000, 777)):
        cache.add_sequence(s)
        cache.append([s], torch.randn(n, 8, 128, generator=g0).to(torch.bfloat16).to(DEV),
                     torch.randn(n, 8, 128, generator=g0).to(torch.bfloat16).to(DEV))
    q = torch.randn(2, 32, 1, 128, generator=g0).to(torch.bfloat16).to(DEV)
    table, lens = cache.block_table([0, 1]), cache.seq_lens([0, 1])
    from gqa_kernels.paged import paged_attention
    fn = lambda: paged_attention(q, cache.k_cache, cache.v_cache, table, lens, True, max_seq_len=3000)
    expect = fn().clone()
    g, out = _capture(fn)
    _replays(g, out, expect)


@pytest.mark.parametrize("shape", [(4, 32, 8, 4096, 4096),   # 2048 items: the dynamic schedule's queues
                                   (1, 32, 8, 1024, 1024)])  # key-split blocks: the merge counters
def test_two_graphs_replayed_concurrently(shape):
    # Two prefills captured into two graphs (on torch's one capture stream),
    # then replayed at the same time on two streams: each captured call has
    # its own counters (queue and merge counters that the kernel leaves
    # zero), so neither replay sees the other's claims.
    from gqa_kernels import gqa_flash_attn
    b, hq, hkv, sq, skv = shape
    print(f"two graphs concurrently {shape}", flush=True)
    ins = [make_inputs(b, hq, hkv, sq, skv, 128, torch.bfloat16, seed=s, device=DEV) for s in (1, 2)]
    expect = [gqa_flash_attn(*x, causal=True) for x in ins]
    graphs = [_capture(lambda x=x: gqa_flash_attn(*x, causal=True)) for x in ins]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(4):
        torch.cuda.synchronize()
        for (g, _), st in zip(graphs, streams):
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                g.replay()
        torch.cuda.synchronize()
        for i, ((_, out), e) in enumerate(zip(graphs, expect)):
            assert torch.equal(out, e), f"replay {rep} of graph {i} differs from the eager result"


def _paged_cache(lens, bs, seed):
    from gqa_kernels.paged import PagedKVCache
    g0 = torch.Generator().manual_seed(seed)
    cache = PagedKVCache(sum(-(-n // bs) for n in lens) + 8, bs, 8, 128, dtype=torch.bfloat16, device=DEV,
                         layout="NHD")
    for s, n in enumerate(lens):
        cache.add_sequence(s)
        cache.append([s], torch.randn(n, 8, 128, generator=g0).to(torch.bfloat16).to(DEV),
                     torch.randn(n, 8, 128, generator=g0).to(torch.bfloat16).to(DEV))
    return cache, g0


@pytest.mark.parametrize("case", ["split_blocks", "chunks", "layer_decode_write"])
def test_paged_routes_in_graph(case):
    """The paged single pass with split blocks (merge counters from the
    capture's own zeroed buffer), the paged key chunks (workspace and the
    combine) and the vLLM-shaped layer's decode step with its K/V write,
    captured and replayed."""
    from gqa_kernels.paged import GQAPagedAttention, PagedAttentionMetadata, paged_attention
    print(f"paged graph {case}", flush=True)
    if case == "layer_decode_write":
        lens = [3000, 700, 1500]
        cache, g0 = _paged_cache(lens, 16, 7)
        slots = torch.tensor(sum((cache.reserve(s, 1) for s in range(3)), []), dtype=torch.int64, device=DEV)
        md = PagedAttentionMetadata(slot_mapping=slots, block_tables=cache.block_table(range(3)),
                                    seq_lens=cache.seq_lens(range(3)), query_len=1, max_seq_len=3001)
        layer = GQAPagedAttention(32, 128, num_kv_heads=8)
        query = torch.randn(3, 32 * 128, generator=g0).to(torch.bfloat16).to(DEV)
        key = torch.randn(3, 8 * 128, generator=g0).to(torch.bfloat16).to(DEV)
        value = torch.randn(3, 8 * 128, generator=g0).to(torch.bfloat16).to(DEV)
        fn = lambda: layer(query, key, value, cache.kv, md)  # the same slots each time: idempotent
    else:
        lens = [3000, 1200] if case == "split_blocks" else [9000]
        cache, g0 = _paged_cache(lens, 16, 11)
        sq = 256 if case == "split_blocks" else 128
        q = torch.randn(len(lens), 32, sq, 128, generator=g0).to(torch.bfloat16).to(DEV)
        table, seq_lens = cache.block_table(range(len(lens))), cache.seq_lens(range(len(lens)))
        route, splits = ("single", 4) if case == "split_blocks" else ("chunks", 8)
        fn = lambda: paged_attention(q, cache.k_cache, cache.v_cache, table, seq_lens, True, max_seq_len=max(lens),
                                     return_lse=True, route=route, splits=splits)
    first = fn()
    expect = tuple(t.clone() for t in first) if isinstance(first, tuple) else first.clone()
    g, out = _capture(fn)
    _replays(g, out, expect)
