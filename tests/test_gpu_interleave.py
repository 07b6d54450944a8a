"""Interleaved calls of every route on one stream: nothing one call leaves
behind changes another's result.

Several paths keep state in device memory between calls: the persistent
prefill's dynamic-schedule counters and the key-split blocks' merge
counters (contiguous and paged; zero on entry, left zero by the last
workgroup), the fused combine's counters, the stream's cached split workspace and counter buffers, and the
no-allocation entry point's fixed per-device buffer.  Each call kind below
is first run alone (synchronised) for its reference result; then a seeded
random sequence of 60 calls of all kinds runs back to back on the stream
with no synchronisation in between, and every result must equal its kind's
reference bit for bit (every route is deterministic: the dynamic schedule,
the key-split merge and the fused combine fix their arithmetic order
independently of which workgroup computes what).  Each kind is also checked
once against the CPU oracle (tests/reference.py:16-34 restated in
oracle/gqa_oracle.py), on row slices where the shape is large.
"""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from helpers import BASELINE_TOL, assert_close, make_inputs, to_np
from oracle.gqa_oracle import gqa_reference

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _kinds():
    """name -> (call returning a tuple of tensors, oracle check)."""
    from gqa_kernels import gqa_flash_attn
    from gqa_kernels import _lib
    from gqa_kernels.gqa_split import LOG2E, split_kv_forward
    from gqa_kernels.paged import paged_attention
    from test_gpu_paged import _check, _paged_inputs

    kinds = {}

    def contiguous(name, B, Hq, Hkv, Sq, Skv, D, causal, lse=False, rows=None):
        q, k, v = make_inputs(B, Hq, Hkv, Sq, Skv, D, seed=Sq + Skv + D, device=DEV)

        def call():
            r = gqa_flash_attn(q, k, v, causal=causal, return_lse=lse)
            return r if lse else (r,)

        def check(out):
            qn, kn, vn = to_np(q), to_np(k), to_np(v)
            if rows is None:
                ref, got = gqa_reference(qn, kn, vn, causal), to_np(out[0])
            else:  # a slice of query rows (the oracle on the whole shape takes too long)
                ref = gqa_reference(qn, kn, vn, causal, rows=rows)
                got = to_np(out[0])[:, :, rows]
            assert_close(got, ref, BASELINE_TOL[torch.bfloat16], name)

        kinds[name] = (call, check)

    # Single pass with key-split blocks (merge counters), persistent kernel
    # with the dynamic schedule (queue counters), key chunks + combine, LSE.
    contiguous("prefill 2048 key-split", 1, 32, 8, 2048, 2048, 128, True, rows=np.arange(1800, 2048))
    contiguous("prefill B=8 4096 dynamic", 8, 32, 8, 4096, 4096, 128, True, rows=np.arange(4000, 4096))
    contiguous("chunks 128 x 16384", 1, 32, 8, 128, 16384, 128, True)
    contiguous("prefill 1024 head_dim 64 lse", 1, 32, 8, 1024, 1024, 64, True, lse=True)
    contiguous("non-causal chunks 300 x 5000", 1, 32, 8, 300, 5000, 128, False)
    # Split-KV decode (cached workspace), verify step, head_dim 64.
    contiguous("decode 8192", 1, 32, 8, 1, 8192, 128, True)
    contiguous("verify B=2 16 x 8192 lse", 2, 32, 8, 16, 8192, 128, True, lse=True)
    contiguous("decode 8192 head_dim 64", 1, 32, 8, 1, 8192, 64, True)

    # Fused one-launch split-KV (its own counters).
    qf, kf, vf = make_inputs(1, 32, 8, 1, 20000, 128, seed=7, device=DEV)

    def fused():
        return split_kv_forward(qf, kf, vf, True, 32, fused=True, return_lse=True)

    def fused_check(out):
        assert_close(to_np(out[0]), gqa_reference(to_np(qf), to_np(kf), to_np(vf), True),
                     BASELINE_TOL[torch.bfloat16], "fused")

    kinds["fused decode 20000"] = (fused, fused_check)

    # No-allocation split-KV (the library's fixed per-device buffer).
    qn_, kn_, vn_ = make_inputs(2, 64, 8, 4, 6000, 128, seed=11, device=DEV)

    def noalloc():
        lib = _lib.load()
        B, Hq, Sq, D = qn_.shape
        o = torch.empty_like(qn_)
        lse = torch.empty(B, Hq, Sq, dtype=torch.float32, device=DEV)
        _lib.check(lib.gqa_split_noalloc_launch(
            qn_.data_ptr(), _lib.strides(qn_), kn_.data_ptr(), _lib.strides(kn_), vn_.data_ptr(), _lib.strides(vn_),
            o.data_ptr(), _lib.strides(o), lse.data_ptr(), 16, B, Hq, 8, Sq, 6000, D, D ** -0.5 * LOG2E, 1,
            _lib.DTYPE_BF16, torch.cuda.current_stream().cuda_stream))
        return o, lse

    def noalloc_check(out):
        assert_close(to_np(out[0]), gqa_reference(to_np(qn_), to_np(kn_), to_np(vn_), True),
                     BASELINE_TOL[torch.bfloat16], "noalloc")

    kinds["noalloc 70B-shaped"] = (noalloc, noalloc_check)

    # Paged decode (16-key token-major pages) and paged chunked prefill.
    for name, (B, Hq, Hkv, Sq, lens, D, bs) in {
            "paged decode bs16": (3, 32, 8, 1, [3000, 17, 5000], 128, 16),
            "paged chunk bs64": (2, 32, 8, 200, [2500, 900], 128, 64)}.items():
        q, kc, vc, table, seq_lens = _paged_inputs(B, Hq, Hkv, Sq, lens, D, bs, torch.bfloat16, seed=bs)
        args = (q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True)

        def pcall(args=args, lens=lens):
            return paged_attention(*args, max_seq_len=max(lens), return_lse=True)

        def pcheck(out, q=q, kc=kc, vc=vc, table=table, seq_lens=seq_lens):
            _check(out[0], out[1], q, kc, vc, table, seq_lens, True, torch.bfloat16)

        kinds[name] = (pcall, pcheck)

    # Paged single pass with split query blocks (merge counters in the same
    # per-stream counter buffer as the prefill's).
    q, kc, vc, table, seq_lens = _paged_inputs(2, 32, 8, 256, [3000, 1200], 128, 16, torch.bfloat16, seed=5)
    sargs = (q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True)

    def scall():
        return paged_attention(*sargs, max_seq_len=3000, return_lse=True, route="single", splits=4)

    def scheck(out, q=q, kc=kc, vc=vc, table=table, seq_lens=seq_lens):
        _check(out[0], out[1], q, kc, vc, table, seq_lens, True, torch.bfloat16)

    kinds["paged split blocks"] = (scall, scheck)
    return kinds


def test_interleaved_calls_match_isolated_calls():
    kinds = _kinds()
    ref = {}
    for name, (call, check) in kinds.items():
        print(f"interleave: isolated {name}", flush=True)
        out = call()
        torch.cuda.synchronize()
        check(out)
        ref[name] = tuple(t.clone() for t in out)
    names = list(kinds)
    rng = random.Random(20261202)
    order = [rng.choice(names) for _ in range(60)]
    print("interleave: sequence " + ", ".join(order), flush=True)
    results = [(name, kinds[name][0]()) for name in order]
    torch.cuda.synchronize()
    for j, (name, out) in enumerate(results):
        for a, b in zip(out, ref[name]):
            assert torch.equal(a, b), f"call {j} ({name}) differs from the isolated call"
    # Every shared counter is left at zero: a repeat of the isolated pass
    # (after the interleaved one) gives the same results again.
    for name, (call, _) in kinds.items():
        out = call()
        torch.cuda.synchronize()
        for a, b in zip(out, ref[name]):
            assert torch.equal(a, b), f"{name}: result changed after the interleaved sequence"


def test_two_streams_concurrently():
    # The cached split workspace and the counter buffers are per (device,
    # stream): calls of every kind issued alternately on two streams run
    # concurrently and still match their isolated results.  (The
    # no-allocation entry point shares one buffer per device and documents
    # that overlapping calls race, so it is left out.)
    kinds = {n: c for n, c in _kinds().items() if not n.startswith("noalloc")}
    ref = {}
    for name, (call, _) in kinds.items():
        out = call()
        torch.cuda.synchronize()
        ref[name] = tuple(t.clone() for t in out)
    names = list(kinds)
    rng = random.Random(7)
    order = [rng.choice(names) for _ in range(40)]
    print("two streams: sequence " + ", ".join(order), flush=True)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    results = []
    for j, name in enumerate(order):
        with torch.cuda.stream(streams[j % 2]):
            results.append((name, kinds[name][0]()))
    torch.cuda.synchronize()
    for j, (name, out) in enumerate(results):
        for a, b in zip(out, ref[name]):
            assert torch.equal(a, b), f"call {j} ({name}, stream {j % 2}) differs from the isolated call"
