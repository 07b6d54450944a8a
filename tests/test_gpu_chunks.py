"""GPU parity of the single pass over key chunks (gqa_fwd_chunks_launch,
route kind "chunks"): every query block runs as several work items over
consecutive key ranges, each writing fp32 partials that the split-KV combine
reduces.  Against the CPU oracle (o and LSE), against the plain single pass
(same math, different summation order), for empty chunks, fully masked rows,
a sequence without keys, and through the public entry point."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BASELINE_TOL, assert_close, errors, make_inputs, oracle, to_np, torch_reference_gpu
from oracle.gqa_oracle import gqa_lse

pytestmark = pytest.mark.gpu

DEV = "cuda"
LSE_TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _chunks(q, k, v, causal, kv_splits, return_lse=False):
    from gqa_kernels.dispatch import chunks_forward
    return chunks_forward(q, k, v, torch.empty_like(q), causal, kv_splits, return_lse)


def _rows(sq, n=64):
    return np.unique(np.concatenate([np.arange(min(sq, 8)), np.linspace(0, sq - 1, n).astype(int),
                                     np.arange(max(0, sq - 8), sq)]))


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,dtype,causal,S", [
    (1, 32, 8, 128, 8192, 128, torch.bfloat16, True, 16),   # the route's shape class
    (1, 32, 8, 128, 8192, 128, torch.bfloat16, False, 16),  # non-causal
    (2, 12, 4, 100, 3000, 128, torch.float16, True, 5),     # G = 3, ragged keys, 5 chunks
    (1, 32, 8, 300, 4096, 64, torch.bfloat16, True, 8),     # head_dim 64 (one workgroup per item)
    (1, 32, 8, 64, 500, 128, torch.bfloat16, True, 16),     # 8 tiles, 16 chunks: 8 empty chunks
    (1, 32, 8, 17, 2048, 128, torch.bfloat16, True, 4),     # 68 packed rows, one block
    (1, 64, 8, 40, 5000, 128, torch.bfloat16, True, 8),     # G = 8, 320 rows: two blocks
])
def test_chunks_match_oracle(B, Hq, Hkv, Sq, Skv, D, dtype, causal, S):
    q, k, v = make_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=Sq + Skv + S, device=DEV)
    print(f"chunks {B},{Hq},{Hkv},{Sq},{Skv},{D},{dtype},causal={causal} S={S}", flush=True)
    o, lse = _chunks(q, k, v, causal, S, return_lse=True)
    torch.cuda.synchronize()
    rows = _rows(Sq)
    ref = oracle(q, k, v, causal, rows=rows)
    assert_close(to_np(o)[:, :, rows], ref, BASELINE_TOL[dtype], "chunks")
    ref_l = gqa_lse(to_np(q), to_np(k), to_np(v), causal, rows=rows)
    assert np.abs(to_np(lse)[:, :, rows] - ref_l).max() <= LSE_TOL
    # the plain single pass: same math, another summation order
    from gqa_kernels.dispatch import single_pass_forward
    o1 = single_pass_forward(q, k, v, torch.empty_like(q), causal, 0)
    torch.cuda.synchronize()
    assert errors(o, o1)[0] <= (1.6e-2 if dtype == torch.bfloat16 else 4e-3)


def test_chunks_fully_masked_rows_and_repeatability():
    # causal with seq_q > seq_kv: rows of positions 0-43 see no key (NaN o,
    # -inf LSE); every call gives the same bits.
    q, k, v = make_inputs(1, 8, 8, 300, 256, 128, torch.bfloat16, seed=4, device=DEV)
    o, lse = _chunks(q, k, v, True, 2, return_lse=True)
    for _ in range(3):  # bitwise (NaN rows included)
        assert torch.equal(_chunks(q, k, v, True, 2).view(torch.int16), o.view(torch.int16))
    torch.cuda.synchronize()
    assert torch.isnan(o[:, :, :44]).all() and not torch.isnan(o[:, :, 44:]).any()
    assert torch.isneginf(lse[:, :, :44]).all() and torch.isfinite(lse[:, :, 44:]).all()
    ref = oracle(q, k, v, True, rows=np.arange(44, 300))
    assert_close(to_np(o)[:, :, 44:], ref, BASELINE_TOL[torch.bfloat16], "masked rows")


def test_chunks_without_keys_gives_zeros():
    # seq_kv = 0: zero rows (tests/reference.py:33-34 over an empty key axis)
    q = torch.randn(1, 32, 100, 128, device=DEV).to(torch.bfloat16)
    k = torch.empty(1, 8, 0, 128, device=DEV, dtype=torch.bfloat16)
    o = _chunks(q, k, k, True, 4)
    torch.cuda.synchronize()
    assert torch.count_nonzero(o) == 0


def test_chunks_route_long_cache():
    # A 128-token chunk of Llama-3.1-8B attention against 131072 keys: the
    # route takes key chunks; checked against fp32 torch attention on the GPU.
    from gqa_kernels import gqa_flash_attn
    from gqa_kernels.dispatch import _cu_count, choose_route
    route = choose_route(1, 32, 8, 128, 131072, _cu_count(0))
    assert route.kind == "chunks", route
    q, k, v = make_inputs(1, 32, 8, 128, 131072, 128, torch.bfloat16, seed=9, device=DEV)
    print(f"chunks route {route}", flush=True)
    o = gqa_flash_attn(q, k, v, causal=True)
    ref = torch_reference_gpu(q, k, v, True)
    torch.cuda.synchronize()
    assert_close(o, ref, BASELINE_TOL[torch.bfloat16], "128 x 131072")
