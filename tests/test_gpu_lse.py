"""GPU parity of the LSE side output (return_lse=True) against the oracle's
gqa_lse, on both routes (single pass, split-KV two-launch and fused), and the
property it exists for: attention over two disjoint key ranges merges
exactly into attention over their union."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BASELINE_TOL, assert_close, make_inputs, oracle, to_np
from oracle.gqa_oracle import gqa_lse

pytestmark = pytest.mark.gpu

DEV = "cuda"
LSE_TOL = 2e-3  # absolute, natural-log units (fp32 accumulation of bf16/fp16 scores)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _lse_err(lse, q, k, v, causal=True):
    ref = gqa_lse(to_np(q), to_np(k), to_np(v), causal)
    got = to_np(lse).astype(np.float64)
    assert got.shape == ref.shape
    fin = np.isfinite(ref)
    assert np.array_equal(np.isneginf(got), ~fin), "-inf rows differ"
    return float(np.abs(got[fin] - ref[fin]).max()) if fin.any() else 0.0


def _route(q, k):
    from gqa_kernels.dispatch import _cu_count, choose_route
    B, Hq, Sq, _ = q.shape
    return choose_route(B, Hq, k.shape[1], Sq, k.shape[2], _cu_count(0))


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,dtype,causal", [
    (1, 32, 8, 1024, 1024, 128, torch.bfloat16, True),    # prefill, single pass
    (2, 32, 8, 300, 700, 64, torch.float16, True),        # chunked, D=64, fp16
    (1, 64, 8, 77, 2000, 128, torch.bfloat16, False),     # G=8, non-causal
    (1, 32, 8, 1, 8192, 128, torch.bfloat16, True),       # decode: split route
    (2, 64, 8, 4, 4096, 128, torch.bfloat16, True),       # 70B-style multi-token decode
    (1, 32, 8, 1, 3000, 64, torch.float16, True),         # decode D=64 fp16, ragged
])
def test_lse_matches_oracle(B, Hq, Hkv, Sq, Skv, D, dtype, causal):
    from gqa_kernels import gqa_flash_attn
    q, k, v = make_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=5, device=DEV)
    o, lse = gqa_flash_attn(q, k, v, causal=causal, return_lse=True)
    torch.cuda.synchronize()
    assert lse.dtype == torch.float32 and tuple(lse.shape) == (B, Hq, Sq)
    assert _lse_err(lse, q, k, v, causal) <= LSE_TOL, _route(q, k)
    # the output is the same as without the side output
    o2 = gqa_flash_attn(q, k, v, causal=causal)
    assert torch.equal(o, o2)


def test_lse_fused_combine_matches_two_launch():
    from gqa_kernels.gqa_split import split_kv_forward
    q, k, v = make_inputs(1, 32, 8, 1, 8192, 128, torch.bfloat16, seed=9, device=DEV)
    o1, l1 = split_kv_forward(q, k, v, True, 16, return_lse=True)
    o2, l2 = split_kv_forward(q, k, v, True, 16, fused=True, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.allclose(l1, l2, rtol=0, atol=1e-5)
    assert _lse_err(l2, q, k, v) <= LSE_TOL


def test_lse_rows_without_keys_are_neg_inf():
    from gqa_kernels import gqa_flash_attn
    # causal with seq_q > seq_kv: the first seq_q - seq_kv rows see no key
    q, k, v = make_inputs(1, 8, 8, 40, 16, 128, torch.bfloat16, seed=2, device=DEV)
    o, lse = gqa_flash_attn(q, k, v, causal=True, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isneginf(lse[:, :, :24]).all() and torch.isfinite(lse[:, :, 24:]).all()
    assert torch.isnan(o[:, :, :24]).all()


@pytest.mark.parametrize("sq,skv", [(1, 8192), (128, 4096)])
def test_lse_merges_disjoint_key_ranges(sq, skv):
    # Non-causal attention over keys [0, h) and [h, skv) merged with the LSEs
    # equals attention over all keys: the use the side output exists for.
    from gqa_kernels import gqa_flash_attn
    q, k, v = make_inputs(1, 32, 8, sq, skv, 128, torch.bfloat16, seed=4, device=DEV)
    h = skv // 3
    o1, l1 = gqa_flash_attn(q, k[:, :, :h], v[:, :, :h], causal=False, return_lse=True)
    o2, l2 = gqa_flash_attn(q, k[:, :, h:], v[:, :, h:], causal=False, return_lse=True)
    l = torch.logaddexp(l1, l2)
    merged = o1.float() * torch.exp(l1 - l)[..., None] + o2.float() * torch.exp(l2 - l)[..., None]
    full, lf = gqa_flash_attn(q, k, v, causal=False, return_lse=True)
    torch.cuda.synchronize()
    assert (lf - l).abs().max().item() <= LSE_TOL
    assert_close(merged, full, BASELINE_TOL[torch.bfloat16], "merged halves")
    assert_close(merged, oracle(q, k, v, causal=False), BASELINE_TOL[torch.bfloat16], "merged vs oracle")
