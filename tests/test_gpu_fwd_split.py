"""GPU parity of the single pass with key-range split of the heaviest causal
query blocks (gqa_fwd_split_launch): against the CPU oracle on row slices,
against the unsplit launch (same math, different summation order), with the
LSE side output, for forced split counts, chunked and fully masked cases,
and across repeated calls (the counters are left zero)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BASELINE_TOL, REF_TOL, assert_close, errors, make_inputs, oracle, to_np
from oracle.gqa_oracle import gqa_lse

pytestmark = pytest.mark.gpu

DEV = "cuda"
LSE_TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _run(q, k, v, causal, n_split, return_lse=False):
    from gqa_kernels.dispatch import single_pass_forward
    o = torch.empty_like(q)
    return single_pass_forward(q, k, v, o, causal, n_split, return_lse)


def _rows(sq, n=96):
    """First, last and evenly spaced query rows (keeps the oracle fast)."""
    return np.unique(np.concatenate([np.arange(min(sq, 16)), np.linspace(0, sq - 1, n).astype(int),
                                     np.arange(max(0, sq - 16), sq)]))


@pytest.mark.parametrize("S", [512, 1024, 2048])
def test_auto_split_prefill_matches_oracle(S):
    from gqa_kernels import gqa_flash_attn
    from gqa_kernels.dispatch import _cu_count, choose_route
    route = choose_route(1, 32, 8, S, S, _cu_count(0), True)
    assert route.kind == "single" and route.fwd_split > 0, route
    q, k, v = make_inputs(1, 32, 8, S, S, 128, torch.bfloat16, seed=S, device=DEV)
    print(f"auto split S={S} n_split={route.fwd_split}", flush=True)
    o, lse = gqa_flash_attn(q, k, v, causal=True, return_lse=True)
    torch.cuda.synchronize()
    rows = _rows(S)
    ref = oracle(q, k, v, True, rows=rows)
    assert_close(to_np(o)[:, :, rows], ref, BASELINE_TOL[torch.bfloat16], f"split S={S}")
    ref_l = gqa_lse(to_np(q), to_np(k), to_np(v), True, rows=rows)
    assert np.abs(to_np(lse)[:, :, rows] - ref_l).max() <= LSE_TOL
    # same result as the unsplit kernel up to summation order
    o0 = _run(q, k, v, True, 0)
    torch.cuda.synchronize()
    assert errors(o, o0)[0] <= 1.6e-2


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,dtype,n_split", [
    (1, 32, 8, 1024, 1024, 128, torch.bfloat16, 1),     # only the heaviest block
    (1, 32, 8, 1024, 1024, 128, torch.bfloat16, 16),    # every block (incl. 1-tile blocks)
    (2, 16, 2, 700, 700, 64, torch.float16, 5),         # G = 8 (32-position blocks), D = 64, ragged
    (1, 32, 8, 1024, 1500, 128, torch.bfloat16, 8),     # chunked: seq_q < seq_kv
    (1, 12, 4, 300, 300, 128, torch.bfloat16, 4),       # G = 3 (85-position blocks)
])
def test_forced_split_matches_oracle(B, Hq, Hkv, Sq, Skv, D, dtype, n_split):
    q, k, v = make_inputs(B, Hq, Hkv, Sq, Skv, D, dtype, seed=n_split + Sq, device=DEV)
    print(f"forced split {B},{Hq},{Hkv},{Sq},{Skv},{D},{dtype} n_split={n_split}", flush=True)
    o, lse = _run(q, k, v, True, n_split, return_lse=True)
    torch.cuda.synchronize()
    rows = _rows(Sq)
    ref = oracle(q, k, v, True, rows=rows)
    assert_close(to_np(o)[:, :, rows], ref, BASELINE_TOL[dtype], "forced split")
    ref_l = gqa_lse(to_np(q), to_np(k), to_np(v), True, rows=rows)
    assert np.abs(to_np(lse)[:, :, rows] - ref_l).max() <= LSE_TOL


def test_split_at_reference_tolerance_x01_inputs():
    # the reference's x0.1 inputs and its tighter bf16 tolerance
    q, k, v = make_inputs(1, 32, 8, 2048, 2048, 128, torch.bfloat16, scale=0.1, seed=3, device=DEV)
    o = _run(q, k, v, True, 32)
    torch.cuda.synchronize()
    rows = _rows(2048)
    assert_close(to_np(o)[:, :, rows], oracle(q, k, v, True, rows=rows), REF_TOL[torch.bfloat16], "x0.1")


def test_split_fully_masked_rows_stay_nan():
    # causal with seq_q > seq_kv: the first 40 rows see no key
    q, k, v = make_inputs(1, 8, 8, 296, 256, 128, torch.bfloat16, seed=4, device=DEV)
    o, lse = _run(q, k, v, True, 2, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isnan(o[:, :, :40]).all() and not torch.isnan(o[:, :, 40:]).any()
    assert torch.isneginf(lse[:, :, :40]).all() and torch.isfinite(lse[:, :, 40:]).all()


def test_split_repeated_calls_leave_counters_zero():
    from gqa_kernels import gqa_split
    q, k, v = make_inputs(1, 32, 8, 1024, 1024, 128, torch.bfloat16, seed=6, device=DEV)
    outs = [_run(q, k, v, True, ns) for ns in (16, 16, 3, 16)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[3])
    assert errors(outs[0], outs[2])[0] <= 1.6e-2
    for buf in gqa_split._counters.values():
        assert int(buf.abs().sum().item()) == 0


@pytest.mark.parametrize("n_split", [1, 8, 16])
def test_split_results_do_not_depend_on_which_half_merges(n_split):
    # Either half of a split block may finish last and merge; the merge is
    # written in terms of the lower and upper half, so every call gives the
    # same bits however the two halves were scheduled.
    q, k, v = make_inputs(1, 32, 8, 1024, 1024, 128, torch.bfloat16, seed=7, device=DEV)
    ref = _run(q, k, v, True, n_split)
    for _ in range(24):
        assert torch.equal(_run(q, k, v, True, n_split), ref)


def test_dynamic_schedule_equals_static_schedule():
    # With at least 8 work items per compute unit the persistent single pass
    # schedules its items dynamically across the XCDs when given counters
    # (gqa_fwd_split_launch, the Python route); items are independent, so
    # the outputs are bit-identical to the static schedule of gqa_fwd_launch,
    # on every call, and the counters are left zero.
    from gqa_kernels import _lib, gqa_split
    from gqa_kernels.dispatch import LOG2E, _cu_count
    B, Hq, Hkv, S, D = 4, 32, 8, 4096, 128
    items = B * Hkv * S // (256 // (Hq // Hkv))
    assert items >= 8 * min(items, _cu_count(0)), "shape too small for the dynamic schedule"
    q, k, v = make_inputs(B, Hq, Hkv, S, S, D, torch.bfloat16, seed=11, device=DEV)
    lib = _lib.load()
    o_static = torch.empty_like(q)
    print(f"dynamic vs static schedule B={B} S={S} items={items}", flush=True)
    _lib.check(lib.gqa_fwd_launch(q.data_ptr(), _lib.strides(q), k.data_ptr(), _lib.strides(k), v.data_ptr(),
                                  _lib.strides(v), o_static.data_ptr(), _lib.strides(o_static), B, Hq, Hkv, S, S,
                                  D, D ** -0.5 * LOG2E, 1, _lib.DTYPE_BF16,
                                  torch.cuda.current_stream().cuda_stream))
    outs = [_run(q, k, v, True, 0) for _ in range(4)]
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o, o_static)
    for buf in gqa_split._counters.values():
        assert int(buf.abs().sum().item()) == 0
    rows = _rows(S, 32)
    ref = oracle(q[:1, :4], k[:1, :1], v[:1, :1], True, rows=rows)
    assert_close(to_np(outs[0])[:1, :4][:, :, rows], ref, BASELINE_TOL[torch.bfloat16], "dynamic schedule")


def test_dynamic_schedule_with_split_blocks_repeats_exactly():
    # Split blocks under the dynamic schedule: either half may run on any
    # XCD; repeated calls give the same bits, close to the unsplit result.
    B, Hq, Hkv, S, D = 4, 32, 8, 4096, 128
    q, k, v = make_inputs(B, Hq, Hkv, S, S, D, torch.bfloat16, seed=12, device=DEV)
    ref = _run(q, k, v, True, 4)
    for _ in range(6):
        assert torch.equal(_run(q, k, v, True, 4), ref)
    o0 = _run(q, k, v, True, 0)
    torch.cuda.synchronize()
    assert errors(ref, o0)[0] <= 1.6e-2
