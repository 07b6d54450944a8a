"""GPU parity of the split-KV decode first pass at head_dim 128 (the
LDS-DMA kernel of gqa_decode.hip) at chunk boundaries: chunks of an odd
number of 64-key tiles (padded with one masked tile), of one partial tile,
and empty chunks (more splits than keys), through both the two-launch and
the fused combine, against the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BASELINE_TOL, assert_close, make_inputs, oracle, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


@pytest.mark.parametrize("sq,skv,S", [
    (1, 4 * 64 * 3, 4),     # 3 tiles per chunk (odd: one padding tile)
    (1, 4 * 64 * 5 + 17, 4),  # 5-6 tiles, ragged end
    (1, 8 * 64, 8),         # one tile per chunk
    (1, 100, 4),            # one partial tile per chunk
    (1, 5, 8),              # splits 5-7 hold no key
    (4, 3 * 64 * 7, 3),     # Sq = 4: the causal diagonal inside the last tile
    (16, 2 * 64 * 9 + 1, 2),  # 32 rows of one block, 9-10 tiles per chunk
])
@pytest.mark.parametrize("fused", [False, True])
def test_decode_chunk_boundaries(sq, skv, S, fused):
    from gqa_kernels.gqa_split import split_kv_forward
    q, k, v = make_inputs(1, 32, 8, sq, skv, 128, torch.bfloat16, seed=skv + S, device=DEV)
    print(f"decode chunks sq={sq} skv={skv} S={S} fused={fused}", flush=True)
    o = split_kv_forward(q, k, v, True, S, fused=fused)
    torch.cuda.synchronize()
    ref = oracle(q, k, v)
    assert_close(o, ref, BASELINE_TOL[torch.bfloat16], f"sq={sq} skv={skv} S={S}")


def test_decode_g8_rows_fill_a_block():
    # The 70B group (G = 8) with 4 query rows: all 32 rows of the block valid.
    from gqa_kernels import gqa_flash_attn
    q, k, v = make_inputs(2, 64, 8, 4, 5000, 128, torch.bfloat16, seed=5, device=DEV)
    o = gqa_flash_attn(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert_close(o, oracle(q, k, v), BASELINE_TOL[torch.bfloat16], "G = 8, Sq = 4")


@pytest.mark.parametrize("Hq,Hkv,sq,skv,S", [
    (32, 8, 9, 3 * 64 * 5 + 11, 4),   # 36 rows: the second 32-row block holds 4
    (32, 8, 16, 4096, 8),             # 64 rows: both blocks full
    (12, 4, 15, 2000, 3),             # G = 3: position 10 straddles the two blocks
    (64, 8, 5, 1000, 2),              # G = 8: 40 rows
    (32, 8, 12, 256, 8),              # 32-key chunks: the causal diagonal crosses chunks
    (32, 8, 16, 10, 2),               # seq_q > seq_kv: rows of positions 0-5 see no key (NaN)
    (32, 8, 17, 3 * 64 * 5 + 11, 4),  # 68 rows: four blocks per workgroup, the last holding 4 rows
    (32, 8, 32, 4096, 8),             # 128 rows: four full blocks
    (12, 4, 30, 2000, 3),             # G = 3, 90 rows: three blocks, the fourth empty
    (64, 8, 16, 1000, 2),             # G = 8: 128 rows
    (32, 8, 32, 20, 2),               # seq_q > seq_kv with four blocks: positions 0-11 see no key
])
@pytest.mark.parametrize("fused", [False, True])
def test_decode_wide_row_blocks(Hq, Hkv, sq, skv, S, fused):
    # 33-128 packed rows per kv head: one workgroup covers two or four
    # 32-row blocks (waves 0-1 / 2-3, or one wave each), streaming each
    # chunk once; the partials and the combine stay per 32-row block.
    from gqa_kernels.gqa_split import split_kv_forward
    from oracle.gqa_oracle import gqa_lse
    q, k, v = make_inputs(1, Hq, Hkv, sq, skv, 128, torch.bfloat16, seed=sq * skv + S, device=DEV)
    print(f"wide row blocks Hq={Hq} Hkv={Hkv} sq={sq} skv={skv} S={S} fused={fused}", flush=True)
    o, lse = split_kv_forward(q, k, v, True, S, fused=fused, return_lse=True)
    torch.cuda.synchronize()
    ref = oracle(q, k, v)
    got = to_np(o)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan), "fully masked rows differ"
    assert_close(got[~nan], ref[~nan], BASELINE_TOL[torch.bfloat16], f"sq={sq} skv={skv} S={S}")
    ref_l = gqa_lse(to_np(q), to_np(k), to_np(v), True)
    fin = np.isfinite(ref_l)
    got_l = to_np(lse)
    assert np.array_equal(np.isneginf(got_l), ~fin)
    assert np.abs(got_l[fin] - ref_l[fin]).max() <= 2e-3


def test_decode_wide_row_blocks_route_and_repeatability():
    # A 16-token verify step at G = 4 through the public entry point (split
    # route, 64-row workgroups): oracle parity, and the same bits on every
    # call (fixed combine order).
    from gqa_kernels import gqa_flash_attn
    from gqa_kernels.dispatch import _cu_count, choose_route
    assert choose_route(2, 32, 8, 16, 20000, _cu_count(0)).kind == "split"
    q, k, v = make_inputs(2, 32, 8, 16, 20000, 128, torch.bfloat16, seed=16, device=DEV)
    o = gqa_flash_attn(q, k, v, causal=True)
    for _ in range(3):
        assert torch.equal(gqa_flash_attn(q, k, v, causal=True), o)
    torch.cuda.synchronize()
    assert_close(o, oracle(q, k, v), BASELINE_TOL[torch.bfloat16], "verify step")


@pytest.mark.parametrize("Hq,Hkv,sq,skv,S", [
    (32, 4, 4, 128 * 64 + 37, 128),  # G * Sq = 32 valid rows x 128 splits: R * S = 4096, the fused limit
    (64, 8, 4, 64 * 64, 64),         # the 70B group, 32 rows x 64 splits
])
def test_decode_fused_combine_at_its_lds_limit(Hq, Hkv, sq, skv, S):
    # The fused combine stages m and l of R valid rows x S splits in LDS; at
    # R * S = 4096 they fill their 16 KiB stage arrays.  It must agree with
    # the two-launch combine (same partials, same arithmetic) and the oracle.
    from gqa_kernels.gqa_split import FUSED_MAX_ROW_SPLITS, split_kv_forward
    assert min(32, Hq // Hkv * sq) * S <= FUSED_MAX_ROW_SPLITS
    q, k, v = make_inputs(1, Hq, Hkv, sq, skv, 128, torch.bfloat16, seed=S + sq, device=DEV)
    print(f"fused combine limit Hq={Hq} Hkv={Hkv} sq={sq} skv={skv} S={S}", flush=True)
    o2, lse2 = split_kv_forward(q, k, v, True, S, fused=False, return_lse=True)
    of, lsef = split_kv_forward(q, k, v, True, S, fused=True, return_lse=True)
    torch.cuda.synchronize()
    # Same partials, combined in a different order: the outputs differ by at
    # most a bf16 rounding step of |o| < 1 (2^-8).
    assert (of.float() - o2.float()).abs().max().item() <= 2 ** -8, "fused and two-launch combines differ"
    assert torch.allclose(lsef, lse2, rtol=0, atol=1e-4)
    assert_close(of, oracle(q, k, v), BASELINE_TOL[torch.bfloat16], f"fused S={S}")
