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
