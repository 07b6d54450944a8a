"""GPU parity of the 16-row split-KV first pass (gqa_decode16_kernel: every
(b, kv head) with at most 16 packed query rows, at head_dim 128 and 64)
against the CPU oracle: every packed-row count 1-16 through group sizes and
query lengths, odd groups (a position's heads split across lanes of
different lane groups), fp16, non-causal, the LSE side output, rows with no
visible key, an empty cache, and paged caches of 8- to 64-key blocks (one
descriptor per instruction, per wave and tile, or per tile) with ragged
sequence lengths."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BASELINE_TOL, REF_TOL, assert_close, make_inputs, oracle, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


@pytest.mark.parametrize("Hq,Hkv,sq", [
    (8, 8, 1), (16, 8, 1), (24, 8, 1), (32, 8, 1), (40, 8, 1), (64, 4, 1), (128, 8, 1),  # G = 1..16, Sq = 1
    (32, 8, 2), (32, 8, 3), (32, 8, 4),      # G = 4: 8, 12, 16 rows
    (24, 8, 5), (40, 8, 3), (56, 8, 2),      # G = 3 (15 rows), 5 (15), 7 (14)
    (8, 8, 16), (16, 8, 8),                  # MHA with 16 positions, G = 2 with 8
])
@pytest.mark.parametrize("S", [3, 16])
@pytest.mark.parametrize("D", [128, 64])
def test_decode16_rows(Hq, Hkv, sq, S, D):
    from gqa_kernels.gqa_split import split_kv_forward
    from oracle.gqa_oracle import gqa_lse
    skv = 64 * 7 * S + 29  # ragged last tile; S * 7 tiles
    q, k, v = make_inputs(1, Hq, Hkv, sq, skv, D, torch.bfloat16, seed=Hq * 31 + sq + S, device=DEV)
    assert (Hq // Hkv) * sq <= 16
    print(f"decode16 Hq={Hq} Hkv={Hkv} sq={sq} S={S} D={D}", flush=True)
    o, lse = split_kv_forward(q, k, v, True, S, return_lse=True)
    torch.cuda.synchronize()
    assert_close(o, oracle(q, k, v), BASELINE_TOL[torch.bfloat16], f"rows {Hq // Hkv * sq}")
    ref_lse = gqa_lse(to_np(q), to_np(k), to_np(v), True)
    np.testing.assert_allclose(to_np(lse), ref_lse, rtol=0, atol=2e-3)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [128, 64])
def test_decode16_fp16(causal, D):
    from gqa_kernels import gqa_flash_attn
    q, k, v = make_inputs(2, 32, 8, 1, 5000, D, torch.float16, scale=0.1, seed=3, device=DEV)
    o = gqa_flash_attn(q, k, v, causal=causal)
    torch.cuda.synchronize()
    assert_close(o, oracle(q, k, v, causal=causal), REF_TOL[torch.float16], f"fp16 causal={causal} D={D}")


@pytest.mark.parametrize("D", [128, 64])
def test_decode16_rows_without_keys_and_empty_cache(D):
    from gqa_kernels.gqa_split import split_kv_forward
    # seq_q > seq_kv under causal: positions 0..sq-skv-1 see no key (NaN rows).
    q, k, v = make_inputs(1, 16, 4, 4, 2, D, torch.bfloat16, seed=9, device=DEV)
    o = split_kv_forward(q, k, v, True, 2)
    torch.cuda.synchronize()
    ref = oracle(q, k, v)
    got = to_np(o)
    nan = np.isnan(ref)
    assert nan.any() and np.array_equal(np.isnan(got), nan)
    np.testing.assert_allclose(got[~nan], ref[~nan], rtol=0, atol=2e-2)
    # An empty cache: zero rows.
    q, k, v = make_inputs(1, 32, 8, 1, 0, D, torch.bfloat16, seed=9, device=DEV)
    o = split_kv_forward(q, k, v, True, 4)
    torch.cuda.synchronize()
    assert torch.count_nonzero(o).item() == 0


@pytest.mark.parametrize("block_size,layout,D", [(16, "NHD", 128), (32, "HND", 128), (32, "NHD", 128),
                                                 (8, "NHD", 64), (16, "NHD", 64), (32, "HND", 64), (64, "NHD", 64),
                                                 (64, "HND", 64)])
@pytest.mark.parametrize("sq", [1, 4])
def test_decode16_paged_medium_blocks(block_size, layout, D, sq):
    # Pages of 16-32 keys: each wave loads 16 consecutive rows of a tile
    # (one page); ragged lengths end inside a wave's share and inside a
    # page; unused slots hold NaN and must never be read.
    from gqa_kernels.paged import paged_attention
    from oracle.gqa_oracle import paged_reference
    B, Hq, Hkv = 3, 32, 8
    lens = [4096 + 7, 1000, 70]
    g = torch.Generator(device="cpu").manual_seed(block_size + sq)
    maxb = max(-(-n // block_size) for n in lens)
    nblk = B * maxb + 5
    perm = torch.randperm(nblk, generator=g)
    table = perm[:B * maxb].view(B, maxb).to(torch.int32)
    shape = (nblk, Hkv, block_size, D) if layout == "HND" else (nblk, block_size, Hkv, D)
    kc = torch.full(shape, float("nan"))
    vc = torch.full(shape, float("nan"))
    for b, n in enumerate(lens):
        kk = torch.randn(n, Hkv, D, generator=g)
        vv = torch.randn(n, Hkv, D, generator=g)
        for j in range(n):
            blk, slot = table[b, j // block_size].item(), j % block_size
            if layout == "HND":
                kc[blk, :, slot] = kk[j]
                vc[blk, :, slot] = vv[j]
            else:
                kc[blk, slot] = kk[j]
                vc[blk, slot] = vv[j]
    kc, vc = kc.to(torch.bfloat16), vc.to(torch.bfloat16)
    if layout == "HND":
        kcv, vcv = kc.transpose(1, 2), vc.transpose(1, 2)
    else:
        kcv, vcv = kc, vc
    q = torch.randn(B, Hq, sq, D, generator=g).to(torch.bfloat16)
    print(f"decode16 paged bs={block_size} {layout} D={D} sq={sq}", flush=True)
    o = paged_attention(q.to(DEV), kcv.to(DEV), vcv.to(DEV), table.to(DEV),
                        torch.tensor(lens, dtype=torch.int32, device=DEV), True, max_seq_len=max(lens))
    torch.cuda.synchronize()
    ref, _ = paged_reference(to_np(q), to_np(kcv), to_np(vcv), table.numpy(), np.array(lens), True)
    assert_close(o, ref, BASELINE_TOL[torch.bfloat16], f"paged bs={block_size} {layout}")
