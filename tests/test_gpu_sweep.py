"""GPU parity over a seeded random sweep of shapes through the drop-in entry
point gqa_flash_attn (and its LSE side output) against the CPU oracle
(tests/reference.py:16-34 restated in oracle/gqa_oracle.py).

The reference's own tests fix one shape family (Llama-3.1-8B, G = 4,
test_correctness.py:48-77); this sweep draws group sizes 1-16, one to eight
kv heads, head_dim 64/128, fp16/bf16, causal and not, batches of 1-3,
single-token decode, multi-token verify, chunked prefill and prefill at
ragged lengths, contiguous and (batch, seq, head, d) strided layouts, and
causal calls with more queries than keys (their leading rows see no key:
NaN in both, as the reference's softmax over an all -inf row).  Every case
goes through choose_route, so the split-KV, single-pass, key-split and
key-chunk routes all meet odd shapes.  Shapes come from a fixed seed, so a
failure names a reproducible case; each is sized for the oracle to finish in
well under a second.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BASELINE_TOL, to_np
from oracle.gqa_oracle import gqa_lse, gqa_reference

pytestmark = pytest.mark.gpu

DEV = "cuda"
LSE_TOL = 2e-3
N_CASES = 64
MAX_FLOP = 6e8  # oracle work per case (4 * D FLOPs per (query, key) pair)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _cases():
    rng = np.random.RandomState(20261202)
    out = []
    while len(out) < N_CASES:
        G = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 16]))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        Hq = G * Hkv
        if Hq > 64:
            continue
        D = int(rng.choice([64, 128]))
        dtype = "bf16" if rng.rand() < 0.7 else "fp16"
        causal = bool(rng.rand() < 0.75)
        kind = str(rng.choice(["decode", "verify", "chunk", "prefill", "overhang"]))
        if kind == "decode":
            Sq, Skv = 1, int(rng.randint(1, 12000))
        elif kind == "verify":
            Sq = int(rng.randint(2, 33))
            Skv = int(rng.randint(Sq, 9000))
        elif kind == "chunk":
            Sq = int(rng.randint(33, 400))
            Skv = int(rng.randint(Sq, 6000))
        elif kind == "prefill":
            Sq = int(rng.randint(1, 1600))
            Skv = Sq if causal else int(rng.randint(1, 1600))
        else:  # more queries than keys
            Skv = int(rng.randint(1, 300))
            Sq = int(rng.randint(Skv + 1, Skv + 200))
        B = int(rng.randint(1, 4))
        if 4.0 * B * Hq * Sq * Skv * D > MAX_FLOP:
            continue
        layout = "bshd" if rng.rand() < 0.25 else "bhsd"
        lse = bool(rng.rand() < 0.3)
        out.append((B, Hq, Hkv, Sq, Skv, D, dtype, causal, kind, layout, lse))
    return out


CASES = _cases()


def _ids(c):
    B, Hq, Hkv, Sq, Skv, D, dtype, causal, kind, layout, lse = c
    return (f"{kind}-B{B}-Hq{Hq}-Hkv{Hkv}-Sq{Sq}-Skv{Skv}-D{D}-{dtype}-{'causal' if causal else 'full'}-{layout}"
            + ("-lse" if lse else ""))


def _draw(B, H, S, D, dtype, layout, g):
    """N(0,1) values rounded to dtype, as a (B, H, S, D) tensor: contiguous,
    or a view of (B, S, H, D) storage (the layout a fused QKV projection
    leaves)."""
    if layout == "bshd":
        return torch.randn(B, S, H, D, generator=g).to(dtype).to(DEV).transpose(1, 2)
    return torch.randn(B, H, S, D, generator=g).to(dtype).to(DEV)


def _compare(got, ref, tol, what):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert np.array_equal(nan_g, nan_r), f"{what}: NaN rows differ ({nan_g.sum()} vs {nan_r.sum()} values)"
    fin = ~nan_r
    if not fin.any():
        return
    d = np.abs(got[fin] - ref[fin])
    assert d.max() <= tol[0], f"{what}: max abs err {d.max():.3e} > {tol[0]:.1e}"
    assert d.mean() <= tol[1], f"{what}: mean abs err {d.mean():.3e} > {tol[1]:.1e}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_sweep(case):
    from gqa_kernels import gqa_flash_attn
    from gqa_kernels.dispatch import _cu_count, choose_route
    B, Hq, Hkv, Sq, Skv, D, dtype_s, causal, kind, layout, want_lse = case
    dtype = torch.bfloat16 if dtype_s == "bf16" else torch.float16
    route = choose_route(B, Hq, Hkv, Sq, Skv, _cu_count(0), causal, D)
    print(f"sweep {_ids(case)} route={route}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(Sq * 7919 + Skv)
    q = _draw(B, Hq, Sq, D, dtype, layout, g)
    k = _draw(B, Hkv, Skv, D, dtype, layout, g)
    v = _draw(B, Hkv, Skv, D, dtype, layout, g)
    if want_lse:
        o, lse = gqa_flash_attn(q, k, v, causal=causal, return_lse=True)
    else:
        o, lse = gqa_flash_attn(q, k, v, causal=causal), None
    torch.cuda.synchronize()
    assert o.shape == q.shape and o.dtype == dtype
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    _compare(to_np(o), gqa_reference(qn, kn, vn, causal), BASELINE_TOL[dtype], _ids(case))
    if lse is not None:
        ref_lse = gqa_lse(qn, kn, vn, causal)
        got_lse = to_np(lse)
        # a row with no visible key: -inf in both
        inf_g, inf_r = np.isneginf(got_lse), np.isneginf(ref_lse)
        assert np.array_equal(inf_g, inf_r), f"{_ids(case)}: rows without keys differ in the LSE"
        fin = ~inf_r
        if fin.any():
            err = np.abs(got_lse[fin].astype(np.float64) - ref_lse[fin])
            assert err.max() <= LSE_TOL, f"{_ids(case)}: LSE max abs err {err.max():.3e}"


# --------------------------------------------------------------------------
# Paged KV cache (gqa_kernels.paged.paged_attention) against the oracle's
# paged_reference: random page sizes 1-256, token-major (NHD) and head-major
# (HND) pages, ragged per-sequence lengths (a sequence may hold no key),
# decode to chunked query blocks; the split-KV route and, where the page size
# allows it, the single pass (plain and with every query block split), then
# the default route (key chunks or split blocks where the plan takes them).
# --------------------------------------------------------------------------
N_PAGED = 40


def _paged_cases():
    rng = np.random.RandomState(7)
    out = []
    while len(out) < N_PAGED:
        G = int(rng.choice([1, 2, 4, 5, 8]))
        Hkv = int(rng.choice([1, 2, 4, 8]))
        Hq = G * Hkv
        if Hq > 64:
            continue
        D = int(rng.choice([64, 128]))
        bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64, 128, 256]))
        B = int(rng.randint(1, 5))
        Sq = int(rng.choice([1, 1, 2, 4, 9, 16, 40, 130]))
        lens = [int(x) for x in rng.randint(0, 6000, size=B)]
        if rng.rand() < 0.3:
            lens[int(rng.randint(0, B))] = int(rng.randint(0, 3))  # (nearly) empty sequence
        dtype = "bf16" if rng.rand() < 0.7 else "fp16"
        causal = bool(rng.rand() < 0.8)
        hnd = bool(rng.rand() < 0.4)
        if 4.0 * Hq * Sq * sum(lens) * D > MAX_FLOP or max(lens) == 0:
            continue
        out.append((B, Hq, Hkv, Sq, lens, D, bs, dtype, causal, hnd))
    return out


PAGED_CASES = _paged_cases()


def _paged_id(c):
    B, Hq, Hkv, Sq, lens, D, bs, dtype, causal, hnd = c
    return (f"B{B}-Hq{Hq}-Hkv{Hkv}-Sq{Sq}-lens{'_'.join(map(str, lens))}-D{D}-bs{bs}-{dtype}-"
            f"{'causal' if causal else 'full'}-{'HND' if hnd else 'NHD'}")


@pytest.mark.parametrize("case", PAGED_CASES, ids=[_paged_id(c) for c in PAGED_CASES])
def test_paged_sweep(case):
    from test_gpu_paged import _check, _paged_inputs
    from gqa_kernels.paged import paged_attention, paged_route, single_pass_min_block
    B, Hq, Hkv, Sq, lens, D, bs, dtype_s, causal, hnd = case
    dtype = torch.bfloat16 if dtype_s == "bf16" else torch.float16
    q, kc, vc, table, seq_lens = _paged_inputs(B, Hq, Hkv, Sq, lens, D, bs, dtype, seed=sum(lens) + bs, hnd=hnd)
    kd, vd = kc.to(DEV), vc.to(DEV)
    if hnd:
        kd, vd = (t.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for t in (kc, vc))
    args = (q.to(DEV), kd, vd, table.to(DEV), seq_lens.to(DEV), causal)
    # Both kernel routes, the single pass with every query block split in
    # two key halves, and the default route (which may take key chunks or
    # split blocks by paged_single_plan).
    legs = [("split", None)]
    if bs >= single_pass_min_block(D):
        n_mblk = -(-Sq // max(1, 256 // (Hq // Hkv)))
        legs += [("single", None), ("single", n_mblk)]
    legs.append((None, None))
    default = paged_route(Hq, Hkv, Sq, bs, D)
    for route, splits in legs:
        print(f"paged sweep {_paged_id(case)} route={route} splits={splits} (default {default})", flush=True)
        o, lse = paged_attention(*args, max_seq_len=max(lens), return_lse=True, route=route, splits=splits)
        torch.cuda.synchronize()
        _check(o, lse, q, kc, vc, table, seq_lens, causal, dtype)
