"""Golden fixtures (tests/golden/gqa_golden.npz, written by make_golden.py).

CPU: the oracle reproduces every stored output (regression of the oracle
itself).  GPU: the HIP path, fed the stored input bits, matches the stored
outputs at the bf16/fp16 gates; fully masked rows must be NaN in both.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.gqa_oracle import gqa_reference

GOLDEN = Path(__file__).resolve().parent / "golden" / "gqa_golden.npz"
TOL = {0: (2e-2, 2e-3), 1: (4e-3, 4e-4)}


def _cases():
    z = np.load(GOLDEN)  # plain arrays only (allow_pickle=False by default)
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


def _decode(z, name):
    meta = z[f"{name}/meta"]
    dt = torch.bfloat16 if meta[7] == 0 else torch.float16
    t = {n: torch.from_numpy(z[f"{name}/{n}"].view(np.int16).copy()).view(dt) for n in "qkv"}
    return meta, t["q"], t["k"], t["v"], z[f"{name}/o"]


def test_golden_file_present():
    z, names = _cases()
    assert len(names) >= 8


@pytest.mark.parametrize("name", _cases()[1])
def test_oracle_reproduces_golden(name):
    z, _ = _cases()
    meta, q, k, v, o = _decode(z, name)
    causal = bool(meta[6])
    got = gqa_reference(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal,
                        dtype=np.float64).astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(o))
    fin = ~np.isnan(o)
    assert np.abs(got[fin] - o[fin]).max() < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("name", _cases()[1])
def test_gpu_matches_golden(name):
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from gqa_kernels import gqa_flash_attn
    z, _ = _cases()
    meta, q, k, v, o = _decode(z, name)
    out = gqa_flash_attn(q.cuda(), k.cuda(), v.cuda(), causal=bool(meta[6]))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    nan = np.isnan(o)
    assert np.array_equal(np.isnan(got), nan)
    d = np.abs(got[~nan].astype(np.float64) - o[~nan])
    mx, mn = TOL[int(meta[7])]
    assert d.max() <= mx and d.mean() <= mn, (d.max(), d.mean())
