"""Write the golden fixtures tests/golden/gqa_golden.npz.

The reference ships no stored vectors (its tests draw random CUDA tensors,
reference tests/test_correctness.py:30-37), so these fixtures come from this
repo's CPU oracle in float64, which tests/test_oracle.py pins against brute
force, closed forms, invariants and torch's SDPA.  Inputs are N(0,1) (x0.1 for
the cases marked so) drawn from a CPU torch generator and rounded to bf16 or
fp16; they are stored as raw 16-bit patterns so the fixture is bit-exact.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
from oracle.gqa_oracle import gqa_reference  # noqa: E402

# name: (B, Hq, Hkv, Sq, Skv, D, dtype, causal, scale)
CASES = {
    "prefill_g4_d64": (1, 8, 2, 64, 64, 64, "bf16", True, 1.0),
    "prefill_ref_scale": (1, 4, 1, 80, 80, 128, "bf16", True, 0.1),
    "decode_g4": (1, 4, 1, 1, 1100, 64, "bf16", True, 1.0),
    "chunked_bottom_right": (1, 8, 2, 16, 200, 64, "bf16", True, 1.0),
    "group8_multitoken": (1, 8, 1, 4, 1040, 64, "bf16", True, 1.0),
    "noncausal_mha_fp16": (1, 4, 4, 33, 65, 64, "fp16", False, 1.0),
    "decode_fp16": (1, 8, 2, 1, 300, 64, "fp16", True, 1.0),
    "masked_rows": (1, 2, 1, 10, 6, 64, "bf16", True, 1.0),
}
TORCH_DT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def make_case(B, Hq, Hkv, Sq, Skv, D, dt, causal, scale, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = (torch.randn(B, Hq, Sq, D, generator=g) * scale).to(TORCH_DT[dt])
    k = (torch.randn(B, Hkv, Skv, D, generator=g) * scale).to(TORCH_DT[dt])
    v = (torch.randn(B, Hkv, Skv, D, generator=g) * scale).to(TORCH_DT[dt])
    o = gqa_reference(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal,
                      dtype=np.float64).astype(np.float32)
    bits = {n: t.view(torch.int16).numpy().view(np.uint16) for n, t in (("q", q), ("k", k), ("v", v))}
    return bits, o


def main():
    arrays = {}
    for i, (name, (B, Hq, Hkv, Sq, Skv, D, dt, causal, scale)) in enumerate(CASES.items()):
        bits, o = make_case(B, Hq, Hkv, Sq, Skv, D, dt, causal, scale, seed=100 + i)
        for n, a in bits.items():
            arrays[f"{name}/{n}"] = a
        arrays[f"{name}/o"] = o
        arrays[f"{name}/meta"] = np.array([B, Hq, Hkv, Sq, Skv, D, int(causal), 0 if dt == "bf16" else 1],
                                          dtype=np.int64)
    out = HERE / "gqa_golden.npz"
    np.savez_compressed(out, **arrays)
    print(f"wrote {out} ({out.stat().st_size} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
