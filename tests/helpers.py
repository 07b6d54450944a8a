"""Shared test helpers: seeded inputs, oracle calls and tolerance checks."""
from __future__ import annotations

import numpy as np
import torch

from oracle.gqa_oracle import gqa_reference

# Reference tolerances (reference tests/test_correctness.py:24-27) for its
# x0.1-scaled inputs, and the N(0,1) gate of the BASELINE configs.
REF_TOL = {torch.bfloat16: (1e-2, 1e-3), torch.float16: (1e-3, 1e-4)}
BASELINE_TOL = {torch.bfloat16: (2e-2, 2e-3), torch.float16: (4e-3, 4e-4)}


def make_inputs(B, Hq, Hkv, Sq, Skv, D, dtype=torch.bfloat16, scale=1.0, seed=0, device="cpu"):
    """q, k, v drawn in that order from a CPU generator in fp32, scaled, then
    rounded to `dtype` (identical bits for the CPU oracle and the GPU kernel)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, Hq, Sq, D, generator=g) * scale
    k = torch.randn(B, Hkv, Skv, D, generator=g) * scale
    v = torch.randn(B, Hkv, Skv, D, generator=g) * scale
    return tuple(t.to(dtype).to(device) for t in (q, k, v))


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def oracle(q, k, v, causal=True, rows=None, dtype=np.float32):
    """Run the CPU oracle on torch tensors (any device); returns numpy."""
    return gqa_reference(to_np(q), to_np(k), to_np(v), causal, rows=rows, dtype=dtype)


def errors(out, ref):
    out = to_np(out) if isinstance(out, torch.Tensor) else np.asarray(out)
    ref = to_np(ref) if isinstance(ref, torch.Tensor) else np.asarray(ref)
    d = np.abs(out.astype(np.float64) - ref.astype(np.float64))
    return float(d.max()), float(d.mean())


def assert_close(out, ref, tol, what=""):
    mx, mn = errors(out, ref)
    max_tol, mean_tol = tol
    assert mx <= max_tol, f"{what} max abs err {mx:.3e} > {max_tol:.1e}"
    assert mn <= mean_tol, f"{what} mean abs err {mn:.3e} > {mean_tol:.1e}"
    return mx, mn


def torch_reference_gpu(q, k, v, causal=True, row_chunk=2048):
    """Plain PyTorch fp32 attention on the GPU (chunked over heads and rows).

    Used for full-size comparisons that the CPU oracle cannot finish in seconds.
    All products are fp32 on contiguous operands.
    """
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = torch.empty(B, Hq, Sq, D, dtype=torch.float32, device=q.device)
    kpos = torch.arange(Skv, device=q.device)
    for b in range(B):
        for kvh in range(Hkv):
            kt = k[b, kvh].float().t().contiguous()
            vv = v[b, kvh].float().contiguous()
            for g in range(G):
                h = kvh * G + g
                for r0 in range(0, Sq, row_chunk):
                    r1 = min(Sq, r0 + row_chunk)
                    s = torch.matmul(q[b, h, r0:r1].float().contiguous(), kt) * (D ** -0.5)
                    if causal:
                        qpos = torch.arange(r0, r1, device=q.device) + (Skv - Sq)
                        s.masked_fill_(qpos[:, None] < kpos[None, :], float("-inf"))
                    out[b, h, r0:r1] = torch.matmul(torch.softmax(s, dim=-1), vv)
    return out
