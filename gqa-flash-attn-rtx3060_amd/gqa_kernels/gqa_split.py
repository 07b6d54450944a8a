"""Split-KV forward for short query blocks against a long KV cache.

Host side of the two-pass flash-decoding path (reference
gqa_kernels/gqa_split.py:153-194): the fp32 partials live in one workspace
allocated here with torch (caller-owned memory: the HIP library never
allocates), then two C-ABI launches run the first pass and the log-sum-exp
combine on torch's current stream.
"""
from __future__ import annotations

import math

import torch

from . import _lib

__all__ = ["split_kv_forward", "workspace_bytes"]

LOG2E = math.log2(math.e)

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}


def workspace_bytes(batch: int, num_heads: int, seq_q: int, head_dim: int, splits: int) -> int:
    """fp32 workspace size: acc (B,Hq,Sq,S,D) then m and l (B,Hq,Sq,S)."""
    return batch * num_heads * seq_q * splits * (head_dim + 2) * 4


def split_kv_forward(q, k, v, causal, splits, workspace=None):
    """Two-pass split-KV forward (first pass + LSE combine).

    ``workspace`` may be a caller-provided fp32 CUDA tensor with at least
    ``workspace_bytes(...) / 4`` elements; otherwise one is allocated.
    """
    lib = _lib.load()
    batch, num_heads, seq_q, head_dim = q.shape
    _, num_kv_heads, seq_kv, _ = k.shape
    scale_log2 = (head_dim ** -0.5) * LOG2E
    dtype = _DTYPES[q.dtype]

    need = workspace_bytes(batch, num_heads, seq_q, head_dim, splits)
    assert need == lib.gqa_split_workspace_bytes(batch, num_heads, seq_q, head_dim, splits)
    if workspace is None:
        workspace = torch.empty(need // 4, dtype=torch.float32, device=q.device)
    else:
        assert workspace.dtype == torch.float32 and workspace.device == q.device
        assert workspace.numel() * 4 >= need, "workspace too small"
    o = torch.empty_like(q)

    stream = torch.cuda.current_stream(q.device).cuda_stream
    _lib.check(
        lib.gqa_split_first_launch(
            q.data_ptr(), _lib.strides(q),
            k.data_ptr(), _lib.strides(k),
            v.data_ptr(), _lib.strides(v),
            workspace.data_ptr(), splits,
            batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim,
            scale_log2, int(bool(causal)), dtype, stream,
        )
    )
    _lib.check(
        lib.gqa_split_reduce_launch(
            workspace.data_ptr(), splits,
            o.data_ptr(), _lib.strides(o),
            batch, num_heads, seq_q, head_dim, dtype, stream,
        )
    )
    return o
