"""gqa_split_noalloc_launch: the split-KV forward with its partials in the
library's fixed per-device buffer (no counterpart in the reference; for
callers that cannot allocate).  It runs the kernels of the workspace entry
points it varies (gqa_split_first_launch, then gqa_split_reduce_lse_launch),
so on the same inputs its output and LSE must equal theirs bit for bit; two
calls in a row, the second smaller, show that nothing left in the shared
buffer by one call leaks into the next.  Sizes above the buffer are refused
before any HIP call (CPU test).  The file name sorts last on purpose, so
that under `pytest -x` a failure here cannot hide the other GPU tests."""
from __future__ import annotations

import pytest
import torch

from helpers import BASELINE_TOL, assert_close, make_inputs, oracle

DEV = "cuda"


def _lib():
    from gqa_kernels import _lib
    return _lib


def _args(q, k, v):
    lib = _lib()
    return (q.data_ptr(), lib.strides(q), k.data_ptr(), lib.strides(k), v.data_ptr(), lib.strides(v))


def _dims(q, k, causal):
    from gqa_kernels.gqa_split import LOG2E
    B, Hq, Sq, D = q.shape
    return (B, Hq, k.shape[1], Sq, k.shape[2], D, D ** -0.5 * LOG2E, int(causal), _lib().DTYPE_BF16)


def _with_workspace(q, k, v, splits, causal):
    """gqa_split_first_launch + gqa_split_reduce_lse_launch, caller workspace."""
    from gqa_kernels.gqa_split import workspace_bytes
    m = _lib()
    lib = m.load()
    B, Hq, Sq, D = q.shape
    stream = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(workspace_bytes(B, Hq, Sq, D, splits) // 4, dtype=torch.float32, device=DEV)
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, Sq, dtype=torch.float32, device=DEV)
    m.check(lib.gqa_split_first_launch(*_args(q, k, v), ws.data_ptr(), splits, *_dims(q, k, causal), stream))
    m.check(lib.gqa_split_reduce_lse_launch(ws.data_ptr(), splits, o.data_ptr(), m.strides(o), lse.data_ptr(),
                                            B, Hq, Sq, D, m.DTYPE_BF16, stream))
    return o, lse


def _noalloc(q, k, v, splits, causal):
    m = _lib()
    lib = m.load()
    B, Hq, Sq, _ = q.shape
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, Sq, dtype=torch.float32, device=DEV)
    m.check(lib.gqa_split_noalloc_launch(*_args(q, k, v), o.data_ptr(), m.strides(o), lse.data_ptr(), splits,
                                         *_dims(q, k, causal), torch.cuda.current_stream().cuda_stream))
    return o, lse


@pytest.mark.gpu
def test_noalloc_equals_workspace_entry_points():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    # Partials shrink from call to call: a 70B-shaped batch (G = 8, 4 query
    # rows, 32 splits: 8.5 MB), the headline decode (131072 keys, 64 splits:
    # 1.06 MB), a short two-row decode (8 splits: 0.27 MB).
    for (B, Hq, Hkv, Sq, Skv, S, causal) in ((2, 64, 8, 4, 8192, 32, True), (1, 32, 8, 1, 131072, 64, True),
                                             (1, 32, 8, 2, 3000, 8, True)):
        print(f"noalloc B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Skv={Skv} splits={S}", flush=True)
        q, k, v = make_inputs(B, Hq, Hkv, Sq, Skv, 128, seed=Skv, device=DEV)
        o_na, lse_na = _noalloc(q, k, v, S, causal)
        o_ws, lse_ws = _with_workspace(q, k, v, S, causal)
        torch.cuda.synchronize()
        assert torch.equal(o_na, o_ws), "output differs from the workspace entry points"
        assert torch.equal(lse_na, lse_ws), "LSE differs from the workspace entry points"
        if Skv <= 4096:
            assert_close(o_na, oracle(q, k, v, causal), BASELINE_TOL[torch.bfloat16], "noalloc vs oracle")


def test_noalloc_rejects_oversized_partials():
    """32 heads x 16 rows x 1024 splits x 130 floats = 272 MB > 16 MiB: the
    call is refused before any HIP call (fake, aligned pointers)."""
    m = _lib()
    lib = m.load()
    st = m.strides(torch.empty(1, 32, 16, 128))
    p = 1 << 20
    from gqa_kernels.gqa_split import LOG2E, workspace_bytes
    assert workspace_bytes(1, 32, 16, 128, 1024) > m.GQA_NOALLOC_SCRATCH_BYTES
    rc = lib.gqa_split_noalloc_launch(p, st, p, st, p, st, p, st, None, 1024, 1, 32, 8, 16, 100000, 128,
                                      128 ** -0.5 * LOG2E, 1, m.DTYPE_BF16, None)
    assert rc == m.GQA_E_SCRATCH
    assert b"GQA_NOALLOC_SCRATCH_BYTES" in lib.gqa_strerror(rc)
    # the largest call that fits is accepted by the size check (rejected
    # later only for its fake stride-0 layout, still before any HIP call)
    assert workspace_bytes(1, 32, 1, 128, 1008) <= m.GQA_NOALLOC_SCRATCH_BYTES
    bad = m._i64x4(0, 0, 0, 0)
    rc = lib.gqa_split_noalloc_launch(p, bad, p, bad, p, bad, p, bad, None, 1008, 1, 32, 8, 1, 100000, 128,
                                      128 ** -0.5 * LOG2E, 1, m.DTYPE_BF16, None)
    assert rc == -4  # GQA_E_STRIDE
