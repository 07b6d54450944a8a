"""Paged single pass with split query blocks (gqa_paged_fwd_split_launch).

The n_split heaviest query blocks of every (sequence, kv head) run as two
work items over the halves of their key range, merged by whichever
finishes last; the result is checked against the CPU oracle
(tests/reference.py:16-34 restated in oracle/gqa_oracle.py, per sequence
over its gathered pages), bit for bit against the contiguous split single
pass at the same count on the same keys, and across repeated calls (the
merge counters are left zero).
"""
from __future__ import annotations

import pytest
import torch

from helpers import make_inputs
from test_gpu_paged import _check, _check_varlen, _paged_inputs, _varlen_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


CASES = [
    # B, Hq, Hkv, Sq, lens, D, bs, n_split, dtype, causal, hnd
    (2, 32, 8, 256, [3000, 1200], 128, 16, 4, torch.bfloat16, True, False),
    (2, 32, 8, 256, [3000, 1200], 128, 64, 2, torch.bfloat16, True, True),
    (3, 32, 8, 130, [2500, 0, 900], 128, 128, 3, torch.float16, True, False),   # an empty sequence
    (1, 32, 8, 512, [4096], 64, 16, 8, torch.bfloat16, True, False),
    (1, 16, 2, 300, [1800], 64, 8, 5, torch.float16, True, True),
    (2, 32, 8, 200, [700, 2100], 128, 32, 4, torch.bfloat16, False, False),     # non-causal
    (1, 64, 8, 96, [5000], 128, 16, 3, torch.bfloat16, True, False),            # G = 8
]


def _ids(c):
    B, Hq, Hkv, Sq, lens, D, bs, ns, dt, causal, hnd = c
    return f"B{B}-G{Hq // Hkv}-Sq{Sq}-L{max(lens)}-D{D}-bs{bs}-ns{ns}-{str(dt)[6:]}-{'c' if causal else 'nc'}" + \
        ("-hnd" if hnd else "")


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_paged_split_matches_oracle(case):
    from gqa_kernels.paged import paged_attention
    B, Hq, Hkv, Sq, lens, D, bs, ns, dt, causal, hnd = case
    q, kc, vc, table, seq_lens = _paged_inputs(B, Hq, Hkv, Sq, lens, D, bs, dt, seed=sum(lens) + ns, hnd=hnd)
    print(f"paged split {_ids(case)}", flush=True)
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), causal)
    o, lse = paged_attention(*args, max_seq_len=max(lens), return_lse=True, route="single", splits=ns)
    o2, lse2 = paged_attention(*args, max_seq_len=max(lens), return_lse=True, route="single", splits=ns)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2), "repeated call differs (merge counters not left zero?)"
    _check(o, lse, q, kc, vc, table, seq_lens, causal, dt)


@pytest.mark.parametrize("bs", [16, 128])
def test_paged_split_variable_query_lengths(bs):
    from gqa_kernels.paged import paged_attention
    Hq, Hkv, D = 32, 8, 128
    lens, qlens = [2000, 900, 3000], [300, 0, 130]
    q, kc, vc, table, seq_lens, starts = _varlen_inputs(Hq, Hkv, D, lens, qlens, bs, torch.bfloat16, seed=7 + bs)
    print(f"paged split varlen bs={bs}", flush=True)
    o, lse = paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True,
                             max_seq_len=max(lens), return_lse=True, route="single", splits=4,
                             query_start=torch.tensor(starts, dtype=torch.int32, device=DEV),
                             query_lens=torch.tensor(qlens, dtype=torch.int32, device=DEV), max_query_len=max(qlens))
    torch.cuda.synchronize()
    _check_varlen(o.cpu(), lse.cpu(), q, kc, vc, table, seq_lens, starts, qlens, True, torch.bfloat16)


@pytest.mark.parametrize("D,bs,ns", [(128, 16, 8), (128, 64, 16), (64, 16, 8)])
def test_paged_split_equals_contiguous_split(D, bs, ns):
    # The same keys contiguous and in shuffled pages, the same split count:
    # the same work items and merges, so the same bits.
    from gqa_kernels.dispatch import single_pass_forward
    from gqa_kernels.paged import paged_attention
    B, Hq, Hkv, Sq, L = 1, 32, 8, 1024, 4096
    q, k, v = make_inputs(B, Hq, Hkv, Sq, L, D, seed=13, device=DEV)
    g = torch.Generator().manual_seed(3)
    nblk = L // bs
    perm = torch.randperm(nblk, generator=g)
    kc = torch.empty(nblk, bs, Hkv, D, dtype=k.dtype, device=DEV)
    vc = torch.empty_like(kc)
    kc[perm] = k[0].transpose(0, 1).reshape(nblk, bs, Hkv, D)
    vc[perm] = v[0].transpose(0, 1).reshape(nblk, bs, Hkv, D)
    table = perm.to(torch.int32).reshape(1, nblk).to(DEV)
    lens = torch.tensor([L], dtype=torch.int32, device=DEV)
    print(f"paged split == contiguous split D={D} bs={bs} n_split={ns}", flush=True)
    o_p = paged_attention(q, kc, vc, table, lens, True, max_seq_len=L, route="single", splits=ns)
    o_c = single_pass_forward(q, k, v, torch.empty_like(q), True, ns)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_c)


def test_paged_default_route_splits_blocks():
    # Two sequences of 512 new tokens over 16384 keys: the plan splits the 8
    # heaviest blocks (measured faster than key chunks), and the default
    # call computes exactly what that forced route computes.
    from gqa_kernels.dispatch import _cu_count
    from gqa_kernels.paged import paged_attention, paged_single_plan
    B, Hq, Hkv, Sq, D, bs = 2, 32, 8, 512, 128, 16
    lens = [16384, 16384]
    plan = paged_single_plan(B, Hq, Hkv, Sq, max(lens), _cu_count(0), True, D)
    assert plan[0] == 0 and plan[1] > 0, plan
    q, kc, vc, table, seq_lens = _paged_inputs(B, Hq, Hkv, Sq, lens, D, bs, torch.bfloat16, seed=19)
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True)
    print(f"paged default route plan {plan}", flush=True)
    o_default = paged_attention(*args, max_seq_len=max(lens))
    o_forced = paged_attention(*args, max_seq_len=max(lens), route="single", splits=plan[1])
    torch.cuda.synchronize()
    assert torch.equal(o_default, o_forced)


def test_paged_split_binding_matches_ctypes(monkeypatch):
    from gqa_kernels import paged
    assert paged._paged_host() is not None
    lens = [3000, 1200]
    q, kc, vc, table, seq_lens = _paged_inputs(2, 32, 8, 256, lens, 128, 16, torch.bfloat16, seed=23)
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), table.to(DEV), seq_lens.to(DEV), True)
    o1, l1 = paged.paged_attention(*args, max_seq_len=max(lens), return_lse=True, route="single", splits=4)
    monkeypatch.setattr(paged, "_paged_host", lambda: None)
    o2, l2 = paged.paged_attention(*args, max_seq_len=max(lens), return_lse=True, route="single", splits=4)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
