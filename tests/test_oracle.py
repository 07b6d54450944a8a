"""Pinning the CPU oracle (CPU only).

The reference ships no golden vectors (its tests draw random CUDA tensors and
compare at tolerance, reference tests/test_correctness.py:30-45), so the
oracle — a restatement of reference tests/reference.py:6-34 — is pinned by
checks that do not retype its formula:

* brute force: scalar fp64 loops over (b, h, i, j) with math.exp;
* closed forms: one visible key, constant V, per-kv-head constant V (head
  map), all-equal keys (prefix mean of V), one dominant logit;
* invariants: chunked rows = last rows of full prefill (bottom-right
  alignment), decode causal = non-causal, key-shift and joint key/value
  permutation invariance, MHA reduction, split-KV = single pass for every
  split count (the log-sum-exp combine of reference gqa_split.py:134-147);
* an independent library: torch.nn.functional.scaled_dot_product_attention in
  fp32 with expanded K/V and an explicit bottom-right mask;
* planted mistakes: mutants of the oracle (upper-left causal alignment, a
  q-head -> kv-head map of h % Hkv, a missing scale, an off-by-one mask, a
  wrong split chunking) must each fail at least one of the pins above.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import gqa_oracle as O


def _rand(B, Hq, Hkv, Sq, Skv, D, seed=0, scale=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, Sq, D)) * scale
    k = rng.standard_normal((B, Hkv, Skv, D)) * scale
    v = rng.standard_normal((B, Hkv, Skv, D))
    return q, k, v


def brute_force(q, k, v, causal):
    """Scalar loops with math.exp, float64, textbook softmax."""
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, Sq, D))
    for b in range(B):
        for h in range(Hq):
            kvh = h // G
            for i in range(Sq):
                qpos = i + Skv - Sq
                logits = []
                for j in range(Skv):
                    if causal and j > qpos:
                        continue
                    dot = 0.0
                    for d in range(D):
                        dot += q[b, h, i, d] * k[b, kvh, j, d]
                    logits.append((j, dot / math.sqrt(D)))
                if not logits:
                    out[b, h, i] = np.nan
                    continue
                mx = max(s for _, s in logits)
                w = [(j, math.exp(s - mx)) for j, s in logits]
                tot = sum(x for _, x in w)
                for j, x in w:
                    out[b, h, i] += (x / tot) * v[b, kvh, j]
    return out


# ---------------------------------------------------------------------------
# Pins, written against an `attn(q, k, v, causal)` callable so that the same
# checks can be run on planted mutants.
# ---------------------------------------------------------------------------
BF_SHAPES = [(2, 4, 2, 1, 5, 8), (1, 4, 2, 3, 5, 8), (1, 4, 1, 17, 17, 4), (2, 2, 2, 3, 70, 4),
             (1, 6, 3, 5, 64, 4), (1, 4, 2, 1, 1, 8)]


def pin_brute_force(attn):
    for i, shp in enumerate(BF_SHAPES):
        q, k, v = _rand(*shp, seed=i)
        for causal in (True, False):
            a = attn(q, k, v, causal)
            b = brute_force(q, k, v, causal)
            if not np.allclose(a, b, atol=1e-10, rtol=1e-9, equal_nan=True):
                return False
    return True


def pin_row0(attn):
    q, k, v = _rand(1, 8, 2, 40, 40, 16, seed=11)
    o = attn(q, k, v, True)
    return np.allclose(o[:, :, 0], v[:, np.arange(8) // 4, 0], atol=1e-12)


def pin_constant_v(attn):
    q, k, v = _rand(2, 6, 3, 9, 30, 16, seed=12)
    v = np.full_like(v, 0.75)
    return all(np.allclose(attn(q, k, v, c), 0.75, atol=1e-12) for c in (True, False))


def pin_head_map(attn):
    q, k, v = _rand(1, 12, 3, 5, 20, 8, seed=13)
    v = np.broadcast_to(np.arange(3.0).reshape(1, 3, 1, 1), v.shape).copy()
    exp = np.broadcast_to((np.arange(12) // 4).reshape(1, 12, 1, 1).astype(float), (1, 12, 5, 8))
    return all(np.allclose(attn(q, k, v, c), exp, atol=1e-12) for c in (True, False))


def pin_uniform_keys(attn):
    # All keys equal -> uniform weights -> prefix mean of V (causal, bottom-right)
    q, k, v = _rand(1, 4, 2, 6, 11, 8, seed=14)
    k = np.broadcast_to(k[:, :, :1], k.shape).copy()
    o = attn(q, k, v, True)
    G = 2
    for h in range(4):
        for i in range(6):
            n = i + 11 - 6 + 1
            if not np.allclose(o[0, h, i], v[0, h // G, :n].mean(axis=0), atol=1e-12):
                return False
    on = attn(q, k, v, False)
    return np.allclose(on, np.broadcast_to(v.mean(axis=2)[:, np.arange(4) // G, None], on.shape), atol=1e-12)


def pin_dominant_logit(attn):
    # One key aligned with the query at large norm dominates: output ~ its V row.
    D = 16
    q, k, v = _rand(1, 2, 1, 1, 9, D, seed=15)
    k[0, 0, 4] = q[0, 0, 0] * 40.0
    o = attn(q, k, v, True)
    return np.allclose(o[0, 0, 0], v[0, 0, 4], atol=1e-6)


def pin_chunked_tail(attn):
    q, k, v = _rand(2, 4, 2, 24, 24, 8, seed=16)
    full = attn(q, k, v, True)
    return all(np.allclose(attn(q[:, :, -sq:], k, v, True), full[:, :, -sq:], atol=1e-12)
               for sq in (1, 5, 23))


def pin_decode_causal(attn):
    q, k, v = _rand(2, 4, 2, 1, 33, 8, seed=17)
    return np.allclose(attn(q, k, v, True), attn(q, k, v, False), atol=1e-12)


def pin_key_shift(attn):
    q, k, v = _rand(1, 4, 2, 7, 19, 8, seed=18)
    u = np.random.default_rng(5).standard_normal(8)
    ok = True
    for c in (True, False):
        ok &= np.allclose(attn(q, k, v, c), attn(q, k + u, v, c), atol=1e-9)
    return ok


def pin_permutation(attn):
    q, k, v = _rand(1, 4, 2, 7, 19, 8, seed=19)
    p = np.random.default_rng(6).permutation(19)
    return np.allclose(attn(q, k, v, False), attn(q, k[:, :, p], v[:, :, p], False), atol=1e-12)


def pin_sdpa(attn):
    for i, (B, Hq, Hkv, Sq, Skv, D) in enumerate([(2, 8, 2, 13, 13, 16), (1, 8, 4, 5, 40, 32),
                                                  (1, 4, 4, 1, 50, 8)]):
        q, k, v = _rand(B, Hq, Hkv, Sq, Skv, D, seed=30 + i)
        G = Hq // Hkv
        tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
        tk = tk.repeat_interleave(G, dim=1)
        tv = tv.repeat_interleave(G, dim=1)
        for causal in (True, False):
            mask = None
            if causal:
                qpos = torch.arange(Sq) + (Skv - Sq)
                mask = qpos[:, None] >= torch.arange(Skv)[None, :]
            ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask).numpy()
            if not np.allclose(attn(q, k, v, causal), ref, atol=1e-10):
                return False
    return True


def pin_split(attn, split=O.split_kv_reference):
    q, k, v = _rand(1, 8, 2, 6, 61, 8, seed=20)
    ok = True
    for causal in (True, False):
        ref = attn(q, k, v, causal)
        for s in (1, 2, 3, 7, 16, 61, 80):
            ok &= np.allclose(split(q, k, v, causal, s), ref, atol=1e-12)
    return ok


PINS = [pin_brute_force, pin_row0, pin_constant_v, pin_head_map, pin_uniform_keys,
        pin_dominant_logit, pin_chunked_tail, pin_decode_causal, pin_key_shift, pin_permutation,
        pin_sdpa, pin_split]


def oracle64(q, k, v, causal):
    return O.gqa_reference(q, k, v, causal, dtype=np.float64)


@pytest.mark.parametrize("pin", PINS, ids=lambda f: f.__name__)
def test_oracle_pinned(pin):
    assert pin(oracle64)


def test_oracle_float32_close_to_float64():
    q, k, v = _rand(1, 8, 2, 50, 300, 64, seed=3)
    a = O.gqa_reference(q, k, v, True, dtype=np.float32)
    b = O.gqa_reference(q, k, v, True, dtype=np.float64)
    assert np.abs(a - b).max() < 1e-5


def test_oracle_rows_subset_and_chunking():
    q, k, v = _rand(2, 4, 2, 37, 50, 8, seed=4)
    full = oracle64(q, k, v, True)
    rows = [0, 5, 36, 17]
    sub = O.gqa_reference(q, k, v, True, rows=rows, dtype=np.float64)
    assert np.array_equal(sub, full[:, :, rows])
    small = O.gqa_reference(q, k, v, True, dtype=np.float64, row_chunk=3)
    assert np.allclose(small, full, atol=1e-14)


def test_fully_masked_rows_nan():
    # seq_q > seq_kv under causal: rows with q_pos < 0 see nothing -> NaN,
    # as torch's softmax over an all -inf row gives (reference.py:33).
    q, k, v = _rand(1, 2, 1, 8, 5, 4, seed=5)
    o = oracle64(q, k, v, True)
    assert np.isnan(o[:, :, :3]).all() and not np.isnan(o[:, :, 3:]).any()
    t = torch.from_numpy
    ref = torch.softmax(torch.full((3, 5), float("-inf")), -1)
    assert torch.isnan(ref).all()
    assert np.allclose(o[:, :, 3:], brute_force(q, k, v, True)[:, :, 3:], atol=1e-12)
    del t


@pytest.mark.parametrize("causal", [True, False])
def test_empty_cache_is_zero(causal):
    # seq_kv = 0: reference.py:25-34 multiplies the softmax over an empty key
    # axis (an empty (Sq, 0) matrix; the mask changes nothing) by an empty V,
    # which torch evaluates to zeros, and so does the oracle; the LSE over no
    # keys is -inf.
    q, k, v = _rand(2, 4, 2, 3, 0, 8, seed=8)
    w = torch.softmax(torch.empty(3, 0, dtype=torch.float64), dim=-1)
    assert torch.equal(w @ torch.empty(0, 8, dtype=torch.float64), torch.zeros(3, 8, dtype=torch.float64))
    o = O.gqa_reference(q, k, v, causal, dtype=np.float64)
    assert o.shape == (2, 4, 3, 8) and np.all(o == 0)
    assert np.isneginf(O.gqa_lse(q, k, v, causal)).all()


def test_split_partials_empty_chunks():
    # Chunks with no visible key: m = -inf, l = 0, acc = 0 (gqa_split.py:79-81).
    q, k, v = _rand(1, 2, 1, 10, 12, 4, seed=6)
    m, l, acc = O.split_partials(q, k, v, True, 6)
    qpos = np.arange(10) + 2
    for s in range(6):
        c0 = s * 2
        empty = qpos < c0
        assert np.isneginf(m[0, :, empty, s]).all()
        assert (l[0, :, empty, s] == 0).all() and (acc[0, :, empty, s] == 0).all()
        assert np.isfinite(m[0, :, ~empty, s]).all()


def test_work_counts():
    assert O.visible_pairs(16384, 16384, True) == 16384 * 16385 // 2
    assert O.visible_pairs(512, 8192, True) == 512 * (8192 - 512) + 512 * 513 // 2
    assert O.visible_pairs(4, 32768, True) == 4 * 32764 + 10
    assert O.visible_pairs(10, 6, True) == sum(max(0, min(6, i - 4 + 1)) for i in range(10))
    assert O.attention_flops(1, 32, 16384, 16384, 128) == 2199157473280
    assert O.attention_bytes(1, 32, 8, 1, 131072, 128) == 536887296


# ---------------------------------------------------------------------------
# Planted mistakes (in the oracle, on the CPU): every mutant must fail a pin.
# ---------------------------------------------------------------------------
def _mut_upper_left(q, k, v, causal):
    # causal aligned top-left (the SDPA convention), not bottom-right
    B, Hq, Sq, D = q.shape
    Skv = k.shape[2]
    if not causal or Sq == Skv:
        return oracle64(q, k, v, causal)
    out = np.empty((B, Hq, Sq, D))
    for i in range(Sq):
        n = min(i + 1, Skv)
        out[:, :, i:i + 1] = O.gqa_reference(q[:, :, i:i + 1], k[:, :, :n], v[:, :, :n], False,
                                             dtype=np.float64)
    return out


def _mut_head_mod(q, k, v, causal):
    Hq, Hkv = q.shape[1], k.shape[1]
    G = Hq // Hkv
    idx = np.arange(Hq) % Hkv  # wrong: should be h // G
    kk = k[:, idx]
    vv = v[:, idx]
    del G
    return O.gqa_reference(q, kk, vv, causal, dtype=np.float64)


def _mut_no_scale(q, k, v, causal):
    return O.gqa_reference(q * math.sqrt(q.shape[-1]), k, v, causal, dtype=np.float64)


def _mut_off_by_one(q, k, v, causal):
    # mask keys >= q_pos instead of > q_pos (a row cannot see itself)
    if not causal:
        return oracle64(q, k, v, causal)
    Sq, Skv = q.shape[2], k.shape[2]
    out = np.empty(q.shape)
    for i in range(Sq):
        n = i + Skv - Sq  # should be + 1
        if n <= 0:
            out[:, :, i] = np.nan
            continue
        out[:, :, i:i + 1] = O.gqa_reference(q[:, :, i:i + 1], k[:, :, :n], v[:, :, :n], False,
                                             dtype=np.float64)
    return out


def _mut_split_chunking(q, k, v, causal, splits):
    # drops the ragged tail: chunk = floor(Skv / S) instead of ceil
    B, Hq, Sq, D = q.shape
    Skv = k.shape[2]
    n = (Skv // splits) * splits
    if n == Skv:
        return O.split_kv_reference(q, k, v, causal, splits)
    return O.split_kv_reference(q[..., :, :], k[:, :, :n], v[:, :, :n], causal and Sq <= n, splits)


@pytest.mark.parametrize("mutant", [_mut_upper_left, _mut_head_mod, _mut_no_scale, _mut_off_by_one],
                         ids=lambda f: f.__name__)
def test_planted_mistake_is_caught(mutant):
    failed = [p.__name__ for p in PINS[:-1] if not p(mutant)]
    assert failed, f"{mutant.__name__} passed every pin"


def test_planted_split_mistake_is_caught():
    assert not pin_split(oracle64, split=_mut_split_chunking)


# ---------------------------------------------------------------------------
# LSE side output: gqa_lse / split_lse pinned by brute force, closed forms,
# the split decomposition, torch.logsumexp, the normalisation identity, and
# planted mistakes.
# ---------------------------------------------------------------------------
def _lse_inputs(seed=7, B=2, Hq=6, Hkv=2, Sq=5, Skv=9, D=16):
    g = np.random.default_rng(seed)
    return (g.standard_normal((B, Hq, Sq, D)), g.standard_normal((B, Hkv, Skv, D)),
            g.standard_normal((B, Hkv, Skv, D)))


def _lse_brute(q, k, v, causal):
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    out = np.empty((B, Hq, Sq))
    for b in range(B):
        for h in range(Hq):
            for i in range(Sq):
                terms = [math.exp(sum(q[b, h, i, d] * k[b, h // (Hq // Hkv), j, d] for d in range(D)) / math.sqrt(D))
                         for j in range(Skv) if not causal or j <= i + Skv - Sq]
                out[b, h, i] = math.log(sum(terms)) if terms else -math.inf
    return out


def test_lse_brute_force():
    q, k, v = _lse_inputs()
    for causal in (True, False):
        assert np.abs(O.gqa_lse(q, k, v, causal) - _lse_brute(q, k, v, causal)).max() < 1e-12


def test_lse_closed_forms():
    q, k, v = _lse_inputs()
    # q = 0: every visible score is 0, lse = ln(number of visible keys)
    z = O.gqa_lse(np.zeros_like(q), k, v, True)
    n_vis = np.arange(q.shape[2]) + (k.shape[2] - q.shape[2]) + 1
    assert np.allclose(z, np.log(n_vis)[None, None, :], atol=1e-13)
    # causal prefill row 0 sees one key: lse = q0.k0 / sqrt(D)
    qs = q[:, :, :4]
    ks, vs = k[:, :, :4], v[:, :, :4]
    one = O.gqa_lse(qs, ks, vs, True)[:, :, 0]
    want = np.einsum("bhd,bhd->bh", qs[:, :, 0], np.repeat(ks[:, :, 0], 3, axis=1)) / 4.0
    assert np.allclose(one, want, atol=1e-13)
    # all keys equal: lse = ln(n) + q.k / sqrt(D)
    keq = np.repeat(k[:, :, :1], k.shape[2], axis=2)
    e = O.gqa_lse(q, keq, v, False)
    dot = np.einsum("bhsd,bhd->bhs", q, np.repeat(k[:, :, 0], 3, axis=1)) / 4.0
    assert np.allclose(e, np.log(k.shape[2]) + dot, atol=1e-12)
    # no visible key (causal, Sq > Skv): -inf
    assert np.all(np.isneginf(O.gqa_lse(q[:, :, :5], k[:, :, :2], v[:, :, :2], True)[:, :, :3]))


def test_lse_split_decomposition_and_torch():
    q, k, v = _lse_inputs(seed=11, Skv=13)
    ref = O.gqa_lse(q, k, v, True)
    for splits in (1, 2, 3, 5, 13, 20):
        m, l, _ = O.split_partials(q, k, v, True, splits)
        assert np.abs(O.split_lse(m, l) - ref).max() < 1e-12
    # torch.logsumexp over the masked, scaled scores (independent library)
    tq, tk = torch.from_numpy(q), torch.from_numpy(k).repeat_interleave(3, dim=1)
    s = tq @ tk.transpose(-1, -2) / 4.0
    mask = torch.arange(13)[None, :] > (torch.arange(5)[:, None] + 8)
    s = s.masked_fill(mask, float("-inf"))
    assert np.abs(torch.logsumexp(s, dim=-1).numpy() - ref).max() < 1e-12


def test_lse_normalises_the_softmax():
    q, k, v = _lse_inputs(seed=3)
    lse = O.gqa_lse(q, k, v, True)
    s = np.einsum("bhsd,bhtd->bhst", q, np.repeat(k, 3, axis=1)) / 4.0
    vis = np.arange(9)[None, :] <= (np.arange(5)[:, None] + 4)
    tot = np.where(vis, np.exp(s - lse[..., None]), 0.0).sum(-1)
    assert np.allclose(tot, 1.0, atol=1e-13)


@pytest.mark.parametrize("mutant", ["log2", "noscale", "upper_left"])
def test_planted_lse_mistake_is_caught(mutant):
    q, k, v = _lse_inputs()
    if mutant == "log2":
        bad = O.gqa_lse(q, k, v, True) / math.log(2.0)
    elif mutant == "noscale":
        bad = O.gqa_lse(q * 4.0, k, v, True)
    else:  # upper-left causal alignment: row i sees keys 0..i
        bad = O.gqa_lse(q, k[:, :, :5], v[:, :, :5], True)
    assert np.abs(bad - _lse_brute(q, k, v, True)).max() > 1e-3
