"""CPU oracle for the GQA flash-attention forward — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or, for cpu_baseline, as the timed CPU
path).  The product path (gqa_kernels) never calls it and has no CPU fallback.

What it restates (numpy, float32 or float64 arithmetic on the exact input
values, which for bf16/fp16 inputs are the bf16/fp16-rounded numbers):

* ``gqa_reference`` — reference tests/reference.py:6-34: each query head h
  reads kv head h // G (reference.py:22-23 repeat_interleave), scores
  q k^T * head_dim^-0.5 (reference.py:25), bottom-right causal mask
  q_pos = i + (seq_kv - seq_q) < k_pos -> -inf (reference.py:27-31), softmax
  over keys (reference.py:33; max-subtracted exp, so a fully masked row is
  NaN exactly as torch's softmax makes it), times V (reference.py:34).
  Unlike the reference it never materialises the expanded K/V and it works
  through the query rows in chunks, so 16K-token prefill fits in memory; the
  arithmetic is the same.  ``rows`` evaluates a subset of query rows.

* ``split_partials`` / ``split_combine`` — the split-KV decomposition of
  reference gqa_kernels/gqa_split.py: chunk s covers keys
  [s*ceil(Skv/S), min((s+1)*ceil(Skv/S), Skv)) (gqa_split.py:55-57); per chunk
  the partial m (max logit in log2 units), l = sum exp2(logit - m) and the
  unnormalised acc = sum exp2(logit - m) v (gqa_split.py:83-112), with
  m = -inf, l = 0, acc = 0 for a chunk with no visible key (gqa_split.py:79-81);
  combine m* = max m, a = exp2(m - m*), o = sum a acc / sum a l
  (gqa_split.py:134-147).

* ``gqa_lse`` — the log-sum-exp of each query row's scaled scores over its
  visible keys, ln sum_k exp(q.k * head_dim^-0.5), natural log (the quantity
  the reference's split combine forms in log2 units as m* + log2 l*,
  gqa_split.py:134-139, without returning it); -inf for a row with no visible
  key.  ``split_lse`` forms it from split partials the way that combine does.

* ``paged_gather`` / ``paged_reference`` — a paged K/V cache (the
  reference's roadmap item, README.md:140-146; not in the reference) read
  back into contiguous per-sequence K/V, and ``gqa_reference`` / ``gqa_lse``
  per sequence over it.

Parity pinning (tests/test_oracle.py): brute-force scalar loops at tiny
shapes, closed forms (one-key row, constant V, constant-per-head V, uniform
keys), invariants (chunked = last rows of prefill, decode causal = non-causal,
key-shift and key-permutation invariance, split == single for every split
count), torch's scaled_dot_product_attention as an independent library, and
planted mistakes that each pin must catch.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = ["gqa_reference", "gqa_lse", "split_partials", "split_combine", "split_kv_reference",
           "split_lse", "paged_gather", "paged_reference", "attention_flops", "attention_bytes",
           "visible_pairs"]

LOG2E = math.log2(math.e)


def _shapes(q, k, v):
    B, Hq, Sq, D = q.shape
    Bk, Hkv, Skv, Dk = k.shape
    if v.shape != k.shape or Bk != B or Dk != D:
        raise ValueError(f"inconsistent shapes q{q.shape} k{k.shape} v{v.shape}")
    if Hq % Hkv:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    return B, Hq, Hkv, Sq, Skv, D


def gqa_reference(q, k, v, causal=True, *, rows=None, dtype=np.float32, row_chunk=1024):
    """Attention output (B, Hq, len(rows) or Sq, D) in ``dtype``.

    q: (B, Hq, Sq, D); k, v: (B, Hkv, Skv, D) — any real array type.
    rows: optional 1-D sequence of query row indices (into seq_q) to evaluate;
    the causal position of row i is still i + Skv - Sq.
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    B, Hq, Hkv, Sq, Skv, D = _shapes(q, k, v)
    G = Hq // Hkv
    scale = D ** -0.5
    sel = np.arange(Sq) if rows is None else np.asarray(rows, dtype=np.int64)
    out = np.empty((B, Hq, len(sel), D), dtype=dtype)
    k_pos = np.arange(Skv)
    for b in range(B):
        for kvh in range(Hkv):
            kk = k[b, kvh].astype(dtype)
            vv = v[b, kvh].astype(dtype)
            for g in range(G):
                h = kvh * G + g
                for r0 in range(0, len(sel), row_chunk):
                    idx = sel[r0:r0 + row_chunk]
                    s = (q[b, h, idx].astype(dtype) @ kk.T) * dtype(scale)
                    if causal:
                        q_pos = idx + (Skv - Sq)
                        s = np.where(q_pos[:, None] < k_pos[None, :], -np.inf, s)
                    with np.errstate(invalid="ignore"):
                        m = s.max(axis=-1, keepdims=True) if Skv else np.zeros((len(idx), 1), dtype)
                        p = np.exp(s - m)
                        p = p / p.sum(axis=-1, keepdims=True)
                    out[b, h, r0:r0 + len(idx)] = p @ vv
    return out


def gqa_lse(q, k, v, causal=True, *, rows=None, dtype=np.float64, row_chunk=1024):
    """Natural-log LSE (B, Hq, len(rows) or Sq) of the scaled scores of each
    query row over its visible keys (max-subtracted, like the output's
    softmax); -inf where no key is visible."""
    q = np.asarray(q)
    k = np.asarray(k)
    B, Hq, Hkv, Sq, Skv, D = _shapes(q, k, np.asarray(v))
    G = Hq // Hkv
    scale = D ** -0.5
    sel = np.arange(Sq) if rows is None else np.asarray(rows, dtype=np.int64)
    out = np.full((B, Hq, len(sel)), -np.inf, dtype=dtype)
    k_pos = np.arange(Skv)
    if Skv == 0:
        return out
    for b in range(B):
        for h in range(Hq):
            kk = k[b, h // G].astype(dtype)
            for r0 in range(0, len(sel), row_chunk):
                idx = sel[r0:r0 + row_chunk]
                s = (q[b, h, idx].astype(dtype) @ kk.T) * dtype(scale)
                if causal:
                    q_pos = idx + (Skv - Sq)
                    s = np.where(q_pos[:, None] < k_pos[None, :], -np.inf, s)
                m = s.max(axis=-1)
                safe = np.where(np.isneginf(m), 0.0, m)
                with np.errstate(divide="ignore"):
                    out[b, h, r0:r0 + len(idx)] = safe + np.log(np.exp(s - safe[:, None]).sum(axis=-1))
    return out


def split_partials(q, k, v, causal, splits, *, dtype=np.float64):
    """Per-chunk partials (m, l, acc) of the split-KV first pass.

    Returns m, l with shape (B, Hq, Sq, splits) and acc with shape
    (B, Hq, Sq, splits, D); m is in log2 units (logit * log2(e)).
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    B, Hq, Hkv, Sq, Skv, D = _shapes(q, k, v)
    G = Hq // Hkv
    c = dtype(D ** -0.5 * LOG2E)
    chunk = -(-Skv // splits)
    m = np.full((B, Hq, Sq, splits), -np.inf, dtype)
    l = np.zeros((B, Hq, Sq, splits), dtype)
    acc = np.zeros((B, Hq, Sq, splits, D), dtype)
    q_pos = np.arange(Sq) + (Skv - Sq)
    for s in range(splits):
        c0, c1 = s * chunk, min((s + 1) * chunk, Skv)
        if c1 <= c0:
            continue
        kp = np.arange(c0, c1)
        for b in range(B):
            for h in range(Hq):
                kvh = h // G
                t = (q[b, h].astype(dtype) @ k[b, kvh, c0:c1].astype(dtype).T) * c
                if causal:
                    t = np.where(q_pos[:, None] < kp[None, :], -np.inf, t)
                mm = t.max(axis=-1)
                safe = np.where(np.isneginf(mm), 0.0, mm)
                p = np.exp2(t - safe[:, None])
                m[b, h, :, s] = mm
                l[b, h, :, s] = p.sum(axis=-1)
                acc[b, h, :, s] = p @ v[b, kvh, c0:c1].astype(dtype)
    return m, l, acc


def split_combine(m, l, acc):
    """Log-sum-exp combine of split partials -> (B, Hq, Sq, D)."""
    with np.errstate(invalid="ignore"):
        mstar = m.max(axis=-1, keepdims=True)
        a = np.exp2(m - mstar)
        lstar = (a * l).sum(axis=-1)
        o = (a[..., None] * acc).sum(axis=-2) / lstar[..., None]
    return o


def split_lse(m, l):
    """Natural-log LSE from split partials (m in log2 units): the combine's
    m* + log2 sum_s exp2(m_s - m*) l_s, times ln 2."""
    with np.errstate(invalid="ignore", divide="ignore"):
        mstar = m.max(axis=-1, keepdims=True)
        lstar = (np.exp2(m - mstar) * l).sum(axis=-1)
        return (mstar[..., 0] + np.log2(lstar)) * math.log(2.0)


def split_kv_reference(q, k, v, causal, splits, *, dtype=np.float64):
    """Split-KV forward on the CPU (first pass + combine)."""
    return split_combine(*split_partials(q, k, v, causal, splits, dtype=dtype))


def paged_gather(k_cache, v_cache, block_table, seq_lens):
    """K and V of each sequence of a paged cache as contiguous arrays.

    k_cache, v_cache: (num_blocks, block_size, Hkv, D); block_table
    (B, max_blocks) and seq_lens (B,) integer arrays.  Key j of sequence b is
    slot j % block_size of block block_table[b, j // block_size] (the layout
    the paged entry points read; the reference has no paged cache, its
    roadmap names one at README.md:140-146).  Returns a list of B pairs of
    (1, Hkv, seq_lens[b], D) arrays, the (batch, kv head, key, d) order of
    reference gqa_kernels/dispatch.py:17-27 with batch 1.
    """
    k_cache = np.asarray(k_cache)
    v_cache = np.asarray(v_cache)
    table = np.asarray(block_table, dtype=np.int64)
    bs = k_cache.shape[1]
    out = []
    for b, n in enumerate(np.asarray(seq_lens, dtype=np.int64)):
        j = np.arange(int(n))
        blk, off = table[b, j // bs], j % bs
        out.append((k_cache[blk, off].transpose(1, 0, 2)[None], v_cache[blk, off].transpose(1, 0, 2)[None]))
    return out


def paged_reference(q, k_cache, v_cache, block_table, seq_lens, causal=True, *, dtype=np.float64):
    """Attention of q (B, Hq, Sq, D) over a paged cache: for each sequence b,
    ``gqa_reference`` of q[b] against its gathered keys (seq_kv = seq_lens[b],
    so the causal alignment is bottom-right per sequence).  Returns
    (o (B, Hq, Sq, D), lse (B, Hq, Sq))."""
    q = np.asarray(q)
    o = np.empty(q.shape, dtype=dtype)
    lse = np.empty(q.shape[:3], dtype=np.float64)
    for b, (kb, vb) in enumerate(paged_gather(k_cache, v_cache, block_table, seq_lens)):
        o[b] = gqa_reference(q[b:b + 1], kb, vb, causal, dtype=dtype)[0]
        lse[b] = gqa_lse(q[b:b + 1], kb, vb, causal)[0]
    return o, lse


def visible_pairs(seq_q: int, seq_kv: int, causal: bool) -> int:
    """Unmasked (query, key) pairs per (batch, q head), bottom-right causal.

    Row i sees keys [0, i + seq_kv - seq_q] clipped to [0, seq_kv); for
    seq_q <= seq_kv the sum is seq_q*(seq_kv - seq_q) + seq_q*(seq_q + 1)/2.
    """
    if not causal:
        return seq_q * seq_kv
    i = np.arange(seq_q, dtype=np.int64)
    return int(np.clip(i + (seq_kv - seq_q) + 1, 0, seq_kv).sum())


def attention_flops(batch, num_heads, seq_q, seq_kv, head_dim, causal=True) -> int:
    """Algorithmic FLOPs: 4 * D per visible (query, key) pair (QK^T + PV)."""
    return 4 * head_dim * batch * num_heads * visible_pairs(seq_q, seq_kv, causal)


def attention_bytes(batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, elem=2) -> int:
    """Algorithmic HBM bytes: K and V read once, Q read once, O written once."""
    return elem * head_dim * (2 * batch * num_kv_heads * seq_kv + 2 * batch * num_heads * seq_q)
