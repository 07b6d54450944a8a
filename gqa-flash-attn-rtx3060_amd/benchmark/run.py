"""Benchmark harness for gqa_flash_attn on MI355X: correctness gate, sweep,
N-trial median, JSON rows.

MI355X counterpart of reference benchmark/run.py (same CLI, same sweep
lengths, same row schema, run.py:181-188 and 268-278).  Baselines: PyTorch
SDPA with K/V pre-expanded to all query heads (reference run.py:57-70), on
its fused flash / memory-efficient backends only; flash-attn2 comes from the
HF Hub in the reference (run.py:23-28), which is not reachable here, so its
column is NaN exactly as the reference prints it when FA2 fails to load.

Usage:
    python gqa-flash-attn-rtx3060_amd/benchmark/run.py                # full sweep, one trial
    python gqa-flash-attn-rtx3060_amd/benchmark/run.py --trials 5     # 5-trial median
    python gqa-flash-attn-rtx3060_amd/benchmark/run.py --quick        # gate + 8K only
    python gqa-flash-attn-rtx3060_amd/benchmark/run.py --correctness  # gate only

Writes <out>/<commit>[_median<N>].json (default out: benchmark/results next to
this file) and prints a markdown table.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

BATCH = 1
NUM_HEADS = 32
NUM_KV_HEADS = 8
HEAD_DIM = 128

# The reference's sweep (run.py:43-45) plus its published lengths.
PREFILL_LENS = (2048, 4096, 6144, 8192, 12288, 16384)
DECODE_LENS = (2048, 4096, 8192, 16384)
CORRECTNESS_LENS = (512, 2048, 4096)

WARMUP = 25
ITERS = 100
GATE_MAX, GATE_MEAN = 1e-2, 1e-3  # reference run.py:98


def _make(torch, seq_q, seq_kv, dtype, gen):
    shape_q = (BATCH, NUM_HEADS, seq_q, HEAD_DIM)
    shape_kv = (BATCH, NUM_KV_HEADS, seq_kv, HEAD_DIM)
    mk = lambda s: (torch.randn(s, generator=gen, device="cuda", dtype=torch.float32) * 0.1).to(dtype)
    return mk(shape_q), mk(shape_kv), mk(shape_kv)


def reference_attention(torch, q, k, v, causal=True):
    """fp32 GQA attention on the GPU (the reference's tests/reference.py:16-34
    semantics: q head h reads kv head h // G, scale D^-0.5, bottom-right causal
    mask), computed per kv head without expanding K/V.  fp32 throughout, with
    contiguous operands for every batched product."""
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = torch.empty(B, Hq, Sq, D, dtype=torch.float32, device=q.device)
    qpos = torch.arange(Sq, device=q.device)[:, None] + (Skv - Sq)
    kpos = torch.arange(Skv, device=q.device)[None, :]
    masked = kpos > qpos
    for b in range(B):
        for h in range(Hkv):
            qq = q[b, h * G:(h + 1) * G].float().reshape(G * Sq, D).contiguous()
            kt = k[b, h].float().t().contiguous()
            s = (qq @ kt).reshape(G, Sq, Skv) * (D ** -0.5)
            if causal:
                s = s.masked_fill(masked, float("-inf"))
            p = torch.softmax(s, dim=-1).reshape(G * Sq, Skv)
            out[b, h * G:(h + 1) * G] = (p @ v[b, h].float().contiguous()).reshape(G, Sq, D)
    return out


def _sdpa_expand(k, v):
    """K/V expanded to every query head once, outside timing (reference run.py:57-61)."""
    group = NUM_HEADS // NUM_KV_HEADS
    return k.repeat_interleave(group, dim=1).contiguous(), v.repeat_interleave(group, dim=1).contiguous()


def _sdpa_call(torch, q, k_exp, v_exp, sdpa_causal):
    """SDPA restricted to its fused backends.  is_causal is upper-left aligned,
    so it is True only for square (prefill) calls (reference run.py:64-70)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    import torch.nn.functional as F
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return F.scaled_dot_product_attention(q, k_exp, v_exp, is_causal=sdpa_causal)


def _err(torch, out, ref):
    d = (out.float() - ref).abs()
    return d.max().item(), d.mean().item()


def correctness_check(torch, gqa_flash_attn, dtype, gen):
    """Gate every kernel (ours and SDPA) against the fp32 reference on the
    reference's cases (run.py:96-141): prefill and decode at 512/2048/4096."""
    print(f"[correctness] gate: max_abs < {GATE_MAX:g}, mean_abs < {GATE_MEAN:g}")
    cases = [(L, L, "prefill") for L in CORRECTNESS_LENS] + [(1, L, "decode") for L in CORRECTNESS_LENS]
    all_ok = True
    for sq, sk, label in cases:
        q, k, v = _make(torch, sq, sk, dtype, gen)
        ref = reference_attention(torch, q, k, v, causal=True)
        mx, mn = _err(torch, gqa_flash_attn(q, k, v, causal=True), ref)
        ok = mx < GATE_MAX and mn < GATE_MEAN
        all_ok &= ok
        print(f"[correctness] {label:<7} L={sk:>5d}  ours: max={mx:.2e} mean={mn:.2e}  {'ok' if ok else 'FAIL'}")
        try:
            k_exp, v_exp = _sdpa_expand(k, v)
            mx, mn = _err(torch, _sdpa_call(torch, q, k_exp, v_exp, sq == sk), ref)
            ok = mx < GATE_MAX and mn < GATE_MEAN
            print(f"[correctness] {label:<7} L={sk:>5d}  sdpa: max={mx:.2e} mean={mn:.2e}  {'ok' if ok else 'FAIL'}")
        except RuntimeError as e:  # no fused SDPA backend for this shape: baseline column stays NaN
            print(f"[correctness] {label:<7} L={sk:>5d}  sdpa: unavailable ({str(e).splitlines()[0][:80]})")
    return all_ok


def _time(torch, fn):
    """Mean ms per call over ITERS back-to-back calls fn(0), fn(1), ...
    after WARMUP (reference run.py:144-158), and the peak memory allocated
    meanwhile (GB)."""
    torch.cuda.synchronize()
    for i in range(WARMUP):
        fn(i)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(ITERS):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / ITERS, torch.cuda.max_memory_allocated() / (1024 ** 3)


# Decode rows read each K/V byte once per call, so back-to-back calls on one
# K/V set would be served by the 256 MB Infinity Cache, not HBM: they rotate
# through as many sets as it takes to stream at least this many bytes.
ROTATE_BYTES = 512 * 2 ** 20


def _n_sets(k, v):
    return max(1, math.ceil(ROTATE_BYTES / (k.numel() * k.element_size() + v.numel() * v.element_size())))


def work(workload, L):
    """Algorithmic FLOPs and bytes of one call (B=1, Hq=32, Hkv=8, D=128)."""
    sq = L if workload == "prefill" else 1
    visible = sq * (sq + 1) // 2 + (L - sq) * sq  # bottom-right causal, sq <= L
    flops = 4 * HEAD_DIM * BATCH * NUM_HEADS * visible
    nbytes = 2 * HEAD_DIM * (2 * BATCH * NUM_KV_HEADS * L + 2 * BATCH * NUM_HEADS * sq)
    return flops, nbytes


def make_row(workload, L, ours_ms, fa2_ms, sdpa_ms, mem_gb):
    """One result row in the reference's schema (run.py:181-188), plus the
    achieved TFLOP/s and GB/s of our kernel."""
    sq = L if workload == "prefill" else 1
    flops, nbytes = work(workload, L)
    return {
        "workload": workload, "seq_kv": L,
        "ours_ms": ours_ms, "fa2_ms": fa2_ms, "sdpa_ms": sdpa_ms,
        "tok_s": sq * 1000.0 / ours_ms,
        "speedup_vs_fa2": fa2_ms / ours_ms,
        "speedup_vs_sdpa": sdpa_ms / ours_ms,
        "peak_mem_gb": mem_gb,
        "tflops": flops / (ours_ms * 1e-3) / 1e12,
        "gbs": nbytes / (ours_ms * 1e-3) / 1e9,
    }


def run_sweep(torch, gqa_flash_attn, prefill_lens, decode_lens, dtype, gen):
    rows = []
    for workload, lens in (("prefill", prefill_lens), ("decode", decode_lens)):
        for L in lens:
            sq = L if workload == "prefill" else 1
            q, k, v = _make(torch, sq, L, dtype, gen)
            # decode: rotate K/V sets (and, for SDPA, expanded sets) past the
            # Infinity Cache; prefill is MFMA-bound and uses one set
            kvs = [(k, v)]
            if workload == "decode":
                kvs += [_make(torch, sq, L, dtype, gen)[1:] for _ in range(_n_sets(k, v) - 1)]
            ours_ms, mem = _time(torch, lambda i: gqa_flash_attn(q, *kvs[i % len(kvs)], causal=True))
            try:
                k_sdpa, v_sdpa = _sdpa_expand(k, v)
                sdpa_kvs = [(k_sdpa, v_sdpa)]
                if workload == "decode":
                    sdpa_kvs += [_sdpa_expand(*kv) for kv in kvs[1:_n_sets(k_sdpa, v_sdpa)]]
                sdpa_ms = _time(torch, lambda i: _sdpa_call(torch, q, *sdpa_kvs[i % len(sdpa_kvs)], sq == L))[0]
                del k_sdpa, v_sdpa, sdpa_kvs
            except RuntimeError:
                sdpa_ms = float("nan")
            del kvs
            row = make_row(workload, L, ours_ms, float("nan"), sdpa_ms, mem)
            rows.append(row)
            print(f"[{workload}] L={L:>5d}  ours={ours_ms:7.3f}ms  fa2=  n/a  ms  sdpa={sdpa_ms:7.3f}ms  "
                  f"vs_sdpa={row['speedup_vs_sdpa']:.2f}x  {row['tflops']:.0f} TFLOP/s  {row['gbs']:.0f} GB/s",
                  flush=True)
            torch.cuda.empty_cache()
    return rows


def aggregate_median(trials):
    """Per (workload, seq_kv) median over trials (reference run.py:191-211)."""
    keys = sorted({(r["workload"], r["seq_kv"]) for trial in trials for r in trial})
    agg = []
    for key in keys:
        cells = [r for trial in trials for r in trial if (r["workload"], r["seq_kv"]) == key]
        med = lambda f: statistics.median(c[f] for c in cells)
        agg.append(make_row(key[0], key[1], med("ours_ms"), med("fa2_ms"), med("sdpa_ms"), med("peak_mem_gb")))
    return agg


def markdown_table(rows):
    out = ["| Workload | seq_kv | ours (ms) | FA2 (ms) | SDPA (ms) | vs FA2 | vs SDPA | TFLOP/s | GB/s | mem (GB) |",
           "|---|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        out.append(f"| {r['workload']} | {r['seq_kv']} | {r['ours_ms']:.3f} | {r['fa2_ms']:.3f} | "
                   f"{r['sdpa_ms']:.3f} | {r['speedup_vs_fa2']:.2f}× | {r['speedup_vs_sdpa']:.2f}× | "
                   f"{r['tflops']:.0f} | {r['gbs']:.0f} | {r['peak_mem_gb']:.2f} |")
    return "\n".join(out)


def _commit():
    # A copy of the tree without git metadata can name its commit.
    if os.environ.get("GQA_COMMIT"):
        return os.environ["GQA_COMMIT"][:7]
    try:
        return subprocess.check_output(["git", "rev-parse", "--short=7", "HEAD"], cwd=HERE,
                                       stderr=subprocess.DEVNULL).decode().strip()
    except Exception:
        return "nogit00"


def main(argv=None):
    p = argparse.ArgumentParser()
    p.add_argument("--trials", type=int, default=1)
    p.add_argument("--quick", action="store_true")
    p.add_argument("--correctness", action="store_true")
    p.add_argument("--dtype", choices=["bf16", "fp16"], default="bf16")
    p.add_argument("--out", type=Path, default=HERE / "results")
    args = p.parse_args(argv)

    import torch
    from gqa_kernels import gqa_flash_attn

    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    gen = torch.Generator(device="cuda").manual_seed(0)
    print(f"device: {torch.cuda.get_device_name(0)}")
    print(f"dtype:  {dtype}")
    print(f"config: H={NUM_HEADS} Hkv={NUM_KV_HEADS} D={HEAD_DIM} batch={BATCH}")
    print("[warn] flash-attn2 not available offline — vs_fa2 column will be NaN\n")

    if not correctness_check(torch, gqa_flash_attn, dtype, gen):
        return 1
    if args.correctness:
        return 0

    prefill = (8192,) if args.quick else PREFILL_LENS
    decode = (8192,) if args.quick else DECODE_LENS
    trials = []
    for i in range(args.trials):
        if args.trials > 1:
            print(f"\n=== trial {i + 1}/{args.trials} ===")
        trials.append(run_sweep(torch, gqa_flash_attn, prefill, decode, dtype, gen))
    rows = aggregate_median(trials) if args.trials > 1 else trials[0]

    args.out.mkdir(parents=True, exist_ok=True)
    commit = _commit()
    suffix = f"_median{args.trials}" if args.trials > 1 else ""
    path = args.out / f"{commit}{suffix}.json"
    with open(path, "w") as f:
        json.dump({
            "commit": commit, "device": torch.cuda.get_device_name(0), "dtype": str(dtype),
            "trials": args.trials,
            "config": {"batch": BATCH, "num_heads": NUM_HEADS, "num_kv_heads": NUM_KV_HEADS,
                       "head_dim": HEAD_DIM, "model": "Llama 3.1 8B attention shape"},
            "env": {"torch": torch.__version__, "hip": getattr(torch.version, "hip", None),
                    "sdpa": "F.scaled_dot_product_attention (flash / memory-efficient backends) "
                            "with pre-expanded K/V",
                    "flash_attn2": "unavailable (HF Hub download; no network)"},
            "rows": rows,
        }, f, indent=2)
    label = f"{args.trials}-trial median" if args.trials > 1 else "single run"
    print(f"\n=== Results ({label}, commit {commit}) -> {path} ===")
    print(markdown_table(rows))
    return 0


if __name__ == "__main__":
    sys.exit(main())
