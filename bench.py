"""Benchmark of sparse_attn_sharedkv on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]

Prints ONE JSON line. The headline workload is BASELINE config 2 (batched
decode B=32, H=64, top-k 512 + window 128, ctx U[8K,32K], bf16, paged
bs=64); `value` is its gathered-KV throughput in GB/s (valid window + top-k
rows x 1152 B, counted once per token since all heads share the row).
The 4K prefill (config 3) is reported beside it in TFLOP/s of useful work
(valid (token, key) pairs x H x 2 x (576 + 512)).

Decode inputs rotate over copies whose touched rows together exceed the
256 MB Infinity Cache, so each call reads HBM, not MALL. Inputs are resident
in HBM before timing starts. The CPU baseline times the oracle (a CPU
restatement of the reference's golden loop) on the host cores.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "decode µs/call + HBM GB/s (B32,H64,k512+w128); prefill TFLOP/s at 4K"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _prepare(inp, **kw):
    from dsv4_amd.api import prepare_sparse_attn_sharedkv
    return prepare_sparse_attn_sharedkv(inp.q, **inp.api_kwargs(), **kw)


def _rotations(inp, n):
    """n copies of the inputs in distinct memory (same values)."""
    from dataclasses import replace
    out = [inp]
    for _ in range(n - 1):
        out.append(replace(inp, q=inp.q.clone(), ori_kv=inp.ori_kv.clone(),
                           cmp_kv=inp.cmp_kv.clone() if inp.cmp_kv is not None else None))
    return out


def time_calls(calls, steps, warmup):
    """Launch calls[i % n] `steps` times between two synchronisations; returns
    (total ms from events on the launch stream, wall ms)."""
    st = torch.cuda.current_stream()
    for i in range(warmup):
        calls[i % len(calls)].launch(st)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(st)
    for i in range(steps):
        calls[i % len(calls)].launch(st)
    e1.record(st)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    return e0.elapsed_time(e1), wall


def cpu_oracle_time(inp, tokens=None, reps=1):
    from oracle import golden_ref as O
    from dsv4_amd import paged
    c = inp.cfg
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        O.golden_paged(inp.q, ori_kv=inp.ori_kv, ori_block_table=inp.ori_bt,
                       cu_seqlens_q=inp.cu_seqlens_q, seqused_kv=inp.seqused_kv, sinks=inp.sinks,
                       softmax_scale=c.scale, cmp_kv=inp.cmp_kv, cmp_block_table=inp.cmp_bt,
                       cmp_sparse_indices=inp.cmp_idx, cmp_ratio=c.cmp_ratio, dv=512,
                       dequant=paged.dequantize_kv_fp8 if c.fp8 else None, tokens=tokens)
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--rotations", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this operator build runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured path)", file=sys.stderr)
        sys.exit(2)

    from dsv4_amd import cases
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    torch.cuda.init()

    # ---------------- decode, config 2 ---------------------------------------
    cfg = cases.CONFIGS["C2"]
    log("building C2 inputs")
    inp = cases.make_inputs(cfg, device="cuda")
    rows = cases.gathered_rows(inp)
    row_bytes = cfg.D * 2
    kv_bytes = rows * row_bytes
    rot = _rotations(inp, args.rotations)
    calls = [_prepare(r) for r in rot]
    torch.cuda.synchronize()
    log(f"C2: T={inp.T} gathered rows={rows} bytes={kv_bytes} splits={calls[0].num_splits} "
        f"rotations={len(calls)} (touched {len(calls) * kv_bytes / 1e6:.0f} MB)")
    ev_ms, wall_ms = time_calls(calls, args.steps, args.warmup)
    us_call = ev_ms * 1e3 / args.steps
    gbs = kv_bytes / (us_call * 1e-6) / 1e9
    log(f"C2 decode: {us_call:.2f} us/call (events), {wall_ms * 1e3 / args.steps:.2f} us wall, "
        f"{gbs:.0f} GB/s")
    # API wall time (host resolution + launch), reported separately
    from dsv4_amd.api import sparse_attn_sharedkv
    kw = inp.api_kwargs()
    for _ in range(3):
        sparse_attn_sharedkv(inp.q, **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        sparse_attn_sharedkv(inp.q, **kw)
    torch.cuda.synchronize()
    api_us = (time.perf_counter() - t0) / 20 * 1e6

    # ---------------- prefill, config 3 --------------------------------------
    prefill = None
    if not args.no_prefill:
        pcfg = cases.CONFIGS["C3"]
        log("building C3 inputs")
        pinp = cases.make_inputs(pcfg, device="cuda")
        prows = cases.gathered_rows(pinp)
        flops = prows * pcfg.H * 2 * (pcfg.D + pcfg.DV)
        pcall = _prepare(pinp)
        pev, _ = time_calls([pcall], args.prefill_steps, 3)
        pus = pev * 1e3 / args.prefill_steps
        tfl = flops / (pus * 1e-6) / 1e12
        prefill = dict(workload="C3 prefill S4096 H64 k512+w128 contiguous", us_per_call=round(pus, 2),
                       tflops=round(tfl, 2), useful_flop=flops, pairs=prows,
                       mfma_frac=round(tfl / BF16_PEAK_TFLOPS, 4), splits=pcall.num_splits)
        log(f"C3 prefill: {pus:.1f} us/call, {tfl:.1f} TFLOP/s ({flops:.4e} useful FLOP)")

    # ---------------- CPU baseline (oracle on host cores) --------------------
    cpu = None
    if not args.no_cpu:
        n = min(len(os.sched_getaffinity(0)), 16)
        torch.set_num_threads(n)
        log(f"CPU baseline on {n} threads")
        host = inp.to("cpu")
        cpu_s = cpu_oracle_time(host, reps=3)
        cpu = dict(value=round(kv_bytes / cpu_s / 1e9, 3), unit="GB/s", cores=n, kind="port",
                   us_per_call=round(cpu_s * 1e6, 1),
                   sample="full C2 decode call (32 tokens), median of 3, torch fp32 oracle")
        if prefill is not None:
            ph = pinp.to("cpu")
            toks = list(range(0, pinp.T, 16))
            ps = cpu_oracle_time(ph, tokens=toks) * pinp.T / len(toks)
            cpu["prefill_tflops"] = round(prefill["useful_flop"] / ps / 1e12, 4)
            cpu["prefill_sample"] = f"{len(toks)} of {pinp.T} C3 tokens (every 16th), scaled"

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ev_ms / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) q/kv, random paged block tables, seeded",
        "config": {"workload": "C2 batched decode B32 S_q1 H64 D576/512 top-k512 + window128, "
                               "ctx U[8K,32K], paged bs64", "B": 32, "H": 64, "topk": 512,
                   "window": 128, "parallelism": "single GPU"},
        "decode_us_per_call": round(us_call, 3),
        "api_us_per_call": round(api_us, 1),
        "gathered_kv_bytes": kv_bytes,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel_time": "event-timed op (fwd + split combine) per call"},
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
