"""Benchmark of sparse_attn_sharedkv on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-traffic]

Prints ONE JSON line. The headline workload is config C2 (batched decode
B=32, H=64, top-k 512 + window 128, ctx U[8K,32K], bf16, paged bs=64);
`value` is its gathered-KV throughput in GB/s per whole call (split kernel +
LSE combine): valid window + top-k rows x 1152 B, counted once per token
since all heads share the row. The 4K prefill (C3) is reported beside it in
TFLOP/s of useful work (valid (token, key) pairs x H x 2 x (576 + 512)).

`roofline` prices the dominant kernel (the split-KV forward kernel of C2)
alone: the same algorithmic bytes divided by its own event-timed average
launch duration. `roofline.traffic` is the HBM bytes one launch of that
kernel moves, from two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE)
run as child processes of this script, each scaled by what the same counter
reads for an elementwise kernel of known size (`--pmc-pass` is that child).

Decode inputs rotate over copies whose touched rows together exceed the
256 MB Infinity Cache, so each call reads HBM, not MALL. Inputs are resident
in HBM before timing starts. The CPU baseline times the oracle (a CPU
restatement of the reference's golden loop) on the host cores.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import shutil
import signal
import subprocess
import sys
import tempfile
import time

import torch

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "decode µs/call + HBM GB/s (B32,H64,k512+w128); prefill TFLOP/s at 4K"
SPLIT_KERNEL = "sas_fwd_kernel"
COMBINE_KERNEL = "sas_combine_kernel"
CAL_KERNEL = "neg_kernel"      # torch.neg on fp32: reads and writes numel*4 bytes
CW_KERNEL = "sas_cache_fp8_kernel"
CAL_NUMEL = 32 << 20           # 128 MiB each way
PMC_ROTATIONS = 4              # 94 MB of gathered rows: beyond the 32 MB of L2


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


def time_launches(launch, n_calls, steps, warmup):
    """Run launch(i, stream) for i in [0, steps) between two synchronisations
    (after `warmup` untimed calls); events are recorded on the launch stream.
    Returns (total event ms, wall ms)."""
    st = torch.cuda.current_stream()
    for i in range(warmup):
        launch(i % n_calls, st)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(st)
    for i in range(steps):
        launch(i % n_calls, st)
    e1.record(st)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    return e0.elapsed_time(e1), wall


def time_cold(launch, steps, flush):
    """Per-call event time with the caches flushed before every call: a
    read of a 1 GB buffer (leaving the 256 MB MALL and the L2s holding other
    lines) runs before each call's start event, outside the timed span.
    Returns the median call in ms."""
    st = torch.cuda.current_stream()
    evs = []
    for _ in range(steps):
        flush()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        launch(st)
        e1.record(st)
        evs.append((e0, e1))
    torch.cuda.synchronize()
    ts = sorted(a.elapsed_time(b) for a, b in evs)
    return ts[len(ts) // 2]


def measured_peaks():
    """HBM: a 2 GiB device copy (read + write bytes / time); bf16 MFMA: an
    8192^3 bf16 GEMM through torch (hipBLASLt)."""
    n = 1 << 29                                     # 2 GiB of fp32
    src = torch.empty(n, device="cuda").normal_()
    dst = torch.empty_like(src)
    ms, _ = time_launches(lambda i, st: dst.copy_(src), 1, 20, 3)
    copy_gbs = 2 * n * 4 / (ms / 20 * 1e-3) / 1e9
    del src, dst
    m = 8192
    a = torch.randn(m, m, device="cuda").to(torch.bfloat16)
    b = torch.randn(m, m, device="cuda").to(torch.bfloat16)
    c = torch.empty(m, m, device="cuda", dtype=torch.bfloat16)
    ms, _ = time_launches(lambda i, st: torch.matmul(a, b, out=c), 1, 20, 3)
    gemm_tf = 2 * m ** 3 / (ms / 20 * 1e-3) / 1e12
    del a, b, c
    # fp32 atomic adds (the backward's row gradients): the library's
    # microbenchmark kernel (each wave adds to a 256-byte run of a row, the
    # backward's pattern; 2048 x 256 threads x 256 adds into 6144 rows of 576
    # floats, the C3 cache's shape), and torch's index_add_ of 2^17 random
    # 576-float rows for comparison. The peak is the larger of the two.
    import ctypes
    from dsv4_amd import _lib
    L = _lib.lib()
    rows, wgs, iters = 6144, 2048, 256
    dst = torch.zeros(rows, 576, device="cuda")
    def kern(i, st):
        _lib.check(L.sas_bench_atomic_add_v1(ctypes.c_void_p(dst.data_ptr()), rows, 576, wgs, iters,
                                             ctypes.c_void_p(st.cuda_stream)), "sas_bench_atomic_add_v1")
    ms, _ = time_launches(kern, 1, 10, 2)
    kern_g = wgs * 256 * iters / (ms / 10 * 1e-3) / 1e9
    n = 1 << 17
    g = torch.Generator(device="cuda").manual_seed(5)
    src = torch.randn(n, 576, device="cuda", generator=g)
    idx = torch.randint(0, rows, (n,), device="cuda", generator=g)
    ms, _ = time_launches(lambda i, st: dst.index_add_(0, idx, src), 1, 10, 2)
    ia_g = n * 576 / (ms / 10 * 1e-3) / 1e9
    del dst, src, idx
    torch.cuda.synchronize()
    return dict(hbm_spec_gbs=HBM_PEAK_GBS, hbm_copy_measured_gbs=round(copy_gbs, 1),
                bf16_spec_tflops=BF16_PEAK_TFLOPS, bf16_gemm_measured_tflops=round(gemm_tf, 1),
                fp32_atomic_measured_g_per_s=round(max(kern_g, ia_g), 1),
                fp32_atomic_kernel_g_per_s=round(kern_g, 1), fp32_atomic_index_add_g_per_s=round(ia_g, 1),
                how="copy: torch copy_ of 2 GiB (read + write bytes); gemm: torch.matmul 8192^3 bf16; "
                    "atomics: the larger of sas_bench_atomic_add_v1 (2048 x 256 threads x 256 adds, "
                    "256-byte runs into 6144 x 576 fp32) and torch index_add_ of 2^17 x 576 fp32")


def usable_cores():
    """Cores this process may run on: the affinity set, capped by the
    cgroup CPU quota when one is set (a job's CPU share)."""
    n = len(os.sched_getaffinity(0))
    note = f"{n} in the affinity set"
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            q = max(1, int(int(quota) / int(period)))
            if q < n:
                note += f", cgroup quota {q}"
                n = q
    except (OSError, ValueError):
        pass
    return n, note


def cpu_oracle_time(inp, tokens=None, min_seconds=0.0, max_reps=1):
    """Median seconds of one oracle pass; repeats until min_seconds of CPU
    work (or max_reps passes) have run."""
    from oracle import golden_ref as O
    from dsv4_amd import paged
    c = inp.cfg
    ts = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        O.golden_paged(inp.q, ori_kv=inp.ori_kv, ori_block_table=inp.ori_bt,
                       cu_seqlens_q=inp.cu_seqlens_q, seqused_kv=inp.seqused_kv, sinks=inp.sinks,
                       softmax_scale=c.scale, cmp_kv=inp.cmp_kv, cmp_block_table=inp.cmp_bt,
                       cmp_sparse_indices=inp.cmp_idx, cmp_ratio=c.cmp_ratio, dv=512,
                       dequant=paged.dequantize_kv_fp8 if c.fp8 else None, tokens=tokens)
        ts.append(time.perf_counter() - t0)
        if len(ts) >= max_reps or time.perf_counter() - t_start >= min_seconds:
            break
    ts.sort()
    return ts[len(ts) // 2], len(ts), time.perf_counter() - t_start


# ---------------------------------------------------------------------------
# HBM traffic from rocprofv3 --pmc (child processes)
# ---------------------------------------------------------------------------

def pmc_pass():
    """Child of a `rocprofv3 --pmc` run: a calibration kernel of known size,
    then PMC_ROTATIONS rounds of C2 decode (split kernel + combine) over
    distinct input copies."""
    from dsv4_amd import cases
    torch.cuda.init()
    src = torch.randn(CAL_NUMEL, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    inp = cases.make_inputs(cases.CONFIGS["C2"], device="cuda")
    calls = [_prepare(r) for r in _rotations(inp, PMC_ROTATIONS)]
    torch.cuda.synchronize()
    for _ in range(3):
        for c in calls:
            c.launch_split()
            c.launch_combine()
    torch.cuda.synchronize()
    del calls, inp
    cw = _cache_write_calls()
    for _ in range(2):
        for c in cw:
            c.launch()
    torch.cuda.synchronize()
    print("[pmc-pass] done", flush=True)


def prefill_pass():
    """Child of a `rocprofv3 --pmc` run for the MFMA counters of the C3
    prefill kernel: a bf16 GEMM of known FLOP (8192^3, hipBLASLt) three
    times, then the C3 forward five times."""
    from dsv4_amd import cases
    torch.cuda.init()
    m = 8192
    a = torch.randn(m, m, device="cuda").to(torch.bfloat16)
    b = torch.randn(m, m, device="cuda").to(torch.bfloat16)
    for _ in range(3):
        torch.matmul(a, b)
    torch.cuda.synchronize()
    del a, b
    inp = cases.make_inputs(cases.CONFIGS["C3"], device="cuda")
    call = _prepare(inp)
    for _ in range(5):
        call.launch()
    torch.cuda.synchronize()
    print(f"[prefill-pass] done: {cases.gathered_rows(inp)} (token, key) pairs", flush=True)


def _read_counter(outdir, counter):
    """{kernel substring: [per-dispatch values]} for the counter."""
    vals = {SPLIT_KERNEL: [], COMBINE_KERNEL: [], CAL_KERNEL: [], CW_KERNEL: []}
    files = glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True)
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") != counter:
                    continue
                name = row.get("Kernel_Name", "")
                for k in vals:
                    if k in name:
                        vals[k].append(float(row["Counter_Value"]))
    return vals


def measure_traffic(kv_bytes_hint=None):
    """HBM bytes per launch of the split kernel (and the combine), each of the
    two counters scaled by its reading for the calibration kernel."""
    prof = shutil.which("rocprofv3")
    if prof is None:
        return None, "rocprofv3 not found"
    res = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        outdir = tempfile.mkdtemp(prefix="sas_pmc_")
        cmd = [prof, "--pmc", counter, "-d", outdir, "-o", "pmc", "--output-format", "csv",
               "--", sys.executable, os.path.abspath(__file__), "--pmc-pass"]
        log(f"pmc pass {counter}")
        p = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                             start_new_session=True)
        try:
            text, _ = p.communicate(timeout=150)
        except subprocess.TimeoutExpired:
            os.killpg(p.pid, signal.SIGKILL)
            p.communicate()
            shutil.rmtree(outdir, ignore_errors=True)
            return None, f"rocprofv3 --pmc {counter} timed out"
        vals = _read_counter(outdir, counter)
        shutil.rmtree(outdir, ignore_errors=True)
        if "[pmc-pass] done" not in text or not vals[SPLIT_KERNEL] or not vals[CAL_KERNEL]:
            tail = " | ".join(text.strip().splitlines()[-3:])
            return None, f"rocprofv3 --pmc {counter} gave no usable rows (rc {p.returncode}): {tail}"
        res[counter] = vals
    out = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        v = res[counter]
        cal = sorted(v[CAL_KERNEL])[len(v[CAL_KERNEL]) // 2] * 1024.0 / (CAL_NUMEL * 4)
        # skip the first pass over the rotations (cold TLB / first touch)
        split = v[SPLIT_KERNEL][PMC_ROTATIONS:] or v[SPLIT_KERNEL]
        comb = v[COMBINE_KERNEL][PMC_ROTATIONS:] or v[COMBINE_KERNEL]
        cw = v[CW_KERNEL][CW_ROTATIONS:] or v[CW_KERNEL]
        out[counter] = dict(
            cal_factor=round(cal, 4),
            split_bytes=sum(split) / len(split) * 1024.0 / cal,
            combine_bytes=(sum(comb) / len(comb) * 1024.0 / cal) if comb else None,
            cache_write_bytes=(sum(cw) / len(cw) * 1024.0 / cal) if cw else None)
    return out, None


# ---------------------------------------------------------------------------


CW_ROWS = 32768        # rows per cache-write call: a 32K-token prefill chunk
CW_ROTATIONS = 8       # distinct inputs and cache blocks: 474 MB touched, beyond the MALL


def _cache_write_calls():
    """CW_ROTATIONS prepared cache writes of CW_ROWS bf16 rows (D = 576, 16
    sequences) into 656-byte fp8 rows through shuffled block tables (bs 64),
    each rotation with its own input rows and cache blocks."""
    from dsv4_amd.cache import prepare_kv_cache_write
    g = torch.Generator(device="cuda").manual_seed(11)
    bs, B = 64, 16
    per_b = CW_ROWS // B
    nblk = per_b // bs
    nb = CW_ROTATIONS * B * nblk
    cache = torch.zeros(nb, bs, 1, 656, dtype=torch.uint8, device="cuda")
    perm = torch.randperm(nb, device="cuda", generator=g).to(torch.int32)
    sid = torch.arange(B, device="cuda", dtype=torch.int32).repeat_interleave(per_b)
    pos = torch.arange(per_b, device="cuda", dtype=torch.int32).repeat(B)
    calls = []
    for r in range(CW_ROTATIONS):
        kv = torch.randn(CW_ROWS, 576, device="cuda", generator=g).to(torch.bfloat16)
        table = perm[r * B * nblk:(r + 1) * B * nblk].reshape(B, nblk).contiguous()
        calls.append(prepare_kv_cache_write(kv, cache, table, sid, pos))
    torch.cuda.synchronize()
    return calls


def bench_cache_write(traffic=None):
    """sas_cache_write_v1 over _cache_write_calls(). Algorithmic HBM bytes per
    row: 1152 read + 656 written + 8 of (batch, position)."""
    bs = 64
    calls = _cache_write_calls()
    ms, _ = time_launches(lambda i, st: calls[i].launch(st), len(calls), 240, 12)
    us = ms * 1e3 / 240
    byts = CW_ROWS * (1152 + 656 + 8)
    gbs = byts / (us * 1e-6) / 1e9
    tr = None
    if traffic and traffic["FETCH_SIZE"].get("cache_write_bytes") and traffic["WRITE_SIZE"].get("cache_write_bytes"):
        tr = round(traffic["FETCH_SIZE"]["cache_write_bytes"] + traffic["WRITE_SIZE"]["cache_write_bytes"])
    return dict(workload=f"fp8 cache write: {CW_ROWS} bf16 rows (D 576) -> 656-byte rows, "
                         f"shuffled block table bs {bs}", kernel=CW_KERNEL, us_per_call=round(us, 3),
                bytes=byts, gbs=round(gbs, 1), hbm_frac=round(gbs / HBM_PEAK_GBS, 4), traffic=tr,
                _log=f"cache write: {us:.2f} us/call, {gbs:.0f} GB/s ({byts} B)")


def bench_decode_configs(names, steps, flush):
    """C1 / C4 / C5 (and C2 for comparison): one whole call per timed span,
    caches flushed before each. Algorithmic bytes = valid (token, key) rows
    x row bytes (1152 for bf16 rows at D = 576, 656 for fp8 rows)."""
    from dsv4_amd import cases
    res = {}
    for name in names:
        cfg = cases.CONFIGS[name]
        inp = cases.make_inputs(cfg, device="cuda")
        rows = cases.gathered_rows(inp)
        rb = 656 if cfg.fp8 else cfg.D * 2
        call = _prepare(inp)
        torch.cuda.synchronize()
        for _ in range(3):
            call.launch()
        ms = time_cold(lambda st: call.launch(st), steps, flush)
        us = ms * 1e3
        byts = rows * rb
        gbs = byts / (us * 1e-6) / 1e9
        # every head of a token attends its rows: 2 x (576 + 512) FLOP per (row, head)
        flop = rows * cfg.H * 2 * (cfg.D + cfg.DV)
        res[name] = dict(workload=cfg.notes, tokens=inp.T, gathered_rows=rows, row_bytes=rb,
                         gathered_bytes=byts, us_per_call=round(us, 3), gbs=round(gbs, 1),
                         hbm_frac=round(gbs / HBM_PEAK_GBS, 4), useful_flop=flop,
                         mfma_frac=round(flop / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4), splits=call.num_splits,
                         timing="median of per-call events, caches flushed before each call")
        log(f"{name}: {us:.2f} us/call (cold), {gbs:.0f} GB/s on {byts} gathered bytes, "
            f"splits {call.num_splits}")
        del call, inp
        torch.cuda.synchronize()
    return res


BWD_FLOP_PER_PAIR_HEAD = 2 * (3 * 576 + 2 * 512)   # q.k, dO.v, dq, dk (D = 576), dv (512)


def bench_backward(dec_inp, pre_inp, atomic_peak=None):
    """sas_bwd_v1 on the C2 decode and C3 prefill inputs: the forward's out /
    LSE, a random bf16 dO, gradient buffers allocated once (the kernel's own
    time: the cache gradients accumulate across the timed launches). Useful
    FLOP per (token, key, head): 2 x (3 x 576 + 2 x 512) = 5504. Row-gradient
    atomics per launch: one fp32 add per (token, key, head group of
    heads_per_workgroup, channel), counted here (with several KV splits the
    dq shares add atomically too, not counted). The launch's atomic rate
    against the measured fp32 atomic peak is the bound that applies (the FLOP
    rate is far below the MFMA peak)."""
    from dsv4_amd import cases
    from dsv4_amd.api import prepare_sparse_attn_sharedkv_backward, sparse_attn_sharedkv
    res = {"kernel": "sas_bwd64_kernel (64-head workgroups, q in registers; MFMA scores, dq and dkv; "
                     "fp32 atomics for dkv); sas_bwd_kernel for H not a multiple of 64; prefills: the "
                     "window rows' dkv by sas_bwd_win_kernel beside it on a side stream",
           "flop_per_pair_head": BWD_FLOP_PER_PAIR_HEAD}
    for key, inp, steps in (("decode", dec_inp, 50), ("prefill", pre_inp, 3)):
        if inp is None:
            continue
        kw = inp.api_kwargs()
        out, lse = sparse_attn_sharedkv(inp.q, return_softmax_lse=True, **kw)
        g = torch.Generator(device="cuda").manual_seed(21)
        dout = torch.randn(out.shape, device="cuda", generator=g).to(out.dtype)
        pb = prepare_sparse_attn_sharedkv_backward(dout, inp.q, out, lse, **kw)
        ms, _ = time_launches(lambda i, st: pb.launch(st), 1, steps, 1)
        us = ms * 1e3 / steps
        pairs = cases.gathered_rows(inp)
        flop = pairs * inp.cfg.H * BWD_FLOP_PER_PAIR_HEAD
        tfl = flop / (us * 1e-6) / 1e12
        hpw = 64 if inp.cfg.H % 64 == 0 else 32 if inp.cfg.H % 32 == 0 else 16
        D = inp.q.shape[-1]
        # the library's default: the key-major window pass for prefills (at
        # least 64 query tokens per batch), whose window rows take one add
        # per (row, 16-head group, channel) instead of one per (token, row)
        win_pass = inp.q.shape[0] >= 64 * len(inp.q_lens)
        win_pairs, win_rows = 0, 0
        for aq, akv in zip(inp.q_lens, inp.kv_lens):
            wl = inp.cfg.win_left
            win_pairs += sum(min(akv - aq + s, wl) + 1 for s in range(aq) if akv - aq + s >= 0)
            win_rows += akv - max(akv - aq - wl, 0) if aq > 0 else 0
        atomics = pairs * (inp.cfg.H // hpw) * D
        if win_pass:
            atomics = ((pairs - win_pairs) * (inp.cfg.H // hpw) + win_rows * (inp.cfg.H // 16)) * D
        rate = atomics / (us * 1e-6) / 1e9
        res[key] = dict(workload=inp.cfg.name, us_per_call=round(us, 1), useful_flop=flop,
                        tflops=round(tfl, 2), mfma_frac=round(tfl / BF16_PEAK_TFLOPS, 5),
                        heads_per_workgroup=hpw, window_pass=win_pass, fp32_row_atomics=atomics,
                        atomic_g_per_s=round(rate, 1),
                        atomic_frac=round(rate / atomic_peak, 3) if atomic_peak else None,
                        atomic_frac_of="peaks.fp32_atomic_measured_g_per_s")
        if win_pass:
            # the same launch with per-token adds for the window rows too
            del pb
            pb = prepare_sparse_attn_sharedkv_backward(dout, inp.q, out, lse, window_pass=False, **kw)
            ms, _ = time_launches(lambda i, st: pb.launch(st), 1, steps, 1)
            res[key]["us_per_call_per_token_adds"] = round(ms * 1e3 / steps, 1)
        del pb, out, lse, dout
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--rotations", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-traffic", action="store_true")
    ap.add_argument("--no-cache-write", action="store_true")
    ap.add_argument("--no-backward", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the C1 / C4 / C5 decode lines")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured copy / GEMM peaks")
    ap.add_argument("--pmc-pass", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--prefill-pass", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this operator build runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured path)", file=sys.stderr)
        sys.exit(2)
    if args.pmc_pass:
        pmc_pass()
        return
    if args.prefill_pass:
        prefill_pass()
        return

    # counter passes run first, in child processes, before this process
    # touches the GPU
    traffic, traffic_note = (None, "skipped (--no-traffic)")
    if not args.no_traffic:
        traffic, traffic_note = measure_traffic()
        log(f"traffic: {traffic if traffic else traffic_note}")

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
    ns = calls[0].num_splits
    log(f"C2: T={inp.T} gathered rows={rows} bytes={kv_bytes} splits={ns} "
        f"rotations={len(calls)} (touched {len(calls) * kv_bytes / 1e6:.0f} MB)")
    ev_ms, wall_ms = time_launches(lambda i, st: calls[i].launch(st), len(calls),
                                   args.steps, args.warmup)
    us_call = ev_ms * 1e3 / args.steps
    gbs = kv_bytes / (us_call * 1e-6) / 1e9
    log(f"C2 decode: {us_call:.2f} us/call (events), {wall_ms * 1e3 / args.steps:.2f} us wall, "
        f"{gbs:.0f} GB/s")
    # the dominant kernel alone (split kernel, partials left in the workspace)
    sp_ms, sp_wall = time_launches(lambda i, st: calls[i].launch_split(st), len(calls),
                                   args.steps, args.warmup)
    us_split = sp_ms * 1e3 / args.steps
    cb_ms, _ = time_launches(lambda i, st: calls[i].launch_combine(st), len(calls),
                             args.steps, args.warmup)
    us_comb = cb_ms * 1e3 / args.steps
    split_gbs = kv_bytes / (us_split * 1e-6) / 1e9
    log(f"C2 split kernel: {us_split:.2f} us/launch ({sp_wall * 1e3 / args.steps:.2f} us wall), "
        f"{split_gbs:.0f} GB/s; combine {us_comb:.2f} us/launch")
    # the same calls captured once in a HIP graph (16 calls, one per input
    # rotation) and replayed: what a serving loop that replays captured
    # launches pays per call
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for c in calls:
                c.launch(side)
    torch.cuda.synchronize()
    # steady state: the first replays after instantiation run slower, and
    # a replay's host cost (~57 µs for these 32 kernel nodes) stays below
    # the GPU time it enqueues
    reps = max(4, 3 * args.steps // len(calls))
    g_ms, _ = time_launches(lambda i, st: graph.replay(), 1, reps, 8)
    us_graph = g_ms * 1e3 / (reps * len(calls))
    log(f"C2 decode in a HIP graph: {us_graph:.2f} us/call")
    # API wall time (host resolution + launch), reported separately
    from dsv4_amd.api import sparse_attn_sharedkv
    # (200 back-to-back calls on one input set; host seqlens as the
    # reference's callers pass them, then already on the device)
    kw = inp.api_kwargs()
    n_api = 200
    for _ in range(20):
        sparse_attn_sharedkv(inp.q, **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_api):
        sparse_attn_sharedkv(inp.q, **kw)
    torch.cuda.synchronize()
    api_us = (time.perf_counter() - t0) / n_api * 1e6
    kwd = dict(kw, cu_seqlens_q=inp.cu_seqlens_q.cuda(), seqused_kv=inp.seqused_kv.cuda())
    for _ in range(20):
        sparse_attn_sharedkv(inp.q, **kwd)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_api):
        sparse_attn_sharedkv(inp.q, **kwd)
    torch.cuda.synchronize()
    api_dev_us = (time.perf_counter() - t0) / n_api * 1e6
    log(f"API call: {api_us:.1f} us (host seqlens), {api_dev_us:.1f} us (device seqlens)")

    # ---------------- prefill, config 3 --------------------------------------
    prefill = None
    if not args.no_prefill:
        pcfg = cases.CONFIGS["C3"]
        log("building C3 inputs")
        pinp = cases.make_inputs(pcfg, device="cuda")
        prows = cases.gathered_rows(pinp)
        flops = prows * pcfg.H * 2 * (pcfg.D + pcfg.DV)
        pcall = _prepare(pinp)
        pev, _ = time_launches(lambda i, st: pcall.launch(st), 1, args.prefill_steps, 3)
        pus = pev * 1e3 / args.prefill_steps
        tfl = flops / (pus * 1e-6) / 1e12
        prefill = dict(workload="C3 prefill S4096 H64 k512+w128 contiguous", us_per_call=round(pus, 2),
                       tflops=round(tfl, 2), useful_flop=flops, pairs=prows,
                       mfma_frac=round(tfl / BF16_PEAK_TFLOPS, 4), splits=pcall.num_splits)
        log(f"C3 prefill: {pus:.1f} us/call, {tfl:.1f} TFLOP/s ({flops:.4e} useful FLOP)")

    # ---------------- the other decode configs (cold caches) ----------------
    flush_buf = torch.empty(1 << 28, device="cuda").normal_()     # 1 GiB

    def flush():
        flush_buf.sum()

    configs = None
    if not args.no_configs:
        configs = bench_decode_configs(["C1", "C2", "C4", "C5"], 50, flush)

    peaks = None
    if not args.no_peaks:
        peaks = measured_peaks()
        log(f"peaks: copy {peaks['hbm_copy_measured_gbs']} GB/s, "
            f"bf16 GEMM {peaks['bf16_gemm_measured_tflops']} TFLOP/s, "
            f"fp32 atomics {peaks['fp32_atomic_measured_g_per_s']} G/s")

    # ---------------- backward (C2 decode, C3 prefill) ----------------------
    backward = None
    if not args.no_backward:
        backward = bench_backward(inp, pinp if prefill is not None else None,
                                  peaks["fp32_atomic_measured_g_per_s"] if peaks else None)
        for k_ in ("decode", "prefill"):
            if backward.get(k_):
                log(f"backward {k_}: {backward[k_]['us_per_call']:.1f} us/call, "
                    f"{backward[k_]['tflops']:.1f} TFLOP/s, {backward[k_]['atomic_g_per_s']:.1f} G atomics/s")

    # ---------------- paged-KV cache writer (fp8 rows) ------------------------
    cwrite = None
    if not args.no_cache_write:
        cwrite = bench_cache_write(traffic)
        log(cwrite.pop("_log"))

    # ---------------- CPU baseline (oracle on host cores) --------------------
    cpu = None
    if not args.no_cpu:
        n, core_note = usable_cores()
        torch.set_num_threads(n)
        log(f"CPU baseline on {n} threads ({core_note})")
        host = inp.to("cpu")
        cpu_s, reps, spent = cpu_oracle_time(host, min_seconds=10.0, max_reps=1000)
        cpu = dict(value=round(kv_bytes / cpu_s / 1e9, 3), unit="GB/s", cores=n, kind="port",
                   cores_note=core_note, us_per_call=round(cpu_s * 1e6, 1),
                   sample=f"full C2 decode call (32 tokens x 64 heads), median of {reps} calls "
                          f"({spent:.1f} s), torch fp32 oracle")
        if prefill is not None:
            ph = pinp.to("cpu")
            ps, _, _ = cpu_oracle_time(ph)
            cpu["prefill_tflops"] = round(prefill["useful_flop"] / ps / 1e12, 4)
            cpu["prefill_s"] = round(ps, 2)
            cpu["prefill_sample"] = f"one full C3 pass ({pinp.T} tokens)"

    tr = None
    if traffic:
        tr = round(traffic["FETCH_SIZE"]["split_bytes"] + traffic["WRITE_SIZE"]["split_bytes"])
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
        "decode_us_per_call_graph": round(us_graph, 3),
        "split_kernel_us": round(us_split, 3),
        "combine_kernel_us": round(us_comb, 3),
        "num_splits": ns,
        "api_us_per_call": round(api_us, 1),
        "api_us_per_call_device_seqlens": round(api_dev_us, 1),
        "gathered_kv_bytes": kv_bytes,
        "roofline": {"bound": "hbm", "achieved": round(split_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(split_gbs / HBM_PEAK_GBS, 4), "traffic": tr,
                     "kernel": f"{SPLIT_KERNEL} (C2 split-KV forward, {ns} splits)",
                     "traffic_detail": traffic if traffic else traffic_note},
        "prefill": prefill,
        "decode_configs": configs,
        "peaks": peaks,
        "cache_write": cwrite,
        "backward": backward,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
