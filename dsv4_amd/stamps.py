"""Phase stamps of the split-KV forward kernel (measurement only).

    python -m dsv4_amd.stamps [C2 C5 C2:4x8x8 ...]

Builds an instrumented copy of ``sas_fwd.hip`` (into ``dsv4_amd/_build/stamp``,
next to the objects ``python -m dsv4_amd.build`` leaves there) in which
thread 0 of every workgroup of ``sas_fwd_kernel`` records when its phases end
into a device array, then launches each named decode workload's split kernel
through that library (the product library ``libsas.so`` is not touched; the
launch arguments come from the normal prepared call) and prints the median
workgroup's phases in microseconds.

Phases: ``resolve`` (index and block-table round trips, compaction),
``qsync`` (query rows in place), ``prologue`` (the ring's first DMA issue,
or for fp8 rows the first row fetch and store), ``first`` (wait for the first
step's rows), then summed over the steps: ``wait`` (later steps' row waits
and step barriers), ``qk``, ``xbar`` (the S-half exchange barrier),
``smax`` (S read-back and softmax), ``pv``, ``prep`` (DMA row addresses) or
for fp8 rows ``fstore`` / ``fload``; ``epi`` (merge, staging, stores) and
``wg`` (the whole workgroup). Workgroup phases come from ``s_memrealtime``
(100 MHz); step phases from ``s_memtime`` (the shader clock), converted with
the clock rate each workgroup measures between its first and last stamp.
The stamps add their own waits (each reads a counter through the scalar
memory path), so a stamped workgroup runs somewhat longer than an unstamped
one. Only the LDS streaming kernel (``sas_fwd_kernel``, the non-pipelined
step loop) is instrumented step by step; the pipelined loops report their
step phases as one total.
"""

from __future__ import annotations

import ctypes
import os
import shutil
import sys
from dataclasses import replace

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build", "stamp")
LIB = os.path.join(OUT, "libsas_stamp.so")
ROWS = 16384   # workgroups recorded
SLOTS = 16     # values per workgroup


def _instrument(src: str) -> str:
    """The forward source with stamps added (each edit checked to apply)."""
    def rep(s, old, new, first=False):
        n = s.count(old)
        assert n == 1 or (first and n > 1), f"stamp edit does not apply to the source: {old[:60]!r}"
        return s.replace(old, new, 1)
    s = src
    s = rep(s, '#include "sas_kern.h"\n',
            '#include "sas_kern.h"\n'
            f'__device__ unsigned long long sas_stamp_buf[{ROWS * SLOTS}];\n'
            'static __device__ __forceinline__ unsigned long long RT() { return __builtin_amdgcn_s_memrealtime(); }\n'
            'static __device__ __forceinline__ unsigned long long CT() { return __builtin_amdgcn_s_memtime(); }\n')
    s = rep(s, "  float m_run, l_run;\n  f32x4 acc[C::NTL];",
            "  float m_run, l_run;\n  f32x4 acc[C::NTL];\n"
            "  unsigned long long ph[8] = {0, 0, 0, 0, 0, 0, 0, 0};\n  unsigned long long c2 = 0, pro = 0;")
    # compute(): QK, exchange barrier, softmax, P.V of the channel-split step
    s = rep(s, """    if constexpr (C::F8R) {
      if (live) qk8(sl, sacc, dma);
    } else {
      if (live) qk(sl, sacc, sodd, dma);
    }
    if constexpr (C::QS) {""", """    const unsigned long long ta = CT();
    if constexpr (C::F8R) {
      if (live) qk8(sl, sacc, dma);
    } else {
      if (live) qk(sl, sacc, sodd, dma);
    }
    const unsigned long long tb = CT();
    ph[1] += tb - ta;
    if constexpr (C::QS) {""")
    s = rep(s, """      lds_barrier();
      if (live) {
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt) {
          if constexpr (C::Q2) sacc[mt] = xs[piece(hw, mt, 0)] + xs[piece(hw, mt, 1)];""",
            """      lds_barrier();
      const unsigned long long tc = CT();
      ph[2] += tc - tb;
      if (live) {
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt) {
          if constexpr (C::Q2) sacc[mt] = xs[piece(hw, mt, 0)] + xs[piece(hw, mt, 1)];""")
    s = rep(s, """        for (int e = 0; e < kSmaxB; ++e) smax_b(e, sv, lsum, pk);
        if constexpr (C::F8R) pv8(sl, pk);
        else pv(sl, pk, [](int) {});
      }
      return;""", """        for (int e = 0; e < kSmaxB; ++e) smax_b(e, sv, lsum, pk);
        const unsigned long long td = CT();
        ph[3] += td - tc;
        if constexpr (C::F8R) pv8(sl, pk);
        else pv(sl, pk, [](int) {});
        ph[4] += CT() - td;
      }
      return;""")
    # step loop: waits, DMA address reads; fp8 row store / fetch
    s = rep(s, """      const int after = it < nsteps ? min(C::NST - 2, nsteps - 1 - it) : 0;
      wait_steps(after);
      step_sync();
      if (it < nsteps || C::QS) {
        const bool more = it + C::NST - 1 < nsteps;
        Dma d;
        if (more) prep(d, (J + C::NST - 1) % C::NST, it + C::NST - 1);""",
            """      const int after = it < nsteps ? min(C::NST - 2, nsteps - 1 - it) : 0;
      const unsigned long long t0 = CT();
      if (it == 0) pro = t0 - c2;
      wait_steps(after);
      step_sync();
      {
        const unsigned long long dt = CT() - t0;
        ph[0] += dt;
        if (it == 0) ph[7] = dt;
      }
      if (it < nsteps || C::QS) {
        const bool more = it + C::NST - 1 < nsteps;
        Dma d;
        const unsigned long long tp = CT();
        if (more) {
          prep(d, (J + C::NST - 1) % C::NST, it + C::NST - 1);
          wait_lgkm0();
        }
        ph[5] += CT() - tp;""")
    s = rep(s, """      step_sync();
      if (it < nsteps || C::QS) compute(slot(J), it, [](int) {});
      if (it + 1 < nsteps) fstore((J + 1) % C::NST);
      if (it + 2 < nsteps) fload(it + 2);""",
            """      const unsigned long long t0 = CT();
      if (it == 0) pro = t0 - c2;
      step_sync();
      {
        const unsigned long long dt = CT() - t0;
        ph[0] += dt;
        if (it == 0) ph[7] = dt;
      }
      if (it < nsteps || C::QS) compute(slot(J), it, [](int) {});
      const unsigned long long t1 = CT();
      if (it + 1 < nsteps) fstore((J + 1) % C::NST);
      const unsigned long long t2 = CT();
      ph[5] += t2 - t1;
      if (it + 2 < nsteps) fload(it + 2);
      ph[6] += CT() - t2;""")
    # workgroup phases (sas_fwd_kernel only: the first match from its body on)
    i = s.index("sas_fwd_kernel(const FwdParams p) {")
    head, tail = s[:i], s[i:]
    tail = rep(tail, "  const int item = item_index(p);\n  if (item < 0) return;", first=True, new=(
               "  const int item = item_index(p);\n  if (item < 0) return;\n"
               "  const unsigned long long s0 = RT(), c0 = CT();"))
    tail = rep(tail, "  const int nvalid = __builtin_amdgcn_readfirstlane(k.nvalid);",
               "  const int nvalid = __builtin_amdgcn_readfirstlane(k.nvalid);\n"
               "  const unsigned long long s1 = RT();", first=True)
    tail = rep(tail, "  f.m_run = seed_sink ? sink * kLog2e : -INFINITY;",
               "  const unsigned long long s2 = RT();\n  f.c2 = CT();\n"
               "  f.m_run = seed_sink ? sink * kLog2e : -INFINITY;")
    tail = rep(tail, "  epilogue<HW, NW, C::CS, QT>(p, k, tid, wave, lane, f.m_run, f.l_run, f.acc);\n}",
               "  const unsigned long long s4 = RT();\n"
               "  epilogue<HW, NW, C::CS, QT>(p, k, tid, wave, lane, f.m_run, f.l_run, f.acc);\n"
               "  const unsigned long long s5 = RT(), c5 = CT();\n"
               "  if (tid == 0) {\n"
               f"    unsigned long long* o = sas_stamp_buf + (size_t)blockIdx.x * {SLOTS};\n"
               "    o[0] = s0; o[1] = s1; o[2] = s2; o[3] = c5 - c0; o[4] = s4; o[5] = s5;\n"
               "    o[6] = f.pro; o[7] = (unsigned long long)f.nsteps;\n"
               "    for (int i = 0; i < 8; ++i) o[8 + i] = f.ph[i];\n  }\n}")
    s = head + tail
    s += ('\nextern "C" int sas_stamp_read(void* dst, size_t bytes) {\n'
          '  return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(sas_stamp_buf), bytes, 0, hipMemcpyDeviceToHost);\n}\n'
          'extern "C" int sas_stamp_clear() {\n'
          f'  static unsigned long long z[{ROWS * SLOTS}];\n'
          '  return (int)hipMemcpyToSymbol(HIP_SYMBOL(sas_stamp_buf), z, sizeof(z), 0, hipMemcpyHostToDevice);\n}\n')
    return s


def build(verbose: bool = False) -> str:
    """Compile the instrumented library; the other objects are the product
    build's (built first when missing)."""
    from . import build as b
    objs = [os.path.join(HERE, "_build", os.path.splitext(src)[0] + ".o") for src, _ in b.SOURCES
            if src != "sas_fwd.hip"]
    if not all(os.path.exists(o) for o in objs):
        b.build(verbose=verbose)
    src_dir = os.path.join(OUT, "src")
    shutil.rmtree(OUT, ignore_errors=True)
    os.makedirs(src_dir)
    for f in os.listdir(b.CSRC):
        shutil.copy(os.path.join(b.CSRC, f), src_dir)
    # the copies include the public header from their own location
    inc = os.path.join(os.path.dirname(HERE), "include")
    for f in os.listdir(src_dir):
        p = os.path.join(src_dir, f)
        with open(p) as fh:
            t = fh.read().replace('"../../include/', '"' + inc + "/")
        with open(p, "w") as fh:
            fh.write(t)
    fwd = os.path.join(src_dir, "sas_fwd.hip")
    with open(fwd) as fh:
        text = _instrument(fh.read())
    with open(fwd, "w") as fh:
        fh.write(text)
    obj = os.path.join(OUT, "sas_fwd_stamp.o")
    extra = dict(b.SOURCES)["sas_fwd.hip"]
    b._run([b.hipcc(), *b.HIP_FLAGS, *extra, "-c", "-o", obj, fwd], verbose)
    b._run([b.hipcc(), *b.HIP_FLAGS, "-shared", "-o", LIB, obj, *objs], verbose)
    return LIB


def run(specs, reps: int = 6, lib: str = LIB) -> list:
    """Median phases (µs) of the median workgroup for each spec
    ``NAME[:HWxNWxNS]`` (head waves x waves x splits, else the planner's)."""
    import numpy as np
    import torch

    from . import _lib, cases
    from .api import prepare_sparse_attn_sharedkv
    L = ctypes.CDLL(lib)
    L.sas_fwd_v1.argtypes = [ctypes.POINTER(_lib.SasFwdArgs), ctypes.c_void_p]
    L.sas_stamp_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    buf = np.zeros((ROWS, SLOTS), dtype=np.uint64)
    out = []
    for spec in specs:
        name, _, plan = spec.partition(":")
        kw = {}
        if plan:
            hw, nw, ns = map(int, plan.split("x"))
            kw = dict(head_waves=hw, waves=nw, num_splits=ns)
        inp0 = cases.make_inputs(cases.CONFIGS[name], device="cuda")
        # 8 copies of the inputs in distinct memory: 7 launches on other
        # copies run between the stamped ones (the caches hold other rows)
        rots = [inp0] + [replace(inp0, q=inp0.q.clone(), ori_kv=inp0.ori_kv.clone(),
                                 cmp_kv=None if inp0.cmp_kv is None else inp0.cmp_kv.clone())
                         for _ in range(7)]
        calls = [prepare_sparse_attn_sharedkv(r.q, **r.api_kwargs(), **kw) for r in rots]
        st = torch.cuda.current_stream()

        def launch(c):
            c.args.flags = _lib.SAS_FWD_NO_COMBINE
            rc = L.sas_fwd_v1(ctypes.byref(c.args), ctypes.c_void_p(st.cuda_stream))
            c.args.flags = 0
            assert rc == 0, f"stamped launch failed ({rc})"
        for c in calls:
            launch(c)
        torch.cuda.synchronize()
        rows = []
        for _ in range(reps):
            for i, c in enumerate(calls):
                if i == len(calls) - 1:
                    torch.cuda.synchronize()
                    assert L.sas_stamp_clear() == 0
                launch(c)
            torch.cuda.synchronize()
            assert L.sas_stamp_read(buf.ctypes.data, buf.nbytes) == 0
            s = buf.astype(np.int64)
            s = s[s[:, 0] > 0]
            ghz = float(np.median(s[:, 3] / np.maximum(s[:, 5] - s[:, 0], 1))) * 0.1
            cyc = lambda v: float(np.median(v)) / (ghz * 1e3)   # noqa: E731
            rt = lambda v: float(np.median(v)) * 0.01           # noqa: E731
            rows.append(dict(
                resolve=rt(s[:, 1] - s[:, 0]), qsync=rt(s[:, 2] - s[:, 1]), prologue=cyc(s[:, 6]),
                first=cyc(s[:, 15]), wait=cyc(s[:, 8] - s[:, 15]), qk=cyc(s[:, 9]), xbar=cyc(s[:, 10]),
                smax=cyc(s[:, 11]), pv=cyc(s[:, 12]), prep_or_fstore=cyc(s[:, 13]), fload=cyc(s[:, 14]),
                steps=rt(s[:, 4] - s[:, 2]), epi=rt(s[:, 5] - s[:, 4]), wg=rt(s[:, 5] - s[:, 0]),
                ghz=ghz, nsteps=float(np.median(s[:, 7])), workgroups=len(s)))
        med = {k: float(np.median([r[k] for r in rows])) for k in rows[0]}
        out.append((spec, calls[0].num_splits, med))
        del calls, rots, inp0
        torch.cuda.synchronize()
    return out


def main(argv=None) -> None:
    specs = (argv if argv is not None else sys.argv[1:]) or ["C2", "C5"]
    build()
    for spec, ns, med in run(specs):
        print(f"{spec} (splits {ns}): " + " ".join(f"{k}={v:.2f}" for k, v in med.items()), flush=True)


if __name__ == "__main__":
    main()
