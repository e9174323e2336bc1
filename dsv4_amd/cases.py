"""Workload definitions and seeded synthetic inputs.

``CONFIGS`` are the five workloads the operator is measured and checked on
(decode B1/H16, batched decode B32/H64, 4K prefill, ragged MTP decode,
long-context fp8 decode). ``REF_SCENARIOS`` are the reference test suite's
six cases (test_sparse_attn_sharedkv.py:81-220: scfa/swa/cfa x decode/prefill,
TND, B=1, N1=64, D=512, block 128).

Seeds (fixed): Q 0, KV 1, indices 2, sinks 3, block tables 4, context
lengths / ragged query lengths 5. All data is synthetic N(0,1).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, replace
from typing import List, Optional

import torch

from . import paged

SEED_Q, SEED_KV, SEED_IDX, SEED_SINK, SEED_BT, SEED_LEN = 0, 1, 2, 3, 4, 5


@dataclass(frozen=True)
class Config:
    name: str
    B: int
    H: int
    D: int = 576                 # q/k head dim (512 latent + 64 rope)
    DV: int = 512                # output / V width (first DV channels)
    sq: tuple = (1,)             # choices for per-sequence query length
    ctx: tuple = (2048, 2048)    # per-sequence kv length, uniform [lo, hi]
    K: int = 0                   # top-k (SCFA); 0 for SWA/CFA
    cmp_ratio: int = 4
    scenario: int = 3            # 1 SWA, 2 CFA, 3 SCFA
    block_size: int = 64
    shuffle: bool = True         # shuffled physical blocks vs identity table
    fp8: bool = False
    prefill: bool = False        # S_q == S_kv (queries are the whole sequence)
    win_left: int = 127
    softmax_scale: Optional[float] = None
    notes: str = ""

    @property
    def scale(self) -> float:
        return self.softmax_scale if self.softmax_scale is not None else 1.0 / math.sqrt(self.D)


CONFIGS = {
    "C1": Config("C1", B=1, H=16, ctx=(2048, 2048), K=64,
                 notes="decode B1 H16 top-k 64 + window 128, 2048 raw / 512 cmp"),
    "C2": Config("C2", B=32, H=64, ctx=(8192, 32768), K=512,
                 notes="batched decode B32 H64 top-k 512 + window 128, ctx U[8K,32K]"),
    "C3": Config("C3", B=1, H=64, ctx=(4096, 4096), K=512, prefill=True, shuffle=False,
                 notes="prefill S4096 H64 causal window 128 + top-k 512, contiguous KV"),
    "C4": Config("C4", B=16, H=128, sq=(1, 2, 4), ctx=(1024, 65536), K=1024,
                 notes="ragged MTP decode B16 S_q in {1,2,4} H128 top-k 1024"),
    "C5": Config("C5", B=8, H=128, ctx=(131072, 131072), K=1024, cmp_ratio=128, fp8=True,
                 notes="long-context fp8 decode B8 H128 ctx 128K r128 top-k 1024"),
}

_REF_COMMON = dict(H=64, D=512, DV=512, block_size=128, softmax_scale=0.04419417)
REF_SCENARIOS = {
    "scfa_decode": Config("scfa_decode", B=1, ctx=(8193, 8193), K=512, cmp_ratio=4,
                          scenario=3, **_REF_COMMON),
    "swa_decode": Config("swa_decode", B=1, ctx=(8193, 8193), K=0, cmp_ratio=4,
                         scenario=1, **_REF_COMMON),
    "cfa_decode": Config("cfa_decode", B=1, ctx=(8193, 8193), K=0, cmp_ratio=128,
                         scenario=2, **_REF_COMMON),
    "scfa_prefill": Config("scfa_prefill", B=1, ctx=(8192, 8192), K=512, cmp_ratio=4,
                           scenario=3, prefill=True, **_REF_COMMON),
    "swa_prefill": Config("swa_prefill", B=1, ctx=(8192, 8192), K=0, cmp_ratio=4,
                          scenario=1, prefill=True, **_REF_COMMON),
    "cfa_prefill": Config("cfa_prefill", B=1, ctx=(8192, 8192), K=0, cmp_ratio=128,
                          scenario=2, prefill=True, **_REF_COMMON),
}


def shrink(cfg: Config, ctx: int, name: Optional[str] = None) -> Config:
    """Same shape family at a smaller context (for CPU-checkable sizes)."""
    return replace(cfg, name=name or f"{cfg.name}@{ctx}", ctx=(ctx, ctx))


def seq_lengths(cfg: Config):
    """Per-sequence (query lengths, kv lengths) from the length seed."""
    g = torch.Generator().manual_seed(SEED_LEN)
    lo, hi = cfg.ctx
    if hi > lo:
        kv = torch.randint(lo, hi + 1, (cfg.B,), generator=g).tolist()
    else:
        kv = [lo] * cfg.B
    if cfg.prefill:
        q = list(kv)
    elif len(cfg.sq) > 1:
        choice = torch.randint(0, len(cfg.sq), (cfg.B,), generator=g).tolist()
        q = [cfg.sq[c] for c in choice]
    else:
        q = [cfg.sq[0]] * cfg.B
    return q, kv


@dataclass
class Inputs:
    cfg: Config
    q: torch.Tensor                       # [T, H, D] bf16
    ori_kv: torch.Tensor                  # [nb, bs, 1, D] bf16 or uint8 [.., 656]
    ori_bt: torch.Tensor                  # [B, w] int32
    cmp_kv: Optional[torch.Tensor]
    cmp_bt: Optional[torch.Tensor]
    cmp_idx: Optional[torch.Tensor]       # [T, 1, K] int32
    cu_seqlens_q: torch.Tensor            # [B+1] int32 (CPU)
    seqused_kv: torch.Tensor              # [B] int32 (CPU)
    sinks: torch.Tensor                   # [H] fp32
    q_lens: List[int] = field(default_factory=list)
    kv_lens: List[int] = field(default_factory=list)

    @property
    def T(self) -> int:
        return int(self.q.shape[0])

    def to(self, device) -> "Inputs":
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return replace(self, q=mv(self.q), ori_kv=mv(self.ori_kv), ori_bt=mv(self.ori_bt),
                       cmp_kv=mv(self.cmp_kv), cmp_bt=mv(self.cmp_bt), cmp_idx=mv(self.cmp_idx),
                       sinks=mv(self.sinks))

    def api_kwargs(self) -> dict:
        c = self.cfg
        return dict(
            ori_kv=self.ori_kv, cmp_kv=self.cmp_kv, cmp_sparse_indices=self.cmp_idx,
            ori_block_table=self.ori_bt, cmp_block_table=self.cmp_bt,
            cu_seqlens_q=self.cu_seqlens_q, seqused_kv=self.seqused_kv, sinks=self.sinks,
            softmax_scale=c.scale, cmp_ratio=c.cmp_ratio if c.scenario >= 2 else None,
            ori_win_left=c.win_left, layout_q="TND", layout_kv="PA_ND",
        )


def topk_indices(q_lens, kv_lens, K, cmp_ratio, gen) -> torch.Tensor:
    """Prefix-valid top-k per query row: distinct, uniform without replacement
    from ``[0, threshold)``, -1 padded (same rule as golden.py:442-473)."""
    rows = []
    for ql, kl in zip(q_lens, kv_lens):
        for s in range(ql):
            thr = max(0, (kl - ql + s + 1) // cmp_ratio)
            row = torch.full((K,), -1, dtype=torch.int32)
            take = min(thr, K)
            if take > 0:
                if thr <= 4 * K:
                    sel = torch.randperm(thr, generator=gen)[:take]
                else:   # sparse draw without materialising a huge permutation
                    sel = torch.unique(torch.randint(0, thr, (2 * take,), generator=gen))
                    while sel.numel() < take:
                        more = torch.randint(0, thr, (take,), generator=gen)
                        sel = torch.unique(torch.cat([sel, more]))
                    sel = sel[torch.randperm(sel.numel(), generator=gen)[:take]]
                row[:take] = sel.to(torch.int32)
            rows.append(row)
    return torch.stack(rows).unsqueeze(1) if rows else torch.empty((0, 1, K), dtype=torch.int32)


def make_inputs(cfg: Config, device="cpu") -> Inputs:
    """Seeded synthetic inputs for ``cfg``; large tensors are drawn on ``device``."""
    q_lens, kv_lens = seq_lengths(cfg)
    T = sum(q_lens)
    dev = torch.device(device)

    def gen(seed):
        return torch.Generator(device=dev).manual_seed(seed)

    q = paged.fill_normal((T, cfg.H, cfg.D), torch.bfloat16, gen(SEED_Q), dev)
    sinks = torch.randn(cfg.H, generator=torch.Generator().manual_seed(SEED_SINK)).float().to(dev)
    gbt = torch.Generator().manual_seed(SEED_BT)
    ori_bt, ori_nb = paged.random_block_table(kv_lens, cfg.block_size, gbt, shuffle=cfg.shuffle)
    gkv = gen(SEED_KV)
    ori = paged.fill_normal((ori_nb, cfg.block_size, 1, cfg.D), torch.bfloat16, gkv, dev)
    cmp_kv = cmp_bt = cmp_idx = None
    if cfg.scenario >= 2:
        cmp_lens = [k // cfg.cmp_ratio for k in kv_lens]
        cmp_bt, cmp_nb = paged.random_block_table(cmp_lens, cfg.block_size, gbt,
                                                  shuffle=cfg.shuffle)
        cmp_kv = paged.fill_normal((cmp_nb, cfg.block_size, 1, cfg.D), torch.bfloat16, gkv, dev)
    if cfg.scenario == 3:
        cmp_idx = topk_indices(q_lens, kv_lens, cfg.K, cfg.cmp_ratio,
                               torch.Generator().manual_seed(SEED_IDX))
    if cfg.fp8:
        ori = paged.quantize_kv_fp8(ori)
        if cmp_kv is not None:
            cmp_kv = paged.quantize_kv_fp8(cmp_kv)
    cu = torch.tensor([0] + list(torch.tensor(q_lens).cumsum(0).tolist()), dtype=torch.int32)
    mv = lambda t: None if t is None else t.to(dev)  # noqa: E731
    return Inputs(cfg=cfg, q=q, ori_kv=ori, ori_bt=mv(ori_bt), cmp_kv=cmp_kv, cmp_bt=mv(cmp_bt),
                  cmp_idx=mv(cmp_idx), cu_seqlens_q=cu,
                  seqused_kv=torch.tensor(kv_lens, dtype=torch.int32), sinks=sinks,
                  q_lens=q_lens, kv_lens=kv_lens)


def gathered_rows(inp: Inputs) -> int:
    """Valid (token, key) pairs: window rows + valid compressed rows."""
    c = inp.cfg
    total = 0
    idx = inp.cmp_idx.cpu() if inp.cmp_idx is not None else None
    t = 0
    for ql, kl in zip(inp.q_lens, inp.kv_lens):
        for s in range(ql):
            sg = kl - ql + s
            total += max(0, sg - max(sg - c.win_left, 0) + 1) if sg >= 0 else 0
            thr = max(0, (sg + 1) // c.cmp_ratio)
            if c.scenario == 2:
                total += thr
            elif c.scenario == 3:
                r = idx[t, 0]
                total += int(((r >= 0) & (r < thr)).sum())
            t += 1
    return total


# Reference suite block pools (test_sparse_attn_sharedkv.py:81-220) and the
# fast-loop shrink (test_sparse_attn_sharedkv_fast.py:72-99).
_REF_BLOCKS = {"scfa": (65, 17, 128), "cfa": (65, 17, 128), "swa": (65, 1, 1)}


def ref_case(name: str, dtype=torch.bfloat16, s1: Optional[int] = None, seed: int = 42) -> Inputs:
    """The reference suite's case ``name`` (``scfa_decode`` ... ``cfa_prefill``),
    optionally shrunk to ``s1`` query tokens, with its data: the same random
    sources in the same order as test_sparse_attn_sharedkv.py:238-391
    (U(-10,10) q and raw KV, U(-5,10) compressed KV, U(-1,1) sinks, numpy
    block permutations seeded ``seed`` / ``seed+1``, indices seeded ``seed+7``)."""
    import numpy as np

    cfg = REF_SCENARIOS[name]
    kind = name.split("_")[0]
    nb1, nb2, bs2 = _REF_BLOCKS[kind]
    kv = cfg.ctx[0]
    S1 = kv if cfg.prefill else 1
    if s1 is not None:
        S1 = kv = s1
        nb1 = -(-s1 // cfg.block_size) + 2
        if cfg.scenario >= 2:
            nb2 = max(1, -(-(s1 // cfg.cmp_ratio) // bs2)) + 1
    torch.manual_seed(seed)
    np.random.seed(seed)
    q = (torch.rand((S1, cfg.H, cfg.D)) * 20 - 10).to(dtype)
    ori_pa, ori_bt, _ = paged.gen_ori_kv_paged(
        B=1, N2=1, D=cfg.D, block_num=nb1, block_size=cfg.block_size, seqused_kv=[kv],
        dtype=dtype, data_range=(-10, 10), rng=np.random.default_rng(seed))
    cmp_pa = cmp_bt = idx = None
    cu = torch.tensor([0, S1], dtype=torch.int32)
    if cfg.scenario >= 2:
        cmp_pa, cmp_bt, _, _ = paged.gen_cmp_kv_paged(
            B=1, N2=1, D=cfg.D, block_num=nb2, block_size=bs2, seqused_kv=[kv],
            cmp_ratio=cfg.cmp_ratio, dtype=dtype, data_range=(-5, 10),
            rng=np.random.default_rng(seed + 1))
    if cfg.scenario == 3:
        g = torch.Generator()
        g.manual_seed(seed + 7)
        idx = paged.gen_cmp_sparse_indices_tnd(B=1, T1=S1, N2=1, K=cfg.K, cu_seqlens_q=cu,
                                               seqused_kv=[kv], cmp_ratio=cfg.cmp_ratio, rng=g)
    sinks = (torch.rand(cfg.H) * 2 - 1).to(torch.float32)
    c = replace(cfg, name=f"{name}@{S1}" if s1 else name, ctx=(kv, kv))
    return Inputs(cfg=c, q=q, ori_kv=ori_pa, ori_bt=ori_bt, cmp_kv=cmp_pa, cmp_bt=cmp_bt,
                  cmp_idx=idx, cu_seqlens_q=cu, seqused_kv=torch.tensor([kv], dtype=torch.int32),
                  sinks=sinks, q_lens=[S1], kv_lens=[kv])
