"""ORACLE (test infrastructure only; never imported by the product path).

CPU restatement of the reference's attention golden
(sparse_attn_sharedkv_tilelang/golden.py:28-244) in torch fp32:

* per query token ``(b, s)``: ``s_global = act_kv - act_q + s`` (golden.py:125);
* window rows ``[max(s_global - win_left, 0), s_global]`` (golden.py:128-131);
* compressed rows from the top-k list, walked in order, stopping at the first
  ``-1`` and looking only at the first ``min(K, threshold)`` entries, keeping
  ``0 <= idx < threshold = floor((s_global + 1) / cmp_ratio)``
  (golden.py:41-66); CFA takes all compressed rows below the threshold
  (golden.py:146-150);
* online softmax over 512-row tiles, window tiles first, seeded with
  ``(max, sum) = (sink_h, 1)``; ``p`` is rounded to the query dtype before
  ``p @ V`` (golden.py:156-196); ``out = acc / sum`` in the query dtype and
  ``lse = max + ln(sum)`` in fp32 (golden.py:198-200).

Generalisations for the measured workloads: ``D_qk`` may exceed ``D_v`` (the
V rows are the first ``D_v`` channels of the shared K=V row; since ``p @ V``
is column-separable this equals golden at ``D_qk`` sliced to ``D_v``), any
head count, and fp8 caches (dequantised to fp32 first, which is the stated
comparison for quantised caches).

Pins (tests/test_oracle.py): the closed-form one-shot softmax with a sink
(golden.py:207-244, itself pinned by the brute-force fp64 mask-matrix form
below and by the online-softmax worked example, out 40.038 without sink and
38.813 with sink 2), gathering through shuffled block tables == gathering
from the dense tensor (golden.py:247-268), column separability of ``D_v``.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

GOLDEN_S2_TILE = 512


def _cmp_rows(idx_row: Sequence[int], threshold: int, cmp_len: int) -> list:
    """Valid compressed positions for one query row (golden.py:41-62)."""
    K = len(idx_row)
    rows = []
    for i in range(min(K, max(threshold, 0))):
        j = int(idx_row[i])
        if j == -1:
            break
        if j >= threshold or j >= cmp_len or j < 0:
            continue
        rows.append(j)
    return rows


def _attend(q: torch.Tensor, tiles, sinks: torch.Tensor, scale: float, dtype, dv: int,
            exact: bool = False, scores_fp64: bool = False):
    """Chunked sink-seeded online softmax for one token (golden.py:156-200).

    ``q`` [G, D] fp32, ``tiles`` list of fp32 [n, D] (already in walk order).
    Returns (out [G, dv] in ``dtype``, lse [G] fp32). With ``exact`` the same
    walk runs in fp64 with no rounding of ``p`` or of the output (a reference
    point for how far golden's own bf16/fp16 roundings move it). With
    ``scores_fp64`` the fp32 walk is unchanged except that ``q k^T`` is
    evaluated in fp64 and rounded once to fp32: an equally valid fp32 score
    (another summation order), used to measure how much golden's output
    depends on the order in which its scores are summed.
    """
    G = q.shape[0]
    wt = torch.float64 if exact else torch.float32
    q = q.to(wt)
    m = sinks.to(wt).clone()
    l = torch.ones(G, dtype=wt)
    acc = torch.zeros((G, dv), dtype=wt)
    for k in tiles:
        if k.shape[0] == 0:
            continue
        k = k.to(wt)
        sc = ((q.double() @ k.double().T).to(wt) if scores_fp64 else q @ k.T) * scale
        m_new = torch.maximum(m, sc.amax(dim=1))
        alpha = torch.exp(m - m_new)
        p = torch.exp(sc - m_new.unsqueeze(1))
        l = alpha * l + p.sum(dim=1)
        pr = p if exact else p.to(dtype).to(torch.float32)
        acc = acc * alpha.unsqueeze(1) + pr @ k[:, :dv]
        m = m_new
    o = acc / l.unsqueeze(1)
    return (o if exact else o.to(dtype)), m + torch.log(l)


def _tiles(rows: torch.Tensor, tile: int):
    return [rows[i:i + tile] for i in range(0, rows.shape[0], tile)]


def golden_bnsd(q_bnsd, ori_k_bnsd, sinks, *, act_q_lens, act_kv_lens, softmax_scale,
                cmp_k_bnsd=None, cmp_sparse_indices=None, cmp_ratio=None, ori_win_left=127,
                dv: Optional[int] = None, s2_tile: int = GOLDEN_S2_TILE):
    """Dense-layout oracle with the signature of golden.py:69-86 (N2 = 1).

    Returns ``(out [B, N1, S1, dv], lse [B, N1, S1])``; padded ``(b, s)``
    slots stay zero (golden.py:97).
    """
    B, N1, S1, D = q_bnsd.shape
    dv = D if dv is None else dv
    dtype = q_bnsd.dtype
    out = torch.zeros((B, N1, S1, dv), dtype=dtype)
    lse = torch.zeros((B, N1, S1), dtype=torch.float32)
    sinks = sinks.float().cpu()
    for b in range(B):
        aq, akv = int(act_q_lens[b]), int(act_kv_lens[b])
        for s in range(aq):
            sg = akv - aq + s
            # window [max(sg - win_left, 0), sg]: empty for sg < 0, as the
            # reference kernel's mask idx <= s_global gives (kernel.py:273-276).
            # golden.py:128-131 slices ori_k[left:sg + 1], which for
            # sg < -1 ends at a negative index and takes rows from the end of
            # the cache (a slicing artefact, not the operator's semantics).
            win = ori_k_bnsd[b, 0, max(sg - ori_win_left, 0):max(sg + 1, 0)].float()
            parts = _tiles(win, s2_tile) if win.shape[0] else []
            if cmp_k_bnsd is not None:
                thr = (sg + 1) // cmp_ratio
                if cmp_sparse_indices is not None:
                    sel = _cmp_rows(cmp_sparse_indices[b, s, 0].tolist(), thr, akv // cmp_ratio)
                    crow = cmp_k_bnsd[b, 0, sel].float() if sel else torch.zeros((0, D))
                else:
                    crow = cmp_k_bnsd[b, 0, :max(thr, 0)].float()
                parts += _tiles(crow, s2_tile)
            o, l_ = _attend(q_bnsd[b, :, s].float(), parts, sinks, softmax_scale, dtype, dv)
            out[b, :, s] = o
            lse[b, :, s] = l_
    return out, lse


def _paged_rows(kv, bt_row, positions, dequant):
    """Rows ``positions`` of one sequence through its block table row."""
    if len(positions) == 0:
        width = 576 if kv.dtype == torch.uint8 else kv.shape[-1]
        return torch.zeros((0, width), dtype=torch.float32)
    bs = kv.shape[1]
    pos = torch.as_tensor(positions, dtype=torch.long)
    phys = bt_row.cpu()[pos // bs].long()
    rows = kv[phys.to(kv.device), (pos % bs).to(kv.device), 0].cpu()  # caches may live on a GPU
    return dequant(rows) if dequant is not None else rows.float()


def golden_paged(q, *, ori_kv, ori_block_table, cu_seqlens_q, seqused_kv, sinks,
                 softmax_scale, cmp_kv=None, cmp_block_table=None, cmp_sparse_indices=None,
                 cmp_ratio=None, ori_win_left=127, dv=512, dequant=None, tokens=None,
                 s2_tile: int = GOLDEN_S2_TILE, exact: bool = False, scores_fp64: bool = False):
    """TND / paged-cache oracle: same math as :func:`golden_bnsd`, rows read
    through block tables (only the rows a token touches are materialised).

    ``q`` [T, H, D]; caches ``[nb, bs, 1, D]`` (or uint8 fp8 rows with
    ``dequant``); ``cmp_sparse_indices`` [T, 1, K] (SCFA) or None with
    ``cmp_kv`` given (CFA). ``tokens`` restricts the computation to a subset
    of packed token ids (others stay zero). Returns (out [T, H, dv], lse [T, H]);
    with ``exact`` both are fp64 and unrounded (see :func:`_attend`).
    """
    q = q.cpu()
    T, H, D = q.shape
    dtype = q.dtype
    cu = [int(x) for x in torch.as_tensor(cu_seqlens_q).cpu().tolist()]
    kvl = [int(x) for x in torch.as_tensor(seqused_kv).cpu().tolist()]
    ori_bt = ori_block_table.cpu()
    cmp_bt = cmp_block_table.cpu() if cmp_block_table is not None else None
    idx = cmp_sparse_indices.cpu() if cmp_sparse_indices is not None else None
    out = torch.zeros((T, H, dv), dtype=torch.float64 if exact else dtype)
    lse = torch.zeros((T, H), dtype=torch.float64 if exact else torch.float32)
    sinks = sinks.float().cpu()
    want = None if tokens is None else set(int(t) for t in tokens)
    for b in range(len(cu) - 1):
        aq, akv = cu[b + 1] - cu[b], kvl[b]
        for s in range(aq):
            t = cu[b] + s
            if want is not None and t not in want:
                continue
            sg = akv - aq + s
            lo = max(sg - ori_win_left, 0)
            win = _paged_rows(ori_kv, ori_bt[b], list(range(lo, sg + 1)), dequant)
            parts = _tiles(win, s2_tile) if win.shape[0] else []
            if cmp_kv is not None:
                thr = (sg + 1) // cmp_ratio
                if idx is not None:
                    sel = _cmp_rows(idx[t, 0].tolist(), thr, akv // cmp_ratio)
                else:
                    sel = list(range(max(thr, 0)))
                parts += _tiles(_paged_rows(cmp_kv, cmp_bt[b], sel, dequant), s2_tile)
            o, l_ = _attend(q[t].float(), parts, sinks, softmax_scale, dtype, dv, exact, scores_fp64)
            out[t] = o
            lse[t] = l_
    return out, lse


def sinks_softmax_closed_form(q, k, *, sinks, softmax_scale, dv=None):
    """One-shot ``softmax([q k^T * scale, sink]) @ [V; 0]`` (golden.py:207-244).

    ``q`` [G, D], ``k`` [n, D]. Returns (out [G, dv] in q's dtype, lse [G]).
    """
    dv = k.shape[-1] if dv is None else dv
    qf, kf = q.float(), k.float()
    sc = (qf @ kf.T) * softmax_scale
    sk = sinks.float().view(-1, 1)
    xmax = torch.cat([sc, sk], dim=1).amax(dim=1, keepdim=True)
    y = torch.exp(sc - xmax)
    denom = y.sum(dim=1, keepdim=True) + torch.exp(sk - xmax)
    p = y / denom
    out = (p.to(q.dtype).float() @ kf[:, :dv]).to(q.dtype)
    return out, (xmax + torch.log(denom)).squeeze(1)


def brute_force_fp64(q, ori_dense, cmp_dense, idx, sinks, *, act_q, act_kv, scale,
                     cmp_ratio, win_left, dv):
    """Independent fp64 formulation for tiny cases: one score row over ALL raw
    positions and ALL compressed positions, with a 0/1 mask built from the
    rule statements (window band, causal compressed threshold, -1 = unused),
    and the sink as an extra logit. ``q`` [S, G, D]; ``ori_dense`` [S2, D];
    ``cmp_dense`` [S3, D]; ``idx`` [S, K] (or None for CFA)."""
    S, G, D = q.shape
    out = torch.zeros((S, G, dv), dtype=torch.float64)
    lse = torch.zeros((S, G), dtype=torch.float64)
    keys = torch.cat([ori_dense, cmp_dense], dim=0).double()
    n_ori = ori_dense.shape[0]
    for s in range(S):
        sg = act_kv - act_q + s
        w = torch.zeros(keys.shape[0], dtype=torch.float64)
        for j in range(n_ori):
            if sg - win_left <= j <= sg and j >= 0:
                w[j] += 1
        thr = math.floor((sg + 1) / cmp_ratio)
        if idx is None:
            for j in range(cmp_dense.shape[0]):
                if j < thr:
                    w[n_ori + j] += 1
        else:
            live = True
            for j in idx[s].tolist()[:max(min(len(idx[s]), thr), 0)]:
                if j == -1:
                    live = False
                if live and 0 <= j < thr:
                    w[n_ori + j] += 1      # duplicates attend twice, as in the list walk
        sc = (q[s].double() @ keys.T) * scale                  # [G, n]
        logits = torch.cat([sc, sinks.double().view(-1, 1)], dim=1)
        wts = torch.cat([w.expand(G, -1), torch.ones((G, 1), dtype=torch.float64)], dim=1)
        mx = logits.masked_fill(wts == 0, -math.inf).amax(dim=1, keepdim=True)
        e = torch.exp(logits - mx) * wts
        z = e.sum(dim=1, keepdim=True)
        vals = torch.cat([keys[:, :dv], torch.zeros((1, dv), dtype=torch.float64)], dim=0)
        out[s] = (e / z) @ vals
        lse[s] = (mx + torch.log(z)).squeeze(1)
    return out, lse
