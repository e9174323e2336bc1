"""ORACLE (test infrastructure only; never imported by the product path).

Backward of sparse_attn_sharedkv on the CPU in fp64, by autograd through
the closed form the forward golden computes (sparse_attn_sharedkv_tilelang/
golden.py:207-244, with golden.py:28-66 / 116-150 choosing each token's
keys): per query token, the window rows and the valid top-k (or dense
compressed) rows, read through the block tables, then

    out = softmax([scale q K^T, sink]) [V; 0],  V = K[:, :dv]

The reference has no backward; this is the mathematics its LSE output is
documented for (api.py:32-35). The gradient of the caches is returned for
the touched rows only, as (flat row index, gradient) pairs per cache.

Pins (tests/test_backward.py): its forward equals golden_paged(exact=True);
central finite differences of the loss on a tiny case match dq, d_kv and
d_sinks; the sink gradient matches the independent closed form
-sum_t exp(sink - lse) (dO . O); a planted mistake (dropping the sink from
the softmax) fails the forward check. :func:`backward_given_forward` (the
explicit FlashAttention-2 formulas from a forward's own out / lse) equals the
autograd gradients when given the exact forward, and a planted sign error in
its dS fails that check.
"""

from __future__ import annotations

from typing import Optional

import torch

from oracle.golden_ref import _cmp_rows


def _rows(bt_row, positions, bs):
    return [int(bt_row[p // bs]) * bs + p % bs for p in positions]


def backward_paged(q, dout, *, ori_kv, ori_block_table, cu_seqlens_q, seqused_kv, sinks, softmax_scale,
                   cmp_kv=None, cmp_block_table=None, cmp_sparse_indices=None, cmp_ratio=None,
                   ori_win_left=127, dv=512, drop_sink: bool = False, tokens=None):
    """Returns dict(out, lse, dq [T,H,D], d_ori=(rows, grads), d_cmp=(rows, grads) or None,
    d_sinks [H]) in fp64. ``drop_sink`` plants a mistake for the oracle's own tests.
    ``tokens`` restricts the loss to those packed token ids (the others have
    zero out / lse / dq and contribute nothing, as if their dout were zero)."""
    q = q.detach().cpu().double()
    dout = dout.detach().cpu().double()
    T, H, D = q.shape
    cu = [int(x) for x in torch.as_tensor(cu_seqlens_q).cpu().tolist()]
    kvl = [int(x) for x in torch.as_tensor(seqused_kv).cpu().tolist()]
    obt = ori_block_table.cpu().tolist()
    cbt = cmp_block_table.cpu().tolist() if cmp_block_table is not None else None
    idx = cmp_sparse_indices.cpu() if cmp_sparse_indices is not None else None
    obs = ori_kv.shape[1]
    cbs = cmp_kv.shape[1] if cmp_kv is not None else 1
    # per token: (ori rows, cmp rows) in golden's order
    plan = {}
    want = None if tokens is None else set(int(x) for x in tokens)
    for b in range(len(cu) - 1):
        aq, akv = cu[b + 1] - cu[b], kvl[b]
        for s in range(aq):
            t = cu[b] + s
            if want is not None and t not in want:
                continue
            sg = akv - aq + s
            lo = max(sg - ori_win_left, 0)
            orows = _rows(obt[b], list(range(lo, sg + 1)), obs)
            crows = []
            if cmp_kv is not None:
                thr = (sg + 1) // cmp_ratio
                sel = (_cmp_rows(idx[t, 0].tolist(), thr, akv // cmp_ratio) if idx is not None
                       else list(range(max(thr, 0))))
                crows = _rows(cbt[b], sel, cbs)
            plan[t] = (orows, crows)
    ou = sorted({r for o, _ in plan.values() for r in o})
    cuq = sorted({r for _, c in plan.values() for r in c})
    ofl = ori_kv.detach().cpu().reshape(-1, D)
    lo_ = torch.tensor(ou, dtype=torch.long)
    oleaf = ofl[lo_].double().requires_grad_(True) if ou else torch.zeros(0, D, dtype=torch.float64)
    omap = {r: i for i, r in enumerate(ou)}
    if cmp_kv is not None and cuq:
        cfl = cmp_kv.detach().cpu().reshape(-1, D)
        cleaf = cfl[torch.tensor(cuq, dtype=torch.long)].double().requires_grad_(True)
    else:
        cleaf = torch.zeros(0, D, dtype=torch.float64)
    cmap = {r: i for i, r in enumerate(cuq)}
    qv = q.clone().requires_grad_(True)
    sk = sinks.detach().cpu().double().clone().requires_grad_(True)
    out = torch.zeros(T, H, dv, dtype=torch.float64)
    lse = torch.zeros(T, H, dtype=torch.float64)
    loss = torch.zeros((), dtype=torch.float64)
    for t, (orows, crows) in plan.items():
        parts = []
        if orows:
            parts.append(oleaf[torch.tensor([omap[r] for r in orows], dtype=torch.long)])
        if crows:
            parts.append(cleaf[torch.tensor([cmap[r] for r in crows], dtype=torch.long)])
        K = torch.cat(parts) if parts else torch.zeros(0, D, dtype=torch.float64)
        sc = (qv[t] @ K.T) * softmax_scale                           # [H, n]
        logits = sc if drop_sink else torch.cat([sc, sk.unsqueeze(1)], dim=1)
        l_ = torch.logsumexp(logits, dim=1)
        pm = torch.exp(logits - l_.unsqueeze(1))[:, :K.shape[0]]
        o = pm @ K[:, :dv]
        out[t] = o.detach()
        lse[t] = l_.detach()
        loss = loss + (o * dout[t]).sum()
    loss.backward()
    res = dict(out=out, lse=lse,
               dq=qv.grad if qv.grad is not None else torch.zeros_like(q),
               d_ori=(lo_, oleaf.grad if ou else torch.zeros(0, D, dtype=torch.float64)),
               d_sinks=sk.grad if sk.grad is not None else torch.zeros(H, dtype=torch.float64))
    res["d_cmp"] = (torch.tensor(cuq, dtype=torch.long),
                    cleaf.grad if (cmp_kv is not None and cuq) else torch.zeros(0, D, dtype=torch.float64)) \
        if cmp_kv is not None else None
    return res


def loss_fp64(q, dout, sinks, ori_kv, cmp_kv, **kw) -> float:
    """sum(dout * out) in fp64 for finite-difference checks (same key sets)."""
    r = backward_paged(q, dout, ori_kv=ori_kv, cmp_kv=cmp_kv, sinks=sinks, **kw)
    return float((r["out"] * dout.double()).sum())


def backward_given_forward(q, dout, out, lse, *, ori_kv, ori_block_table, cu_seqlens_q, seqused_kv, sinks,
                           softmax_scale, cmp_kv=None, cmp_block_table=None, cmp_sparse_indices=None,
                           cmp_ratio=None, ori_win_left=127, dv=512, tokens=None, plant_sign: bool = False):
    """The backward as a FlashAttention-2 style pass defines it, in fp64, from
    a forward's own outputs ``out`` [T, H, dv] and ``lse`` [T, H] (the inputs
    sas_bwd_v1 takes): over each token's key set (golden.py:28-66, 116-150),

        P_j = exp(scale q.k_j - lse),  Delta = dout . out,
        dS_j = P_j (dout . v_j - Delta),
        dq = scale sum_j dS_j k_j,  d k_j += scale dS_j q,  d v_j += P_j dout,
        d sink = -exp(sink - lse) Delta.

    With the exact forward (out, lse of :func:`backward_paged`) this equals
    the autograd gradients; with a rounded forward output it is what any
    backward that takes that output computes. Same return layout as
    :func:`backward_paged` (without out / lse). ``plant_sign`` flips the sign
    of Delta in dS, a planted mistake for the oracle's own tests."""
    q = q.detach().cpu().double()
    dout = dout.detach().cpu().double()
    out = out.detach().cpu().double()
    lse = lse.detach().cpu().double()
    T, H, D = q.shape
    cu = [int(x) for x in torch.as_tensor(cu_seqlens_q).cpu().tolist()]
    kvl = [int(x) for x in torch.as_tensor(seqused_kv).cpu().tolist()]
    obt = ori_block_table.cpu().tolist()
    cbt = cmp_block_table.cpu().tolist() if cmp_block_table is not None else None
    idx = cmp_sparse_indices.cpu() if cmp_sparse_indices is not None else None
    obs = ori_kv.shape[1]
    cbs = cmp_kv.shape[1] if cmp_kv is not None else 1
    ofl = ori_kv.detach().cpu().reshape(-1, D).double()
    cfl = cmp_kv.detach().cpu().reshape(-1, D).double() if cmp_kv is not None else None
    sk = sinks.detach().cpu().double()
    want = None if tokens is None else set(int(x) for x in tokens)
    dq = torch.zeros(T, H, D, dtype=torch.float64)
    d_ori, d_cmp = {}, {}
    d_sinks = torch.zeros(H, dtype=torch.float64)
    for b in range(len(cu) - 1):
        aq, akv = cu[b + 1] - cu[b], kvl[b]
        for s in range(aq):
            t = cu[b] + s
            if want is not None and t not in want:
                continue
            sg = akv - aq + s
            lo = max(sg - ori_win_left, 0)
            orows = _rows(obt[b], list(range(lo, sg + 1)), obs)
            crows = []
            if cmp_kv is not None:
                thr = (sg + 1) // cmp_ratio
                sel = (_cmp_rows(idx[t, 0].tolist(), thr, akv // cmp_ratio) if idx is not None
                       else list(range(max(thr, 0))))
                crows = _rows(cbt[b], sel, cbs)
            delta = (dout[t] * out[t]).sum(-1)                                   # [H]
            d_sinks -= torch.exp(sk - lse[t]) * delta
            keys = [(ofl, d_ori, r) for r in orows] + [(cfl, d_cmp, r) for r in crows]
            if not keys:
                continue
            K = torch.stack([src[r] for src, _, r in keys])                      # [n, D]
            P = torch.exp((q[t] @ K.T) * softmax_scale - lse[t].unsqueeze(1))   # [H, n]
            sgn = -1.0 if plant_sign else 1.0
            dS = P * (dout[t] @ K[:, :dv].T - sgn * delta.unsqueeze(1))          # [H, n]
            dq[t] = softmax_scale * dS @ K
            dK = softmax_scale * dS.T @ q[t]                                     # [n, D]
            dK[:, :dv] += P.T @ dout[t]
            for i, (_, acc, r) in enumerate(keys):
                acc[r] = acc[r] + dK[i] if r in acc else dK[i].clone()

    def pairs(acc):
        rows = sorted(acc)
        return (torch.tensor(rows, dtype=torch.long),
                torch.stack([acc[r] for r in rows]) if rows else torch.zeros(0, D, dtype=torch.float64))

    return dict(dq=dq, d_ori=pairs(d_ori), d_cmp=pairs(d_cmp) if cmp_kv is not None else None,
                d_sinks=d_sinks)
