"""ORACLE (test infrastructure only; never imported by the product path).

CPU restatement of the reference metadata scheduler
(sparse_attn_sharedkv_tilelang/metadata.py:258-1086), used by tests to check
the product's C++ scheduler on arbitrary inputs. Pure-Python integers, so
arithmetic is unbounded like the reference's (the C++ port must reproduce
that, e.g. for ``ori_win_left = -1`` where pre-tokens are INT64_MAX).

Pinned by: ``tests/golden/metadata_fixtures.json`` (72 input/output vectors
written from the reference scheduler, including the design note's worked
example B=2/aic=3), and the reference's own invariants
(test_sparse_attn_sharedkv.py:721-924).
"""

from __future__ import annotations

INT64_MAX = (1 << 63) - 1
AIC_CORE_NUM, AIV_CORE_NUM, META_SIZE = 36, 72, 1024
WIN_N, WIN_T, CMP_N, CMP_T = 0, 1, 2, 3


def _ints(x):
    if x is None:
        return []
    if hasattr(x, "tolist"):
        return [int(v) for v in x.reshape(-1).tolist()]
    return [int(v) for v in x]


class _S1G:
    """Per-(batch, s1g row) block/cost cache (metadata.py:155-177)."""

    __slots__ = ("b", "row", "s2_start", "s2_end", "win_start", "win_end", "cmp_start",
                 "cmp_end", "cost", "last_cost", "blocks", "win_blocks", "win_cost",
                 "win_last", "win_normal", "cmp_blocks", "cmp_cost", "cmp_last",
                 "cmp_normal", "cmp_tail", "win_tail")

    def __init__(self):
        for k in self.__slots__:
            setattr(self, k, 0)


def metadata_ref(*, num_heads_q, num_heads_kv, head_dim, cu_seqlens_q=None,
                 cu_seqlens_ori_kv=None, cu_seqlens_cmp_kv=None, seqused_q=None,
                 seqused_kv=None, batch_size=0, max_seqlen_q=0, max_seqlen_kv=0,
                 ori_topk=0, cmp_topk=0, cmp_ratio=-1, ori_mask_mode=4, cmp_mask_mode=3,
                 ori_win_left=127, ori_win_right=0, layout_q="BSND", layout_kv="PA_ND",
                 has_ori_kv=True, has_cmp_kv=True, aic_core_num=24, aiv_core_num=48,
                 device=None):
    """Return the int32[1024] schedule as a Python list (metadata.py:1018-1086)."""
    cu_q, cu_kv = _ints(cu_seqlens_q), _ints(cu_seqlens_ori_kv)
    sq, skv = _ints(seqused_q), _ints(seqused_kv)
    nkv = num_heads_kv
    aic, aiv = aic_core_num, aiv_core_num

    # ParamsInit (metadata.py:359-389)
    if sq:
        B = len(sq)
    elif layout_q == "TND" and cu_q:
        B = len(cu_q) - 1
    else:
        B = batch_size
    if ori_mask_mode == 0:
        pre, nxt, attn_mode = INT64_MAX, INT64_MAX, 0
    elif ori_mask_mode == 3:
        pre, nxt, attn_mode = INT64_MAX, 0, 1
    else:
        pre = ori_win_left if ori_win_left > -1 else INT64_MAX
        nxt, attn_mode = 0, 1
    is_s1g = layout_q in ("BSND", "BSH", "TND")
    G = 0 if nkv == 0 else num_heads_q // nkv
    is_cfa = has_cmp_kv and cmp_topk <= 0
    is_scfa = has_cmp_kv and cmp_topk > 0
    mbase, s2base = G, 512

    def s1_len(b):  # metadata.py:393-398
        if sq:
            return sq[b]
        if layout_q == "TND" and cu_q:
            return cu_q[b + 1] - cu_q[b]
        return max_seqlen_q

    def s2_len(b):  # metadata.py:400-407
        if skv:
            return skv[b]
        if layout_kv == "TND" and cu_kv:
            return cu_kv[b + 1] - cu_kv[b]
        return max_seqlen_kv

    def cost(m, s2):  # metadata.py:428-438 (window and cmp costs are identical)
        return 6 * ((m + 15) >> 4) + 10 * ((s2 + 63) >> 6)

    # SplitInfo (metadata.py:671-683)
    s1g_num = [(s1_len(b) * G + mbase - 1) // mbase if mbase else 0 for b in range(B)]
    s1g_tail = [(s1_len(b) * G) % mbase if mbase else 0 for b in range(B)]
    s2_num = [(s2_len(b) + s2base - 1) // s2base for b in range(B)]
    all_zero = not any(s1g_num[b] != 0 and s2_num[b] != 0 for b in range(B))

    def batch_ctx(b):  # metadata.py:505-510, 409-426
        s1, s2 = s1_len(b), s2_len(b)
        pre_lu = s1 - s2 + pre if ori_mask_mode == 4 else pre
        if ori_mask_mode in (0, 1, 2):
            nxt_lu = nxt
        elif ori_mask_mode == 3:
            nxt_lu = s2 - s1
        elif ori_mask_mode == 4:
            nxt_lu = s2 - s1 + nxt
        else:
            nxt_lu = nxt
        return (b, s1, s2, pre_lu, nxt_lu)

    def fill_s1g(row, bc, c):  # metadata.py:634-667
        b, s1, s2, pre_lu, nxt_lu = bc
        if s1g_num[b] == 0:
            c.cost = c.last_cost = c.win_normal = c.win_last = 0
            c.cmp_normal = c.cmp_last = c.blocks = 0
            c.s2_start = c.cmp_start = c.s2_end = 0
            return
        c.b, c.row = b, row
        # s2 token range (metadata.py:479-501)
        if s1 == 0 or s2 == 0:
            f, l_ = 0, 0
        elif not attn_mode:
            f, l_ = 0, s2 - 1
        else:
            g0 = row * mbase
            g1 = min(g0 + mbase, s1 * G) - 1
            if is_s1g:
                a0, a1 = g0 // G, g1 // G
            elif g0 // s1 == g1 // s1:
                a0, a1 = g0 % s1, g1 % s1
            else:
                a0, a1 = 0, s1
            f, l_ = a0 - pre_lu, a1 + nxt_lu
        # block range and tails (metadata.py:512-547)
        if f >= s2 or l_ < 0 or l_ < f:
            f = l_ = 0
            c.win_start = c.win_end = c.win_tail = 0
        else:
            f = max(0, min(f, s2 - 1))
            l_ = max(0, min(l_, s2 - 1))
            c.win_start = 0
            c.win_end = (l_ - f) // s2base + 1
            c.win_tail = (l_ - f + 1) % s2base
        c.cmp_start = c.win_end
        last_tok = (l_ + 1) // cmp_ratio if (has_cmp_kv and cmp_ratio > 0) else 0
        act = last_tok if is_cfa else (min(last_tok, cmp_topk) if is_scfa else 0)
        c.cmp_end = c.cmp_start if act == 0 else c.cmp_start + (act - 1) // s2base + 1
        c.cmp_tail = act % s2base
        # cost table (metadata.py:440-477)
        tail = s1g_tail[b]
        tc = [[0] * 4 for _ in range(4)]
        tc[WIN_N][WIN_N] = cost(mbase, s2base)
        tc[WIN_T][WIN_N] = 0 if tail == 0 else cost(tail, s2base)
        tc[WIN_N][WIN_T] = 0 if c.win_tail == 0 else cost(mbase, c.win_tail)
        tc[WIN_T][WIN_T] = 0 if (tail == 0 or c.win_tail == 0) else cost(tail, c.win_tail)
        if has_cmp_kv:
            tc[CMP_N][CMP_N] = cost(mbase, s2base)
            tc[CMP_T][CMP_N] = 0 if tail == 0 else cost(tail, s2base)
            tc[CMP_N][CMP_T] = 0 if c.cmp_tail == 0 else cost(mbase, c.cmp_tail)
            tc[CMP_T][CMP_T] = 0 if (tail == 0 or c.cmp_tail == 0) else cost(tail, c.cmp_tail)
        last_row = row == s1g_num[b] - 1 and tail != 0
        # window part (metadata.py:549-584) and cmp part (586-621)
        for kind, start, end, tl in ((WIN_N, c.win_start, c.win_end, c.win_tail),
                                     (CMP_N, c.cmp_start, c.cmp_end, c.cmp_tail)):
            if start >= end:
                nb = tot = lst = nrm = 0
            else:
                nb = end - start
                has_tail = 1 if tl != 0 else 0
                normal = nb - has_tail
                r = kind + 1 if last_row else kind          # row type: tail or normal
                tot = tc[r][kind] * normal + tc[r][kind + 1] * has_tail
                lst = tc[r][kind + 1] if has_tail else tc[r][kind]
                nrm = tc[r][kind]
            if kind == WIN_N:
                c.win_blocks, c.win_cost, c.win_last, c.win_normal = nb, tot, lst, nrm
            else:
                c.cmp_blocks, c.cmp_cost, c.cmp_last, c.cmp_normal = nb, tot, lst, nrm
        # merge (metadata.py:623-632)
        c.s2_start = c.win_start if c.win_blocks > 0 else c.cmp_start
        if c.cmp_blocks > 0:
            c.last_cost, c.s2_end = c.cmp_last, c.cmp_end
        else:
            c.last_cost, c.s2_end = c.win_last, c.win_end
        c.blocks = c.win_blocks + c.cmp_blocks
        c.cost = c.win_cost + c.cmp_cost

    out = [0] * META_SIZE
    bn2_end = [0] * aic
    m_end = [0] * aic
    s2_end = [0] * aic
    used = 0
    if all_zero:  # metadata.py:959-964
        used = 1
        if aic > 0:
            bn2_end[0] = B * nkv
    else:
        # CostInfo (metadata.py:685-714)
        bcost, bblock, blast = [0] * B, [0] * B, [0] * B
        total_cost = 0
        max_row_cost = 0
        for b in range(B):
            if s1_len(b) == 0 or s2_len(b) == 0:
                continue
            bc, c = batch_ctx(b), _S1G()
            for row in range(s1g_num[b]):
                fill_s1g(row, bc, c)
                bcost[b] += c.cost
                bblock[b] += c.blocks
                max_row_cost = max(max_row_cost, c.cost)
                if c.blocks > 0:
                    blast[b] = c.last_cost
            total_cost += bcost[b] * nkv
        # SplitPlan (metadata.py:898-923); supportFd is False in the reference,
        # so the block-level pass, forced assignment and FD records never run.
        if aic > 0:
            cur_b = cur_bn2 = cur_row = 0
            unassigned = total_cost
            bn2_cost, bn2_block = bcost[0], bblock[0]
            bc, c = batch_ctx(0), _S1G()
            fill_s1g(0, bc, c)
            cur_s2 = c.s2_start
            finished = False
            max_cost = 0
            core = 0
            for i in range(aic):
                if finished or unassigned <= 0:
                    break
                core = i
                avg = unassigned // max(1, aic - i)
                limit = max(avg, max_row_cost)
                ccost = cblock = 0
                # AssignByBatch (metadata.py:718-745)
                if not finished:
                    while bn2_cost == 0 or limit + blast[cur_b] // 2 >= ccost + bn2_cost:
                        ccost += bn2_cost
                        cblock += bn2_block
                        cur_bn2 += 1
                        if cur_bn2 == B * nkv:
                            cur_row = cur_s2 = 0
                            finished = True
                            break
                        if cur_bn2 // nkv != cur_b:
                            cur_b = cur_bn2 // nkv
                            bc = batch_ctx(cur_b)
                        bn2_cost, bn2_block = bcost[cur_b], bblock[cur_b]
                        cur_row = 0
                        fill_s1g(cur_row, bc, c)
                        cur_s2 = c.s2_start
                # AssignByRow (metadata.py:747-764)
                if not finished:
                    while limit + c.last_cost // 2 >= ccost + c.cost:
                        ccost += c.cost
                        cblock += c.blocks
                        bn2_cost = max(0, bn2_cost - c.cost)
                        bn2_block = max(0, bn2_block - c.blocks)
                        while True:
                            cur_row += 1
                            fill_s1g(cur_row, bc, c)
                            if c.blocks != 0:
                                break
                        cur_s2 = c.s2_start
                bn2_end[i], m_end[i], s2_end[i] = cur_bn2, cur_row, cur_s2
                max_cost = max(max_cost, ccost)
                unassigned -= ccost
            used = core + 1
        used = max(used, 1)
    # GenMetaData (metadata.py:974-1009)
    for i in range(AIC_CORE_NUM):
        if i >= used or i >= aic:
            continue
        r = 8 * i
        out[r] = 1
        if i > 0:
            out[r + 1], out[r + 2], out[r + 3] = bn2_end[i - 1], m_end[i - 1], s2_end[i - 1]
        out[r + 4], out[r + 5], out[r + 6] = bn2_end[i], m_end[i], s2_end[i]
    return out
