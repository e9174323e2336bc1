// Host-side work scheduler for sparse_attn_sharedkv, bit-exact with the
// reference scheduler (sparse_attn_sharedkv_tilelang/metadata.py:258-1086,
// itself a port of the Ascend AICPU SparseAttnSharedkvMetadata kernel).
//
// The schedule is a cost-balanced partition of (batch*kv_head, s1g-row) work
// over `aic_core_num` cores. Each row's cost counts 512-token KV blocks of the
// sliding window and of the compressed pass at 6*ceil(m/16) + 10*ceil(s2/64).
// Cores are filled greedily, first by whole (batch, kv-head) units, then by
// rows, each allowed to overshoot its limit by half of the last block's cost.
// The flash-decode (block-level split) path is disabled in the reference
// (supportFd = false, metadata.py:323-325), so the FD section stays zero and
// only the FA rows are written.
//
// Arithmetic on token ranges uses 128-bit integers: the reference computes in
// unbounded Python integers and, e.g., ori_win_left = -1 makes the pre-token
// bound INT64_MAX before offsets are added.

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/sas.h"
#include "sas_common.h"

namespace {

using i64 = int64_t;
using i128 = __int128;

constexpr i64 kInt64Max = INT64_MAX;
constexpr i64 kS2Base = 512;
constexpr i64 kMaxRowSkip = int64_t(1) << 26;  // guard for the row-skip loop

enum BlockType { WIN_N = 0, WIN_T = 1, CMP_N = 2, CMP_T = 3 };

inline i128 floordiv(i128 a, i128 b) {
  i128 q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}
inline i128 floormod(i128 a, i128 b) { return a - floordiv(a, b) * b; }

inline i64 block_cost(i64 m, i64 s2) {  // metadata.py:428-438
  return 6 * ((m + 15) >> 4) + 10 * ((s2 + 63) >> 6);
}

struct RowCache {  // metadata.py:155-177
  i64 b = 0, row = 0;
  i64 s2_start = 0, s2_end = 0, win_start = 0, win_end = 0, cmp_start = 0, cmp_end = 0;
  i64 cost = 0, last_cost = 0, blocks = 0;
  i64 win_blocks = 0, win_cost = 0, win_last = 0, win_normal = 0;
  i64 cmp_blocks = 0, cmp_cost = 0, cmp_last = 0, cmp_normal = 0;
  i64 cmp_tail = 0, win_tail = 0;
};

struct BatchCtx {  // metadata.py:146-151
  i64 b = 0, s1 = 0, s2 = 0;
  i128 pre_lu = 0, next_lu = 0;
};

struct Scheduler {
  // inputs
  i64 heads_q, heads_kv;
  std::vector<i64> cu_q, cu_kv, seq_q, seq_kv;
  i64 batch_arg, max_q, max_kv, cmp_topk, cmp_ratio;
  i64 mask_mode, win_left;
  std::string layout_q, layout_kv;
  bool has_cmp;
  i64 aic, aiv;
  // derived (metadata.py:359-389)
  i64 B = 0, G = 0, mbase = 0;
  i128 pre = 0, nxt = 0;
  int attn_mode = 1;
  bool is_s1g = true, is_cfa = false, is_scfa = false;
  std::vector<i64> s1g_num, s1g_tail, s2_num;
  bool all_zero = true;

  i64 s1_len(i64 b) const {  // metadata.py:393-398
    if (!seq_q.empty()) return seq_q[b];
    if (layout_q == "TND" && !cu_q.empty()) return cu_q[b + 1] - cu_q[b];
    return max_q;
  }
  i64 s2_len(i64 b) const {  // metadata.py:400-407
    if (!seq_kv.empty()) return seq_kv[b];
    if (layout_kv == "TND" && !cu_kv.empty()) return cu_kv[b + 1] - cu_kv[b];
    return max_kv;
  }

  void init() {
    if (!seq_q.empty()) B = (i64)seq_q.size();
    else if (layout_q == "TND" && !cu_q.empty()) B = (i64)cu_q.size() - 1;
    else B = batch_arg;
    if (mask_mode == 0) { pre = kInt64Max; nxt = kInt64Max; attn_mode = 0; }
    else if (mask_mode == 3) { pre = kInt64Max; nxt = 0; attn_mode = 1; }
    else { pre = win_left > -1 ? (i128)win_left : (i128)kInt64Max; nxt = 0; attn_mode = 1; }
    is_s1g = layout_q == "BSND" || layout_q == "BSH" || layout_q == "TND";
    G = heads_q / heads_kv;
    if (has_cmp) { if (cmp_topk > 0) is_scfa = true; else is_cfa = true; }
    mbase = G;
    s1g_num.assign(B, 0); s1g_tail.assign(B, 0); s2_num.assign(B, 0);
    for (i64 b = 0; b < B; ++b) {  // metadata.py:671-683
      i64 s1 = s1_len(b), s2 = s2_len(b);
      s1g_num[b] = (i64)floordiv((i128)s1 * G + mbase - 1, mbase);
      s1g_tail[b] = (i64)floormod((i128)s1 * G, mbase);
      s2_num[b] = (i64)floordiv((i128)s2 + kS2Base - 1, kS2Base);
      if (s1g_num[b] != 0 && s2_num[b] != 0) all_zero = false;
    }
  }

  BatchCtx batch_ctx(i64 b) const {  // metadata.py:505-510, 409-426
    BatchCtx c;
    c.b = b; c.s1 = s1_len(b); c.s2 = s2_len(b);
    c.pre_lu = mask_mode == 4 ? (i128)c.s1 - c.s2 + pre : pre;
    if (mask_mode == 0 || mask_mode == 1 || mask_mode == 2) c.next_lu = nxt;
    else if (mask_mode == 3) c.next_lu = (i128)c.s2 - c.s1;
    else if (mask_mode == 4) c.next_lu = (i128)c.s2 - c.s1 + nxt;
    else c.next_lu = nxt;
    return c;
  }

  void fill_row(i64 row, const BatchCtx& bc, RowCache& c) const {  // metadata.py:634-667
    if (s1g_num[bc.b] == 0) {
      c.cost = c.last_cost = c.win_normal = c.win_last = 0;
      c.cmp_normal = c.cmp_last = c.blocks = 0;
      c.s2_start = c.cmp_start = c.s2_end = 0;
      return;
    }
    c.b = bc.b; c.row = row;
    // token range of the row (metadata.py:479-501)
    i128 f, l;
    if (bc.s1 == 0 || bc.s2 == 0) { f = 0; l = 0; }
    else if (!attn_mode) { f = 0; l = (i128)bc.s2 - 1; }
    else {
      i128 g0 = (i128)row * mbase;
      i128 g1 = std::min<i128>(g0 + mbase, (i128)bc.s1 * G) - 1;
      i128 a0, a1;
      if (is_s1g) { a0 = floordiv(g0, G); a1 = floordiv(g1, G); }
      else if (floordiv(g0, bc.s1) == floordiv(g1, bc.s1)) {
        a0 = floormod(g0, bc.s1); a1 = floormod(g1, bc.s1);
      } else { a0 = 0; a1 = bc.s1; }
      f = a0 - bc.pre_lu;
      l = a1 + bc.next_lu;
    }
    // block ranges and tails (metadata.py:512-547)
    if (f >= bc.s2 || l < 0 || l < f) {
      f = 0; l = 0;
      c.win_start = c.win_end = c.win_tail = 0;
    } else {
      f = std::max<i128>(0, std::min<i128>(f, bc.s2 - 1));
      l = std::max<i128>(0, std::min<i128>(l, bc.s2 - 1));
      c.win_start = 0;
      c.win_end = (i64)floordiv(l - f, kS2Base) + 1;
      c.win_tail = (i64)floormod(l - f + 1, kS2Base);
    }
    c.cmp_start = c.win_end;
    i64 last_tok = (has_cmp && cmp_ratio > 0) ? (i64)floordiv(l + 1, cmp_ratio) : 0;
    i64 act = is_cfa ? last_tok : (is_scfa ? std::min(last_tok, cmp_topk) : 0);
    c.cmp_end = act == 0 ? c.cmp_start : c.cmp_start + (i64)floordiv((i128)act - 1, kS2Base) + 1;
    c.cmp_tail = (i64)floormod(act, kS2Base);
    // per-type block costs (metadata.py:440-477)
    i64 tail = s1g_tail[bc.b];
    i64 tc[4][4] = {};
    tc[WIN_N][WIN_N] = block_cost(mbase, kS2Base);
    tc[WIN_T][WIN_N] = tail == 0 ? 0 : block_cost(tail, kS2Base);
    tc[WIN_N][WIN_T] = c.win_tail == 0 ? 0 : block_cost(mbase, c.win_tail);
    tc[WIN_T][WIN_T] = (tail == 0 || c.win_tail == 0) ? 0 : block_cost(tail, c.win_tail);
    if (has_cmp) {
      tc[CMP_N][CMP_N] = block_cost(mbase, kS2Base);
      tc[CMP_T][CMP_N] = tail == 0 ? 0 : block_cost(tail, kS2Base);
      tc[CMP_N][CMP_T] = c.cmp_tail == 0 ? 0 : block_cost(mbase, c.cmp_tail);
      tc[CMP_T][CMP_T] = (tail == 0 || c.cmp_tail == 0) ? 0 : block_cost(tail, c.cmp_tail);
    }
    const bool last_row = row == s1g_num[bc.b] - 1 && tail != 0;
    // window part (metadata.py:549-584), compressed part (586-621)
    auto part = [&](int kind, i64 start, i64 end, i64 tl, i64& nb, i64& tot, i64& lst,
                    i64& nrm) {
      if (start >= end) { nb = tot = lst = nrm = 0; return; }
      nb = end - start;
      i64 has_tail = tl != 0 ? 1 : 0;
      i64 normal = nb - has_tail;
      int r = last_row ? kind + 1 : kind;
      tot = tc[r][kind] * normal + tc[r][kind + 1] * has_tail;
      lst = has_tail ? tc[r][kind + 1] : tc[r][kind];
      nrm = tc[r][kind];
    };
    part(WIN_N, c.win_start, c.win_end, c.win_tail, c.win_blocks, c.win_cost, c.win_last,
         c.win_normal);
    part(CMP_N, c.cmp_start, c.cmp_end, c.cmp_tail, c.cmp_blocks, c.cmp_cost, c.cmp_last,
         c.cmp_normal);
    // merge (metadata.py:623-632)
    c.s2_start = c.win_blocks > 0 ? c.win_start : c.cmp_start;
    if (c.cmp_blocks > 0) { c.last_cost = c.cmp_last; c.s2_end = c.cmp_end; }
    else { c.last_cost = c.win_last; c.s2_end = c.win_end; }
    c.blocks = c.win_blocks + c.cmp_blocks;
    c.cost = c.win_cost + c.cmp_cost;
  }

  int run(int32_t* out) {
    init();
    std::vector<i64> bn2_end(std::max<i64>(aic, 1), 0), m_end(std::max<i64>(aic, 1), 0),
        s2_end(std::max<i64>(aic, 1), 0);
    i64 used = 0;
    if (all_zero) {  // metadata.py:959-964
      used = 1;
      bn2_end[0] = B * heads_kv;
    } else {
      // per-batch costs (metadata.py:685-714)
      std::vector<i64> bcost(B, 0), bblock(B, 0), blast(B, 0);
      i64 total_cost = 0, max_row_cost = 0;
      for (i64 b = 0; b < B; ++b) {
        if (s1_len(b) == 0 || s2_len(b) == 0) continue;
        BatchCtx bc = batch_ctx(b);
        RowCache c;
        for (i64 row = 0; row < s1g_num[b]; ++row) {
          fill_row(row, bc, c);
          bcost[b] += c.cost;
          bblock[b] += c.blocks;
          max_row_cost = std::max(max_row_cost, c.cost);
          if (c.blocks > 0) blast[b] = c.last_cost;
        }
        total_cost += bcost[b] * heads_kv;
      }
      // greedy assignment (metadata.py:718-764, 872-923)
      if (aic > 0) {
        i64 cur_b = 0, cur_bn2 = 0, cur_row = 0, cur_s2;
        i64 unassigned = total_cost;
        i64 bn2_cost = bcost[0], bn2_block = bblock[0];
        BatchCtx bc = batch_ctx(0);
        RowCache c;
        fill_row(0, bc, c);
        cur_s2 = c.s2_start;
        bool finished = false;
        i64 core = 0;
        for (i64 i = 0; i < aic; ++i) {
          if (finished || unassigned <= 0) break;
          core = i;
          i64 avg = (i64)floordiv(unassigned, std::max<i64>(1, aic - i));
          i64 limit = std::max(avg, max_row_cost);
          i64 ccost = 0, cblock = 0;
          // whole (batch, kv-head) units
          while (bn2_cost == 0 || limit + blast[cur_b] / 2 >= ccost + bn2_cost) {
            ccost += bn2_cost;
            cblock += bn2_block;
            cur_bn2 += 1;
            if (cur_bn2 == B * heads_kv) { cur_row = 0; cur_s2 = 0; finished = true; break; }
            if (cur_bn2 / heads_kv != cur_b) { cur_b = cur_bn2 / heads_kv; bc = batch_ctx(cur_b); }
            bn2_cost = bcost[cur_b];
            bn2_block = bblock[cur_b];
            cur_row = 0;
            fill_row(cur_row, bc, c);
            cur_s2 = c.s2_start;
          }
          // single rows
          if (!finished) {
            while (limit + c.last_cost / 2 >= ccost + c.cost) {
              ccost += c.cost;
              cblock += c.blocks;
              bn2_cost = std::max<i64>(0, bn2_cost - c.cost);
              bn2_block = std::max<i64>(0, bn2_block - c.blocks);
              i64 guard = 0;
              do {
                cur_row += 1;
                fill_row(cur_row, bc, c);
                if (++guard > kMaxRowSkip)
                  return sas::set_error(SAS_EINVAL, "metadata: row scan does not terminate");
              } while (c.blocks == 0);
              cur_s2 = c.s2_start;
            }
          }
          bn2_end[i] = cur_bn2; m_end[i] = cur_row; s2_end[i] = cur_s2;
          unassigned -= ccost;
        }
        used = core + 1;
      }
      used = std::max<i64>(used, 1);
    }
    // output rows (metadata.py:974-1009)
    std::memset(out, 0, sizeof(int32_t) * SAS_META_SIZE);
    for (i64 i = 0; i < SAS_AIC_CORE_NUM; ++i) {
      if (i >= used || i >= aic) continue;
      int32_t* r = out + i * SAS_FA_METADATA_SIZE;
      r[0] = 1;
      if (i > 0) { r[1] = (int32_t)bn2_end[i - 1]; r[2] = (int32_t)m_end[i - 1]; r[3] = (int32_t)s2_end[i - 1]; }
      r[4] = (int32_t)bn2_end[i]; r[5] = (int32_t)m_end[i]; r[6] = (int32_t)s2_end[i];
      r[7] = 0;
    }
    return SAS_OK;
  }
};

std::vector<i64> to_vec(const int32_t* p, int64_t n) {
  std::vector<i64> v;
  if (p && n > 0) v.assign(p, p + n);
  return v;
}

}  // namespace

extern "C" int sas_metadata_v1(const SasMetaParams* p, int32_t* out) {
  sas::clear_error();
  if (!p || !out) return sas::set_error(SAS_EINVAL, "metadata: null argument");
  if (p->num_heads_kv <= 0 || p->num_heads_q < p->num_heads_kv)
    return sas::set_error(SAS_EINVAL, "metadata: need num_heads_kv > 0 and num_heads_q >= num_heads_kv "
                          "(got %lld, %lld)", (long long)p->num_heads_q, (long long)p->num_heads_kv);
  if (p->aic_core_num < 1 || p->aiv_core_num < 0)
    return sas::set_error(SAS_EINVAL, "metadata: aic_core_num must be >= 1");
  Scheduler s;
  s.heads_q = p->num_heads_q;
  s.heads_kv = p->num_heads_kv;
  s.cu_q = to_vec(p->cu_seqlens_q, p->n_cu_seqlens_q);
  s.cu_kv = to_vec(p->cu_seqlens_ori_kv, p->n_cu_seqlens_ori_kv);
  s.seq_q = to_vec(p->seqused_q, p->n_seqused_q);
  s.seq_kv = to_vec(p->seqused_kv, p->n_seqused_kv);
  s.batch_arg = p->batch_size;
  s.max_q = p->max_seqlen_q;
  s.max_kv = p->max_seqlen_kv;
  s.cmp_topk = p->cmp_topk;
  s.cmp_ratio = p->cmp_ratio;
  s.mask_mode = p->ori_mask_mode;
  s.win_left = p->ori_win_left;
  s.layout_q = p->layout_q ? p->layout_q : "BSND";
  s.layout_kv = p->layout_kv ? p->layout_kv : "PA_ND";
  s.has_cmp = p->has_cmp_kv != 0;
  s.aic = p->aic_core_num;
  s.aiv = p->aiv_core_num;
  // batch count sanity: every per-batch array must cover B entries
  i64 B;
  if (!s.seq_q.empty()) B = (i64)s.seq_q.size();
  else if (s.layout_q == "TND" && !s.cu_q.empty()) B = (i64)s.cu_q.size() - 1;
  else B = s.batch_arg;
  if (B < 0) return sas::set_error(SAS_EINVAL, "metadata: negative batch size");
  if (!s.seq_kv.empty() && (i64)s.seq_kv.size() < B)
    return sas::set_error(SAS_EINVAL, "metadata: seqused_kv has %lld entries, batch is %lld",
                          (long long)s.seq_kv.size(), (long long)B);
  if (s.seq_kv.empty() && s.layout_kv == "TND" && !s.cu_kv.empty() && (i64)s.cu_kv.size() < B + 1)
    return sas::set_error(SAS_EINVAL, "metadata: cu_seqlens_ori_kv too short");
  return s.run(out);
}
