// The reference's cost-balanced work schedule for sparse_attn_sharedkv
// (sparse_attn_sharedkv_tilelang/metadata.py:258-1015, a port of the Ascend
// AICPU SparseAttnSharedkvMetadata kernel), shared by the host entry point
// (sas_metadata_v1, sas_metadata.cpp) and the device one
// (sas_metadata_device_v1, sas_sched.hip).
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
// Token-range arithmetic is templated on its integer type W. The reference
// computes in unbounded Python integers, and e.g. ori_win_left = -1 makes the
// pre-token bound INT64_MAX before offsets are added: the host uses 128-bit
// integers. The device uses 64-bit ones with the two bounds saturated at
// 2^40 (Sched::derive): every other quantity is an int32 length or a
// difference of them, so a bound of 2^40 or more clamps the row's token
// range exactly as INT64_MAX does (and 128-bit division would cost the
// device hundreds of instructions per use).
#pragma once

#include <cstdint>
#include <vector>

#if defined(__HIPCC__)
#define SAS_HD __host__ __device__
#else
#define SAS_HD
#endif

namespace sas {
namespace sched {

using i64 = int64_t;

constexpr i64 kInt64Max = INT64_MAX;
constexpr i64 kS2Base = 512;
constexpr i64 kMaxRowSkip = int64_t(1) << 26;   // the host's guard of the row-skip loop
constexpr i64 kSatBound = int64_t(1) << 40;     // device: saturated INT64_MAX bounds

enum Layout { kLayoutOther = 0, kLayoutTND = 1, kLayoutBSND = 2, kLayoutBSH = 3 };
enum BlockType { WIN_N = 0, WIN_T = 1, CMP_N = 2, CMP_T = 3 };

template <typename T> SAS_HD inline T smax(T a, T b) { return a < b ? b : a; }
template <typename T> SAS_HD inline T smin(T a, T b) { return b < a ? b : a; }

template <typename W>
SAS_HD inline W floordiv(W a, W b) {
  // non-negative operands below 2^32 (nearly every use): a 32-bit division,
  // the same quotient (the device has no 64-bit divider)
  if (a >= 0 && b > 0 && a <= (W)0xffffffffu && b <= (W)0xffffffffu) return (W)((uint32_t)a / (uint32_t)b);
  W q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}
template <typename W>
SAS_HD inline W floormod(W a, W b) { return a - floordiv(a, b) * b; }

SAS_HD inline i64 block_cost(i64 m, i64 s2) {   // metadata.py:428-438
  return 6 * ((m + 15) >> 4) + 10 * ((s2 + 63) >> 6);
}

// What the scheduler reads; the arrays are host or device pointers by side.
struct Inputs {
  i64 heads_q, heads_kv;
  const int32_t* cu_q; i64 n_cu_q;
  const int32_t* cu_kv; i64 n_cu_kv;
  const int32_t* seq_q; i64 n_seq_q;
  const int32_t* seq_kv; i64 n_seq_kv;
  i64 batch_arg, max_q, max_kv, cmp_topk, cmp_ratio, mask_mode, win_left;
  int layout_q, layout_kv;   // Layout
  int has_cmp;
  i64 aic;
  // per-batch query / KV lengths already read from the arrays above (the
  // device scheduler's LDS copy), or null
  const i64* len_q;
  const i64* len_kv;
};

// One s1g row's blocks and costs (metadata.py:155-177)
struct RowCache {
  i64 s2_start = 0, s2_end = 0, win_start = 0, win_end = 0, cmp_start = 0, cmp_end = 0;
  i64 cost = 0, last_cost = 0, blocks = 0;
  i64 win_blocks = 0, win_cost = 0, win_last = 0, win_normal = 0;
  i64 cmp_blocks = 0, cmp_cost = 0, cmp_last = 0, cmp_normal = 0;
  i64 cmp_tail = 0, win_tail = 0;
};

template <typename W>
struct BatchCtx {   // metadata.py:146-151
  i64 b = 0, s1 = 0, s2 = 0;
  W pre_lu = 0, next_lu = 0;
};

template <typename W>
struct Sched {
  Inputs in;
  // derived (metadata.py:359-389)
  i64 B = 0, G = 0, mbase = 0;
  W pre = 0, nxt = 0;
  int attn_mode = 1;
  bool is_s1g = true, is_cfa = false, is_scfa = false;

  SAS_HD i64 s1_len(i64 b) const {   // metadata.py:393-398
    if (in.len_q) return in.len_q[b];
    if (in.n_seq_q > 0) return in.seq_q[b];
    if (in.layout_q == kLayoutTND && in.n_cu_q > 0) return (i64)in.cu_q[b + 1] - in.cu_q[b];
    return in.max_q;
  }
  SAS_HD i64 s2_len(i64 b) const {   // metadata.py:400-407
    if (in.len_kv) return in.len_kv[b];
    if (in.n_seq_kv > 0) return in.seq_kv[b];
    if (in.layout_kv == kLayoutTND && in.n_cu_kv > 0) return (i64)in.cu_kv[b + 1] - in.cu_kv[b];
    return in.max_kv;
  }
  SAS_HD i64 batch_count() const {
    if (in.n_seq_q > 0) return in.n_seq_q;
    if (in.layout_q == kLayoutTND && in.n_cu_q > 0) return in.n_cu_q - 1;
    return in.batch_arg;
  }

  // saturate: true for the 64-bit device arithmetic
  SAS_HD void derive(bool saturate) {
    B = batch_count();
    const W big = saturate ? (W)kSatBound : (W)kInt64Max;
    if (in.mask_mode == 0) { pre = big; nxt = big; attn_mode = 0; }
    else if (in.mask_mode == 3) { pre = big; nxt = 0; attn_mode = 1; }
    else {
      pre = in.win_left > -1 ? (saturate ? (W)smin<i64>(in.win_left, kSatBound) : (W)in.win_left) : big;
      nxt = 0;
      attn_mode = 1;
    }
    is_s1g = in.layout_q == kLayoutBSND || in.layout_q == kLayoutBSH || in.layout_q == kLayoutTND;
    G = in.heads_q / in.heads_kv;
    if (in.has_cmp) { if (in.cmp_topk > 0) is_scfa = true; else is_cfa = true; }
    mbase = G;
  }

  // per-batch row count, tail and KV block count (metadata.py:671-683)
  SAS_HD void batch_dims(i64 b, i64& s1g_num, i64& s1g_tail, i64& s2_num) const {
    const i64 s1 = s1_len(b), s2 = s2_len(b);
    s1g_num = (i64)floordiv<W>((W)s1 * G + mbase - 1, (W)mbase);
    s1g_tail = (i64)floormod<W>((W)s1 * G, (W)mbase);
    s2_num = (i64)floordiv<W>((W)s2 + kS2Base - 1, (W)kS2Base);
  }

  SAS_HD BatchCtx<W> batch_ctx(i64 b) const {   // metadata.py:505-510, 409-426
    BatchCtx<W> c;
    c.b = b; c.s1 = s1_len(b); c.s2 = s2_len(b);
    c.pre_lu = in.mask_mode == 4 ? (W)c.s1 - c.s2 + pre : pre;
    if (in.mask_mode == 0 || in.mask_mode == 1 || in.mask_mode == 2) c.next_lu = nxt;
    else if (in.mask_mode == 3) c.next_lu = (W)c.s2 - c.s1;
    else if (in.mask_mode == 4) c.next_lu = (W)c.s2 - c.s1 + nxt;
    else c.next_lu = nxt;
    return c;
  }

  // row `row` of batch bc.b, whose row count and tail are s1g_num, tail
  // (metadata.py:634-667)
  SAS_HD void fill_row(i64 row, const BatchCtx<W>& bc, i64 s1g_num, i64 tail, RowCache& c) const {
    if (s1g_num == 0) {
      c.cost = c.last_cost = c.win_normal = c.win_last = 0;
      c.cmp_normal = c.cmp_last = c.blocks = 0;
      c.s2_start = c.cmp_start = c.s2_end = 0;
      return;
    }
    // token range of the row (metadata.py:479-501)
    W f, l;
    if (bc.s1 == 0 || bc.s2 == 0) { f = 0; l = 0; }
    else if (!attn_mode) { f = 0; l = (W)bc.s2 - 1; }
    else {
      const W g0 = (W)row * mbase;
      const W g1 = smin<W>(g0 + mbase, (W)bc.s1 * G) - 1;
      W a0, a1;
      if (is_s1g) { a0 = floordiv<W>(g0, (W)G); a1 = floordiv<W>(g1, (W)G); }
      else if (floordiv<W>(g0, (W)bc.s1) == floordiv<W>(g1, (W)bc.s1)) {
        a0 = floormod<W>(g0, (W)bc.s1); a1 = floormod<W>(g1, (W)bc.s1);
      } else { a0 = 0; a1 = bc.s1; }
      f = a0 - bc.pre_lu;
      l = a1 + bc.next_lu;
    }
    // block ranges and tails (metadata.py:512-547)
    if (f >= bc.s2 || l < 0 || l < f) {
      f = 0; l = 0;
      c.win_start = c.win_end = c.win_tail = 0;
    } else {
      f = smax<W>(0, smin<W>(f, (W)bc.s2 - 1));
      l = smax<W>(0, smin<W>(l, (W)bc.s2 - 1));
      c.win_start = 0;
      c.win_end = (i64)floordiv<W>(l - f, (W)kS2Base) + 1;
      c.win_tail = (i64)floormod<W>(l - f + 1, (W)kS2Base);
    }
    c.cmp_start = c.win_end;
    const i64 last_tok = (in.has_cmp && in.cmp_ratio > 0) ? (i64)floordiv<W>(l + 1, (W)in.cmp_ratio) : 0;
    const i64 act = is_cfa ? last_tok : (is_scfa ? smin<i64>(last_tok, in.cmp_topk) : 0);
    c.cmp_end = act == 0 ? c.cmp_start : c.cmp_start + (i64)floordiv<W>((W)act - 1, (W)kS2Base) + 1;
    c.cmp_tail = (i64)floormod<W>((W)act, (W)kS2Base);
    // per-type block costs (metadata.py:440-477)
    i64 tc[4][4] = {};
    tc[WIN_N][WIN_N] = block_cost(mbase, kS2Base);
    tc[WIN_T][WIN_N] = tail == 0 ? 0 : block_cost(tail, kS2Base);
    tc[WIN_N][WIN_T] = c.win_tail == 0 ? 0 : block_cost(mbase, c.win_tail);
    tc[WIN_T][WIN_T] = (tail == 0 || c.win_tail == 0) ? 0 : block_cost(tail, c.win_tail);
    if (in.has_cmp) {
      tc[CMP_N][CMP_N] = block_cost(mbase, kS2Base);
      tc[CMP_T][CMP_N] = tail == 0 ? 0 : block_cost(tail, kS2Base);
      tc[CMP_N][CMP_T] = c.cmp_tail == 0 ? 0 : block_cost(mbase, c.cmp_tail);
      tc[CMP_T][CMP_T] = (tail == 0 || c.cmp_tail == 0) ? 0 : block_cost(tail, c.cmp_tail);
    }
    const bool last_row = row == s1g_num - 1 && tail != 0;
    // window part (metadata.py:549-584), compressed part (586-621)
    auto part = [&](int kind, i64 start, i64 end, i64 tl, i64& nb, i64& tot, i64& lst, i64& nrm) {
      if (start >= end) { nb = tot = lst = nrm = 0; return; }
      nb = end - start;
      const i64 has_tail = tl != 0 ? 1 : 0;
      const i64 normal = nb - has_tail;
      const int r = last_row ? kind + 1 : kind;
      tot = tc[r][kind] * normal + tc[r][kind + 1] * has_tail;
      lst = has_tail ? tc[r][kind + 1] : tc[r][kind];
      nrm = tc[r][kind];
    };
    part(WIN_N, c.win_start, c.win_end, c.win_tail, c.win_blocks, c.win_cost, c.win_last, c.win_normal);
    part(CMP_N, c.cmp_start, c.cmp_end, c.cmp_tail, c.cmp_blocks, c.cmp_cost, c.cmp_last, c.cmp_normal);
    // merge (metadata.py:623-632)
    c.s2_start = c.win_blocks > 0 ? c.win_start : c.cmp_start;
    if (c.cmp_blocks > 0) { c.last_cost = c.cmp_last; c.s2_end = c.cmp_end; }
    else { c.last_cost = c.win_last; c.s2_end = c.win_end; }
    c.blocks = c.win_blocks + c.cmp_blocks;
    c.cost = c.win_cost + c.cmp_cost;
  }
};

// The per-row figures the greedy assignment needs
struct RowInfo {
  i64 cost, blocks, last_cost, s2_start;
};

// The row phase of a core's fill (metadata.py:750-764): rows of the current
// unit, from the current one (c), each taken while it fits its limit plus
// half its last block's cost; rows without blocks are stepped over. Returns
// false when one step runs over more than max_skip rows without blocks.
template <typename W, typename RowFn>
SAS_HD bool scan_rows(RowFn& row_info, i64 cur_b, const BatchCtx<W>& bc, i64 limit, i64 max_skip, i64& cur_row,
                      RowInfo& c, i64& cur_s2, i64& ccost, i64& cblock, i64& bn2_cost, i64& bn2_block) {
  while (limit + c.last_cost / 2 >= ccost + c.cost) {
    ccost += c.cost;
    cblock += c.blocks;
    bn2_cost = smax<i64>(0, bn2_cost - c.cost);
    bn2_block = smax<i64>(0, bn2_block - c.blocks);
    i64 guard = 0;
    do {
      cur_row += 1;
      c = row_info(cur_b, bc, cur_row);
      if (++guard > max_skip) return false;
    } while (c.blocks == 0);
    cur_s2 = c.s2_start;
  }
  return true;
}

// Greedy assignment of the cores (metadata.py:718-764, 872-923, 959-964).
// `bat` gives, per batch b, its row count / tail and summed cost / blocks /
// last block cost: bat.num(b), bat.tail(b), bat.cost(b), bat.block(b),
// bat.last(b); `row_info(b, bc, row)` one row's figures; `scan(cur_b, bc,
// limit, cur_row, c, cur_s2, ccost, cblock, bn2_cost, bn2_block)` the row
// phase, scan_rows's contract (the device runs it with the whole workgroup).
// Core i's end (bn2, m, s2) goes to ends[i] for i < cap (zeroed by the
// caller). Returns the number of cores used, or -1 when a row scan steps
// over more than max_skip rows without blocks.
template <typename W, typename Bat, typename RowFn, typename ScanFn>
SAS_HD i64 assign(const Sched<W>& s, const Bat& bat, i64 total_cost, i64 max_row_cost, bool all_zero,
                  RowFn&& row_info, i64 (*ends)[3], i64 cap, ScanFn&& scan) {
  const i64 aic = s.in.aic, B = s.B, hkv = s.in.heads_kv;
  if (all_zero) {
    if (cap > 0) { ends[0][0] = B * hkv; ends[0][1] = 0; ends[0][2] = 0; }
    return 1;
  }
  i64 used = 0;
  if (aic > 0) {
    i64 cur_b = 0, cur_bn2 = 0, cur_row = 0, cur_s2;
    i64 unassigned = total_cost;
    i64 bn2_cost = bat.cost(0), bn2_block = bat.block(0);
    BatchCtx<W> bc = s.batch_ctx(0);
    RowInfo c = row_info(0, bc, 0);
    cur_s2 = c.s2_start;
    bool finished = false;
    i64 core = 0;
    for (i64 i = 0; i < aic; ++i) {
      if (finished || unassigned <= 0) break;
      core = i;
      const i64 avg = (i64)floordiv<i64>(unassigned, smax<i64>(1, aic - i));
      const i64 limit = smax(avg, max_row_cost);
      i64 ccost = 0, cblock = 0;
      // whole (batch, kv-head) units
      while (bn2_cost == 0 || limit + bat.last(cur_b) / 2 >= ccost + bn2_cost) {
        ccost += bn2_cost;
        cblock += bn2_block;
        cur_bn2 += 1;
        if (cur_bn2 == B * hkv) { cur_row = 0; cur_s2 = 0; finished = true; break; }
        if (cur_bn2 / hkv != cur_b) { cur_b = cur_bn2 / hkv; bc = s.batch_ctx(cur_b); }
        bn2_cost = bat.cost(cur_b);
        bn2_block = bat.block(cur_b);
        cur_row = 0;
        c = row_info(cur_b, bc, cur_row);
        cur_s2 = c.s2_start;
      }
      // single rows
      if (!finished && !scan(cur_b, bc, limit, cur_row, c, cur_s2, ccost, cblock, bn2_cost, bn2_block)) return -1;
      if (i < cap) { ends[i][0] = cur_bn2; ends[i][1] = cur_row; ends[i][2] = cur_s2; }
      unassigned -= ccost;
    }
    used = core + 1;
  }
  return smax<i64>(used, 1);
}

// Output rows (metadata.py:974-1009): fa[36][8] (enable, bn2_start, m_start,
// s2_start, bn2_end, m_end, s2_end, first_fd_ws), then zeros.
SAS_HD inline void write_rows(i64 aic, i64 used, const i64 (*ends)[3], int32_t* out, int meta_size,
                              int aic_rows, int row_size) {
  for (int i = 0; i < meta_size; ++i) out[i] = 0;
  for (i64 i = 0; i < aic_rows; ++i) {
    if (i >= used || i >= aic) continue;
    int32_t* r = out + i * row_size;
    r[0] = 1;
    if (i > 0) { r[1] = (int32_t)ends[i - 1][0]; r[2] = (int32_t)ends[i - 1][1]; r[3] = (int32_t)ends[i - 1][2]; }
    r[4] = (int32_t)ends[i][0]; r[5] = (int32_t)ends[i][1]; r[6] = (int32_t)ends[i][2];
    r[7] = 0;
  }
}

// The whole schedule on the host, sequentially (sas_metadata_v1 with W =
// 128-bit; the tests also run it with the device's 64-bit saturated
// arithmetic). Writes the int32[SAS_META_SIZE] rows (meta_size, aic_rows,
// row_size: SAS_META_SIZE, SAS_AIC_CORE_NUM, SAS_FA_METADATA_SIZE); returns
// the cores used, or -1 when a row scan steps over max_skip empty rows.
template <typename W>
i64 run_host(const Inputs& in, bool saturate, i64 max_skip, int32_t* out, int meta_size = 1024,
             int aic_rows = 36, int row_size = 8) {
  struct Batches {
    std::vector<i64> n, tl, c, bl, la;
    i64 num(i64 b) const { return n[b]; }
    i64 tail(i64 b) const { return tl[b]; }
    i64 cost(i64 b) const { return c[b]; }
    i64 block(i64 b) const { return bl[b]; }
    i64 last(i64 b) const { return la[b]; }
  };
  Sched<W> s;
  s.in = in;
  s.derive(saturate);
  const i64 B = s.B;
  Batches bat;
  const size_t nb = (size_t)smax<i64>(B, 0);
  bat.n.assign(nb, 0); bat.tl.assign(nb, 0); bat.c.assign(nb, 0); bat.bl.assign(nb, 0); bat.la.assign(nb, 0);
  bool all_zero = true;
  for (i64 b = 0; b < B; ++b) {
    i64 s2n = 0;
    s.batch_dims(b, bat.n[b], bat.tl[b], s2n);
    if (bat.n[b] != 0 && s2n != 0) all_zero = false;
  }
  // per-batch costs (metadata.py:685-714)
  i64 total_cost = 0, max_row_cost = 0;
  if (!all_zero) {
    for (i64 b = 0; b < B; ++b) {
      if (s.s1_len(b) == 0 || s.s2_len(b) == 0) continue;
      const BatchCtx<W> bc = s.batch_ctx(b);
      RowCache c;
      for (i64 row = 0; row < bat.n[b]; ++row) {
        s.fill_row(row, bc, bat.n[b], bat.tl[b], c);
        bat.c[b] += c.cost;
        bat.bl[b] += c.blocks;
        max_row_cost = smax(max_row_cost, c.cost);
        if (c.blocks > 0) bat.la[b] = c.last_cost;
      }
      total_cost += bat.c[b] * in.heads_kv;
    }
  }
  auto row_info = [&](i64 b, const BatchCtx<W>& bc, i64 row) {
    RowCache c;
    s.fill_row(row, bc, bat.n[b], bat.tl[b], c);
    return RowInfo{c.cost, c.blocks, c.last_cost, c.s2_start};
  };
  std::vector<i64> ends(3 * (size_t)smax<i64>(in.aic, 1), 0);
  auto* e3 = reinterpret_cast<i64(*)[3]>(ends.data());
  auto scan = [&](i64 b, const BatchCtx<W>& bc, i64 limit, i64& cur_row, RowInfo& c, i64& cur_s2, i64& ccost,
                  i64& cblock, i64& bn2_cost, i64& bn2_block) {
    return scan_rows<W>(row_info, b, bc, limit, max_skip, cur_row, c, cur_s2, ccost, cblock, bn2_cost, bn2_block);
  };
  const i64 used = assign(s, bat, total_cost, max_row_cost, all_zero, row_info, e3, in.aic, scan);
  if (used < 0) return -1;
  write_rows(in.aic, used, e3, out, meta_size, aic_rows, row_size);
  return used;
}

}  // namespace sched
}  // namespace sas
