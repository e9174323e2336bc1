// Device entry point of the work scheduler (sas_metadata_device_v1): the
// reference's int32[1024] schedule (sparse_attn_sharedkv_tilelang/
// metadata.py:258-1086) computed on the GPU from device-resident sequence
// lengths, so a caller whose lengths live on the device gets the tensor with
// no device -> host copy and no synchronisation (the reference reads them
// back to the host for this, api.py:210, 336, 361). The schedule is
// sas_sched.h, the host entry point's own code, with 64-bit token arithmetic.
//
// One workgroup of 256 threads:
//  1. per-batch row counts and tails (threads over batches) and their
//     exclusive scan;
//  2. every s1g row's cost, blocks, last block cost and first KV block
//     (threads over all rows of all batches): summed per batch with LDS
//     atomics, the largest row cost and each batch's last row with blocks;
//     the first kRowsMax rows' figures are kept in LDS;
//  3. each batch's last block cost, the total cost;
//  4. the greedy core assignment, run by every thread on the same figures
//     (so each holds the same state): the unit phase by each thread alone,
//     the row phase by the workgroup together, 256 rows at a time (prefix
//     sums of the candidate rows' costs, the first row that does not fit);
//     rows past kRowsMax, and rows past a batch's end that the scan steps
//     onto, are computed on the spot. Then every thread writes the output
//     rows.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "../../include/sas.h"
#include "sas_common.h"
#include "sas_sched.h"

namespace sas {
namespace {

using sched::i64;
using DevSched = sched::Sched<i64>;

constexpr int kThreads = 256;
constexpr int kMaxB = 1024;      // batches
constexpr int kRowsMax = 5120;   // rows whose figures stay in LDS
constexpr i64 kMaxRows = i64(1) << 22;   // rows in all
// The assignment's row scan past a batch's last row: stopped (and reported)
// after this many rows without blocks. The host scans up to 2^26 rows before
// it reports the same failure; here the bound is the row count itself, so
// within the 2^22 rows above the device reports the failure exactly where
// the host does.
constexpr i64 kDevRowSkip = kMaxRows;
// rows the row phase takes one at a time before it scans windows
constexpr int kSeqRows = 1;

struct Shared {
  i64 s1[kMaxB], s2[kMaxB];   // query / KV length of each batch
  i64 num[kMaxB], tail[kMaxB], first[kMaxB + 1], last[kMaxB];
  unsigned long long cost[kMaxB], block[kMaxB];
  long long lastrow[kMaxB];
  int32_t r_cost[kRowsMax], r_block[kRowsMax], r_last[kRowsMax], r_s2[kRowsMax];
  long long maxrow, total;
  int nonzero, used;
  i64 ends[SAS_AIC_CORE_NUM][3];
  // row-phase scratch: per-wave sums and first / last indices, one row's figures
  i64 w_cost[kThreads / 64], w_block[kThreads / 64];
  int w_first[kThreads / 64], w_fail[kThreads / 64], w_last[kThreads / 64];
  sched::RowInfo pick;
};

struct DevBatches {
  const Shared& s;
  __device__ i64 num(i64 b) const { return s.num[b]; }
  __device__ i64 tail(i64 b) const { return s.tail[b]; }
  __device__ i64 cost(i64 b) const { return (i64)s.cost[b]; }
  __device__ i64 block(i64 b) const { return (i64)s.block[b]; }
  __device__ i64 last(i64 b) const { return s.last[b]; }
};

__device__ sched::RowInfo compute_row(const DevSched& sc, const Shared& sh, i64 b,
                                      const sched::BatchCtx<i64>& bc, i64 row) {
  sched::RowCache c;
  sc.fill_row(row, bc, sh.num[b], sh.tail[b], c);
  return sched::RowInfo{c.cost, c.blocks, c.last_cost, c.s2_start};
}

// A row's figures: from LDS for the first kRowsMax rows of the batches,
// computed otherwise.
__device__ sched::RowInfo row_at(const DevSched& sc, const Shared& sh, i64 b, const sched::BatchCtx<i64>& bc,
                                 i64 row) {
  const i64 g = sh.first[b] + row;
  if (row < sh.num[b] && g < kRowsMax) return sched::RowInfo{sh.r_cost[g], sh.r_block[g], sh.r_last[g], sh.r_s2[g]};
  return compute_row(sc, sh, b, bc, row);
}

// Inclusive prefix sums of (a, b) over the workgroup's threads in order;
// the totals come back in ta, tb.
__device__ void block_scan2(Shared& sh, int tid, i64& a, i64& b, i64& ta, i64& tb) {
  const int lane = tid & 63, w = tid >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const i64 xa = __shfl_up(a, off), xb = __shfl_up(b, off);
    if (lane >= off) { a += xa; b += xb; }
  }
  if (lane == 63) { sh.w_cost[w] = a; sh.w_block[w] = b; }
  __syncthreads();
  i64 oa = 0, ob = 0;
  ta = 0; tb = 0;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) {
    if (i < w) { oa += sh.w_cost[i]; ob += sh.w_block[i]; }
    ta += sh.w_cost[i]; tb += sh.w_block[i];
  }
  a += oa;
  b += ob;
  __syncthreads();   // the per-wave sums are read before the next use
}

// The workgroup's smallest thread index with f0 / f1 set and largest with
// f2 set (kThreads / -1 when none).
__device__ void block_first(Shared& sh, int tid, bool f0, bool f1, bool f2, int& i0, int& i1, int& i2) {
  const int lane = tid & 63, w = tid >> 6;
  const unsigned long long m0 = __ballot(f0), m1 = __ballot(f1), m2 = __ballot(f2);
  if (lane == 0) {
    sh.w_first[w] = m0 ? w * 64 + __ffsll((long long)m0) - 1 : kThreads;
    sh.w_fail[w] = m1 ? w * 64 + __ffsll((long long)m1) - 1 : kThreads;
    sh.w_last[w] = m2 ? w * 64 + 63 - __clzll((long long)m2) : -1;
  }
  __syncthreads();
  i0 = kThreads; i1 = kThreads; i2 = -1;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) {
    i0 = min(i0, sh.w_first[i]);
    i1 = min(i1, sh.w_fail[i]);
    i2 = max(i2, sh.w_last[i]);
  }
  __syncthreads();
}

// The row phase (sched::scan_rows) with the whole workgroup: every thread
// calls it with the same state and gets the same state back. After the
// current row is taken, windows of kThreads rows follow: the candidates are
// the rows with blocks, a candidate fits while limit + last / 2 >= ccost +
// (the costs of the window's candidates up to and including it), and the
// first one that does not fit ends the phase as the next current row (with
// the candidates before it taken); a window without it is taken whole.
__device__ bool par_scan(const DevSched& sc, Shared& sh, int tid, i64 b, const sched::BatchCtx<i64>& bc,
                         i64 limit, i64 max_skip, i64& cur_row, sched::RowInfo& c, i64& cur_s2, i64& ccost,
                         i64& cblock, i64& bn2_cost, i64& bn2_block) {
  static_assert(kDevRowSkip >= kThreads, "a step inside one window stays within the skip bound");
  if (!(limit + c.last_cost / 2 >= ccost + c.cost)) return true;
  ccost += c.cost;
  cblock += c.blocks;
  bn2_cost = sched::smax<i64>(0, bn2_cost - c.cost);
  bn2_block = sched::smax<i64>(0, bn2_block - c.blocks);
  i64 gap = 0;   // rows stepped since the last row taken
  i64 base = cur_row + 1;
  // First a few rows one at a time, as scan_rows does: the phase often ends
  // at the next row (at a unit's end); then, if it has not ended, windows.
  for (int k = 0; k < kSeqRows; ++k) {
    sched::RowInfo r{};
    bool found = false;
    for (int q = 0; q < kSeqRows && !found; ++q) {
      r = row_at(sc, sh, b, bc, base);
      if (++gap > max_skip) return false;
      if (r.blocks != 0) found = true;
      else base += 1;
    }
    if (!found) break;   // the windows go on from `base`, `gap` rows stepped
    cur_row = base;
    c = r;
    cur_s2 = c.s2_start;
    if (!(limit + c.last_cost / 2 >= ccost + c.cost)) return true;
    ccost += c.cost;
    cblock += c.blocks;
    bn2_cost = sched::smax<i64>(0, bn2_cost - c.cost);
    bn2_block = sched::smax<i64>(0, bn2_block - c.blocks);
    gap = 0;
    base = cur_row + 1;
  }
  const i64 start = base;
  for (;; base += kThreads) {
    // a scan longer than all rows plus the skip bound ends as a failure
    // (bounds the loop whatever the figures)
    if (base - start > kMaxRows + kDevRowSkip) return false;
    const sched::RowInfo ri = row_at(sc, sh, b, bc, base + tid);
    const bool cand = ri.blocks != 0;
    i64 pc = cand ? ri.cost : 0, pb = cand ? ri.blocks : 0, tc, tb;
    block_scan2(sh, tid, pc, pb, tc, tb);
    const bool fail = cand && !(limit + ri.last_cost / 2 >= ccost + pc);
    int first, fi, last;
    block_first(sh, tid, cand, fail, cand, first, fi, last);
    if (first == kThreads) {   // no candidate: the step goes on
      gap += kThreads;
      if (gap > max_skip) return false;
      continue;
    }
    if (gap + first + 1 > max_skip) return false;
    if (fi < kThreads) {
      // candidates before fi are taken; fi is the next current row
      if (tid == fi) { sh.pick = ri; sh.w_cost[0] = pc - ri.cost; sh.w_block[0] = pb - ri.blocks; }
      __syncthreads();
      const i64 sc_ = sh.w_cost[0], sb_ = sh.w_block[0];
      ccost += sc_;
      cblock += sb_;
      bn2_cost = sched::smax<i64>(0, bn2_cost - sc_);
      bn2_block = sched::smax<i64>(0, bn2_block - sb_);
      cur_row = base + fi;
      c = sh.pick;
      cur_s2 = c.s2_start;
      __syncthreads();   // sh.pick / sums read before the scratch is reused
      return true;
    }
    ccost += tc;
    cblock += tb;
    bn2_cost = sched::smax<i64>(0, bn2_cost - tc);
    bn2_block = sched::smax<i64>(0, bn2_block - tb);
    gap = kThreads - 1 - last;
  }
}

__global__ void __launch_bounds__(kThreads) sas_sched_kernel(const sched::Inputs in, int32_t* out) {
  __shared__ Shared sh;
  const int tid = threadIdx.x;
  // The lengths are read from global memory once, into LDS, where the
  // schedule then reads them (Inputs::len_q / len_kv).
  DevSched sc;
  sc.in = in;
  sc.derive(true);
  const i64 B = sc.B;
  for (i64 b = tid; b < B; b += kThreads) { sh.s1[b] = sc.s1_len(b); sh.s2[b] = sc.s2_len(b); }
  sc.in.len_q = sh.s1;
  sc.in.len_kv = sh.s2;
  if (tid == 0) { sh.maxrow = 0; sh.total = 0; sh.nonzero = 0; sh.used = 1; }
  for (int i = tid; i < SAS_AIC_CORE_NUM * 3; i += kThreads) sh.ends[i / 3][i % 3] = 0;
  __syncthreads();

  // 1. per-batch dims (metadata.py:671-683)
  for (i64 b = tid; b < B; b += kThreads) {
    i64 s2n = 0;
    sc.batch_dims(b, sh.num[b], sh.tail[b], s2n);
    if (sh.num[b] != 0 && s2n != 0) sh.nonzero = 1;
    sh.cost[b] = 0;
    sh.block[b] = 0;
    sh.lastrow[b] = -1;
    sh.last[b] = 0;
  }
  __syncthreads();
  // exclusive scan of the row counts: each thread sums its run of
  // ceil(B / 256) batches, then a scan over the threads' sums
  {
    const i64 per = (B + kThreads - 1) / kThreads;
    const i64 b0 = tid * per, b1 = sched::smin<i64>(b0 + per, B);
    i64 run = 0;
    for (i64 b = b0; b < b1; ++b) run += sched::smax<i64>(sh.num[b], 0);   // (a negative count has no rows)
    __shared__ i64 part[kThreads];
    part[tid] = run;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
      const i64 v = tid >= off ? part[tid - off] : 0;
      __syncthreads();
      part[tid] += v;
      __syncthreads();
    }
    i64 acc = part[tid] - run;
    for (i64 b = b0; b < b1; ++b) { sh.first[b] = acc; acc += sched::smax<i64>(sh.num[b], 0); }
    if (tid == kThreads - 1) sh.first[B] = part[tid];
  }
  __syncthreads();

  // 2. every row (metadata.py:685-714): batches with no query or no KV
  // tokens add no cost (their rows' figures are still kept for the scan).
  // Beyond kMaxRows rows in all (~8 µs of this loop per thread) the call
  // reports failure instead of running for seconds.
  const i64 total_rows = sh.first[B];
  if (total_rows > kMaxRows) {
    for (int i = tid; i < SAS_META_SIZE; i += kThreads) out[i] = i == 0 ? -1 : 0;
    return;
  }
  // Each thread's rows lie in non-decreasing batches: its sums for the
  // current batch are added to LDS when the batch changes (and at the end),
  // one set of LDS atomics per batch a thread meets instead of per row.
  {
    i64 cb = -1, acc_c = 0, acc_b = 0, acc_last = -1, acc_max = 0;
    auto flush = [&] {
      if (cb < 0) return;
      atomicAdd(&sh.cost[cb], (unsigned long long)acc_c);
      atomicAdd(&sh.block[cb], (unsigned long long)acc_b);
      if (acc_last >= 0) atomicMax(&sh.lastrow[cb], (long long)acc_last);
    };
    for (i64 g = tid; g < total_rows; g += kThreads) {
      i64 lo = 0, hi = B;   // largest b with first[b] <= g
      while (hi - lo > 1) {
        const i64 mid = (lo + hi) / 2;
        if (sh.first[mid] <= g) lo = mid; else hi = mid;
      }
      const i64 b = lo, row = g - sh.first[b];
      const auto bc = sc.batch_ctx(b);
      const sched::RowInfo r = compute_row(sc, sh, b, bc, row);
      if (g < kRowsMax) {
        sh.r_cost[g] = (int32_t)r.cost;
        sh.r_block[g] = (int32_t)r.blocks;
        sh.r_last[g] = (int32_t)r.last_cost;
        sh.r_s2[g] = (int32_t)r.s2_start;
      }
      if (bc.s1 == 0 || bc.s2 == 0) continue;
      if (b != cb) {
        flush();
        cb = b; acc_c = 0; acc_b = 0; acc_last = -1;
      }
      acc_c += r.cost;
      acc_b += r.blocks;
      acc_max = sched::smax<i64>(acc_max, r.cost);
      if (r.blocks > 0) acc_last = row;   // rows of a batch come in increasing order
    }
    flush();
    if (acc_max > 0) atomicMax(&sh.maxrow, (long long)acc_max);
  }
  __syncthreads();

  // 3. each batch's last block cost, the total cost
  for (i64 b = tid; b < B; b += kThreads) {
    if (sh.lastrow[b] >= 0) {
      const i64 g = sh.first[b] + sh.lastrow[b];
      sh.last[b] = g < kRowsMax ? (i64)sh.r_last[g]
                                : compute_row(sc, sh, b, sc.batch_ctx(b), sh.lastrow[b]).last_cost;
    }
    if (sh.cost[b]) atomicAdd((unsigned long long*)&sh.total, (unsigned long long)((i64)sh.cost[b] * in.heads_kv));
  }
  __syncthreads();

  // 4. the assignment (metadata.py:718-764, 872-923, 959-964): every thread
  // runs it on the same LDS figures and holds the same state, so the row
  // phase's barriers are taken by all; the ends / used written by all are
  // equal
  {
    auto row_info = [&](i64 b, const sched::BatchCtx<i64>& bc, i64 row) { return row_at(sc, sh, b, bc, row); };
    auto scan = [&](i64 b, const sched::BatchCtx<i64>& bc, i64 limit, i64& cur_row, sched::RowInfo& c,
                    i64& cur_s2, i64& ccost, i64& cblock, i64& bn2_cost, i64& bn2_block) {
      return par_scan(sc, sh, tid, b, bc, limit, kDevRowSkip, cur_row, c, cur_s2, ccost, cblock, bn2_cost,
                      bn2_block);
    };
    const i64 used = sched::assign(sc, DevBatches{sh}, (i64)sh.total, (i64)sh.maxrow, sh.nonzero == 0, row_info,
                                   sh.ends, SAS_AIC_CORE_NUM, scan);
    __syncthreads();
    if (tid == 0) sh.used = (int)used;
  }
  __syncthreads();
  // output rows (metadata.py:974-1009); a row scan that does not end leaves
  // out[0] = -1 (where the host entry point returns SAS_EINVAL)
  const i64 used = sh.used;
  for (int i = tid; i < SAS_META_SIZE; i += kThreads) {
    const int core = i / SAS_FA_METADATA_SIZE, f = i % SAS_FA_METADATA_SIZE;
    int32_t v = 0;
    if (used < 0) {
      v = i == 0 ? -1 : 0;
    } else if (core < SAS_AIC_CORE_NUM && core < used && core < in.aic) {
      switch (f) {
        case 0: v = 1; break;
        case 1: case 2: case 3: v = core > 0 ? (int32_t)sh.ends[core - 1][f - 1] : 0; break;
        case 4: case 5: case 6: v = (int32_t)sh.ends[core][f - 4]; break;
        default: v = 0;
      }
    }
    out[i] = v;
  }
}

int layout_of(const char* s, const char* dflt) {
  const char* l = s ? s : dflt;
  auto eq = [](const char* a, const char* b) {
    while (*a && *a == *b) { ++a; ++b; }
    return *a == *b;
  };
  if (eq(l, "TND")) return sched::kLayoutTND;
  if (eq(l, "BSND")) return sched::kLayoutBSND;
  if (eq(l, "BSH")) return sched::kLayoutBSH;
  return sched::kLayoutOther;
}

}  // namespace
}  // namespace sas

extern "C" int sas_metadata_device_v1(const SasMetaParams* p, int32_t* out, void* stream) {
  using namespace sas;
  clear_error();
  if (!p || !out) return set_error(SAS_EINVAL, "metadata (device): null argument");
  if (p->num_heads_kv <= 0 || p->num_heads_q < p->num_heads_kv)
    return set_error(SAS_EINVAL, "metadata (device): need num_heads_kv > 0 and num_heads_q >= num_heads_kv "
                     "(got %lld, %lld)", (long long)p->num_heads_q, (long long)p->num_heads_kv);
  if (p->aic_core_num < 1 || p->aiv_core_num < 0)
    return set_error(SAS_EINVAL, "metadata (device): aic_core_num must be >= 1");
  sched::Inputs in{};
  in.heads_q = p->num_heads_q;
  in.heads_kv = p->num_heads_kv;
  in.cu_q = p->cu_seqlens_q; in.n_cu_q = p->cu_seqlens_q ? std::max<int64_t>(p->n_cu_seqlens_q, 0) : 0;
  in.cu_kv = p->cu_seqlens_ori_kv;
  in.n_cu_kv = p->cu_seqlens_ori_kv ? std::max<int64_t>(p->n_cu_seqlens_ori_kv, 0) : 0;
  in.seq_q = p->seqused_q; in.n_seq_q = p->seqused_q ? std::max<int64_t>(p->n_seqused_q, 0) : 0;
  in.seq_kv = p->seqused_kv; in.n_seq_kv = p->seqused_kv ? std::max<int64_t>(p->n_seqused_kv, 0) : 0;
  in.batch_arg = p->batch_size;
  in.max_q = p->max_seqlen_q;
  in.max_kv = p->max_seqlen_kv;
  in.cmp_topk = p->cmp_topk;
  in.cmp_ratio = p->cmp_ratio;
  in.mask_mode = p->ori_mask_mode;
  in.win_left = p->ori_win_left;
  in.layout_q = layout_of(p->layout_q, "BSND");
  in.layout_kv = layout_of(p->layout_kv, "PA_ND");
  in.has_cmp = p->has_cmp_kv != 0;
  in.aic = p->aic_core_num;
  int64_t B;
  if (in.n_seq_q > 0) B = in.n_seq_q;
  else if (in.layout_q == sched::kLayoutTND && in.n_cu_q > 0) B = in.n_cu_q - 1;
  else B = in.batch_arg;
  if (B < 0) return set_error(SAS_EINVAL, "metadata (device): negative batch size");
  if (B > kMaxB) return set_error(SAS_EINVAL, "metadata (device): at most %d batches (got %lld)", kMaxB, (long long)B);
  if (in.n_seq_kv > 0 && in.n_seq_kv < B)
    return set_error(SAS_EINVAL, "metadata (device): seqused_kv has %lld entries, batch is %lld",
                     (long long)in.n_seq_kv, (long long)B);
  if (in.n_seq_kv == 0 && in.layout_kv == sched::kLayoutTND && in.n_cu_kv > 0 && in.n_cu_kv < B + 1)
    return set_error(SAS_EINVAL, "metadata (device): cu_seqlens_ori_kv too short");
  hipLaunchKernelGGL(sas_sched_kernel, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, in, out);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SAS_ELAUNCH, "sas_sched launch: %s", hipGetErrorString(e));
  return SAS_OK;
}
