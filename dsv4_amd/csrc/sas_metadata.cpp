// Host entry point of the work scheduler for sparse_attn_sharedkv, bit-exact
// with the reference scheduler (sparse_attn_sharedkv_tilelang/metadata.py:
// 258-1086, itself a port of the Ascend AICPU SparseAttnSharedkvMetadata
// kernel). The schedule itself (row costs, greedy core assignment, output
// rows) is sas_sched.h, shared with the device entry point; here it runs with
// 128-bit token arithmetic, as the reference computes in unbounded integers.

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/sas.h"
#include "sas_common.h"
#include "sas_sched.h"

namespace {

using sas::sched::i64;
using i128 = __int128;

int layout_of(const char* s, const char* dflt) {
  const std::string l = s ? s : dflt;
  if (l == "TND") return sas::sched::kLayoutTND;
  if (l == "BSND") return sas::sched::kLayoutBSND;
  if (l == "BSH") return sas::sched::kLayoutBSH;
  return sas::sched::kLayoutOther;
}

int run(const sas::sched::Inputs& in, int32_t* out) {
  if (sas::sched::run_host<i128>(in, false, sas::sched::kMaxRowSkip, out) < 0)
    return sas::set_error(SAS_EINVAL, "metadata: row scan does not terminate");
  return SAS_OK;
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
  sas::sched::Inputs in{};
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
  // batch count sanity: every per-batch array must cover B entries
  i64 B;
  if (in.n_seq_q > 0) B = in.n_seq_q;
  else if (in.layout_q == sas::sched::kLayoutTND && in.n_cu_q > 0) B = in.n_cu_q - 1;
  else B = in.batch_arg;
  if (B < 0) return sas::set_error(SAS_EINVAL, "metadata: negative batch size");
  if (in.n_seq_kv > 0 && in.n_seq_kv < B)
    return sas::set_error(SAS_EINVAL, "metadata: seqused_kv has %lld entries, batch is %lld",
                          (long long)in.n_seq_kv, (long long)B);
  if (in.n_seq_kv == 0 && in.layout_kv == sas::sched::kLayoutTND && in.n_cu_kv > 0 && in.n_cu_kv < B + 1)
    return sas::set_error(SAS_EINVAL, "metadata: cu_seqlens_ori_kv too short");
  return run(in, out);
}
