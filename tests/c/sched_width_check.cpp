// The work schedule (dsv4_amd/csrc/sas_sched.h) with the host's 128-bit
// token arithmetic and with the device's 64-bit arithmetic whose INT64_MAX
// bounds are saturated at 2^40: the same rows on seeded random inputs that
// include windows around and far beyond 2^40, every mask mode and layout,
// empty batches and sequences. Usage: sched_width_check [cases] [seed];
// prints "ok <cases>" or the first difference.

#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "../../dsv4_amd/csrc/sas_sched.h"

using sas::sched::i64;
using i128 = __int128;

int main(int argc, char** argv) {
  const int n = argc > 1 ? atoi(argv[1]) : 20000;
  std::mt19937_64 rng(argc > 2 ? strtoull(argv[2], nullptr, 10) : 2026);
  auto pick = [&](std::initializer_list<i64> v) { return *(v.begin() + rng() % v.size()); };
  const i64 big = i64(1) << 40;
  for (int it = 0; it < n; ++it) {
    const i64 B = pick({0, 1, 2, 3, 7, 16, 48});
    std::vector<int32_t> ql(B), kl(B), cu(B + 1, 0);
    for (i64 b = 0; b < B; ++b) {
      ql[b] = (int32_t)pick({0, 1, 2, 3, 5, 64, 65, 200, 513});
      kl[b] = (int32_t)std::max<i64>(0, ql[b] + pick({-3, 0, 1, 7, 511, 512, 513, 4000, 70000}));
      cu[b + 1] = cu[b] + ql[b];
    }
    sas::sched::Inputs in{};
    const i64 hkv = pick({1, 1, 2, 4});
    in.heads_kv = hkv;
    in.heads_q = hkv * pick({1, 3, 16, 64, 128});
    in.layout_q = (int)pick({0, 1, 2, 3});
    in.layout_kv = (int)pick({0, 1});
    const bool use_seq_kv = rng() % 5 != 0;
    if (use_seq_kv) { in.seq_kv = kl.data(); in.n_seq_kv = B; }
    std::vector<int32_t> cukv(B + 1, 0);
    for (i64 b = 0; b < B; ++b) cukv[b + 1] = cukv[b] + kl[b];
    if (!use_seq_kv && in.layout_kv == sas::sched::kLayoutTND && B > 0) { in.cu_kv = cukv.data(); in.n_cu_kv = B + 1; }
    if (in.layout_q == sas::sched::kLayoutTND && B > 0) { in.cu_q = cu.data(); in.n_cu_q = B + 1; }
    else if (rng() % 2 && B > 0) { in.seq_q = ql.data(); in.n_seq_q = B; }
    in.batch_arg = B;
    i64 mq = 0, mk = 0;
    for (i64 b = 0; b < B; ++b) { mq = std::max<i64>(mq, ql[b]); mk = std::max<i64>(mk, kl[b]); }
    in.max_q = mq;
    in.max_kv = mk;
    in.has_cmp = rng() % 10 < 7;
    in.cmp_ratio = in.has_cmp ? pick({1, 4, 128, 0, -1}) : -1;
    in.cmp_topk = in.has_cmp ? pick({0, 64, 512, 2048}) : 0;
    in.mask_mode = pick({0, 1, 2, 3, 4, 4, 4, 5});
    in.win_left = pick({-7, -1, 0, 1, 127, 511, 512, big - 1, big, big + 5, i64(1) << 50, i64(1) << 62,
                        INT64_MAX - 1});
    in.aic = pick({1, 2, 5, 24, 36, 40});
    int32_t a[1024], b[1024];
    const i64 ua = sas::sched::run_host<i128>(in, false, i64(1) << 12, a);
    const i64 ub = sas::sched::run_host<i64>(in, true, i64(1) << 12, b);
    bool same = ua == ub;
    if (same && ua >= 0)
      for (int i = 0; i < 1024; ++i) same = same && a[i] == b[i];
    if (!same) {
      printf("case %d differs: B=%" PRId64 " mask=%" PRId64 " win_left=%" PRId64 " layout_q=%d used %" PRId64
             " vs %" PRId64 "\n", it, B, in.mask_mode, in.win_left, in.layout_q, ua, ub);
      return 1;
    }
  }
  printf("ok %d\n", n);
  return 0;
}
