/*
 * Native (C) caller of libsas's C ABI, as an FFI binding of the reference's
 * operator would be: include/sas.h only, no Python. Reads scheduler cases
 * from stdin, one per line:
 *   name nhq nhkv hd B max_sq max_skv ori_topk cmp_topk ratio ori_mask
 *   cmp_mask win_l win_r layout_q layout_kv has_ori has_cmp aic aiv
 *   n cu_seqlens_q... n seqused_kv... n seqused_q...
 * and prints "name v0 .. v1023" (sas_metadata_v1's int32[1024]) per case,
 * then checks argument errors of the other entry points on the host and
 * prints "ABI ok" (or "ABI FAIL <what>").
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sas.h"

static int read_arr(int32_t** out, int64_t* n) {
  long long m;
  if (scanf("%lld", &m) != 1) return 0;
  *n = m;
  *out = m ? (int32_t*)malloc(sizeof(int32_t) * (size_t)m) : NULL;
  for (long long i = 0; i < m; ++i) {
    int v;
    if (scanf("%d", &v) != 1) return 0;
    (*out)[i] = v;
  }
  return 1;
}

#define CHECK(cond, what)                                  \
  do {                                                     \
    if (!(cond)) {                                         \
      printf("ABI FAIL %s (%s)\n", what, sas_last_error()); \
      return 1;                                            \
    }                                                      \
  } while (0)

int main(void) {
  char name[128], lq[16], lkv[16];
  long long v[19];
  while (scanf("%127s", name) == 1) {
    if (strcmp(name, "END") == 0) break;
    for (int i = 0; i < 13; ++i)
      if (scanf("%lld", &v[i]) != 1) return 2;
    if (scanf("%15s %15s", lq, lkv) != 2) return 2;
    for (int i = 13; i < 17; ++i)
      if (scanf("%lld", &v[i]) != 1) return 2;
    SasMetaParams p;
    memset(&p, 0, sizeof(p));
    p.num_heads_q = v[0]; p.num_heads_kv = v[1]; p.head_dim = v[2];
    p.batch_size = v[3]; p.max_seqlen_q = v[4]; p.max_seqlen_kv = v[5];
    p.ori_topk = v[6]; p.cmp_topk = v[7]; p.cmp_ratio = v[8];
    p.ori_mask_mode = v[9]; p.cmp_mask_mode = v[10]; p.ori_win_left = v[11]; p.ori_win_right = v[12];
    p.layout_q = lq; p.layout_kv = lkv;
    p.has_ori_kv = (int32_t)v[13]; p.has_cmp_kv = (int32_t)v[14];
    p.aic_core_num = v[15]; p.aiv_core_num = v[16];
    int32_t *cu = NULL, *skv = NULL, *sq = NULL;
    if (!read_arr(&cu, &p.n_cu_seqlens_q) || !read_arr(&skv, &p.n_seqused_kv) || !read_arr(&sq, &p.n_seqused_q))
      return 2;
    p.cu_seqlens_q = cu; p.seqused_kv = skv; p.seqused_q = sq;
    int32_t out[SAS_META_SIZE];
    const int rc = sas_metadata_v1(&p, out);
    printf("%s %d", name, rc);
    for (int i = 0; i < SAS_META_SIZE; ++i) printf(" %d", out[i]);
    printf("\n");
    free(cu); free(skv); free(sq);
  }

  /* argument errors, host side only (no device memory is touched) */
  CHECK(sas_metadata_v1(NULL, NULL) == SAS_EINVAL, "metadata null");
  SasFwdArgs a;
  memset(&a, 0, sizeof(a));
  a.T = 4; a.B = 1; a.H = 64; a.D = 576; a.DV = 512; a.K = 512; a.scenario = SAS_SCFA;
  a.q_dtype = a.kv_dtype = SAS_DT_BF16; a.cmp_ratio = 4; a.win_left = 127; a.softmax_scale = 0.04f;
  int32_t splits = -1;
  size_t ws = 1;
  CHECK(sas_fwd_plan(&a, &splits, &ws) == SAS_OK && splits >= 1, "fwd plan");
  CHECK(sas_fwd_v1(&a, NULL) == SAS_EINVAL && strstr(sas_last_error(), "null"), "fwd null pointers");
  a.D = 100;
  CHECK(sas_fwd_plan(&a, &splits, &ws) == SAS_EINVAL && strstr(sas_last_error(), "D must be"), "fwd bad D");
  SasBwdArgs b;
  memset(&b, 0, sizeof(b));
  b.fwd = a;
  b.fwd.D = 576; b.fwd.kv_dtype = SAS_DT_FP8_E4M3_ROW656;
  CHECK(sas_bwd_v1(&b, NULL) == SAS_EINVAL && strstr(sas_last_error(), "fp8"), "bwd fp8 cache");
  SasCacheWriteArgs w;
  memset(&w, 0, sizeof(w));
  w.N = 0; w.B = 1; w.D = 576; w.kv_stride = 576; w.bt_stride = 1; w.block_size = 64; w.num_blocks = 1;
  CHECK(sas_cache_write_v1(&w, NULL) == SAS_OK, "cache write empty");
  w.N = 3;
  CHECK(sas_cache_write_v1(&w, NULL) == SAS_EINVAL, "cache write null");
  SasCombineArgs c;
  memset(&c, 0, sizeof(c));
  CHECK(sas_combine_v1(&c, NULL) == SAS_EINVAL, "combine null");
  CHECK(strstr(sas_version(), "gfx950") != NULL, "version");
  printf("ABI ok\n");
  return 0;
}
