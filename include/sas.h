/*
 * sas.h — C ABI of libsas.so, the MI355X (gfx950) implementation of
 * sparse_attn_sharedkv: fused sliding-window + top-k compressed-KV attention
 * over one shared K=V latent cache, with online softmax and per-head sinks.
 *
 * Plain pointers and sizes only. Device pointers are HIP device addresses;
 * `stream` is a hipStream_t passed as void*. Functions return SAS_OK (0) or
 * an error code, with a message available from sas_last_error() (thread-local).
 * The library never allocates or frees caller memory and keeps no pointer
 * after a call returns.
 */
#ifndef SAS_H_
#define SAS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Metadata layout, sparse_attn_sharedkv_tilelang/metadata.py:38-60. */
#define SAS_META_SIZE 1024
#define SAS_AIC_CORE_NUM 36
#define SAS_AIV_CORE_NUM 72
#define SAS_FA_METADATA_SIZE 8
#define SAS_FD_METADATA_SIZE 8

enum {
  SAS_OK = 0,
  SAS_EINVAL = 1,  /* bad argument / unsupported shape */
  SAS_ELAUNCH = 2, /* HIP launch or runtime error */
  SAS_ENOWS = 3    /* workspace missing or too small */
};

/* Element formats. */
enum {
  SAS_DT_BF16 = 0,
  SAS_DT_FP16 = 1,
  /* 656-byte fp8 cache row: 512 e4m3fn latent | 4 fp32 scales (one per 128
     latent channels) | 64 bf16 rope channels. Dequantised value =
     e4m3(byte) * scale[channel / 128]. */
  SAS_DT_FP8_E4M3_ROW656 = 2
};

/* Index-source scenario, sparse_attn_sharedkv_tilelang/api.py:196-202. */
enum { SAS_SWA = 1, SAS_CFA = 2, SAS_SCFA = 3 };

/*
 * Scheduler inputs; mirrors the keyword arguments of
 * sparse_attn_sharedkv_metadata (sparse_attn_sharedkv_tilelang/metadata.py:
 * 1018-1045). Optional int32 arrays are (pointer, element count) pairs with
 * a NULL pointer / zero count when absent. Layouts are the reference strings
 * ("BSND", "BSH", "TND", "BNSD", "PA_ND", ...).
 */
typedef struct SasMetaParams {
  int64_t num_heads_q, num_heads_kv, head_dim;
  int64_t batch_size, max_seqlen_q, max_seqlen_kv;
  int64_t ori_topk, cmp_topk, cmp_ratio;
  int64_t ori_mask_mode, cmp_mask_mode, ori_win_left, ori_win_right;
  const char* layout_q;
  const char* layout_kv;
  int32_t has_ori_kv, has_cmp_kv;
  int64_t aic_core_num, aiv_core_num;
  const int32_t* cu_seqlens_q;      int64_t n_cu_seqlens_q;
  const int32_t* cu_seqlens_ori_kv; int64_t n_cu_seqlens_ori_kv;
  const int32_t* cu_seqlens_cmp_kv; int64_t n_cu_seqlens_cmp_kv;
  const int32_t* seqused_q;         int64_t n_seqused_q;
  const int32_t* seqused_kv;        int64_t n_seqused_kv;
} SasMetaParams;

/*
 * Host-side cost-balanced schedule, bit-exact with the reference scheduler.
 * Replaces sparse_attn_sharedkv_tilelang/metadata.py:1018-1086
 * (_MetadataScheduler.run, metadata.py:258-1015). Writes int32[1024]:
 * fa[36][8] (enable, bn2_start, m_start, s2_start, bn2_end, m_end, s2_end,
 * first_fd_ws) followed by fd[72][8] and zero padding.
 */
int sas_metadata_v1(const SasMetaParams* p, int32_t* out /* [SAS_META_SIZE] */);

/*
 * The same schedule computed on the GPU, for callers whose sequence lengths
 * live there: no device -> host copy and no synchronisation, where the
 * reference reads them back to the host for it (api.py:210, 336, 361;
 * metadata.py:1018-1086). The SasMetaParams arrays (cu_seqlens_*,
 * seqused_*) are DEVICE pointers with their host-side lengths; `out` is a
 * device int32[SAS_META_SIZE], written by one launch on `stream`. Bit-exact
 * with sas_metadata_v1. At most 1024 batches (SAS_EINVAL beyond). A call
 * whose schedule sas_metadata_v1 rejects with SAS_EINVAL on the data (a row
 * scan that does not end), or whose batches hold more than 2^22 query rows in
 * all, leaves out[0] = -1 (no valid schedule has a negative core flag).
 */
int sas_metadata_device_v1(const SasMetaParams* p, int32_t* out /* device [SAS_META_SIZE] */, void* stream);

/*
 * Forward arguments; the device tensors of the reference kernel callable
 * (sparse_attn_sharedkv_tilelang/kernel.py:158-178) plus dims and strides.
 * q/out are flat token-major [T, H, D] / [T, H, DV]; q_prefix/act_q give each
 * batch's first packed token and query length (TND: cu_seqlens_q[:-1] and
 * lengths; BSND: b*S_max and S_max). With act_q = NULL, q_prefix is
 * cu_seqlens_q itself ([B + 1], the lengths being its differences), so a
 * TND caller passes its device cu_seqlens_q unchanged. Caches are
 * [num_blocks, block_size, 1, row] with row = D elements (bf16/fp16) or 656
 * bytes (fp8 rows).
 */
typedef struct SasFwdArgs {
  const void* q;                 /* [T, H, D] q_dtype */
  const void* ori_kv;            /* paged raw KV */
  const int32_t* ori_block_table;/* [B, ori_bt_stride] */
  const void* cmp_kv;            /* paged compressed KV (CFA/SCFA) or NULL */
  const int32_t* cmp_block_table;/* [B, cmp_bt_stride] or NULL */
  const int32_t* cmp_indices;    /* [T, 1, K] (SCFA) or NULL */
  const int32_t* q_prefix;       /* [B], or [B + 1] = cu_seqlens_q when act_q is NULL */
  const int32_t* act_q;          /* [B] or NULL */
  const int32_t* act_kv;         /* [B] seqused_kv */
  const float* sinks;            /* [H] */
  void* out;                     /* [T, H, DV] q_dtype */
  float* lse;                    /* [T, H] */
  void* workspace;               /* split-KV partials; size from sas_fwd_plan */
  size_t workspace_bytes;
  int64_t T, B, H, D, DV;
  int64_t ori_block_size, ori_bt_stride, ori_num_blocks;
  int64_t cmp_block_size, cmp_bt_stride, cmp_num_blocks;
  int64_t K;                     /* SCFA: top-k width; CFA: compressed slots per row */
  int32_t scenario;              /* SAS_SWA / SAS_CFA / SAS_SCFA */
  int32_t q_dtype;               /* SAS_DT_BF16 or SAS_DT_FP16 */
  int32_t kv_dtype;              /* q_dtype, or SAS_DT_FP8_E4M3_ROW656 with bf16 q */
  int32_t cmp_ratio;
  int32_t win_left;              /* ori_win_left (window = win_left + 1 rows) */
  float softmax_scale;
  int32_t num_splits;            /* KV splits per token, 1..65536; 0 = choose
                                    automatically (at most 64, more when a token's
                                    win_left + 1 + K key slots exceed 64 x 1280;
                                    at most 65536 x 1280 slots per token).
                                    Above 1 on a window-only call, it selects the
                                    streaming schedule over the one-split exact one */
  int32_t head_waves;            /* waves sharing each KV tile (16 heads each): 1, 2, 4;
                                    the other waves/head_waves groups stream disjoint rows;
                                    0 = choose automatically */
  int32_t flags;                 /* SAS_FWD_* bits, 0 by default */
  int32_t waves;                 /* waves per workgroup: 4 or 8 (fp8 rows: 4);
                                    0 = choose automatically. 8 also selects the
                                    streaming schedule where a split's rows would
                                    fit one LDS ring (window-only calls, 16-head
                                    groups), which then runs 4 waves */
} SasFwdArgs;

/* SasFwdArgs.flags: with more than one split, stop after the split kernel and
   leave the partials in the workspace (part_o at offset 0, part_ml after
   T*S*H*DV partial elements, S = the planned split count; layout as in
   SasCombineArgs); the caller then runs
   sas_combine_v1 itself, e.g. to time or overlap the two kernels apart. */
#define SAS_FWD_NO_COMBINE 1

/* SasFwdArgs.flags of a sas_bwd_v1 call (the forward rejects them): how the
   window rows' gradients are summed. SAS_BWD_WINDOW_TOKENS: one fp32 add per
   (token, row, head group, channel). SAS_BWD_WINDOW_KEYS: a key-major pass
   sums each window row's gradient over the tokens whose window holds it and
   adds it once per 16-head group; it runs beside the per-token kernel on a
   side stream of the library (one per device, created on first use, forked
   from and joined back to `stream` by events; one after the other on
   `stream` while it is being captured). Neither flag: the key-major pass for
   calls with at least 64 query tokens per batch on average that are not
   being captured, per-token adds otherwise. The results agree up to fp32
   summation order. */
#define SAS_BWD_WINDOW_TOKENS 2   /* per-token adds for window rows */
#define SAS_BWD_WINDOW_KEYS 4     /* the key-major window pass */

/*
 * Split count the library would use (after auto-selection) and the
 * workspace bytes it needs for these arguments (0 when no split is used).
 */
int sas_fwd_plan(const SasFwdArgs* a, int32_t* num_splits, size_t* workspace_bytes);

/*
 * Launch the fused forward on `stream`: one workgroup per (token, head group,
 * KV split), gather through block tables into LDS, bf16/fp16 MFMA for QK^T and
 * PV, sink-seeded online softmax, and (when splits > 1) the LSE combine.
 * Replaces the jitted callable of kernel.py:156-178 / api.py:372-384.
 */
int sas_fwd_v1(const SasFwdArgs* a, void* stream);

/*
 * sas_fwd_v1 without any allocation by caller or library, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The split partials go to a 16 MiB (16777216-byte) device array of the
 * library (one per device, held until the process ends) instead of a caller
 * workspace: `workspace` / `workspace_bytes` are ignored, and a call whose
 * plan needs more (the workspace size sas_fwd_plan reports) fails with
 * SAS_ENOWS. SAS_FWD_NO_COMBINE is rejected. `stream` must belong to the
 * current device. Calls that overlap on one device share the array and race:
 * serialise them (one stream, or events).
 */
int sas_fwd_noalloc_v1(const SasFwdArgs* a, void* stream);

/*
 * Split-KV LSE combine (no counterpart launched by the reference: its
 * flash-decode fields stay zero, metadata.py:323-325): for each (token, head)
 * M = max(sink, m_i), L = e^(sink-M) + sum_i l_i e^(m_i-M),
 * out = sum_i e^(m_i-M) O_i / L, lse = M + ln L.
 * part_o [T, S, H, DV]: the unnormalised O_i scaled by 2^e, with one integer
 * e per (token, split, head) and 256-channel half (O_i = value * 2^-e,
 * exactly); elements are fp16 when out_dtype is bf16 (e puts each half's
 * largest |value| in [2^14, 2^15)) and fp32 when out_dtype is fp16 (e = 0 as
 * written by sas_fwd_v1); part_ml [T, S, H, 4] fp32: (running max in log2 units, running
 * sum, e of channels 0-255, e of channels 256-511). A negative running sum
 * marks a padded token (out = 0, lse = 0).
 */
typedef struct SasCombineArgs {
  const void* part_o;
  const float* part_ml;
  const float* sinks;
  void* out;
  float* lse;
  int64_t T, S, H, DV;           /* S: 1..65536 splits */
  int32_t out_dtype;             /* SAS_DT_BF16 or SAS_DT_FP16 */
} SasCombineArgs;

int sas_combine_v1(const SasCombineArgs* a, void* stream);

/*
 * Backward of sas_fwd_v1 (no counterpart launched by the reference, whose
 * LSE output is documented as the input of a FlashAttention-v2 style
 * backward, api.py:32-35, 176-184). `fwd` holds the forward's arguments:
 * q, caches (in the query dtype; fp8 rows are not differentiated), tables,
 * indices, seqlens, sinks, and its outputs `out` / `lse`, which are inputs
 * here; its workspace / head-group / wave fields are ignored, num_splits
 * (> 0) sets the KV split count (0: chosen to fill the CUs with splits of
 * at least 128 key slots; the forward's own plan does not carry over). Over the forward's
 * key set J of each (token, head), with P_j = exp(scale q.k_j - lse),
 * Delta = dout . out, dS_j = P_j (dout . v_j - Delta):
 *   dq = scale sum_j dS_j k_j                      (zero on entry; written or accumulated)
 *   d_kv[row j] += scale dS_j q + [P_j dout, 0]    (accumulated, V = the first DV channels)
 *   d_sinks[h] += -exp(sink_h - lse) Delta         (accumulated)
 * All four outputs must be zeroed by the caller first; cache rows (and dq
 * with several KV splits) receive atomic fp32 adds, so their summation order
 * varies. Tokens with more than 1280 key slots (win_left + 1 + K) are split
 * across several workgroups. fwd.flags may hold SAS_BWD_WINDOW_TOKENS or
 * SAS_BWD_WINDOW_KEYS (how the window rows' gradients are summed; same
 * result up to fp32 summation order).
 */
typedef struct SasBwdArgs {
  SasFwdArgs fwd;
  const void* dout;              /* [T, H, DV] q_dtype */
  float* dq;                     /* [T, H, D] fp32, zero on entry */
  float* d_ori_kv;               /* [ori_num_blocks, ori_block_size, 1, D] fp32 */
  float* d_cmp_kv;               /* [cmp_num_blocks, cmp_block_size, 1, D] fp32; NULL for SWA */
  float* d_sinks;                /* [H] fp32 */
} SasBwdArgs;

int sas_bwd_v1(const SasBwdArgs* a, void* stream);

/*
 * Paged-KV cache writer (no counterpart in the reference, whose tests build
 * paged caches on the host in the layout of golden.py:315-408; this is the
 * device-side producer of that layout). Input row r (of N) goes to the cache
 * row of batch seq_ids[r] at logical position positions[r]: physical block
 * block_table[b * bt_stride + pos / block_size], offset pos % block_size.
 * Rows with a negative position, a batch outside [0, B), a position past the
 * table, or a table entry outside [0, num_blocks) (-1 = unused) are skipped.
 * cache_dtype == kv_dtype: the D channels are copied. cache_dtype ==
 * SAS_DT_FP8_E4M3_ROW656 (bf16 kv, D = 576): per 128 latent channels
 * scale = amax / 448 is stored and byte = e4m3fn(clamp(x * inv, -448, 448))
 * with inv = 448 / amax (both 1 for an all-zero group), rounded to nearest
 * even; rope channels copied as bf16. Rows written by one
 * call must be distinct (two rows to one cache row race).
 */
typedef struct SasCacheWriteArgs {
  const void* kv;                /* [N, kv_stride] kv_dtype, 16-byte aligned rows */
  const int32_t* seq_ids;        /* [N] batch of each row */
  const int32_t* positions;      /* [N] logical position in that batch's cache */
  const int32_t* block_table;    /* [B, bt_stride] */
  void* cache;                   /* [num_blocks, block_size, 1, row] */
  int64_t N, B, D, kv_stride;    /* kv_stride in elements */
  int64_t bt_stride, block_size, num_blocks;
  int32_t kv_dtype;              /* SAS_DT_BF16 or SAS_DT_FP16 */
  int32_t cache_dtype;           /* kv_dtype, or SAS_DT_FP8_E4M3_ROW656 */
} SasCacheWriteArgs;

int sas_cache_write_v1(const SasCacheWriteArgs* a, void* stream);

/* Thread-local message of the last failed call on this thread ("" if none). */
const char* sas_last_error(void);

/* Library version string. */
const char* sas_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SAS_H_ */
