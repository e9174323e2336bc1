// Paged-KV cache writer for MI355X (gfx950): scatter new latent KV rows
// through a block table into the paged cache the forward kernels read,
// either as a plain bf16 / fp16 row copy or quantised into 656-byte fp8 rows
// (512 e4m3fn latent bytes | 4 fp32 scales, one per 128 latent channels |
// 64 bf16 rope channels).
//
// The reference has no cache writer: its tests build paged caches on the
// host (golden.py:315-408: row `pos` of batch b lives in physical block
// block_table[b, pos // block_size] at offset pos % block_size, -1 marks an
// unused table entry). This kernel writes rows in that layout on the device.
//
// One row per wave, four waves per workgroup. HBM-bound byte work: each
// lane moves 16 bytes in and (fp8) 8 bytes out per row; no LDS, no MFMA.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "../../include/sas.h"
#include "sas_common.h"


namespace sas {
namespace {

constexpr int kRow656 = 656, kLatent = 512, kScaleOff = 512, kRopeOff = 528;
constexpr float kE4m3Max = 448.f;

struct CwParams {
  const uint8_t* kv;
  const int32_t* seq_ids;
  const int32_t* positions;
  const int32_t* bt;
  uint8_t* cache;
  long long kv_stride_b;   // bytes between input rows
  int N, B, D, bt_stride, bs, nblocks;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Each wave handles kRowsPerWave consecutive rows: their data loads are
// issued first, then the destinations of all of them are resolved together
// (two dependent rounds of independent scalar loads: batch / position, then
// the table entry), so the data and index latencies overlap. Measured on the
// 32768-row fp8 write: 1 row per wave 16.5 us, 2 rows 29.0 us, 4 rows
// 28.5 us, 8 rows 24.7 us; a grid-stride loop over 1024 / 2048 / 4096
// workgroups whose waves load the next row while storing the current one:
// 18.7 / 17.7 / 18.2 us.
#ifndef SAS_CW_ROWS_PER_WAVE
#define SAS_CW_ROWS_PER_WAVE 1
#endif
constexpr int kRowsPerWave = SAS_CW_ROWS_PER_WAVE;
constexpr int kWaves = 4;

// Destination rows of input rows r0 .. r0 + kRowsPerWave - 1, null where a
// row is skipped (past N, negative position, batch out of range, position
// past the table, unused or out-of-range block). Wave-uniform; the table is
// read at a clamped index for skipped rows.
__device__ __forceinline__ void dest_rows(const CwParams& p, int r0, int row_bytes,
                                          uint8_t* (&dst)[kRowsPerWave]) {
  int b[kRowsPerWave], pos[kRowsPerWave], lb[kRowsPerWave], blk[kRowsPerWave];
  bool ok[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int r = min(r0 + i, p.N - 1);
    b[i] = p.seq_ids[r];
    pos[i] = p.positions[r];
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    ok[i] = r0 + i < p.N && b[i] >= 0 && b[i] < p.B && pos[i] >= 0 && pos[i] / p.bs < p.bt_stride;
    lb[i] = ok[i] ? pos[i] / p.bs : 0;
    blk[i] = p.bt[ok[i] ? (size_t)b[i] * p.bt_stride + lb[i] : 0];
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    ok[i] = ok[i] && blk[i] >= 0 && blk[i] < p.nblocks;
    dst[i] = ok[i] ? p.cache + ((size_t)blk[i] * p.bs + (pos[i] - lb[i] * p.bs)) * row_bytes : nullptr;
  }
}

// Plain copy: D 16-bit channels per row (D * 2 / 16 chunks of 16 bytes,
// at most 2 per lane for D <= 1024).
__global__ void __launch_bounds__(64 * kWaves) sas_cache_copy_kernel(const CwParams p) {
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * kRowsPerWave;
  if (r0 >= p.N) return;
  const int nch = p.D / 8;
  uint4 v[kRowsPerWave][2];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const uint8_t* src = p.kv + (size_t)min(r0 + i, p.N - 1) * p.kv_stride_b;
#pragma unroll
    for (int k = 0; k < 2; ++k)   // every lane loads (a clamped chunk), as in the fp8 kernel
      v[i][k] = *reinterpret_cast<const uint4*>(src + min(lane + 64 * k, nch - 1) * 16);
  }
  uint8_t* dst[kRowsPerWave];
  dest_rows(p, r0, p.D * 2, dst);
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    if (!dst[i]) continue;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int c = lane + 64 * k;
      if (c < nch) *reinterpret_cast<uint4*>(dst[i] + c * 16) = v[i][k];
    }
  }
}

// fp8 rows from bf16 input (D = 576): lane l quantises latent channels
// 8l .. 8l + 7 (group l / 16: the 16 lanes of a group reduce their amax with
// xor shuffles), lanes 0-7 copy the 64 rope channels, the first lane of each
// group writes its scale. scale = amax / 448 and inv = 448 / amax (both 1
// for an all-zero group), byte = e4m3fn(clamp(x * inv, -448, 448)), as
// dsv4_amd.paged.quantize_kv_fp8.
__device__ __forceinline__ void put_fp8_row(uint8_t* dst, const uint4& w, const uint4& rope, int lane) {
  const float x[8] = {bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y),
                      bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
  float amax = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(x[k]));
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  const float scale = amax > 0.f ? amax / kE4m3Max : 1.f;
  const float inv = amax > 0.f ? kE4m3Max / amax : 1.f;
  // v_cvt_pk_fp8_f32: two floats -> two OCP e4m3fn bytes, nearest even
  // (the same bytes as torch's float8_e4m3fn conversion for every bf16
  // input; 2x faster here than a bit-level encoder)
  uint32_t q[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int t = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(x[4 * h] * inv, -kE4m3Max, kE4m3Max),
                                            __builtin_amdgcn_fmed3f(x[4 * h + 1] * inv, -kE4m3Max, kE4m3Max),
                                            0, false);
    t = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(x[4 * h + 2] * inv, -kE4m3Max, kE4m3Max),
                                        __builtin_amdgcn_fmed3f(x[4 * h + 3] * inv, -kE4m3Max, kE4m3Max),
                                        t, true);
    q[h] = (uint32_t)t;
  }
  *reinterpret_cast<uint2*>(dst + lane * 8) = make_uint2(q[0], q[1]);
  if ((lane & 15) == 0) *reinterpret_cast<float*>(dst + kScaleOff + (lane >> 4) * 4) = scale;
  if (lane < 8) *reinterpret_cast<uint4*>(dst + kRopeOff + lane * 16) = rope;
}

__global__ void __launch_bounds__(64 * kWaves) sas_cache_fp8_kernel(const CwParams p) {
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * kRowsPerWave;
  if (r0 >= p.N) return;
  uint4 w[kRowsPerWave], rope[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const uint8_t* src = p.kv + (size_t)min(r0 + i, p.N - 1) * p.kv_stride_b;
    w[i] = *reinterpret_cast<const uint4*>(src + lane * 16);
    // every lane loads (lanes 8-63 re-read lane l & 7's chunk: the same
    // lines): a load under a divergent branch made the compiler wait for
    // the loads in flight before it (32768-row write 16.7-17.2 -> 16.4-16.5 us)
    rope[i] = *reinterpret_cast<const uint4*>(src + kLatent * 2 + (lane & 7) * 16);
  }
  uint8_t* dst[kRowsPerWave];
  dest_rows(p, r0, kRow656, dst);
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i)
    if (dst[i]) put_fp8_row(dst[i], w[i], rope[i], lane);
}

}  // namespace
}  // namespace sas

extern "C" int sas_cache_write_v1(const SasCacheWriteArgs* a, void* stream) {
  using namespace sas;
  clear_error();
  if (!a) return set_error(SAS_EINVAL, "cache_write: null args");
  if (a->N < 0 || a->B < 1 || a->bt_stride < 1 || a->block_size < 1 || a->num_blocks < 1)
    return set_error(SAS_EINVAL, "cache_write: bad sizes");
  if (a->N == 0) return SAS_OK;
  if (!a->kv || !a->seq_ids || !a->positions || !a->block_table || !a->cache)
    return set_error(SAS_EINVAL, "cache_write: null device pointer");
  if (a->kv_dtype != SAS_DT_BF16 && a->kv_dtype != SAS_DT_FP16)
    return set_error(SAS_EINVAL, "cache_write: kv dtype must be bf16 or fp16");
  const bool fp8 = a->cache_dtype == SAS_DT_FP8_E4M3_ROW656;
  if (fp8 && (a->kv_dtype != SAS_DT_BF16 || a->D != 576))
    return set_error(SAS_EINVAL, "cache_write: fp8 rows need bf16 kv with D = 576");
  if (!fp8 && a->cache_dtype != a->kv_dtype)
    return set_error(SAS_EINVAL, "cache_write: cache dtype must be the kv dtype or fp8 rows");
  if (a->D < 8 || a->D % 8 || a->D > 1024)
    return set_error(SAS_EINVAL, "cache_write: D must be a multiple of 8 in [8, 1024]");
  if (a->kv_stride < a->D || (a->kv_stride * 2) % 16)
    return set_error(SAS_EINVAL, "cache_write: kv row stride must be >= D and 16-byte aligned");
  if (((uintptr_t)a->kv | (uintptr_t)a->cache) % 16)
    return set_error(SAS_EINVAL, "cache_write: kv and cache must be 16-byte aligned");
  if (a->N > INT32_MAX / 64 || a->B > INT32_MAX || a->bt_stride > INT32_MAX ||
      (double)a->num_blocks * a->block_size > 2147483000.0)
    return set_error(SAS_EINVAL, "cache_write: sizes beyond 32-bit indexing");
  CwParams p{};
  p.kv = (const uint8_t*)a->kv;
  p.seq_ids = a->seq_ids;
  p.positions = a->positions;
  p.bt = a->block_table;
  p.cache = (uint8_t*)a->cache;
  p.kv_stride_b = (long long)a->kv_stride * 2;
  p.N = (int)a->N; p.B = (int)a->B; p.D = (int)a->D;
  p.bt_stride = (int)a->bt_stride; p.bs = (int)a->block_size; p.nblocks = (int)a->num_blocks;
  constexpr int kRowsPerBlock = kWaves * kRowsPerWave;
  const dim3 grid((unsigned)((a->N + kRowsPerBlock - 1) / kRowsPerBlock)), block(64 * kWaves);
  hipStream_t st = (hipStream_t)stream;
  if (fp8) hipLaunchKernelGGL(sas_cache_fp8_kernel, grid, block, 0, st, p);
  else hipLaunchKernelGGL(sas_cache_copy_kernel, grid, block, 0, st, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SAS_ELAUNCH, "cache_write launch: %s", hipGetErrorString(e));
  return SAS_OK;
}
