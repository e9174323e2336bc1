// sparse_attn_sharedkv backward for MI355X (gfx950): dQ, dKV (the shared
// K = V cache rows) and d(sink) from the forward's output and LSE.
//
// No counterpart in the reference, which documents its LSE output as the
// input of a FlashAttention-v2 style backward (api.py:32-35, 176-184). For a
// query token t and head h over the forward's key set J (window rows and the
// valid top-k rows, resolved by the forward's own slot resolution) and the
// sink:
//   P_j = exp(scale q.k_j - lse),  P_sink = exp(sink - lse)
//   dP_j = dO . v_j (v_j = the first 512 channels of k_j),  Delta = dO . O
//   dS_j = P_j (dP_j - Delta)
//   dq = scale sum_j dS_j k_j
//   dkv_j += scale dS_j q  +  [P_j dO, 0]   (summed over heads and tokens)
//   dsink += -P_sink Delta                   (the sink's value row is zero)
//
// One workgroup per (token, head group, KV split). The fp32 atomic adds of
// the row gradients, one per (token, row, head group, channel), bound the
// backward, so head groups are as wide as registers and LDS allow: 64 heads
// (sas_bwd64_kernel, q in registers) when H is a multiple of 64, else 32
// (8 waves, two 16-head groups sharing the row tile) or 16 heads (4 waves)
// with q and dO in LDS (sas_bwd_kernel). With few tokens the token's key
// slots are split over several workgroups (as in the forward), which then add
// their dq shares atomically. Rows stream through LDS in chunks of 16 (the
// next chunk's loads in flight in registers): S^T and dP^T are 16x16x32
// MFMAs, P and dS go to an LDS table, then dq (dS . K, accumulated across
// chunks in registers) and the chunk's dkv rows (dS^T . Q + P^T . dO, summed
// over the heads, added to the fp32 gradient cache rows with atomics) are
// 16x16x16 MFMAs per 16-channel tile.

#include <mutex>
#include <type_traits>
#include <utility>

#include "sas_kern.h"

namespace sas {
namespace {

constexpr int kBwdRows = 16;   // rows per chunk (= lanes per head)
#ifndef SAS_BWD_NG
#define SAS_BWD_NG 2   // 16-head groups per workgroup when H is a multiple of 32 (1 or 2)
#endif
#ifndef SAS_BWD64
#define SAS_BWD64 1    // 1: 64-head workgroups (sas_bwd64_kernel) when H is a multiple of 64
#endif

struct BwdParams {
  FwdParams f;
  const uint8_t* out;   // [T, H, 512] q dtype
  const uint8_t* dout;  // [T, H, 512] q dtype
  float* dq;            // [T, H, D] fp32
  float* d_ori;         // [ori rows, D] fp32, accumulated
  float* d_cmp;         // [cmp rows, D] fp32, accumulated (null for SWA)
  float* d_sinks;       // [H] fp32, accumulated
  int win_pass;         // 1: window rows' gradients come from sas_bwd_win_kernel (the per-token kernels skip them)
  int win_tiles;        // sas_bwd_win_kernel: 64-position row tiles per batch
};

// f(integral_constant<int, j>) for j = 0 .. N-1, with no loop: arrays
// indexed this way are split into registers, while an array indexed inside a
// loop (even one unrolled later) is first moved to LDS or scratch memory by
// the compiler, which made each row-chunk prefetch a load waited for at once.
template <typename F, int... I>
__device__ __forceinline__ void unroll_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void unroll(F&& f) {
  unroll_impl(f, std::make_integer_sequence<int, N>{});
}
template <typename QT>
__device__ __forceinline__ float to_f(uint16_t v) {
  return (float)__builtin_bit_cast(QT, v);
}

// c + a.x * b.x + a.y * b.y for two packed 16-bit pairs (v_dot2c_f32_bf16 /
// v_dot2c_f32_f16)
template <typename QT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  typedef QT v2 __attribute__((ext_vector_type(2)));
  if constexpr (std::is_same<QT, __bf16>::value)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
}

// two packed 16-bit values (low half first) -> floats
template <typename QT>
__device__ __forceinline__ float2 unpack2(uint32_t w) {
  return make_float2(to_f<QT>((uint16_t)(w & 0xffffu)), to_f<QT>((uint16_t)(w >> 16)));
}

// Sum over the 16 lanes of a DPP row (a head's lanes), returned in every
// lane: quad_perm [1,0,3,2] and [2,3,0,1] (lane xor 1, xor 2), then
// row_half_mirror and row_mirror pair the quads and the halves.
__device__ __forceinline__ float sum16(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x140, 0xF, 0xF, false));
  return x;
}

// NG 16-head groups per workgroup (1 or 2; 4 NG waves): the groups share
// the row tile and their dkv contributions are summed (chained MFMAs) before
// one set of atomics, so NG = 2 halves the row-gradient atomics.
template <int D, typename QT, int NG>
__global__ void __launch_bounds__(256 * NG) sas_bwd_kernel(const BwdParams bp) {
  constexpr int NT = 256 * NG;                 // threads
  constexpr int NHD = 16 * NG;                 // heads per workgroup
  constexpr int CP = D / 16;                   // channels per part
  constexpr int CH = D / 8;                    // 16-byte chunks per row
  constexpr int KS = D * 2 + 16;               // LDS row stride (bytes)
  constexpr int QS = D * 2 + 16, OS = kDV * 2 + 16;   // padded q / dO row strides (bytes)
  __shared__ __attribute__((aligned(16))) uint8_t lds_k[kBwdRows * KS];
  __shared__ __attribute__((aligned(16))) uint8_t lds_q[NHD * QS];
  __shared__ __attribute__((aligned(16))) uint8_t lds_do[NHD * OS];
  __shared__ float lds_pd[kBwdRows][NHD][2];   // (P, scale dS) per row and head
  __shared__ float lds_hd[NHD][2];              // per head: Delta, lse (log2 units)

  const FwdParams& p = bp.f;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int item = item_index(p);
  if (item < 0) return;
  Tok k = item_of(p, item);
  resolve<256, D * 2>(p, k, tid, lane, wave, [] {});
  const int hgw = wave >> 2, wl = wave & 3;    // head group in the workgroup, wave in the group
  const int h = (tid & 255) >> 4, part = tid & 15;
  const int hw = hgw * 16 + h;                 // head in the workgroup
  const int hq = k.hg * NHD + hw;
  const int t = k.t;
  if (k.padded) {   // dq stays zero (the caller zeroes it)
    return;
  }

  // this thread's q / dO channels as packed pairs (dO zero past channel
  // 512), Delta = dO . O over the head's 16 lanes
  const uint32_t* dog = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(bp.dout) +
                                                          ((size_t)t * p.H + hq) * kDV);
  const uint32_t* og = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(bp.out) +
                                                         ((size_t)t * p.H + hq) * kDV);
  constexpr int CP2 = CP / 2;
  float dpart = 0.f;
#pragma unroll
  for (int i = 0; i < CP2; ++i) {
    const int c2 = part * CP2 + i;   // channel pair
    if (2 * c2 < kDV) dpart = dot2<QT>(dog[c2], og[c2], dpart);
  }
  // dq by MFMA: wave wl of head group hgw owns 16-channel tiles wl, wl + 4,
  // ...; lane (g4, c16) holds the group's heads 4 g4 .. 4 g4 + 3 of channel
  // 16 ct + c16
  constexpr int NDT = (D / 16 + 3) / 4;
  const int c16 = lane & 15, g4 = lane >> 4;
  f32x4 dqt[NDT];
#pragma unroll
  for (int j = 0; j < NDT; ++j) dqt[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float delta = sum16(dpart);
  const float lse2 = p.lse[(size_t)t * p.H + hq] * kLog2e;
  if (part == 0) { lds_hd[hw][0] = delta; lds_hd[hw][1] = lse2; }
  if (part == 0 && k.sp == 0) {
    const float psink = __builtin_amdgcn_exp2f(p.sinks[hq] * kLog2e - lse2);
    atomicAdd(bp.d_sinks + hq, -psink * delta);
  }
  {
    const uint4* qs = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.q) +
                                                     ((size_t)t * p.H + k.hg * NHD) * D);
    const uint4* ds = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(bp.dout) +
                                                     ((size_t)t * p.H + k.hg * NHD) * kDV);
    stage_chunks<NHD * D / 8, NT>(qs, tid, [&](int i, const uint4& v) {
      *reinterpret_cast<uint4*>(lds_q + (i / (D / 8)) * QS + (i % (D / 8)) * 16) = v;
    });
    stage_chunks<NHD * kDV / 8, NT>(ds, tid, [&](int i, const uint4& v) {
      *reinterpret_cast<uint4*>(lds_do + (i / (kDV / 8)) * OS + (i % (kDV / 8)) * 16) = v;
    });
  }
  const float scale = p.scale_log2 / kLog2e;
  const uint64_t ori_lo = reinterpret_cast<uint64_t>(p.ori_kv);
  const uint64_t ori_n = (uint64_t)p.ori_nblocks * p.ori_bs * (D * 2);
  const uint64_t cmp_lo = reinterpret_cast<uint64_t>(p.cmp_kv);
  // col4(base, stride, ct): the 16-bit values of rows 4 g4 .. 4 g4 + 3 of
  // `base` at channel 16 ct + c16, packed as an MFMA operand, by one
  // transposed read: lane (g4, c16) addresses row 4 g4 + c16 / 4 at channels
  // 16 ct + 4 (c16 & 3) .. + 3 and receives its channel of the four rows
  // (rows padded by 16 bytes, so the row groups spread over the banks)
  auto col4 = [&](const uint8_t* base, int stride, int ct) {
    const uint8_t* a = base + (4 * g4 + (c16 >> 2)) * stride + (ct * 16 + 4 * (c16 & 3)) * 2;
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4*)(a)));
  };

  // Row chunks are double-buffered through registers: the loads of chunk
  // c + 1 are issued right after chunk c is in LDS and land during its
  // compute (rows past the end repeat the last row: their P and dS are 0).
  constexpr int NLD = (kBwdRows * CH + NT - 1) / NT;
  uint4 rbuf[NLD];
  auto load_rows = [&](int c0n) {
    const int nrn = min(kBwdRows, k.nvalid - c0n);
    unroll<NLD>([&](auto J) {
      constexpr int j = decltype(J)::value;
      const int i = tid + NT * j;
      if (i < kBwdRows * CH) {
        const int r = i / CH, c = i - r * CH;
        rbuf[j] = gld16(lds_rows[c0n + min(r, nrn - 1)] + c * 16);
      }
    });
  };
  if (k.nvalid > 0) load_rows(0);

  for (int c0 = 0; c0 < k.nvalid; c0 += kBwdRows) {
    const int nr = min(kBwdRows, k.nvalid - c0);
    unroll<NLD>([&](auto J) {
      constexpr int j = decltype(J)::value;
      const int i = tid + NT * j;
      if (i < kBwdRows * CH) {
        const int r = i / CH, c = i - r * CH;
        *reinterpret_cast<uint4*>(lds_k + r * KS + c * 16) = rbuf[j];
      }
    });
    __syncthreads();
    if (c0 + kBwdRows < k.nvalid) load_rows(c0 + kBwdRows);
    // S^T[key][head] = K . Q^T and dP^T = V . dO^T by 16x16x32 MFMA, the
    // whole tile in the first wave of head group hgw (A = 8 channels of key
    // c16 from the row tile, B = the same channels of head c16 from the q /
    // dO tile); lane (g4, c16) holds keys 4 g4 .. + 3 of head c16 and writes
    // their P and scale dS to the table.
    if (wl == 0) {
      f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f}, dacc = sacc;
      const uint8_t* kb = lds_k + c16 * KS + g4 * 16;
      const uint8_t* qb = lds_q + (hgw * 16 + c16) * QS + g4 * 16;
      const uint8_t* ob = lds_do + (hgw * 16 + c16) * OS + g4 * 16;
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) {
        const uint4 kf = *reinterpret_cast<const uint4*>(kb + ks * 64);
        sacc = mfma32k<QT>(kf, *reinterpret_cast<const uint4*>(qb + ks * 64), sacc);
        if (ks < kDV / 32) dacc = mfma32k<QT>(kf, *reinterpret_cast<const uint4*>(ob + ks * 64), dacc);
      }
      const int hh = hgw * 16 + c16;
      const float dl = lds_hd[hh][0], l2 = lds_hd[hh][1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 4 * g4 + i;
        float pr = 0.f, dsr = 0.f;
        if (key < nr) {
          pr = __builtin_amdgcn_exp2f(sacc[i] * p.scale_log2 - l2);
          dsr = pr * (dacc[i] - dl) * scale;
        }
        lds_pd[key][hh][0] = pr;
        lds_pd[key][hh][1] = dsr;
      }
    }
    __syncthreads();
    // dq[head][ch] += dS[head][key] . K[key][ch]: A = keys 4 g4 .. + 3 of the
    // group's head c16 (dS rounded to the query dtype), B = the same keys of
    // channel 16 ct + c16 from the row tile (rows past nr carry dS = 0)
    {
      uint2 a_dq;
      a_dq.x = pack2<QT>(lds_pd[4 * g4][hgw * 16 + c16][1], lds_pd[4 * g4 + 1][hgw * 16 + c16][1]);
      a_dq.y = pack2<QT>(lds_pd[4 * g4 + 2][hgw * 16 + c16][1], lds_pd[4 * g4 + 3][hgw * 16 + c16][1]);
#pragma unroll
      for (int j = 0; j < NDT; ++j) {
        const int ct = wl + 4 * j;
        if (ct < D / 16) dqt[j] = mfma16k<QT>(a_dq, col4(lds_k, KS, ct), dqt[j]);
      }
    }
    // dkv rows of the chunk by 16x16x16 MFMA: per 16-channel tile ct (wave
    // w takes tiles w, w + 4 NG, ...), dK[key][ch] = sum over the head
    // groups of dS[key][head] . Q[head][ch] (+ P[key][head] . dO[head][ch]
    // for ch < 512), one chained MFMA per group. A = 4 heads (4 g4 .. + 3)
    // of key c16 from the (P, dS) table, rounded to the query dtype; B = the
    // same 4 heads of channel 16 ct + c16 from the q / dO tiles. Lane (g4,
    // c16) then holds keys 4 g4 .. + 3 of channel 16 ct + c16 and adds them
    // to the rows' fp32 gradients (64-byte runs per key).
    {
      uint2 a_ds[NG], a_p[NG];
#pragma unroll
      for (int gg = 0; gg < NG; ++gg) {
        const int hb = gg * 16 + 4 * g4;
        a_ds[gg].x = pack2<QT>(lds_pd[c16][hb][1], lds_pd[c16][hb + 1][1]);
        a_ds[gg].y = pack2<QT>(lds_pd[c16][hb + 2][1], lds_pd[c16][hb + 3][1]);
        a_p[gg].x = pack2<QT>(lds_pd[c16][hb][0], lds_pd[c16][hb + 1][0]);
        a_p[gg].y = pack2<QT>(lds_pd[c16][hb + 2][0], lds_pd[c16][hb + 3][0]);
      }
      float* grow[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 4 * g4 + i;
        const uint64_t a = lds_rows[c0 + min(key, nr - 1)];
        grow[i] = key < nr ? (a - ori_lo < ori_n ? (bp.win_pass ? nullptr : bp.d_ori + (a - ori_lo) / (D * 2) * D)
                                                 : bp.d_cmp + (a - cmp_lo) / (D * 2) * D)
                           : nullptr;
      }
      // a chunk of window rows only, under the window pass: no dkv here
      const bool any_row = __ballot(grow[0] || grow[1] || grow[2] || grow[3]) != 0;
      for (int ct = wave; any_row && ct < D / 16; ct += 4 * NG) {
        const int ch = ct * 16 + c16;
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int gg = 0; gg < NG; ++gg) {
          acc = mfma16k<QT>(a_ds[gg], col4(lds_q + gg * 16 * QS, QS, ct), acc);
          if (ct < kDV / 16) acc = mfma16k<QT>(a_p[gg], col4(lds_do + gg * 16 * OS, OS, ct), acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (grow[i]) atomicAdd(grow[i] + ch, acc[i]);
      }
    }
    __syncthreads();
  }
  // one split: the workgroup owns its heads' dq; several: each adds its share
  float* dqb = bp.dq + ((size_t)t * p.H + k.hg * NHD + hgw * 16 + 4 * g4) * D + c16;
#pragma unroll
  for (int j = 0; j < NDT; ++j) {
    const int ct = wl + 4 * j;
    if (ct >= D / 16) break;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (p.nsplit == 1) dqb[(size_t)i * D + ct * 16] = dqt[j][i];
      else atomicAdd(dqb + (size_t)i * D + ct * 16, dqt[j][i]);
    }
  }
}

// 64-head workgroups (H a multiple of 64): 8 waves, wave w = 2 g + hh holds
// head group g (16 heads) and channel half hh. The dkv atomics are one per
// (token, row, channel) for all 64 heads, half those of 32-head workgroups,
// and the row-gradient atomics bound the backward. The q / dO tiles of 64
// heads (141 KB) do not fit beside the row tile in LDS, so q lives in
// registers, spread over the waves: each wave holds its head group's Q^T
// fragments for its half of the S = K Q^T channels and, for its dkv channel
// tiles (w, w + 8, ...), the q B-operands of all four head groups; dO stays
// in LDS. Per 16-row chunk: each wave sums its channel half of S^T and dP^T
// (16x16x32 MFMA), the pair adds the halves through LDS (own + other, the
// same bits in both waves), P and scale dS go to the (P, dS) table, then dq
// over the wave's head group and channel half, and the dkv tiles (dS^T . Q +
// P^T . dO summed over the four groups) with one atomic add per value.
template <int D, typename QT>
__global__ void __launch_bounds__(512) sas_bwd64_kernel(const BwdParams bp) {
  constexpr int NT = 512, NHD = 64;
  constexpr int CH = D / 8;                // 16-byte chunks per row
  constexpr int KS = D * 2 + 16;           // row tile stride (bytes)
  constexpr int QSTR = D * 2 + 16;         // staged q row stride (bytes)
  constexpr int OS = kDV * 2 + 16;         // dO row stride (bytes)
  constexpr int KSH = D / 64;              // S k-steps (32 channels) per channel half
  constexpr int VSH = kDV / 64;            // dP k-steps per channel half
  constexpr int NCT = D / 16;              // 16-channel tiles
  constexpr int MT = (NCT + 7) / 8;        // dkv tiles per wave (at most)
  constexpr int DQT = NCT / 2;             // dq tiles per wave (its channel half)
  static_assert(NCT % 2 == 0 && KSH * 2 * 32 == D, "channel halves");
  // q is staged here for the register loads, then dO takes the space
  __shared__ __attribute__((aligned(16))) uint8_t lds_qo[NHD * QSTR];
  // row chunks, double-buffered, filled by LDS-DMA: chunk position P of a
  // buffer is row P / KCH, 16-byte chunk P % KCH (the last chunk of a padded
  // row, and positions past the chunk, take a dummy copy)
  constexpr int KCH = KS / 16;                              // chunks per padded row
  constexpr int NKDMA = (kBwdRows * KCH + 63) / 64;         // DMA instructions per chunk
  static_assert(KS % 16 == 0 && KCH == CH + 1, "padded row = chunks + one");
  __shared__ __attribute__((aligned(16))) uint8_t lds_kb[2][NKDMA * 64 * 16];
  __shared__ float lds_pd[kBwdRows][NHD][2];   // (P, scale dS) per row and head
  __shared__ float lds_hd[NHD][2];             // per head: Delta, lse (log2 units)
  __shared__ f32x4 lds_x[8][2][64];            // S^T / dP^T channel halves per wave

  const FwdParams& p = bp.f;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int item = item_index(p);
  if (item < 0) return;
  Tok k = item_of(p, item);
  resolve<256, D * 2>(p, k, tid, lane, wave, [] {});
  const int g = wave >> 1, hh = wave & 1;
  const int c16 = lane & 15, g4 = lane >> 4;
  const int t = k.t, h0 = k.hg * NHD;
  if (k.padded) return;   // dq stays zero (the caller zeroes it)

  // Delta = dO . O: 8 threads per head, 64 channels each, 8-lane sums
  {
    const int hd = tid >> 3, part = tid & 7, hq = h0 + hd;
    const uint32_t* dog = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(bp.dout) +
                                                            ((size_t)t * p.H + hq) * kDV) + part * 32;
    const uint32_t* og = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(bp.out) +
                                                           ((size_t)t * p.H + hq) * kDV) + part * 32;
    float dpart = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) dpart = dot2<QT>(dog[i], og[i], dpart);
    dpart += __shfl_xor(dpart, 1);
    dpart += __shfl_xor(dpart, 2);
    dpart += __shfl_xor(dpart, 4);
    const float lse2 = p.lse[(size_t)t * p.H + hq] * kLog2e;
    if (part == 0) {
      lds_hd[hd][0] = dpart;
      lds_hd[hd][1] = lse2;
      if (k.sp == 0) {
        const float psink = __builtin_amdgcn_exp2f(p.sinks[hq] * kLog2e - lse2);
        atomicAdd(bp.d_sinks + hq, -psink * dpart);
      }
    }
  }
  // col4(base, stride, ct): the 16-bit values of rows 4 g4 .. 4 g4 + 3 of
  // `base` at channel 16 ct + c16, packed as an MFMA operand, by one
  // transposed read (rows padded by 16 bytes)
  auto col4 = [&](const uint8_t* base, int stride, int ct) {
    const uint8_t* a = base + (4 * g4 + (c16 >> 2)) * stride + (ct * 16 + 4 * (c16 & 3)) * 2;
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4*)(a)));
  };
  // q of the 64 heads staged in LDS, read into registers: qs = this wave's
  // Q^T fragments (head 16 g + c16, channels 32 (hh KSH + ks) + 8 g4 ..),
  // qk[m][gg] = q of heads 16 gg + 4 g4 .. + 3 at channel 16 (wave + 8 m) + c16
  uint4 qs[KSH];
  uint2 qk[MT][4];
  {
    const uint4* qg = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.q) +
                                                     ((size_t)t * p.H + h0) * D);
    stage_chunks<NHD * CH, NT>(qg, tid, [&](int i, const uint4& v) {
      *reinterpret_cast<uint4*>(lds_qo + (i / CH) * QSTR + (i % CH) * 16) = v;
    });
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < KSH; ++ks)
      qs[ks] = *reinterpret_cast<const uint4*>(lds_qo + (16 * g + c16) * QSTR + ((hh * KSH + ks) * 32 + 8 * g4) * 2);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int ct = wave + 8 * m;
#pragma unroll
      for (int gg = 0; gg < 4; ++gg)
        qk[m][gg] = ct < NCT ? col4(lds_qo + gg * 16 * QSTR, QSTR, ct) : make_uint2(0, 0);
    }
    __syncthreads();   // every wave has its q before dO overwrites it
    const uint4* ds = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(bp.dout) +
                                                     ((size_t)t * p.H + h0) * kDV);
    stage_chunks<NHD * kDV / 8, NT>(ds, tid, [&](int i, const uint4& v) {
      *reinterpret_cast<uint4*>(lds_qo + (i / (kDV / 8)) * OS + (i % (kDV / 8)) * 16) = v;
    });
  }
  const float scale = p.scale_log2 / kLog2e;
  const uint64_t ori_lo = reinterpret_cast<uint64_t>(p.ori_kv);
  const uint64_t ori_n = (uint64_t)p.ori_nblocks * p.ori_bs * (D * 2);
  const uint64_t cmp_lo = reinterpret_cast<uint64_t>(p.cmp_kv);
  f32x4 dqt[DQT];
#pragma unroll
  for (int j = 0; j < DQT; ++j) dqt[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Row chunks by LDS-DMA into two buffers: chunk c + 1 is issued right
  // after chunk c is in LDS and lands during its compute (rows past the end
  // repeat the last row: their P and dS are 0). The DMA is not tracked by
  // the compiler; its completion is waited for explicitly. The only vector-
  // memory operations a wave issues after its DMA of a chunk are its
  // row-gradient atomics of the chunk before, natom of them, so waiting
  // until at most natom operations are in flight (rounded down) covers the
  // DMA without waiting for the atomics. (With the rows loaded through
  // registers the compiler waited for everything in flight, the atomics
  // included: the atomics were issued in branches it could not count.)
  auto dma_rows = [&](int b, int c0n) {
    const int nrn = min(kBwdRows, k.nvalid - c0n);
    const uint32_t rb = __builtin_amdgcn_readfirstlane(lds_addr_of(lds_rows + c0n));
    const uint32_t kb0 = lds_addr_of(lds_kb[b]);
    for (int o = wave; o < NKDMA; o += 8) {   // wave-uniform
      const int P = o * 64 + lane, r = P / KCH, c = P - r * KCH;
      const bool real = r < kBwdRows && c < CH;
      const uint64_t a = *reinterpret_cast<const LDS_AS uint64_t*>(
          (size_t)(rb + 8u * (uint32_t)(real ? min(r, nrn - 1) : 0)));
      dma16(reinterpret_cast<const void*>(a + (real ? (uint64_t)c * 16 : 0)),
            __builtin_amdgcn_readfirstlane(kb0 + (uint32_t)o * 64 * 16));
    }
  };
  auto wait_vm_atmost = [](int n) {   // n wave-uniform; rounded down to a multiple of 4
    if (n >= 16) wait_vm<16>();
    else if (n >= 12) wait_vm<12>();
    else if (n >= 8) wait_vm<8>();
    else if (n >= 4) wait_vm<4>();
    else wait_vm<0>();
  };
  int ntile = 0;   // dkv tiles of this wave: ct = wave + 8 m < NCT
#pragma unroll
  for (int m = 0; m < MT; ++m) ntile += wave + 8 * m < NCT;
  int natom = 0;   // atomic instructions this wave issued since its last DMA
  if (k.nvalid > 0) dma_rows(0, 0);

  for (int c0 = 0, ci = 0; c0 < k.nvalid; c0 += kBwdRows, ++ci) {
    const int nr = min(kBwdRows, k.nvalid - c0);
    const uint8_t* lds_k = lds_kb[ci & 1];
    wait_vm_atmost(natom);   // my DMA of this chunk
    lds_barrier();           // everyone's (and, the first time, dO) in LDS
    if (c0 + kBwdRows < k.nvalid) dma_rows((ci + 1) & 1, c0 + kBwdRows);
    // this wave's channel half of S^T = K . Q^T and dP^T = V . dO^T for its
    // head group: A = 8 channels of key c16, B = the same channels of head c16
    {
      f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f}, dacc = sacc;
      const uint8_t* kb = lds_k + c16 * KS + g4 * 16;
      const uint8_t* ob = lds_qo + (16 * g + c16) * OS + g4 * 16;
#pragma unroll
      for (int ks = 0; ks < KSH; ++ks)
        sacc = mfma32k<QT>(*reinterpret_cast<const uint4*>(kb + (hh * KSH + ks) * 64), qs[ks], sacc);
#pragma unroll
      for (int vs = 0; vs < VSH; ++vs) {
        const int off = (hh * VSH + vs) * 64;
        dacc = mfma32k<QT>(*reinterpret_cast<const uint4*>(kb + off), *reinterpret_cast<const uint4*>(ob + off), dacc);
      }
      lds_x[wave][0][lane] = sacc;
      lds_x[wave][1][lane] = dacc;
      lds_barrier();
      sacc += lds_x[wave ^ 1][0][lane];
      dacc += lds_x[wave ^ 1][1][lane];
      // lane (g4, c16): keys 4 g4 .. + 3 of head 16 g + c16; one wave of the
      // pair writes their P and scale dS
      if (hh == 0) {
        const int hd = 16 * g + c16;
        const float dl = lds_hd[hd][0], l2 = lds_hd[hd][1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = 4 * g4 + i;
          float pr = 0.f, dsr = 0.f;
          if (key < nr) {
            pr = __builtin_amdgcn_exp2f(sacc[i] * p.scale_log2 - l2);
            dsr = pr * (dacc[i] - dl) * scale;
          }
          lds_pd[key][hd][0] = pr;
          lds_pd[key][hd][1] = dsr;
        }
      }
    }
    lds_barrier();
    // dq[head][ch] += dS[head][key] . K[key][ch] over this wave's head group
    // and channel half (A = keys 4 g4 .. + 3 of head c16; B = the same keys
    // of channel 16 ct + c16, rows past nr carry dS = 0)
    {
      const int hd = 16 * g + c16;
      uint2 a_dq;
      a_dq.x = pack2<QT>(lds_pd[4 * g4][hd][1], lds_pd[4 * g4 + 1][hd][1]);
      a_dq.y = pack2<QT>(lds_pd[4 * g4 + 2][hd][1], lds_pd[4 * g4 + 3][hd][1]);
#pragma unroll
      for (int j = 0; j < DQT; ++j) dqt[j] = mfma16k<QT>(a_dq, col4(lds_k, KS, hh * DQT + j), dqt[j]);
    }
    // dkv rows of the chunk, tiles ct = wave + 8 m: dK[key][ch] = sum over
    // the four head groups of dS[key][head] . Q[head][ch] (+ P[key][head] .
    // dO[head][ch] for ch < 512); A = 4 heads (4 g4 .. + 3) of key c16 from
    // the table, rounded to the query dtype; lane (g4, c16) then holds keys
    // 4 g4 .. + 3 of channel 16 ct + c16 and adds them to the fp32 gradients
    {
      uint2 a_ds[4], a_p[4];
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        const int hb = gg * 16 + 4 * g4;
        a_ds[gg].x = pack2<QT>(lds_pd[c16][hb][1], lds_pd[c16][hb + 1][1]);
        a_ds[gg].y = pack2<QT>(lds_pd[c16][hb + 2][1], lds_pd[c16][hb + 3][1]);
        a_p[gg].x = pack2<QT>(lds_pd[c16][hb][0], lds_pd[c16][hb + 1][0]);
        a_p[gg].y = pack2<QT>(lds_pd[c16][hb + 2][0], lds_pd[c16][hb + 3][0]);
      }
      float* grow[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 4 * g4 + i;
        const uint64_t a = lds_rows[c0 + min(key, nr - 1)];
        grow[i] = key < nr ? (a - ori_lo < ori_n ? (bp.win_pass ? nullptr : bp.d_ori + (a - ori_lo) / (D * 2) * D)
                                                 : bp.d_cmp + (a - cmp_lo) / (D * 2) * D)
                           : nullptr;
      }
      // a chunk of window rows only, under the window pass: no dkv here
      const bool any_row = __ballot(grow[0] || grow[1] || grow[2] || grow[3]) != 0;
      // the atomic instructions issued below: one per (tile, i) with some lane's row
      int nrow_i = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) nrow_i += __ballot(grow[i] != nullptr) != 0;
      natom = any_row ? ntile * nrow_i : 0;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const int ct = wave + 8 * m;
        if (ct >= NCT || !any_row) break;   // wave-uniform
        const int ch = ct * 16 + c16;
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
          acc = mfma16k<QT>(a_ds[gg], qk[m][gg], acc);
          if (ct < kDV / 16) acc = mfma16k<QT>(a_p[gg], col4(lds_qo + gg * 16 * OS, OS, ct), acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (grow[i]) atomicAdd(grow[i] + ch, acc[i]);
      }
    }
    lds_barrier();
  }
  // one split: the workgroup owns its heads' dq; several: each adds its share
  float* dqb = bp.dq + ((size_t)t * p.H + h0 + 16 * g + 4 * g4) * D + c16;
#pragma unroll
  for (int j = 0; j < DQT; ++j) {
    const int ct = hh * DQT + j;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (p.nsplit == 1) dqb[(size_t)i * D + ct * 16] = dqt[j][i];
      else atomicAdd(dqb + (size_t)i * D + ct * 16, dqt[j][i]);
    }
  }
}

// ---------------------------------------------------------------------------
// key-major pass over the window rows
// ---------------------------------------------------------------------------
//
// A window row (position pos of batch b's raw cache) is a key of every token
// of b whose window [max(s_g - win_left, 0), s_g] covers it: up to
// win_left + 1 consecutive tokens of a prefill. The per-token kernels add one
// fp32 atomic per (token, row, channel) for it; this pass instead keeps a
// tile of 64 consecutive positions resident, streams the tokens that attend
// any of them, and sums each row's gradient over those tokens in registers,
// adding it once per 16-head group at the end (C3 prefill: 2.97e8 of the
// 1.20e9 row atomics). Workgroup = (batch, 64-position tile, 16-head group),
// 4 waves; wave w owns rows 16 w .. 16 w + 15 of the tile, their K^T
// fragments in registers for the whole token loop, and their dkv^T
// accumulators [576 channels x 16 rows]. Per token (q, dO and O of the 16
// heads staged in LDS, double-buffered, the loads of the token two ahead in
// flight in registers):
//   S[head][row] = Q . K^T and dP = dO . V^T   (16x16x32 MFMA, A = q / dO
//     rows from LDS, B = the wave's K^T registers; lane (g4, c16) holds
//     heads 4 g4 .. + 3 of row c16)
//   P = exp(scale S - lse), dS = P (dP - Delta) scale, masked to the
//     token's window and valid rows, rounded to the query dtype
//   dkv^T[ch][row] += Q^T[ch][head] . dS[head][row] (+ dO^T . P for the 512
//     V channels)   (16x16x16 MFMA, A = a transposed read of the q / dO
//     tile, B = dS / P exactly in the S accumulator's layout)
// P, dS and their rounding are those of the per-token kernels, so the sum
// differs from theirs only in fp32 summation order. Row validity follows
// resolve(): position below act_kv, block inside the table, table entry
// inside the cache. It runs beside the per-token kernel on a side stream
// (SideStream below); sas_bwd_v1 chooses it for prefills.
constexpr int kWinRows = 64;   // positions per tile (16 per wave)

template <int D, typename QT>
__global__ void __launch_bounds__(256) sas_bwd_win_kernel(const BwdParams bp) {
  constexpr int HG = 16;                   // heads per workgroup
  constexpr int CH = D / 8;                // 16-byte chunks per row
  constexpr int KSN = D / 32;              // S k-steps
  constexpr int VSN = kDV / 32;            // dP k-steps
  constexpr int NCT = D / 16;              // dkv channel tiles
  constexpr int RS = D * 2 + 16;           // row / q stride in LDS (bytes)
  constexpr int OS = kDV * 2 + 16;         // dO stride in LDS (bytes)
  constexpr int QL = (HG * CH + 255) / 256;   // q chunks per thread (16 threads per head)
  constexpr int OL = kDV / 8 / 16;            // dO / O chunks per thread
  static_assert(OL == 4 && HG * 16 == 256, "thread (head, part) layout");
  __shared__ __attribute__((aligned(16))) uint8_t lds_r[kWinRows * RS];
  __shared__ __attribute__((aligned(16))) uint8_t lds_tq[2][HG * RS];
  __shared__ __attribute__((aligned(16))) uint8_t lds_to[2][HG * OS];
  __shared__ float lds_th[2][HG][2];       // per buffer and head: Delta, lse (log2 units)
  __shared__ uint64_t lds_wr[kWinRows];    // row addresses (0: invalid row)

  const FwdParams& p = bp.f;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int c16 = lane & 15, g4 = lane >> 4;
  const int nhgw = p.H / HG;
  const int hg = (int)(blockIdx.x % nhgw), rest = (int)(blockIdx.x / nhgw);
  const int tile = rest % bp.win_tiles, b = rest / bp.win_tiles;
  const int p0 = tile * kWinRows;
  const bool cu = p.act_q == nullptr;
  const int qp = p.q_prefix[b];
  const int aq = cu ? p.q_prefix[b + 1] - qp : p.act_q[b];
  const int akv = p.act_kv[b];
  const int sg0 = akv - aq;                // causal position of the batch's first token
  // tokens whose window meets [p0, p0 + 64): s_g in [p0, p0 + 63 + win_left]
  // and in [max(sg0, 0), akv - 1]
  const long long sg_lo = p0 > sg0 ? (p0 > 0 ? p0 : 0) : (sg0 > 0 ? sg0 : 0);
  const long long sg_top = (long long)p0 + kWinRows - 1 + p.win_left;
  long long sg_hi = sg_top < (long long)akv - 1 ? sg_top : (long long)akv - 1;
  // (and tokens inside [0, T): lengths that point past the query tensor
  // bring no token in)
  const long long sg_tend = (long long)sg0 + (long long)p.T - 1 - qp;
  if (sg_tend < sg_hi) sg_hi = sg_tend;
  if (aq <= 0 || qp < 0 || qp >= p.T || sg_lo > sg_hi) return;   // uniform: no token of this tile
  const int h0 = hg * HG;

  // row tile: addresses (as resolve() validates them), then the rows
  if (tid < kWinRows) {
    const int pos = p0 + tid;
    const int blk = pos / p.ori_bs;
    uint64_t a = 0;
    if (pos < akv && blk < p.ori_bt_stride) {
      const int phys = p.ori_bt[(size_t)b * p.ori_bt_stride + blk];
      if (phys >= 0 && phys < p.ori_nblocks)
        a = reinterpret_cast<uint64_t>(p.ori_kv) + (uint64_t)((uint32_t)(phys * p.ori_bs + pos - blk * p.ori_bs)) * (D * 2);
    }
    lds_wr[tid] = a;
  }
  __syncthreads();
  for (int i = tid; i < kWinRows * CH; i += 256) {
    const int r = i / CH, c = i - r * CH;
    const uint64_t a = lds_wr[r];
    *reinterpret_cast<uint4*>(lds_r + r * RS + c * 16) = a ? gld16(a + c * 16) : make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  // this wave's rows: K^T operands (row c16, channels 32 ks + 8 g4 ..) and
  // the lane's row position / validity
  uint4 kf[KSN];
#pragma unroll
  for (int ks = 0; ks < KSN; ++ks)
    kf[ks] = *reinterpret_cast<const uint4*>(lds_r + (16 * wave + c16) * RS + (32 * ks + 8 * g4) * 2);
  const int pos = p0 + 16 * wave + c16;
  const bool rok = lds_wr[16 * wave + c16] != 0;
  const int wpos0 = p0 + 16 * wave;        // the wave's first position

  f32x4 acc[NCT];
#pragma unroll
  for (int j = 0; j < NCT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float scale = p.scale_log2 / kLog2e;

  // Token staging: thread (head th = tid / 16, part tp = tid % 16) loads its
  // share of a token's q, dO and O into one of two register sets, two tokens
  // ahead of the token being computed (one token ahead left the global
  // round trip exposed: 3 µs per token on the C3 prefill), and stores it
  // into the LDS buffer of the same index, with the head's Delta = dO . O.
  const int th = tid >> 4, tp = tid & 15;
  uint4 rq[2][QL], rd[2][OL], ro[2][OL];
  float rl[2] = {0.f, 0.f};
  auto load_tok = [&](auto S, long long sg) __attribute__((always_inline)) {
    constexpr int sl = decltype(S)::value;
    const size_t t = (size_t)qp + (size_t)(sg - sg0);
    const uint4* qg = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.q) + (t * p.H + h0 + th) * D);
    const uint4* dg = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(bp.dout) + (t * p.H + h0 + th) * kDV);
    const uint4* og = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(bp.out) + (t * p.H + h0 + th) * kDV);
    unroll<QL>([&](auto J) {
      constexpr int j = decltype(J)::value;
      const int c = tp + 16 * j;
      rq[sl][j] = c < CH ? qg[c] : make_uint4(0, 0, 0, 0);
    });
    unroll<OL>([&](auto J) {
      constexpr int j = decltype(J)::value;
      rd[sl][j] = dg[tp * OL + j];
      ro[sl][j] = og[tp * OL + j];
    });
    rl[sl] = p.lse[t * p.H + h0 + th];
  };
  auto store_tok = [&](auto S) __attribute__((always_inline)) {
    constexpr int sl = decltype(S)::value;
    unroll<QL>([&](auto J) {
      constexpr int j = decltype(J)::value;
      const int c = tp + 16 * j;
      if (c < CH) *reinterpret_cast<uint4*>(lds_tq[sl] + th * RS + c * 16) = rq[sl][j];
    });
    float dp = 0.f;
    unroll<OL>([&](auto J) {
      constexpr int j = decltype(J)::value;
      *reinterpret_cast<uint4*>(lds_to[sl] + th * OS + (tp * OL + j) * 16) = rd[sl][j];
      dp = dot2<QT>(rd[sl][j].x, ro[sl][j].x, dp);
      dp = dot2<QT>(rd[sl][j].y, ro[sl][j].y, dp);
      dp = dot2<QT>(rd[sl][j].z, ro[sl][j].z, dp);
      dp = dot2<QT>(rd[sl][j].w, ro[sl][j].w, dp);
    });
    dp = sum16(dp);   // Delta of head th (its 16 lanes)
    if (tp == 0) { lds_th[sl][th][0] = dp; lds_th[sl][th][1] = rl[sl] * kLog2e; }
  };
  // A operand: the 16-bit values of heads 4 g4 .. + 3 at channel 16 ct +
  // c16, by one transposed read (rows padded by 16 bytes)
  auto col4 = [&](const uint8_t* base, int stride, int ct) __attribute__((always_inline)) {
    const uint8_t* a = base + (4 * g4 + (c16 >> 2)) * stride + (ct * 16 + 4 * (c16 & 3)) * 2;
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4*)(a)));
  };
  auto compute = [&](int buf, long long sg) __attribute__((always_inline)) {
    const long long wlo = sg - p.win_left > 0 ? sg - p.win_left : 0;
    if (wpos0 + 15 < wlo || wpos0 > sg) return;   // wave-uniform: none of my rows in this window
    const uint8_t* tq = lds_tq[buf];
    const uint8_t* to = lds_to[buf];
    // With one wave per SIMD nothing else hides an LDS read's latency, so
    // every operand read is issued kPfA (S, dP) or kPfC (dkv) MFMAs ahead
    // of its use.
    constexpr int kPfA = 4, kPfC = 8;
    auto qfrag = [&](int ks) __attribute__((always_inline)) {
      return *reinterpret_cast<const uint4*>(tq + c16 * RS + (32 * ks + 8 * g4) * 2);
    };
    auto ofrag = [&](int ks) __attribute__((always_inline)) {
      return *reinterpret_cast<const uint4*>(to + c16 * OS + (32 * ks + 8 * g4) * 2);
    };
    // two accumulation chains each for S and dP (even / odd k-steps)
    f32x4 sc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}}, dc[2] = {sc[0], sc[0]};
    uint4 qa[kPfA], oa[kPfA];
#pragma unroll
    for (int i = 0; i < kPfA; ++i) { qa[i] = qfrag(i); oa[i] = ofrag(i); }
#pragma unroll
    for (int ks = 0; ks < KSN; ++ks) {
      const uint4 a = qa[ks % kPfA];
      if (ks + kPfA < KSN) qa[ks % kPfA] = qfrag(ks + kPfA);
      sc[ks & 1] = mfma32k<QT>(a, kf[ks], sc[ks & 1]);
      if (ks < VSN) {
        const uint4 o = oa[ks % kPfA];
        if (ks + kPfA < VSN) oa[ks % kPfA] = ofrag(ks + kPfA);
        dc[ks & 1] = mfma32k<QT>(o, kf[ks], dc[ks & 1]);
      }
    }
    const f32x4 s_ = sc[0] + sc[1], d_ = dc[0] + dc[1];
    // lane (g4, c16): heads 4 g4 + i of row c16
    const bool in = rok && pos >= wlo && pos <= sg;
    float pr[4], ds[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * g4 + i;
      pr[i] = in ? __builtin_amdgcn_exp2f(s_[i] * p.scale_log2 - lds_th[buf][h][1]) : 0.f;
      ds[i] = pr[i] * (d_[i] - lds_th[buf][h][0]) * scale;
    }
    const uint2 b_p = make_uint2(pack2<QT>(pr[0], pr[1]), pack2<QT>(pr[2], pr[3]));
    const uint2 b_ds = make_uint2(pack2<QT>(ds[0], ds[1]), pack2<QT>(ds[2], ds[3]));
    // dkv: every tile's dS MFMA, then every V tile's P MFMA (a tile's two
    // adds 36 MFMAs apart instead of back to back)
    uint2 cq[kPfC];
#pragma unroll
    for (int i = 0; i < kPfC; ++i) cq[i] = col4(tq, RS, i);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const uint2 a = cq[ct % kPfC];
      cq[ct % kPfC] = ct + kPfC < NCT ? col4(tq, RS, ct + kPfC) : col4(to, OS, ct + kPfC - NCT);
      acc[ct] = mfma16k<QT>(a, b_ds, acc[ct]);
    }
#pragma unroll
    for (int ct = 0; ct < kDV / 16; ++ct) {
      const uint2 o = cq[(NCT + ct) % kPfC];
      if (ct + kPfC < kDV / 16) cq[(NCT + ct) % kPfC] = col4(to, OS, ct + kPfC);
      acc[ct] = mfma16k<QT>(o, b_p, acc[ct]);
    }
  };
  // one token from register set / LDS buffer S: store it, start the loads
  // of the token two ahead into the freed registers, then (after the
  // barrier, by which every wave has left the compute that last read
  // buffer S) compute it. The loads go out unconditionally (past
  // the last token they re-read it), and the barrier waits for the LDS
  // stores only:
  // a conditional load, or a barrier that also drains the loads in flight
  // (__syncthreads), made every token wait for the next one's loads.
  const std::integral_constant<int, 0> S0;
  const std::integral_constant<int, 1> S1;
  auto step = [&](auto S, long long sg, long long sg_next2) __attribute__((always_inline)) {
    store_tok(S);
    load_tok(S, sg_next2);
    lds_barrier();
    compute(decltype(S)::value, sg);
  };
  load_tok(S0, sg_lo);
  load_tok(S1, sg_lo + 1 <= sg_hi ? sg_lo + 1 : sg_hi);
  for (long long sg = sg_lo; sg <= sg_hi; sg += 2) {
    step(S0, sg, sg + 2 <= sg_hi ? sg + 2 : sg_hi);
    if (sg + 1 <= sg_hi) step(S1, sg + 1, sg + 3 <= sg_hi ? sg + 3 : sg_hi);   // uniform
  }
  // lane (g4, c16): channels 16 ct + 4 g4 .. + 3 of row c16
  if (rok) {
    const uint64_t a = lds_wr[16 * wave + c16];
    float* gr = bp.d_ori + (a - reinterpret_cast<uint64_t>(p.ori_kv)) / (D * 2) * D + 4 * g4;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) atomicAdd(gr + ct * 16 + i, acc[ct][i]);
  }
}

template <int D, typename QT>
int launch_bwd_win(const BwdParams& bp, int nblocks, hipStream_t st) {
  hipLaunchKernelGGL((sas_bwd_win_kernel<D, QT>), dim3(nblocks), dim3(256), 0, st, bp);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SAS_ELAUNCH, "sas_bwd_win launch: %s", hipGetErrorString(e));
  return SAS_OK;
}

// The window pass runs beside the per-token kernel, on a side stream of the
// library's (one per device, created on first use, default priority; forked
// from and joined back to the caller's stream by events): the per-token
// kernel is bound by the device's fp32 atomic rate, which 128 of the 256 CUs
// already reach (sas_bench_atomic_add_v1 with 128 four-wave workgroups:
// 323 G adds/s, with 2048: 326), so the window pass's workgroups take CUs it
// does not need. The two kernels write disjoint outputs (the per-token
// kernel skips the window rows' gradients). Calls made under stream capture
// run the two kernels one after the other on the caller's stream.
struct SideStream {
  hipStream_t st = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_side_mu;
SideStream g_side[64];

int side_stream(SideStream** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return set_error(SAS_ELAUNCH, "bwd: no device for the window pass's side stream");
  }
  SideStream& s = g_side[dev];
  if (!s.st) {
    if (hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&s.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&s.join, hipEventDisableTiming) != hipSuccess) {
      const hipError_t e = hipGetLastError();
      return set_error(SAS_ELAUNCH, "bwd: side stream: %s", hipGetErrorString(e));
    }
  }
  *out = &s;
  return SAS_OK;
}

template <int D, typename QT>
int launch_bwd64(const BwdParams& bp, int nblocks, hipStream_t st) {
  hipLaunchKernelGGL((sas_bwd64_kernel<D, QT>), dim3(nblocks), dim3(512), 0, st, bp);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SAS_ELAUNCH, "sas_bwd64 launch: %s", hipGetErrorString(e));
  return SAS_OK;
}

template <int D, typename QT, int NG>
int launch_bwd(const BwdParams& bp, int nblocks, hipStream_t st) {
  hipLaunchKernelGGL((sas_bwd_kernel<D, QT, NG>), dim3(nblocks), dim3(256 * NG), 0, st, bp);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SAS_ELAUNCH, "sas_bwd launch: %s", hipGetErrorString(e));
  return SAS_OK;
}

template <int D, typename QT>
int launch_bwd_ng(const BwdParams& bp, int ng, int nblocks, hipStream_t st) {
  return ng == 2 ? launch_bwd<D, QT, 2>(bp, nblocks, st) : launch_bwd<D, QT, 1>(bp, nblocks, st);
}

}  // namespace
}  // namespace sas

extern "C" int sas_bwd_v1(const SasBwdArgs* ba, void* stream) {
  using namespace sas;
  clear_error();
  if (!ba) return set_error(SAS_EINVAL, "bwd: null args");
  const SasFwdArgs* a = &ba->fwd;
  if (a->T < 0 || a->B < 1 || a->H < 1 || a->H % 16) return set_error(SAS_EINVAL, "bwd: bad T/B/H (H a multiple of 16)");
  if (a->D != 512 && a->D != 576) return set_error(SAS_EINVAL, "bwd: D must be 512 or 576");
  if (a->DV != kDV) return set_error(SAS_EINVAL, "bwd: DV must be 512");
  if (a->scenario < SAS_SWA || a->scenario > SAS_SCFA) return set_error(SAS_EINVAL, "bwd: bad scenario");
  if (a->q_dtype != SAS_DT_BF16 && a->q_dtype != SAS_DT_FP16) return set_error(SAS_EINVAL, "bwd: q dtype");
  if (a->kv_dtype != a->q_dtype) return set_error(SAS_EINVAL, "bwd: the cache must be in the query dtype (no fp8 rows)");
  if (a->win_left < 0) return set_error(SAS_EINVAL, "bwd: win_left out of range");
  if (a->scenario >= SAS_CFA && (a->cmp_ratio < 1 || a->K < 0)) return set_error(SAS_EINVAL, "bwd: bad cmp_ratio/K");
  const long long nslots = (long long)a->win_left + 1 + (a->scenario >= SAS_CFA ? a->K : 0);
  if (a->T == 0) return SAS_OK;
  if (!a->q || !a->ori_kv || !a->ori_block_table || !a->q_prefix || !a->act_kv || !a->sinks ||
      !a->out || !a->lse || !ba->dout || !ba->dq || !ba->d_ori_kv || !ba->d_sinks)
    return set_error(SAS_EINVAL, "bwd: null device pointer");
  if (a->scenario >= SAS_CFA && (!a->cmp_kv || !a->cmp_block_table || !ba->d_cmp_kv))
    return set_error(SAS_EINVAL, "bwd: CFA/SCFA need cmp_kv, cmp_block_table and d_cmp_kv");
  if (a->scenario == SAS_SCFA && !a->cmp_indices) return set_error(SAS_EINVAL, "bwd: SCFA needs cmp_indices");
  if (a->ori_block_size < 1 || a->ori_bt_stride < 1 || a->ori_num_blocks < 1)
    return set_error(SAS_EINVAL, "bwd: bad ori cache geometry");
  if (a->scenario >= SAS_CFA && (a->cmp_block_size < 1 || a->cmp_bt_stride < 1 || a->cmp_num_blocks < 1))
    return set_error(SAS_EINVAL, "bwd: bad cmp cache geometry");
  if ((double)a->ori_num_blocks * a->ori_block_size > 2147483000.0 ||
      (double)a->cmp_num_blocks * std::max<int64_t>(a->cmp_block_size, 1) > 2147483000.0)
    return set_error(SAS_EINVAL, "bwd: cache has more than 2^31 rows");

  BwdParams bp{};
  FwdParams& fp = bp.f;
  fp.q = (const uint8_t*)a->q;
  fp.ori_kv = (const uint8_t*)a->ori_kv;
  fp.ori_bt = a->ori_block_table;
  fp.cmp_kv = (const uint8_t*)a->cmp_kv;
  fp.cmp_bt = a->cmp_block_table;
  fp.cmp_idx = a->cmp_indices;
  fp.q_prefix = a->q_prefix;
  fp.act_q = a->act_q;
  fp.act_kv = a->act_kv;
  fp.sinks = a->sinks;
  fp.lse = a->lse;
  fp.T = (int)a->T; fp.B = (int)a->B; fp.H = (int)a->H;
  fp.ori_bs = (int)a->ori_block_size; fp.ori_bt_stride = (int)a->ori_bt_stride;
  fp.ori_nblocks = (int)a->ori_num_blocks;
  fp.cmp_bs = (int)std::max<int64_t>(a->cmp_block_size, 1);
  fp.cmp_bt_stride = (int)std::max<int64_t>(a->cmp_bt_stride, 1);
  fp.cmp_nblocks = (int)a->cmp_num_blocks;
  fp.K = (int)a->K; fp.scenario = a->scenario;
  fp.cmp_ratio = std::max(1, a->cmp_ratio); fp.win_left = a->win_left;
  fp.scale_log2 = a->softmax_scale * kLog2e;
  // KV splits: the caller's count, else enough (token, head group, split)
  // workgroups to fill the CUs, each split at least 128 slots (C2, 640 slots
  // per token, 32 tokens: 2 / 3 / 4 / 5 / 6 / 8 / 10 splits 110 / 89 / 79 /
  // 78 / 78 / 84 / 106 µs: below ~128 slots a workgroup's fixed cost and the
  // extra dq adds outweigh the CUs it adds)
  // 64 heads per workgroup when H allows, else two 16-head groups (each
  // doubling halves the dkv atomics)
  const bool b64 = SAS_BWD64 && a->H % 64 == 0;
  const int ng = b64 ? 4 : a->H % 32 == 0 ? SAS_BWD_NG : 1;
  fp.nhg = (int)a->H / (16 * ng);
  int ns = a->num_splits;
  if (ns <= 0) {
    // enough (token, head groups, split) workgroups for 8 waves per CU (one
    // 8-wave workgroup per CU: 64 heads; 32 heads; two of 4 waves: 16 heads)
    const long long items = a->T * fp.nhg;
    const long long wgs = ng == 1 ? 2LL * device_cus() : (long long)device_cus();
    const long long want = (wgs + items - 1) / items;
    ns = (int)std::min<long long>(want, std::max<long long>(1, nslots / 128));
  }
  // at most 64 splits of the planner's own choice; up to kMaxBwdSplits when
  // the token's slots need them or the caller asks
  constexpr long long kMaxBwdSplits = 1 << 16;
  ns = (int)std::max<long long>(1, std::min<long long>(ns, a->num_splits > 0 ? kMaxBwdSplits : 64));
  long long sps = (nslots + ns - 1) / ns;
  if (sps > kMaxSlots) {
    // a workgroup resolves at most kMaxSlots slots: more splits (dq is then
    // accumulated atomically across them)
    const long long need = (nslots + kMaxSlots - 1) / kMaxSlots;
    if (need > kMaxBwdSplits) return set_error(SAS_EINVAL, "bwd: too many key slots per token (%lld)", nslots);
    ns = (int)need;
    sps = (nslots + ns - 1) / ns;
  }
  fp.nsplit = (int)((nslots + sps - 1) / sps);
  fp.slots_per_split = (int)sps;
  bp.out = (const uint8_t*)a->out;
  bp.dout = (const uint8_t*)ba->dout;
  bp.dq = ba->dq;
  bp.d_ori = ba->d_ori_kv;
  bp.d_cmp = ba->d_cmp_kv;
  bp.d_sinks = ba->d_sinks;
  fp.nxcd = device_xcds();
  const long long nblocks_ll = (long long)((a->T + fp.nxcd - 1) / fp.nxcd) * fp.nhg * fp.nsplit * fp.nxcd;
  if (nblocks_ll > INT_MAX) return set_error(SAS_EINVAL, "bwd: %lld workgroups beyond one launch", nblocks_ll);
  const int nblocks = (int)nblocks_ll;
  // The key-major window pass (sas_bwd_win_kernel): by default when query
  // tokens share window rows (at least 64 query tokens per batch on
  // average, a prefill) and the call is not being captured, else when asked.
  // On the C3 prefill it takes the window rows' 2.97e8 atomics out of the
  // per-token kernel (3.97 -> 3.46 ms) and costs 575 µs itself (each token's
  // q / dO / O streamed by ~3 tiles: ~200 µs of loads; ~310 µs of MFMA and
  // LDS work with one wave per SIMD; ~180 µs per-token staging and
  // barriers); run after it, 4.03 against 3.97 ms, run beside it on the side
  // stream, 3.70 ms. Decode-like calls (one token per batch) share no rows,
  // and the pass's grid covers every position a block table can address:
  // per-token adds there.
  if ((a->flags & SAS_BWD_WINDOW_TOKENS) && (a->flags & SAS_BWD_WINDOW_KEYS))
    return set_error(SAS_EINVAL, "bwd: SAS_BWD_WINDOW_TOKENS and SAS_BWD_WINDOW_KEYS together");
  bool capturing = false;
  {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) {
      (void)hipGetLastError();
      cs = hipStreamCaptureStatusActive;   // unknown: as if capturing
    }
    capturing = cs != hipStreamCaptureStatusNone;
  }
  const bool win = (a->flags & SAS_BWD_WINDOW_KEYS) ||
                   (!(a->flags & SAS_BWD_WINDOW_TOKENS) && !capturing && a->T >= 64 * a->B);
  long long win_blocks = 0;
  if (win) {
    const long long tiles = ((long long)a->ori_bt_stride * a->ori_block_size + kWinRows - 1) / kWinRows;
    win_blocks = (long long)a->B * tiles * (a->H / 16);
    if (tiles > INT_MAX || win_blocks > INT_MAX)
      return set_error(SAS_EINVAL, "bwd: %lld window-pass workgroups beyond one launch", win_blocks);
    bp.win_pass = 1;
    bp.win_tiles = (int)tiles;
  }
  hipStream_t st = (hipStream_t)stream;
  // window pass beside the per-token kernel (see SideStream)
  std::unique_lock<std::mutex> side_lock(g_side_mu, std::defer_lock);
  SideStream* side = nullptr;
  if (win && win_blocks > 0) {
    if (!capturing) {
      side_lock.lock();
      const int src = side_stream(&side);
      if (src) return src;
      // fork: the side stream starts after everything the caller queued
      // before this call (the inputs), not after the per-token kernel
      if (hipEventRecord(side->fork, st) != hipSuccess || hipStreamWaitEvent(side->st, side->fork, 0) != hipSuccess) {
        const hipError_t e = hipGetLastError();
        return set_error(SAS_ELAUNCH, "bwd: fork to the side stream: %s", hipGetErrorString(e));
      }
    }
  }
  int rc;
  if (b64) {
    if (a->q_dtype == SAS_DT_BF16)
      rc = a->D == 576 ? launch_bwd64<576, __bf16>(bp, nblocks, st) : launch_bwd64<512, __bf16>(bp, nblocks, st);
    else
      rc = a->D == 576 ? launch_bwd64<576, _Float16>(bp, nblocks, st) : launch_bwd64<512, _Float16>(bp, nblocks, st);
  } else if (a->q_dtype == SAS_DT_BF16) {
    rc = a->D == 576 ? launch_bwd_ng<576, __bf16>(bp, ng, nblocks, st)
                     : launch_bwd_ng<512, __bf16>(bp, ng, nblocks, st);
  } else {
    rc = a->D == 576 ? launch_bwd_ng<576, _Float16>(bp, ng, nblocks, st)
                     : launch_bwd_ng<512, _Float16>(bp, ng, nblocks, st);
  }
  if (rc || !win || win_blocks == 0) return rc;
  hipStream_t wst = side ? side->st : st;
  if (a->q_dtype == SAS_DT_BF16)
    rc = a->D == 576 ? launch_bwd_win<576, __bf16>(bp, (int)win_blocks, wst)
                     : launch_bwd_win<512, __bf16>(bp, (int)win_blocks, wst);
  else
    rc = a->D == 576 ? launch_bwd_win<576, _Float16>(bp, (int)win_blocks, wst)
                     : launch_bwd_win<512, _Float16>(bp, (int)win_blocks, wst);
  if (side) {
    // join: the caller's stream continues once the window pass is done
    if (hipEventRecord(side->join, side->st) != hipSuccess || hipStreamWaitEvent(st, side->join, 0) != hipSuccess) {
      const hipError_t e = hipGetLastError();
      return set_error(SAS_ELAUNCH, "bwd: join from the side stream: %s", hipGetErrorString(e));
    }
  }
  return rc;
}
