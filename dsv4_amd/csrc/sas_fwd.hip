// sparse_attn_sharedkv forward for MI355X (gfx950 / CDNA4).
//
// One workgroup of 4 waves per (query token, head group, KV split). The
// token's key slots are the sliding window (win_left + 1 slots) followed by
// the top-k compressed entries (or the dense compressed prefix for CFA).
//
//  1. Resolve the workgroup's slot range to physical cache rows through the
//     block tables, drop masked slots (window band, idx < 0, idx >= causal
//     threshold) and compact the survivors, in order, into LDS.
//  2. The 4 waves form HW head-waves x KW key-groups (HW * KW = 4). A wave
//     owns 16 query heads; a key-group owns a contiguous share of the rows and
//     streams it in steps of 32 rows through an HW-deep ring of LDS slots.
//     Rows move HBM -> LDS with global_load_lds_dwordx4 (no register staging,
//     up to 4 x 36 KB in flight per CU), stored row-major with an XOR swizzle
//     of 16-byte chunks so both operand reads below are bank-conflict free.
//     fp8 rows go through registers instead (dequantised to bf16 on the way).
//  3. Per step and wave:  S^T[32 keys x 16 heads] = K . Q^T  (16x16x32 MFMA,
//     A from LDS, Q^T resident in VGPRs), sink-seeded online softmax in the
//     log2 domain, P rounded to the query dtype, then
//     O^T[512 x 16 heads] += V^T . P^T where the V^T operand comes straight
//     from the row-major tile with ds_read_b64_tr_b16 and P^T is already in
//     the register layout the MFMA wants (the S^T accumulator layout).
//  4. Key-groups merge through LDS (max / sum rescale); the result is the
//     output + LSE, or with several KV splits an unnormalised partial that
//     the LSE combine kernel merges.
//
// Semantics follow sparse_attn_sharedkv_tilelang/kernel.py:254-277 (work
// decode), :628-722 (window / compressed masks), :594-617 (sink seed),
// :877 (P cast), :1135-1145 (LSE), and golden.py:69-204.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "../../include/sas.h"
#include "sas_common.h"

#define LDS_AS __attribute__((address_space(3)))

namespace {

constexpr int kTR = 32;           // rows per pipeline step
constexpr int kDV = 512;          // output / V channels
constexpr int kMaxSlots = 1280;   // slot range one workgroup may own
constexpr int kXcds = 8;          // MI355X: 8 XCDs, workgroups dealt round-robin
constexpr int kSplitTarget = 128; // workgroups the automatic split count aims for
constexpr int kRow656 = 656;      // fp8 cache row bytes
constexpr int kChunksMax = 72;    // 16-byte chunks of a 576-channel bf16 row
constexpr int kSlotChunks = kTR * kChunksMax;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazyLog2 = 8.f;   // O / l rescale threshold (log2 units)

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

// Four statically distinct LDS slots: the compiler tracks LDS-DMA writes per
// buffer, so reads of one slot never wait on loads still landing in another.
__shared__ __attribute__((aligned(16))) uint4 lds_slot0[kSlotChunks];
__shared__ __attribute__((aligned(16))) uint4 lds_slot1[kSlotChunks];
__shared__ __attribute__((aligned(16))) uint4 lds_slot2[kSlotChunks];
__shared__ __attribute__((aligned(16))) uint4 lds_slot3[kSlotChunks];
__shared__ int lds_rows[kMaxSlots];
__shared__ int lds_cnt[8];
__shared__ float lds_ml[4][2][16];

__device__ __forceinline__ uint4* slot_by_index(int i) {
  return i == 0 ? lds_slot0 : i == 1 ? lds_slot1 : i == 2 ? lds_slot2 : lds_slot3;
}

template <int S>
__device__ __forceinline__ uint4* slot_ptr() {
  if constexpr (S == 0) return lds_slot0;
  else if constexpr (S == 1) return lds_slot1;
  else if constexpr (S == 2) return lds_slot2;
  else return lds_slot3;
}

struct FwdParams {
  const uint8_t* q;
  const uint8_t* ori_kv;
  const int32_t* ori_bt;
  const uint8_t* cmp_kv;
  const int32_t* cmp_bt;
  const int32_t* cmp_idx;
  const int32_t* q_prefix;
  const int32_t* act_q;
  const int32_t* act_kv;
  const float* sinks;
  uint8_t* out;
  float* lse;
  float* part_o;
  float* part_ml;
  int T, B, H;
  int ori_bs, ori_bt_stride, ori_nblocks;
  int cmp_bs, cmp_bt_stride, cmp_nblocks;
  int K, scenario, cmp_ratio, win_left;
  float scale_log2;
  int nsplit, slots_per_split, nhg, items, per_xcd;
};

// ---------------------------------------------------------------------------
// element helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even (finite inputs)
  return u >> 16;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

template <typename QT>
__device__ __forceinline__ uint32_t to_bits(float f);
template <>
__device__ __forceinline__ uint32_t to_bits<__bf16>(float f) { return f32_to_bf16_bits(f); }
template <>
__device__ __forceinline__ uint32_t to_bits<_Float16>(float f) { return f32_to_f16_bits(f); }

// OCP e4m3fn byte -> float (bias 7, subnormals m * 2^-9; 0x7f/0xff NaN are
// never produced by the cache writer, which saturates at 448).
__device__ __forceinline__ float e4m3_to_f32(uint32_t v) {
  const uint32_t e = (v >> 3) & 0xfu, m = v & 7u;
  float f = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0.001953125f;
  return (v & 0x80u) ? -f : f;
}

template <typename QT>
__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, const f32x4& c);
template <>
__device__ __forceinline__ f32x4 mfma16<__bf16>(const uint4& a, const uint4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16<_Float16>(const uint4& a, const uint4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Chunk swizzle inside each aligned group of 8 chunks of a row: row r keeps
// logical chunk c at position c ^ swz(r). With it, 8 lanes reading the same
// chunk of rows r..r+7 (QK^T operand) and 16 lanes reading 4 rows x 2 chunks
// (transposed PV operand) each touch distinct banks.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

// 16 bytes per lane global -> LDS (lane i lands at lds_addr + 16 i). Issued
// as inline asm so the compiler does not track it: its LDS-DMA tracking
// cannot tell the slots apart for transposed LDS reads and would wait for
// every load in flight. Completion is ordered explicitly with wait_vm<>()
// and lds_barrier(); loads return in order, so the compiler's own vmcnt
// waits for its loads stay conservative.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_addr) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(src), "s"(lds_addr)
      : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
  return (uint32_t)(uintptr_t)(const LDS_AS void*)p;
}

// s_waitcnt vmcnt(N) leaving expcnt / lgkmcnt alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}
// LDS reads done, then a workgroup barrier (no memory fence: in-flight LDS
// DMA of other slots keeps streaming across it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
}

// ---------------------------------------------------------------------------
// forward kernel
// ---------------------------------------------------------------------------

// HW head-waves x KW key-groups; D = q/k channels; QT = query dtype;
// KVF: 0 = cache rows in the query dtype, 1 = 656-byte fp8 rows.
template <int HW, int D, typename QT, int KVF>
struct Cfg {
  static constexpr int KW = 4 / HW;
  static constexpr int NST = HW;                 // ring depth per key-group
  static constexpr int CH = D / 8;               // 16-byte chunks per bf16 row
  static constexpr int KS = D / 32;              // QK^T k-steps
  static constexpr int GT = HW * 64;             // threads per key-group
  static constexpr int OPS = kTR * CH / GT;      // DMA ops per thread per step
  static constexpr int ROWB = KVF ? kRow656 : D * 2;
  // fp8 register staging: 40 work chunks per row (32 latent x 16 values, 8 rope)
  static constexpr int FCPR = 40;
  static constexpr int FOPS = (kTR * FCPR + GT - 1) / GT;
  static_assert(kTR * CH % GT == 0, "uniform DMA op count");
};

template <int HW, int D, typename QT, int KVF>
struct Fwd {
  using C = Cfg<HW, D, QT, KVF>;
  const FwdParams& p;
  const int lane, c16, g, kw, hw, gt;
  const int* rows;     // this key-group's compacted row ids
  int nrows;           // rows this key-group owns
  int nsteps, nsteps_max, dummy;
  uint4 qf[C::KS];
  float m_run, l_run;
  f32x4 acc[kDV / 16];
  uint4 fbuf[KVF ? C::FOPS : 1];
  float fsc[KVF ? C::FOPS : 1];

  __device__ Fwd(const FwdParams& p_, int lane_, int wave)
      : p(p_), lane(lane_), c16(lane_ & 15), g(lane_ >> 4), kw(wave / HW), hw(wave % HW),
        gt((wave % HW) * 64 + lane_) {}

  __device__ __forceinline__ const uint8_t* row_ptr(int id) const {
    return id >= 0 ? p.ori_kv + (size_t)id * C::ROWB : p.cmp_kv + (size_t)(-id - 2) * C::ROWB;
  }

  // -- bf16 / fp16 rows: DMA one 32-row step into slot SLOT --------------------
  template <int SLOT>
  __device__ __forceinline__ void issue(int step) {
    uint4* slot = slot_ptr<SLOT>();
    const int* rp = rows + step * kTR;
    const int nk = min(kTR, nrows - step * kTR);
#pragma unroll
    for (int j = 0; j < C::OPS; ++j) {
      const int blk = j * C::GT + hw * 64;          // wave-uniform chunk base
      const int P = blk + lane;
      const int r = P / C::CH, pc = P - r * C::CH;
      const int c = pc ^ swz(r);
      const int id = r < nk ? rp[r] : dummy;
      dma16(row_ptr(id) + c * 16, __builtin_amdgcn_readfirstlane(lds_addr_of(slot + blk)));
    }
  }

  // -- fp8 rows: global -> registers, dequantised into slot on store ---------
  __device__ __forceinline__ void fload(int step) {
    const int* rp = rows + step * kTR;
    const int nk = min(kTR, nrows - step * kTR);
#pragma unroll
    for (int k = 0; k < C::FOPS; ++k) {
      const int e = gt + k * C::GT;
      const int r = e / C::FCPR, c = e - r * C::FCPR;
      fbuf[k] = make_uint4(0, 0, 0, 0);
      fsc[k] = 0.f;
      if (e < kTR * C::FCPR && r < nk) {
        const uint8_t* src = row_ptr(rp[r]);
        if (c < 32) {
          fbuf[k] = *reinterpret_cast<const uint4*>(src + c * 16);
          fsc[k] = *reinterpret_cast<const float*>(src + 512 + 4 * (c >> 3));
        } else {
          fbuf[k] = *reinterpret_cast<const uint4*>(src + 528 + (c - 32) * 16);
        }
      }
    }
  }
  template <int SLOT>
  __device__ __forceinline__ void fstore() {
    uint4* slot = slot_ptr<SLOT>();
#pragma unroll
    for (int k = 0; k < C::FOPS; ++k) {
      const int e = gt + k * C::GT;
      if (e >= kTR * C::FCPR) continue;
      const int r = e / C::FCPR, c = e - r * C::FCPR;
      uint4* row = slot + r * C::CH;
      const int sw = swz(r);
      if (c < 32) {
        const uint32_t w[4] = {fbuf[k].x, fbuf[k].y, fbuf[k].z, fbuf[k].w};
        uint32_t o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t b0 = (w[i >> 1] >> ((i & 1) * 16)) & 0xffu;
          const uint32_t b1 = (w[i >> 1] >> ((i & 1) * 16 + 8)) & 0xffu;
          o[i] = f32_to_bf16_bits(e4m3_to_f32(b0) * fsc[k]) |
                 (f32_to_bf16_bits(e4m3_to_f32(b1) * fsc[k]) << 16);
        }
        row[(2 * c) ^ sw] = make_uint4(o[0], o[1], o[2], o[3]);
        row[(2 * c + 1) ^ sw] = make_uint4(o[4], o[5], o[6], o[7]);
      } else {
        row[(64 + c - 32) ^ sw] = fbuf[k];
      }
    }
  }

  // -- one 32-key step of attention for this wave's 16 heads ----------------
  template <int SLOT>
  __device__ __forceinline__ void compute(int step) {
    const uint4* slot = slot_ptr<SLOT>();
    const int nk = min(kTR, nrows - step * kTR);
    f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    // K operand: rows c16 and 16 + c16 share swz(); logical chunk 4ks + g only
    // changes in its low 3 bits with ks & 1, the rest is an immediate offset.
    // Reads run kPfK k-steps ahead of the MFMAs that consume them.
    const int ksw = swz(c16);
    const uint4* qrow = slot + c16 * C::CH;
    const int qo0 = g ^ ksw, qo1 = (4 + g) ^ ksw;
    auto kfrag = [&](int ks, int mt) {
      return qrow[mt * 16 * C::CH + (ks >> 1) * 8 + ((ks & 1) ? qo1 : qo0)];
    };
    constexpr int kPfK = 3;
    uint4 af[kPfK][2];
#pragma unroll
    for (int i = 0; i < kPfK; ++i) { af[i][0] = kfrag(i, 0); af[i][1] = kfrag(i, 1); }
    // even / odd k-steps accumulate separately: four independent MFMA chains
    f32x4 sodd[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      const uint4 a0 = af[ks % kPfK][0], a1 = af[ks % kPfK][1];
      if (ks + kPfK < C::KS) {
        af[ks % kPfK][0] = kfrag(ks + kPfK, 0);
        af[ks % kPfK][1] = kfrag(ks + kPfK, 1);
      }
      if (ks & 1) {
        sodd[0] = mfma16<QT>(a0, qf[ks], sodd[0]);
        sodd[1] = mfma16<QT>(a1, qf[ks], sodd[1]);
      } else {
        sacc[0] = mfma16<QT>(a0, qf[ks], sacc[0]);
        sacc[1] = mfma16<QT>(a1, qf[ks], sacc[1]);
      }
    }
    // schedule: the prefetch reads first, then per k-step 2 MFMAs + 2 reads
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kPfK, 0);
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      if (ks + kPfK < C::KS) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    sacc[0] += sodd[0];
    sacc[1] += sodd[1];
    float sv[2][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = mt * 16 + g * 4 + j;
        const float x = key < nk ? sacc[mt][j] * p.scale_log2 : -INFINITY;
        sv[mt][j] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    // Lazy rescale: m_run is a reference max, moved (and O, l rescaled) only
    // when some head's max rises more than kLazyLog2 above it, so P <= 2^8.
    // out = acc / l and lse = m_run + log2 l are exact for any reference.
    if (__ballot(mloc > m_run + kLazyLog2)) {
      const float m_new = fmaxf(m_run, mloc);
      const float alpha = exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int mt = 0; mt < kDV / 16; ++mt) acc[mt] *= alpha;
    }
    float lsum = 0.f;
    uint32_t pk[4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      float pv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pv[j] = exp2f(sv[mt][j] - m_run);
        lsum += pv[j];
      }
      pk[mt * 2 + 0] = to_bits<QT>(pv[0]) | (to_bits<QT>(pv[1]) << 16);
      pk[mt * 2 + 1] = to_bits<QT>(pv[2]) | (to_bits<QT>(pv[3]) << 16);
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    l_run += lsum;
    const uint4 pfrag = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    // V^T operand by transposed reads: lanes of group g address rows
    // 4g + c16/4 (and +16), channels mt*16 + 4*(c16&3); each lane receives
    // 4 keys of channel mt*16 + c16. Reads run kPfV channel tiles ahead.
    const int vr = 4 * g + (c16 >> 2);
    const int vsw = swz(vr);
    const int vb = (c16 & 3) >> 1;
    const char* vbase = reinterpret_cast<const char*>(slot) + vr * C::CH * 16 + (c16 & 1) * 8;
    // logical chunk 2mt + vb: its low 3 bits cycle with mt & 3
    int voff[4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) voff[q4] = ((2 * q4 + vb) ^ vsw) * 16;
    auto vfrag = [&](int mt) {
      const char* a0 = vbase + (mt >> 2) * 128 + voff[mt & 3];
      const i16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4*)(a0));
      const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4*)(a0 + 16 * C::CH * 16));
      const uint2 u0 = __builtin_bit_cast(uint2, v0), u1 = __builtin_bit_cast(uint2, v1);
      return make_uint4(u0.x, u0.y, u1.x, u1.y);
    };
    constexpr int kPfV = 4;
    uint4 vf[kPfV];
#pragma unroll
    for (int i = 0; i < kPfV; ++i) vf[i] = vfrag(i);
#pragma unroll
    for (int mt = 0; mt < kDV / 16; ++mt) {
      const uint4 a = vf[mt % kPfV];
      if (mt + kPfV < kDV / 16) vf[mt % kPfV] = vfrag(mt + kPfV);
      acc[mt] = mfma16<QT>(a, pfrag, acc[mt]);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kPfV, 1);
#pragma unroll
    for (int mt = 0; mt < kDV / 16; ++mt) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      if (mt + kPfV < kDV / 16) __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    }
  }

  // -- the step loop of key-group KWI (slots KWI*NST .. +NST-1) ---------------
  template <int KWI, int J>
  __device__ __forceinline__ void step_j(int it0) {
    constexpr int SLOT = KWI * C::NST + J;
    const int it = it0 + J;
    if (it >= nsteps_max) return;                       // uniform over the workgroup
    if constexpr (!KVF) {
      // my DMA for step `it` done (steps after it may still stream), then all waves
      const int after = it < nsteps ? min(C::NST - 1, nsteps - 1 - it) : 0;
      if (after <= 0) wait_vm<0>();
      else if (after == 1) wait_vm<C::OPS>();
      else if (after == 2) wait_vm<(C::NST > 2 ? 2 * C::OPS : 0)>();
      else wait_vm<(C::NST > 3 ? 3 * C::OPS : 0)>();
      lds_barrier();
      if (it < nsteps) compute<SLOT>(it);
      lds_barrier();
      if (it + C::NST < nsteps) issue<SLOT>(it + C::NST);
    } else {
      // fp8: registers hold step it+1; slot (it & 1) of the group holds step it
      lds_barrier();
      if (it < nsteps) compute<SLOT>(it);
      if (it + 1 < nsteps) {
        constexpr int NEXT = KWI * C::NST + ((J + 1) % C::NST);
        fstore<NEXT>();
      }
      if (it + 2 < nsteps) fload(it + 2);
    }
  }

  template <int KWI>
  __device__ __forceinline__ void run_group() {
    if constexpr (!KVF) {
#pragma unroll
      for (int j = 0; j < C::NST; ++j) {
        if (j < nsteps) {
          if (j == 0) issue<KWI * C::NST + 0>(0);
          if constexpr (C::NST > 1) if (j == 1) issue<KWI * C::NST + 1>(1);
          if constexpr (C::NST > 2) if (j == 2) issue<KWI * C::NST + 2>(2);
          if constexpr (C::NST > 3) if (j == 3) issue<KWI * C::NST + 3>(3);
        }
      }
    } else {
      if (nsteps > 0) { fload(0); fstore<KWI * C::NST>(); }
      if (nsteps > 1) fload(1);
    }
    for (int it0 = 0; it0 < nsteps_max; it0 += C::NST) {
      step_j<KWI, 0>(it0);
      if constexpr (C::NST > 1) step_j<KWI, 1>(it0);
      if constexpr (C::NST > 2) step_j<KWI, 2>(it0);
      if constexpr (C::NST > 3) step_j<KWI, 3>(it0);
    }
  }
};

template <int HW, int D, typename QT, int KVF>
__global__ void __launch_bounds__(256)
sas_fwd_kernel(const FwdParams p) {
  using C = Cfg<HW, D, QT, KVF>;
  static_assert(!KVF || HW >= 2, "fp8 staging needs a ring of at least 2 slots");
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  // XCD-aware item mapping: XCD x = blockIdx % 8 owns a contiguous item range,
  // so all splits / head groups of a token (and neighbouring tokens) share L2.
  const int item = (int)(blockIdx.x % kXcds) * p.per_xcd + (int)(blockIdx.x / kXcds);
  if (item >= p.items) return;
  const int per_tok = p.nhg * p.nsplit;
  const int t = item / per_tok;
  const int hg = (item % per_tok) / p.nsplit;
  const int sp = item % p.nsplit;

  // token -> (batch, position): largest b with q_prefix[b] <= t
  int lo = 0, hi = p.B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.q_prefix[mid] <= t) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int s = t - p.q_prefix[b];
  const int aq = p.act_q[b], akv = p.act_kv[b];
  const bool padded = s < 0 || s >= aq;
  const int sg = akv - aq + s;                               // causal position
  const int nwin = (padded || sg < 0) ? 0 : min(sg, p.win_left) + 1;
  const int wlo = sg - nwin + 1;                             // = max(sg - win_left, 0)
  const int thr = (padded || sg + 1 <= 0) ? 0 : (sg + 1) / p.cmp_ratio;
  const int wincap = p.win_left + 1;
  const int nslots = wincap + (p.scenario >= 2 ? p.K : 0);
  const int s0 = sp * p.slots_per_split;
  const int s1 = min(s0 + p.slots_per_split, nslots);

  // The first slot chunk's top-k index is fetched before Q (loads return in
  // order, so waiting for the index never waits for Q); Q's latency then
  // overlaps the block-table lookups of the slot resolution.
  int idx_first = 0;
  {
    const int j = s0 + tid;
    if (p.scenario == SAS_SCFA && j < s1 && j >= wincap && !padded)
      idx_first = p.cmp_idx[(size_t)t * p.K + (j - wincap)];
  }
  // Q^T operand in registers (head hq, channels ks*32 + 8g .. +8)
  Fwd<HW, D, QT, KVF> f(p, lane, wave);
  const int hq = hg * (16 * HW) + f.hw * 16 + f.c16;
  {
    const uint4* qp = reinterpret_cast<const uint4*>(p.q + ((size_t)t * p.H + hq) * D * 2);
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) f.qf[ks] = qp[ks * 4 + f.g];
  }

  // ---- 1. resolve + compact slot range [s0, s1) -------------------------
  // Stored ids: raw rows as id >= 0, compressed rows as -(id + 2).
  int nvalid = 0;
  for (int c0 = s0; c0 < s1; c0 += 256) {
    const int j = c0 + tid;
    int rid = -1;
    if (j < s1 && !padded) {
      if (j < wincap) {
        if (j < nwin) {
          const int pos = wlo + j;
          const int blk = pos / p.ori_bs;
          if (blk < p.ori_bt_stride) {
            const int phys = p.ori_bt[(size_t)b * p.ori_bt_stride + blk];
            if (phys >= 0 && phys < p.ori_nblocks) rid = phys * p.ori_bs + pos % p.ori_bs;
          }
        }
      } else {
        const int k = j - wincap;
        const int idx = p.scenario != SAS_SCFA ? k
                        : c0 == s0 ? idx_first : p.cmp_idx[(size_t)t * p.K + k];
        if (idx >= 0 && idx < thr) {
          const int blk = idx / p.cmp_bs;
          if (blk < p.cmp_bt_stride) {
            const int phys = p.cmp_bt[(size_t)b * p.cmp_bt_stride + blk];
            if (phys >= 0 && phys < p.cmp_nblocks) rid = -(phys * p.cmp_bs + idx % p.cmp_bs + 2);
          }
        }
      }
    }
    const bool v = rid != -1;
    const uint64_t mask = __ballot(v);
    const int before = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) lds_cnt[wave] = __popcll(mask);
    lds_barrier();
    int wpre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int cw = lds_cnt[w];
      wpre += w < wave ? cw : 0;
      tot += cw;
    }
    if (v) lds_rows[nvalid + wpre + before] = rid;
    nvalid += tot;
    lds_barrier();
  }

  // key-group shares: whole 32-row steps, group 0 first
  const int per = ((nvalid + C::KW * kTR - 1) / (C::KW * kTR)) * kTR;
  const int gbeg = min(nvalid, f.kw * per);
  f.rows = lds_rows + gbeg;
  f.nrows = min(nvalid, gbeg + per) - gbeg;
  f.nsteps = (f.nrows + kTR - 1) / kTR;
  f.nsteps_max = per / kTR;
  f.dummy = nvalid > 0 ? lds_rows[0] : 0;

  // retire every load the compiler tracks (Q, tables, indices) before the
  // DMA ring starts, so none of its own vmcnt waits lands inside the loop
  __builtin_amdgcn_s_waitcnt(0);
  const bool seed_sink = p.nsplit == 1 && f.kw == 0;
  f.m_run = seed_sink ? p.sinks[hq] * kLog2e : -INFINITY;
  f.l_run = seed_sink ? 1.f : 0.f;
#pragma unroll
  for (int i = 0; i < kDV / 16; ++i) f.acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- 2./3. pipelined step loop of this wave's key-group -----------------
  if (f.kw == 0) f.template run_group<0>();
  if constexpr (C::KW > 1) { if (f.kw == 1) f.template run_group<1>(); }
  if constexpr (C::KW > 2) { if (f.kw == 2) f.template run_group<2>(); }
  if constexpr (C::KW > 3) { if (f.kw == 3) f.template run_group<3>(); }

  // ---- 4. merge key-groups, epilogue --------------------------------------
  float M = f.m_run, L = f.l_run, w_self = 1.f;
  if constexpr (C::KW > 1) {
    if (f.g == 0) { lds_ml[wave][0][f.c16] = f.m_run; lds_ml[wave][1][f.c16] = f.l_run; }
    __syncthreads();
    M = -INFINITY;
#pragma unroll
    for (int k = 0; k < C::KW; ++k) M = fmaxf(M, lds_ml[k * HW + f.hw][0][f.c16]);
    L = 0.f;
#pragma unroll
    for (int k = 0; k < C::KW; ++k) {
      const float mk = lds_ml[k * HW + f.hw][0][f.c16];
      const float wk = mk == -INFINITY ? 0.f : exp2f(mk - M);
      L += wk * lds_ml[k * HW + f.hw][1][f.c16];
      if (k == f.kw) w_self = wk;
    }
    // scaled O of every wave -> its own slot as [head 16][512] fp32 (32 KB)
    float* obuf = reinterpret_cast<float*>(slot_by_index(wave));
#pragma unroll
    for (int mt = 0; mt < kDV / 16; ++mt) {
      const f32x4 v = f.acc[mt] * w_self;
      *reinterpret_cast<float4*>(obuf + f.c16 * kDV + mt * 16 + f.g * 4) =
          make_float4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();
  }

  const int nhead_wg = 16 * HW;
  if constexpr (C::KW == 1) {
    if (p.nsplit == 1) {
      const float inv = padded ? 0.f : 1.f / L;
      uint16_t* op = reinterpret_cast<uint16_t*>(p.out) + ((size_t)t * p.H + hq) * kDV;
#pragma unroll
      for (int mt = 0; mt < kDV / 16; ++mt) {
        const uint32_t w0 = to_bits<QT>(f.acc[mt][0] * inv) | (to_bits<QT>(f.acc[mt][1] * inv) << 16);
        const uint32_t w1 = to_bits<QT>(f.acc[mt][2] * inv) | (to_bits<QT>(f.acc[mt][3] * inv) << 16);
        *reinterpret_cast<uint2*>(op + mt * 16 + f.g * 4) = make_uint2(w0, w1);
      }
      if (f.g == 0) p.lse[(size_t)t * p.H + hq] = padded ? 0.f : M * kLn2 + logf(L);
    } else {
      const size_t row = ((size_t)t * p.nsplit + sp) * p.H + hq;
      float* po = p.part_o + row * kDV;
#pragma unroll
      for (int mt = 0; mt < kDV / 16; ++mt)
        *reinterpret_cast<float4*>(po + mt * 16 + f.g * 4) =
            make_float4(f.acc[mt][0], f.acc[mt][1], f.acc[mt][2], f.acc[mt][3]);
      if (f.g == 0) {
        p.part_ml[row * 2 + 0] = M;
        p.part_ml[row * 2 + 1] = padded ? -1.f : L;  // l < 0 marks a padded token
      }
    }
  } else {
    // every thread sums (head, 4 channels) items over the KW waves of its head-wave
    const float* mlb = &lds_ml[0][0][0];
    for (int e = tid; e < nhead_wg * (kDV / 4); e += 256) {
      const int hh = e / (kDV / 4), c4 = e % (kDV / 4);
      const int hwi = hh >> 4, hl = hh & 15;
      float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int k = 0; k < C::KW; ++k) {
        const float* ob = reinterpret_cast<const float*>(slot_by_index(k * HW + hwi));
        const float4 v = *reinterpret_cast<const float4*>(ob + hl * kDV + c4 * 4);
        o.x += v.x; o.y += v.y; o.z += v.z; o.w += v.w;
      }
      const int h = hg * nhead_wg + hh;
      if (p.nsplit == 1) {
        // recompute this head's merged sum (the seed sink sits in key-group 0)
        float Mh = -INFINITY, Lh = 0.f;
#pragma unroll
        for (int k = 0; k < C::KW; ++k) Mh = fmaxf(Mh, mlb[((k * HW + hwi) * 2 + 0) * 16 + hl]);
#pragma unroll
        for (int k = 0; k < C::KW; ++k) {
          const float mk = mlb[((k * HW + hwi) * 2 + 0) * 16 + hl];
          Lh += (mk == -INFINITY ? 0.f : exp2f(mk - Mh)) * mlb[((k * HW + hwi) * 2 + 1) * 16 + hl];
        }
        const float inv = padded ? 0.f : 1.f / Lh;
        const uint32_t w0 = to_bits<QT>(o.x * inv) | (to_bits<QT>(o.y * inv) << 16);
        const uint32_t w1 = to_bits<QT>(o.z * inv) | (to_bits<QT>(o.w * inv) << 16);
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + ((size_t)t * p.H + h) * kDV + c4 * 4) =
            make_uint2(w0, w1);
        if (c4 == 0) p.lse[(size_t)t * p.H + h] = padded ? 0.f : Mh * kLn2 + logf(Lh);
      } else {
        const size_t row = ((size_t)t * p.nsplit + sp) * p.H + h;
        *reinterpret_cast<float4*>(p.part_o + row * kDV + c4 * 4) = o;
        if (c4 == 0) {
          float Mh = -INFINITY, Lh = 0.f;
#pragma unroll
          for (int k = 0; k < C::KW; ++k) Mh = fmaxf(Mh, mlb[((k * HW + hwi) * 2 + 0) * 16 + hl]);
#pragma unroll
          for (int k = 0; k < C::KW; ++k) {
            const float mk = mlb[((k * HW + hwi) * 2 + 0) * 16 + hl];
            Lh += (mk == -INFINITY ? 0.f : exp2f(mk - Mh)) * mlb[((k * HW + hwi) * 2 + 1) * 16 + hl];
          }
          p.part_ml[row * 2 + 0] = Mh;
          p.part_ml[row * 2 + 1] = padded ? -1.f : Lh;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// split-KV combine
// ---------------------------------------------------------------------------

constexpr int kCombineThreads = 256;
constexpr int kMaxCombineSplits = 64;

// One workgroup per (token, 2 heads), thread = (head, 4 channels). Each
// thread derives its head's merge weights from the small (m, l) partials and
// streams its S partial rows once; loads are independent, so they overlap.
template <typename QT>
__global__ void __launch_bounds__(kCombineThreads)
sas_combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                   const float* __restrict__ sinks, uint8_t* __restrict__ out,
                   float* __restrict__ lse, int S, int H) {
  constexpr int kHeads = kCombineThreads / (kDV / 4);  // 2
  const int nhb = (H + kHeads - 1) / kHeads;
  const int t = blockIdx.x / nhb;
  const int c4 = threadIdx.x % (kDV / 4);
  const int h = (blockIdx.x % nhb) * kHeads + threadIdx.x / (kDV / 4);
  if (h >= H) return;
  const size_t row0 = (size_t)t * S * H + h;
  const float sink2 = sinks[h] * kLog2e;
  float M = sink2;
  bool pad = false;
#pragma unroll 8
  for (int s = 0; s < S; ++s) {
    const float2 ml = *reinterpret_cast<const float2*>(part_ml + (row0 + (size_t)s * H) * 2);
    M = fmaxf(M, ml.x);
    pad |= ml.y < 0.f;
  }
  float L = exp2f(sink2 - M);
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
  for (int s = 0; s < S; ++s) {
    const size_t r = row0 + (size_t)s * H;
    const float2 ml = *reinterpret_cast<const float2*>(part_ml + r * 2);
    const float4 v = *reinterpret_cast<const float4*>(part_o + r * kDV + c4 * 4);
    const float w = exp2f(ml.x - M);
    L += w * ml.y;
    o.x += w * v.x; o.y += w * v.y; o.z += w * v.z; o.w += w * v.w;
  }
  const float il = pad ? 0.f : 1.f / L;
  const uint32_t w0 = to_bits<QT>(o.x * il) | (to_bits<QT>(o.y * il) << 16);
  const uint32_t w1 = to_bits<QT>(o.z * il) | (to_bits<QT>(o.w * il) << 16);
  *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + ((size_t)t * H + h) * kDV + c4 * 4) =
      make_uint2(w0, w1);
  if (c4 == 0) lse[(size_t)t * H + h] = pad ? 0.f : M * kLn2 + logf(L);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

struct Plan {
  int hw, nhg, nslots, nsplit, sps;
  size_t ws;
};

int make_plan(const SasFwdArgs* a, Plan* pl) {
  if (!a) return sas::set_error(SAS_EINVAL, "null args");
  if (a->T < 0 || a->B < 1 || a->H < 1) return sas::set_error(SAS_EINVAL, "bad T/B/H");
  if (a->D != 512 && a->D != 576) return sas::set_error(SAS_EINVAL, "D must be 512 or 576 (got %lld)", (long long)a->D);
  if (a->DV != kDV) return sas::set_error(SAS_EINVAL, "DV must be 512 (got %lld)", (long long)a->DV);
  if (a->H % 16) return sas::set_error(SAS_EINVAL, "H must be a multiple of 16 (got %lld)", (long long)a->H);
  if (a->scenario < SAS_SWA || a->scenario > SAS_SCFA) return sas::set_error(SAS_EINVAL, "bad scenario");
  if (a->flags & ~SAS_FWD_NO_COMBINE) return sas::set_error(SAS_EINVAL, "unknown flags 0x%x", a->flags);
  if (a->win_left < 0 || a->win_left > 8191) return sas::set_error(SAS_EINVAL, "win_left out of range");
  if (a->scenario >= SAS_CFA && (a->cmp_ratio < 1 || a->K < 0)) return sas::set_error(SAS_EINVAL, "bad cmp_ratio/K");
  const bool fp8 = a->kv_dtype == SAS_DT_FP8_E4M3_ROW656;
  // head-waves per workgroup: 4 whenever H allows it (64 heads share every
  // gathered tile, so each KV row crosses HBM->LDS once per token); 2 or 1
  // only for head counts that are not a multiple of 64.
  int hw = a->head_waves;
  if (hw <= 0) hw = 4;
  if (hw != 1 && hw != 2 && hw != 4) return sas::set_error(SAS_EINVAL, "head_waves must be 1, 2 or 4");
  while (hw > 1 && a->H % (16 * hw)) hw >>= 1;
  if (fp8) {  // fp8 staging registers only fit with 4 head-waves (or 2 when H = 32k)
    if (a->H % 32) return sas::set_error(SAS_EINVAL, "fp8 cache rows need H a multiple of 32");
    hw = a->H % 64 ? 2 : 4;
  }
  pl->hw = hw;
  pl->nhg = (int)a->H / (16 * hw);
  pl->nslots = a->win_left + 1 + (a->scenario >= SAS_CFA ? (int)a->K : 0);
  int ns = a->num_splits;
  if (ns <= 0) {
    // about half a workgroup per CU: every extra split adds a partial
    // write + combine read of 2 KB per head, which past ~128 workgroups
    // costs more than the extra streaming parallelism gains; splits no
    // smaller than one 32-row step
    const long long items = std::max<long long>(1, (long long)a->T * pl->nhg);
    const long long want = (kSplitTarget + items - 1) / items;
    const int max_by_step = std::max(1, (pl->nslots + kTR - 1) / kTR);
    ns = (int)std::min<long long>(std::max<long long>(want, 1), max_by_step);
  }
  ns = std::max(1, std::min(ns, kMaxCombineSplits));
  int sps = (pl->nslots + ns - 1) / ns;
  if (sps > kMaxSlots) {
    ns = (pl->nslots + kMaxSlots - 1) / kMaxSlots;
    if (ns > kMaxCombineSplits) return sas::set_error(SAS_EINVAL, "too many key slots per token");
    sps = (pl->nslots + ns - 1) / ns;
  }
  ns = (pl->nslots + sps - 1) / sps;  // drop empty trailing splits
  pl->nsplit = std::max(ns, 1);
  pl->sps = sps;
  pl->ws = pl->nsplit > 1 ? (size_t)a->T * pl->nsplit * a->H * (kDV + 2) * sizeof(float) : 0;
  return SAS_OK;
}

template <int HW, int D, typename QT, int KVF>
int launch_fwd(const FwdParams& fp, int nblocks, hipStream_t st) {
  hipLaunchKernelGGL((sas_fwd_kernel<HW, D, QT, KVF>), dim3(nblocks), dim3(256), 0, st, fp);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return sas::set_error(SAS_ELAUNCH, "sas_fwd launch: %s", hipGetErrorString(e));
  return SAS_OK;
}

template <int D, typename QT, int KVF>
int dispatch_hw(int hw, const FwdParams& fp, int nb, hipStream_t st) {
  if constexpr (!KVF) {
    if (hw == 1) return launch_fwd<1, D, QT, KVF>(fp, nb, st);
  }
  if (hw == 2) return launch_fwd<2, D, QT, KVF>(fp, nb, st);
  if (hw == 4) return launch_fwd<4, D, QT, KVF>(fp, nb, st);
  return sas::set_error(SAS_EINVAL, "unsupported head grouping");
}

int combine_impl(const SasCombineArgs* a, hipStream_t st) {
  if (!a || !a->part_o || !a->part_ml || !a->sinks || !a->out || !a->lse)
    return sas::set_error(SAS_EINVAL, "combine: null pointer");
  if (a->DV != kDV || a->S < 1 || a->S > kMaxCombineSplits || a->H < 1 || a->T < 0)
    return sas::set_error(SAS_EINVAL, "combine: bad dims (S must be 1..64, DV 512)");
  if (a->T == 0) return SAS_OK;
  constexpr int kHeads = kCombineThreads / (kDV / 4);
  const dim3 grid((unsigned)(a->T * ((a->H + kHeads - 1) / kHeads)));
  if (a->out_dtype == SAS_DT_BF16)
    hipLaunchKernelGGL(sas_combine_kernel<__bf16>, grid, dim3(kCombineThreads), 0, st, a->part_o,
                       a->part_ml, a->sinks, (uint8_t*)a->out, a->lse, (int)a->S, (int)a->H);
  else if (a->out_dtype == SAS_DT_FP16)
    hipLaunchKernelGGL(sas_combine_kernel<_Float16>, grid, dim3(kCombineThreads), 0, st, a->part_o,
                       a->part_ml, a->sinks, (uint8_t*)a->out, a->lse, (int)a->S, (int)a->H);
  else
    return sas::set_error(SAS_EINVAL, "combine: bad out dtype");
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return sas::set_error(SAS_ELAUNCH, "sas_combine launch: %s", hipGetErrorString(e));
  return SAS_OK;
}

}  // namespace

extern "C" int sas_fwd_plan(const SasFwdArgs* a, int32_t* num_splits, size_t* workspace_bytes) {
  sas::clear_error();
  Plan pl;
  const int rc = make_plan(a, &pl);
  if (rc) return rc;
  if (num_splits) *num_splits = pl.nsplit;
  if (workspace_bytes) *workspace_bytes = pl.ws;
  return SAS_OK;
}

extern "C" int sas_fwd_v1(const SasFwdArgs* a, void* stream) {
  sas::clear_error();
  Plan pl;
  int rc = make_plan(a, &pl);
  if (rc) return rc;
  if (a->T == 0) return SAS_OK;
  if (!a->q || !a->ori_kv || !a->ori_block_table || !a->q_prefix || !a->act_q || !a->act_kv ||
      !a->sinks || !a->out || !a->lse)
    return sas::set_error(SAS_EINVAL, "null device pointer");
  if (a->scenario >= SAS_CFA && (!a->cmp_kv || !a->cmp_block_table))
    return sas::set_error(SAS_EINVAL, "CFA/SCFA need cmp_kv and cmp_block_table");
  if (a->scenario == SAS_SCFA && !a->cmp_indices) return sas::set_error(SAS_EINVAL, "SCFA needs cmp_indices");
  if (a->ori_block_size < 1 || a->ori_bt_stride < 1 || a->ori_num_blocks < 1)
    return sas::set_error(SAS_EINVAL, "bad ori cache geometry");
  if (a->scenario >= SAS_CFA && (a->cmp_block_size < 1 || a->cmp_bt_stride < 1 || a->cmp_num_blocks < 1))
    return sas::set_error(SAS_EINVAL, "bad cmp cache geometry");
  if ((double)a->ori_num_blocks * a->ori_block_size > 2147483000.0 ||
      (double)a->cmp_num_blocks * std::max<int64_t>(a->cmp_block_size, 1) > 2147483000.0)
    return sas::set_error(SAS_EINVAL, "cache has more than 2^31 rows");
  const bool fp8 = a->kv_dtype == SAS_DT_FP8_E4M3_ROW656;
  if (fp8 && (a->q_dtype != SAS_DT_BF16 || a->D != 576))
    return sas::set_error(SAS_EINVAL, "fp8 cache rows need bf16 q and D=576");
  if (!fp8 && a->kv_dtype != a->q_dtype) return sas::set_error(SAS_EINVAL, "kv dtype must match q dtype");
  if (a->q_dtype != SAS_DT_BF16 && a->q_dtype != SAS_DT_FP16) return sas::set_error(SAS_EINVAL, "q dtype");
  if (pl.nsplit > 1 && (!a->workspace || a->workspace_bytes < pl.ws))
    return sas::set_error(SAS_ENOWS, "workspace of %zu bytes required", pl.ws);

  FwdParams fp;
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
  fp.out = (uint8_t*)a->out;
  fp.lse = a->lse;
  fp.part_o = pl.nsplit > 1 ? (float*)a->workspace : nullptr;
  fp.part_ml = pl.nsplit > 1 ? (float*)a->workspace + (size_t)a->T * pl.nsplit * a->H * kDV : nullptr;
  fp.T = (int)a->T; fp.B = (int)a->B; fp.H = (int)a->H;
  fp.ori_bs = (int)a->ori_block_size; fp.ori_bt_stride = (int)a->ori_bt_stride;
  fp.ori_nblocks = (int)a->ori_num_blocks;
  fp.cmp_bs = (int)std::max<int64_t>(a->cmp_block_size, 1);
  fp.cmp_bt_stride = (int)std::max<int64_t>(a->cmp_bt_stride, 1);
  fp.cmp_nblocks = (int)a->cmp_num_blocks;
  fp.K = (int)a->K; fp.scenario = a->scenario;
  fp.cmp_ratio = std::max(1, a->cmp_ratio); fp.win_left = a->win_left;
  fp.scale_log2 = a->softmax_scale * kLog2e;
  fp.nsplit = pl.nsplit; fp.slots_per_split = pl.sps; fp.nhg = pl.nhg;
  fp.items = (int)(a->T * pl.nhg * pl.nsplit);
  fp.per_xcd = (fp.items + kXcds - 1) / kXcds;
  const int nblocks = fp.per_xcd * kXcds;
  hipStream_t st = (hipStream_t)stream;

  if (fp8) rc = dispatch_hw<576, __bf16, 1>(pl.hw, fp, nblocks, st);
  else if (a->q_dtype == SAS_DT_BF16)
    rc = a->D == 576 ? dispatch_hw<576, __bf16, 0>(pl.hw, fp, nblocks, st)
                     : dispatch_hw<512, __bf16, 0>(pl.hw, fp, nblocks, st);
  else
    rc = a->D == 576 ? dispatch_hw<576, _Float16, 0>(pl.hw, fp, nblocks, st)
                     : dispatch_hw<512, _Float16, 0>(pl.hw, fp, nblocks, st);
  if (rc) return rc;
  if (pl.nsplit > 1 && !(a->flags & SAS_FWD_NO_COMBINE)) {
    SasCombineArgs ca;
    ca.part_o = fp.part_o; ca.part_ml = fp.part_ml; ca.sinks = a->sinks;
    ca.out = a->out; ca.lse = a->lse;
    ca.T = a->T; ca.S = pl.nsplit; ca.H = a->H; ca.DV = kDV;
    ca.out_dtype = a->q_dtype;
    return combine_impl(&ca, st);
  }
  return SAS_OK;
}

extern "C" int sas_combine_v1(const SasCombineArgs* a, void* stream) {
  sas::clear_error();
  return combine_impl(a, (hipStream_t)stream);
}
