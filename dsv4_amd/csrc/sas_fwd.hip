// sparse_attn_sharedkv forward for MI355X (gfx950 / CDNA4).
//
// One workgroup per (query token, head group, KV split). The token's key
// slots are the sliding window (win_left + 1 slots) followed by the top-k
// compressed entries (or the dense compressed prefix for CFA). A workgroup
//   1. resolves its slot range to physical cache rows through the block
//      tables, dropping masked slots (window band, idx < 0, idx >= causal
//      threshold) and compacting the rest in order into LDS;
//   2. streams the valid rows in tiles of 32 from HBM into LDS with 16-byte
//      loads (next tile prefetched into registers while the current one is
//      computed), storing each tile twice: row-major K for QK^T and a
//      transposed V^T (first 512 channels) for PV;
//   3. per wave (16 query heads; the KV row is shared by all heads):
//        S^T[32 keys x 16 heads] = K_tile . Q^T      (16x16x32 MFMA, Q in VGPRs)
//        sink-seeded online softmax in the log2 domain, P rounded to q dtype
//        O^T[512 x 16 heads]    += V^T_tile . P^T    (16x16x32 MFMA)
//      Computing the transposed products keeps P in exactly the register
//      layout the PV MFMA consumes, so P never passes through LDS;
//   4. writes out = O / l and lse = m + ln l, or, with several splits,
//      unnormalised partials (O, m, l) for the LSE combine kernel.
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

namespace {

constexpr int kTile = 32;         // keys per tile
constexpr int kDV = 512;          // output / V channels
constexpr int kMaxSlots = 1280;   // slot range one workgroup may own
constexpr int kXcds = 8;          // MI355X: 8 XCDs, workgroups dealt round-robin
constexpr int kRow656 = 656;      // fp8 cache row bytes
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

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

// Position of key r (0..31) inside a V^T row: lane group g of the S^T MFMA
// output holds keys {4g..4g+3} and {16+4g..16+4g+3}; they become the 8
// consecutive k of that lane's PV operand, so V^T stores them adjacently.
__device__ __forceinline__ int vt_pos(int r) {
  return r < 16 ? ((r >> 2) << 3) + (r & 3) : (((r - 16) >> 2) << 3) + 4 + (r & 3);
}

// ---------------------------------------------------------------------------
// forward kernel
// ---------------------------------------------------------------------------

// KVF: 0 = cache rows in the query dtype (D elements), 1 = 656-byte fp8 rows.
template <int NW, int D, typename QT, int KVF>
struct Cfg {
  // Always 4 waves: all of them gather; the first NW (16 heads each) compute.
  static constexpr int NT = 256;
  static constexpr int KS = D / 32;                 // k-steps of the QK^T MFMA
  static constexpr int LDK = D + 8;                 // K tile row stride (elements)
  static constexpr int LDV = kTile + 8;             // V^T row stride (elements)
  // 16-byte work chunks per row: bf16/fp16 rows -> D/8; fp8 rows -> 32 latent
  // chunks (16 values each) + 8 rope chunks.
  static constexpr int CPR = KVF ? 40 : D / 8;
  static constexpr int CPT = (kTile * CPR + NT - 1) / NT;  // chunks per thread per tile
  static constexpr int ROWB = KVF ? kRow656 : D * 2;
  static constexpr size_t LDS_K = (size_t)kTile * LDK * 2;
  static constexpr size_t LDS_V = (size_t)kDV * LDV * 2;
  static constexpr size_t LDS = LDS_K + LDS_V + sizeof(int) * (kMaxSlots + 2 * NW + 4);
};

template <int NW, int D, typename QT, int KVF>
__global__ void __launch_bounds__(256)
sas_fwd_kernel(const FwdParams p) {
  using C = Cfg<NW, D, QT, KVF>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t* Ks = reinterpret_cast<uint16_t*>(smem);
  uint16_t* Vt = reinterpret_cast<uint16_t*>(smem + C::LDS_K);
  int* s_rows = reinterpret_cast<int*>(smem + C::LDS_K + C::LDS_V);
  int* s_cnt = s_rows + kMaxSlots;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c16 = lane & 15, g = lane >> 4;
  const bool computes = wave < NW;

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

  // ---- 1. resolve + compact slot range [s0, s1) -------------------------
  // Stored ids: raw rows as id >= 0, compressed rows as -(id + 2).
  int nvalid = 0;
  for (int c0 = s0; c0 < s1; c0 += C::NT) {
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
        const int idx = p.scenario == SAS_SCFA ? p.cmp_idx[(size_t)t * p.K + k] : k;
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
    if (lane == 0) s_cnt[wave] = __popcll(mask);
    __syncthreads();
    int wpre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < C::NT / 64; ++w) {
      const int cw = s_cnt[w];
      wpre += w < wave ? cw : 0;
      tot += cw;
    }
    if (v) s_rows[nvalid + wpre + before] = rid;
    nvalid += tot;
    __syncthreads();
  }
  const int ntiles = (nvalid + kTile - 1) / kTile;

  // ---- Q^T operand in registers: head hq, channels ks*32 + 8g .. +8 ------
  const int hq = hg * (16 * NW) + (computes ? wave : 0) * 16 + c16;
  uint4 qf[C::KS];
  if (computes) {
    const uint4* qp = reinterpret_cast<const uint4*>(p.q + ((size_t)t * p.H + hq) * D * 2);
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) qf[ks] = qp[ks * 4 + g];
  }

  // online-softmax state for head hq (replicated over the 4 lane groups)
  float m_run, l_run;
  if (p.nsplit == 1) { m_run = p.sinks[hq] * kLog2e; l_run = 1.f; }
  else { m_run = -INFINITY; l_run = 0.f; }
  f32x4 acc[kDV / 16];
#pragma unroll
  for (int i = 0; i < kDV / 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- 2./3. tile loop ----------------------------------------------------
  uint4 buf[C::CPT];
  float bsc[KVF ? C::CPT : 1];

  auto row_ptr = [&](int id) -> const uint8_t* {
    return id >= 0 ? p.ori_kv + (size_t)id * C::ROWB : p.cmp_kv + (size_t)(-id - 2) * C::ROWB;
  };
  auto prefetch = [&](int it) {
    const int base = it * kTile;
#pragma unroll
    for (int k = 0; k < C::CPT; ++k) {
      const int e = tid + k * C::NT;
      const int r = e / C::CPR, c = e % C::CPR;
      buf[k] = make_uint4(0, 0, 0, 0);
      if constexpr (KVF) bsc[k] = 0.f;
      if (e < kTile * C::CPR && base + r < nvalid) {
        const uint8_t* rp = row_ptr(s_rows[base + r]);
        if constexpr (!KVF) {
          buf[k] = *reinterpret_cast<const uint4*>(rp + c * 16);
        } else {
          if (c < 32) {
            buf[k] = *reinterpret_cast<const uint4*>(rp + c * 16);
            bsc[k] = *reinterpret_cast<const float*>(rp + 512 + 4 * (c >> 3));
          } else {
            buf[k] = *reinterpret_cast<const uint4*>(rp + 528 + (c - 32) * 16);
          }
        }
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int k = 0; k < C::CPT; ++k) {
      const int e = tid + k * C::NT;
      if (e >= kTile * C::CPR) continue;
      const int r = e / C::CPR, c = e % C::CPR;
      const int vp = vt_pos(r);
      if constexpr (!KVF) {
        *reinterpret_cast<uint4*>(Ks + r * C::LDK + c * 8) = buf[k];
        if (c * 8 < kDV) {
          const uint32_t w[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            Vt[(c * 8 + 2 * i) * C::LDV + vp] = (uint16_t)(w[i] & 0xffffu);
            Vt[(c * 8 + 2 * i + 1) * C::LDV + vp] = (uint16_t)(w[i] >> 16);
          }
        }
      } else if (c < 32) {  // KVF: 16 e4m3 latent values -> bf16 (value * group scale)
        const uint32_t w[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
        uint32_t o[8];
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const uint32_t lo8 = (w[i >> 2] >> ((i & 3) * 8)) & 0xffu;
          const uint32_t hi8 = (w[i >> 2] >> (((i + 1) & 3) * 8)) & 0xffu;
          const uint32_t a = f32_to_bf16_bits(e4m3_to_f32(lo8) * bsc[k]);
          const uint32_t bb = f32_to_bf16_bits(e4m3_to_f32(hi8) * bsc[k]);
          o[i >> 1] = a | (bb << 16);
          Vt[(c * 16 + i) * C::LDV + vp] = (uint16_t)a;
          Vt[(c * 16 + i + 1) * C::LDV + vp] = (uint16_t)bb;
        }
        *reinterpret_cast<uint4*>(Ks + r * C::LDK + c * 16) = make_uint4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<uint4*>(Ks + r * C::LDK + c * 16 + 8) = make_uint4(o[4], o[5], o[6], o[7]);
      } else {
        *reinterpret_cast<uint4*>(Ks + r * C::LDK + 512 + (c - 32) * 8) = buf[k];
      }
    }
  };

  if (ntiles > 0) prefetch(0);
  for (int it = 0; it < ntiles; ++it) {
    __syncthreads();  // previous tile fully consumed
    store_tile();
    __syncthreads();
    if (it + 1 < ntiles) prefetch(it + 1);
    if (!computes) continue;
    const int nk = min(kTile, nvalid - it * kTile);

    // S^T = K_tile . Q^T : two 16-key M tiles
    f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const uint4 a = *reinterpret_cast<const uint4*>(Ks + (mt * 16 + c16) * C::LDK + ks * 32 + g * 8);
        sacc[mt] = mfma16<QT>(a, qf[ks], sacc[mt]);
      }
    }
    // online softmax (log2 domain) for head hq over this tile's keys
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
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = exp2f(m_run - m_new);
    float lsum = 0.f;
    uint32_t pk[4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      float pv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pv[j] = exp2f(sv[mt][j] - m_new);
        lsum += pv[j];
      }
      pk[mt * 2 + 0] = to_bits<QT>(pv[0]) | (to_bits<QT>(pv[1]) << 16);
      pk[mt * 2 + 1] = to_bits<QT>(pv[2]) | (to_bits<QT>(pv[3]) << 16);
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    l_run = l_run * alpha + lsum;
    m_run = m_new;
    const uint4 pfrag = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    // O^T = alpha * O^T + V^T_tile . P^T
#pragma unroll
    for (int mt = 0; mt < kDV / 16; ++mt) {
      const uint4 a = *reinterpret_cast<const uint4*>(Vt + (mt * 16 + c16) * C::LDV + g * 8);
      acc[mt] *= alpha;
      acc[mt] = mfma16<QT>(a, pfrag, acc[mt]);
    }
  }

  // ---- 4. epilogue ----------------------------------------------------------
  if (!computes) return;
  if (p.nsplit == 1) {
    const float inv = padded ? 0.f : 1.f / l_run;
    uint16_t* op = reinterpret_cast<uint16_t*>(p.out) + ((size_t)t * p.H + hq) * kDV;
#pragma unroll
    for (int mt = 0; mt < kDV / 16; ++mt) {
      const uint32_t w0 = to_bits<QT>(acc[mt][0] * inv) | (to_bits<QT>(acc[mt][1] * inv) << 16);
      const uint32_t w1 = to_bits<QT>(acc[mt][2] * inv) | (to_bits<QT>(acc[mt][3] * inv) << 16);
      *reinterpret_cast<uint2*>(op + mt * 16 + g * 4) = make_uint2(w0, w1);
    }
    if (g == 0) p.lse[(size_t)t * p.H + hq] = padded ? 0.f : m_run * kLn2 + logf(l_run);
  } else {
    const size_t row = ((size_t)t * p.nsplit + sp) * p.H + hq;
    float* po = p.part_o + row * kDV;
#pragma unroll
    for (int mt = 0; mt < kDV / 16; ++mt)
      *reinterpret_cast<float4*>(po + mt * 16 + g * 4) =
          make_float4(acc[mt][0], acc[mt][1], acc[mt][2], acc[mt][3]);
    if (g == 0) {
      p.part_ml[row * 2 + 0] = m_run;
      p.part_ml[row * 2 + 1] = padded ? -1.f : l_run;  // l < 0 marks a padded token
    }
  }
}

// ---------------------------------------------------------------------------
// split-KV combine
// ---------------------------------------------------------------------------

constexpr int kCombineThreads = 256;
constexpr int kMaxCombineSplits = 64;

template <typename QT>
__global__ void __launch_bounds__(kCombineThreads)
sas_combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                   const float* __restrict__ sinks, uint8_t* __restrict__ out,
                   float* __restrict__ lse, int S, int H, int hpb) {
  // one workgroup per (token, block of hpb heads)
  extern __shared__ float cw[];  // [hpb][S] weights, then [hpb] 1/L
  float* inv_l = cw + hpb * S;
  const int nhb = (H + hpb - 1) / hpb;
  const int t = blockIdx.x / nhb;
  const int h0 = (blockIdx.x % nhb) * hpb;
  const int nh = min(hpb, H - h0);
  for (int hh = threadIdx.x; hh < nh; hh += blockDim.x) {
    const int h = h0 + hh;
    const float sink2 = sinks[h] * kLog2e;
    float M = sink2;
    bool pad = false;
    for (int s = 0; s < S; ++s) {
      const float* ml = part_ml + (((size_t)t * S + s) * H + h) * 2;
      M = fmaxf(M, ml[0]);
      pad |= ml[1] < 0.f;
    }
    float L = exp2f(sink2 - M);
    for (int s = 0; s < S; ++s) {
      const float* ml = part_ml + (((size_t)t * S + s) * H + h) * 2;
      const float w = exp2f(ml[0] - M);
      cw[hh * S + s] = pad ? 0.f : w;
      L += pad ? 0.f : w * ml[1];
    }
    inv_l[hh] = pad ? 0.f : 1.f / L;
    lse[(size_t)t * H + h] = pad ? 0.f : M * kLn2 + logf(L);
  }
  __syncthreads();
  const int nq = kDV / 4;
  for (int e = threadIdx.x; e < nh * nq; e += blockDim.x) {
    const int hh = e / nq, c4 = e % nq, h = h0 + hh;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < S; ++s) {
      const float w = cw[hh * S + s];
      const float4 v = *reinterpret_cast<const float4*>(part_o + (((size_t)t * S + s) * H + h) * kDV + c4 * 4);
      o.x += w * v.x; o.y += w * v.y; o.z += w * v.z; o.w += w * v.w;
    }
    const float il = inv_l[hh];
    const uint32_t w0 = to_bits<QT>(o.x * il) | (to_bits<QT>(o.y * il) << 16);
    const uint32_t w1 = to_bits<QT>(o.z * il) | (to_bits<QT>(o.w * il) << 16);
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + ((size_t)t * H + h) * kDV + c4 * 4) =
        make_uint2(w0, w1);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

int heads_per_wg(int H) {
  for (int nw : {4, 2, 1})
    if (H % (16 * nw) == 0) return 16 * nw;
  return 0;
}

struct Plan {
  int nw, nhg, nslots, nsplit, sps;
  size_t ws;
};

int make_plan(const SasFwdArgs* a, Plan* pl) {
  if (!a) return sas::set_error(SAS_EINVAL, "null args");
  if (a->T < 0 || a->B < 1 || a->H < 1) return sas::set_error(SAS_EINVAL, "bad T/B/H");
  if (a->D != 512 && a->D != 576) return sas::set_error(SAS_EINVAL, "D must be 512 or 576 (got %lld)", (long long)a->D);
  if (a->DV != kDV) return sas::set_error(SAS_EINVAL, "DV must be 512 (got %lld)", (long long)a->DV);
  const int hpw = heads_per_wg((int)a->H);
  if (!hpw) return sas::set_error(SAS_EINVAL, "H must be a multiple of 16 (got %lld)", (long long)a->H);
  if (a->scenario < SAS_SWA || a->scenario > SAS_SCFA) return sas::set_error(SAS_EINVAL, "bad scenario");
  if (a->win_left < 0 || a->win_left > 8191) return sas::set_error(SAS_EINVAL, "win_left out of range");
  if (a->scenario >= SAS_CFA && (a->cmp_ratio < 1 || a->K < 0)) return sas::set_error(SAS_EINVAL, "bad cmp_ratio/K");
  pl->nw = hpw / 16;
  pl->nhg = (int)a->H / hpw;
  pl->nslots = a->win_left + 1 + (a->scenario >= SAS_CFA ? (int)a->K : 0);
  int ns = a->num_splits;
  const int per_tok = pl->nhg;
  if (ns <= 0) {
    // aim for ~2 workgroups per CU (256 CUs), at least 32 slots per split
    const long long target = 512;
    long long want = (target + (long long)a->T * per_tok - 1) / std::max<long long>(1, (long long)a->T * per_tok);
    const int max_by_tile = std::max(1, (pl->nslots + kTile - 1) / kTile);
    ns = (int)std::min<long long>(std::max<long long>(want, 1), max_by_tile);
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

template <int NW, int D, typename QT, int KVF>
int launch_fwd(const FwdParams& fp, int nblocks, hipStream_t st) {
  using C = Cfg<NW, D, QT, KVF>;
  auto kern = sas_fwd_kernel<NW, D, QT, KVF>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS) != hipSuccess)
      return sas::set_error(SAS_ELAUNCH, "hipFuncSetAttribute failed");
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(nblocks), dim3(C::NT), C::LDS, st, fp);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return sas::set_error(SAS_ELAUNCH, "sas_fwd launch: %s", hipGetErrorString(e));
  return SAS_OK;
}

template <int D, typename QT, int KVF>
int dispatch_nw(int nw, const FwdParams& fp, int nb, hipStream_t st) {
  switch (nw) {
    case 1: return launch_fwd<1, D, QT, KVF>(fp, nb, st);
    case 2: return launch_fwd<2, D, QT, KVF>(fp, nb, st);
    case 4: return launch_fwd<4, D, QT, KVF>(fp, nb, st);
  }
  return sas::set_error(SAS_EINVAL, "unsupported head grouping");
}

int combine_impl(const SasCombineArgs* a, hipStream_t st) {
  if (!a || !a->part_o || !a->part_ml || !a->sinks || !a->out || !a->lse)
    return sas::set_error(SAS_EINVAL, "combine: null pointer");
  if (a->DV != kDV || a->S < 1 || a->S > kMaxCombineSplits || a->H < 1 || a->T < 0)
    return sas::set_error(SAS_EINVAL, "combine: bad dims (S must be 1..64, DV 512)");
  if (a->T == 0) return SAS_OK;
  const int hpb = (int)std::min<int64_t>(a->H, 16);
  const int nhb = (int)((a->H + hpb - 1) / hpb);
  const size_t sm = sizeof(float) * (size_t)hpb * (a->S + 1);
  const dim3 grid((unsigned)(a->T * nhb));
  if (a->out_dtype == SAS_DT_BF16)
    hipLaunchKernelGGL(sas_combine_kernel<__bf16>, grid, dim3(kCombineThreads), sm, st, a->part_o,
                       a->part_ml, a->sinks, (uint8_t*)a->out, a->lse, (int)a->S, (int)a->H, hpb);
  else if (a->out_dtype == SAS_DT_FP16)
    hipLaunchKernelGGL(sas_combine_kernel<_Float16>, grid, dim3(kCombineThreads), sm, st, a->part_o,
                       a->part_ml, a->sinks, (uint8_t*)a->out, a->lse, (int)a->S, (int)a->H, hpb);
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

  if (fp8) rc = dispatch_nw<576, __bf16, 1>(pl.nw, fp, nblocks, st);
  else if (a->q_dtype == SAS_DT_BF16)
    rc = a->D == 576 ? dispatch_nw<576, __bf16, 0>(pl.nw, fp, nblocks, st)
                     : dispatch_nw<512, __bf16, 0>(pl.nw, fp, nblocks, st);
  else
    rc = a->D == 576 ? dispatch_nw<576, _Float16, 0>(pl.nw, fp, nblocks, st)
                     : dispatch_nw<512, _Float16, 0>(pl.nw, fp, nblocks, st);
  if (rc) return rc;
  if (pl.nsplit > 1) {
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
