// sparse_attn_sharedkv forward for MI355X (gfx950 / CDNA4).
//
// One workgroup per (query token, head group, KV split); NW = 4 or 8 waves.
// The token's key slots are the sliding window (win_left + 1 slots) followed
// by the top-k compressed entries (or the dense compressed prefix for CFA).
//
//  1. Resolve the workgroup's slot range to cache rows through the block
//     tables, drop masked slots (window band, idx < 0, idx >= causal
//     threshold) and compact the survivors' row addresses, in order, into LDS
//     (resolve() in sas_kern.h: two global round trips).
//  2. The waves form HW head-waves (16 query heads each) x CS channel halves x
//     KW key-groups. A key-group owns a contiguous share of the rows and
//     streams it in steps of TR rows (32, or 16 when every wave is its own
//     key-group) through a ring of LDS slots. Rows move HBM -> LDS with
//     global_load_lds_dwordx4 (no register staging), issued between the QK^T
//     MFMAs of the step before, into the slot that step freed; one workgroup
//     barrier per step. Tiles are row-major with an XOR swizzle of 16-byte
//     chunks that keeps both operand reads below bank-conflict free. fp8 rows
//     reach LDS the same way and stay fp8 there in the 32-head 8-wave plan
//     (each operand fragment converted to bf16 in registers); the other fp8
//     plans convert them through registers into bf16 slots. With one wave
//     per key-group the step loop has no workgroup barrier.
//  3. Per step and wave:  S^T[TR keys x 16 heads] = K . Q^T  (16x16x32 MFMA,
//     A from LDS, Q^T resident in VGPRs), sink-seeded online softmax in the
//     log2 domain, P rounded to the query dtype, then
//     O^T[channels x 16 heads] += V^T . P^T where the V^T operand comes
//     straight from the row-major tile with ds_read_b64_tr_b16 and P^T is
//     already in the register layout the MFMA wants (the S^T accumulator
//     layout). With 8 waves the two waves of a 16-head pair split O by
//     channels and share QK^T: by channels (each sums half of S; 32-head
//     groups) or by keys (each takes half of the step's keys and hands its
//     P to the other; 64-head groups).
//  4. Key-groups merge through LDS (max / sum rescale); the result is the
//     output + LSE, or with several KV splits an unnormalised partial (fp16
//     scaled by a power of two for bf16 outputs, fp32 for fp16) that the LSE
//     combine kernel merges with the sink.
//
// Semantics follow sparse_attn_sharedkv_tilelang/kernel.py:254-277 (work
// decode), :628-722 (window / compressed masks), :594-617 (sink seed),
// :877 (P cast), :1135-1145 (LSE), and golden.py:69-204.

#include "sas_kern.h"

#include <mutex>

#ifndef SAS_PFK
#define SAS_PFK 3   // K operand k-steps read ahead (32-row steps)
#endif
#ifndef SAS_KG2_SPLIT_MERGE
#define SAS_KG2_SPLIT_MERGE 1   // two key-groups each merge and store half the channels
#endif
#ifndef SAS_F8_PFK
#define SAS_F8_PFK 2   // fp8-resident: K fragments read ahead
#endif
#ifndef SAS_F8_PFV
#define SAS_F8_PFV 2   // fp8-resident: V^T fragments read ahead
#endif
#ifndef SAS_FP8_RESIDENT
#define SAS_FP8_RESIDENT 2   // fp8 mode of the 32-head 8-wave plan (1: rows converted into bf16 slots)
#endif
#ifndef SAS_PFV
#define SAS_PFV 4   // V^T operand channel tiles read ahead (32-row steps)
#endif
#ifndef SAS_KSPLIT
#define SAS_KSPLIT 1   // 64-head 8-wave plan: QK^T split across the wave pair by keys (1) or channels (0)
#endif


namespace sas {
namespace {

// ---------------------------------------------------------------------------
// forward kernel
// ---------------------------------------------------------------------------

// NW waves = HW head-waves x CS channel-halves x KW key-groups; D = q/k
// channels; QT = query dtype; KVF: 0 = cache rows in the query dtype,
// 1 / 2 = 656-byte fp8 rows (converted into bf16 slots / kept fp8 in LDS).
// With 8 waves (2 per SIMD, 256 registers each) a wave holds the O of its
// 16 heads for half of the 512 V channels (CS = 2), and the pair shares
// the QK^T work (by channels, or by keys with KSP).
template <int HW, int NW, int D, typename QT, int KVF>
struct Cfg {
  // KVF == 2: fp8 rows stay fp8 in LDS (LDS-DMA like bf16 rows) and each
  // operand fragment is converted to bf16 in registers just before its
  // MFMA; a 656-byte slot row lets two key-groups hold three 32-row slots
  // each. (KVF == 1: rows are converted once, through registers, into bf16
  // slots of 16 rows.)
  static constexpr bool F8R = KVF == 2;
  static constexpr int CS = NW == 8 ? 2 : 1;
  static constexpr int WK = HW * CS;                        // waves sharing a key-group's slots
  static constexpr int KW = NW / WK;
  static constexpr int NTL = kDV / 16 / CS;                 // 16-channel O tiles per wave
  // With two channel halves the QK^T k-steps are split as well (but see KSP
  // below): each wave of a pair sums S over its half of the D channels and
  // the pair adds the two halves through LDS (no QK^T work is duplicated).
  // The exchange buffer takes the ring rows above kRingRows.
  static constexpr bool QS = CS == 2;
  // Key-split QK^T (the 64-head, 8-wave, one-key-group plan with
  // SAS_KSPLIT): the two waves of a pair each compute S over all D channels
  // for one 16-key half of the step, run the softmax of their own keys and
  // exchange P (with their reference max) instead of S halves; O stays
  // split by channels.
  static constexpr bool KSP = SAS_KSPLIT && !KVF && NW == 8 && HW == 4;
  static constexpr int kRingRows = QS ? 96 : kLdsRows;
  // rows per step: 32, or 16 when 32-row slots would leave a ring shallower than 2
  static constexpr int TR = F8R ? 32 : kRingRows / (KW * 32) < 2 ? 16 : 32;
  static constexpr int PFK = F8R ? SAS_F8_PFK : TR == 16 ? 4 : SAS_PFK;   // K operand reads ahead
  static constexpr int PFV = F8R ? SAS_F8_PFV : TR == 16 ? 8 : SAS_PFV;   // V^T operand reads ahead
  // two QK^T accumulation chains (one suffices for the half k-range of a
  // channel-split wave, which shares its SIMD with a second wave)
  static constexpr bool CH2 = !QS || KSP;
  // Paired QK^T (channel-split waves, 32-row steps): the head-waves 2h and
  // 2h + 1 of a channel half share their K operand reads. Each of the two
  // computes S for both their head tiles over one 16-row half of the step
  // (two MFMAs per K fragment read, half the K reads of a wave per head),
  // and the S pieces meet in LDS in the layout P.V reads.
  static constexpr bool Q2 = QS && TR == 32 && HW % 2 == 0 && !KSP;
  static constexpr int NQ = Q2 ? 2 : 1;                     // head tiles in a wave's QK^T
  // 8 waves: the workgroup's query rows reach LDS by DMA (waves 4-7, which
  // do no slot resolution), one row per head from row kQRow0 on, in the
  // swizzled K-tile layout; every wave then reads its Q^T fragments there.
  // The rows lie outside the slots of the first ring fill.
  static constexpr bool QL = QS;
  static constexpr int kQRow0 = kLdsRows - 16 * HW;
  static constexpr int MT = TR / 16;                        // 16-key tiles per step
  static constexpr int NST = F8R ? 3 : kRingRows / (KW * TR) > 4 ? 4 : kRingRows / (KW * TR);   // ring depth per key-group
  // fp8-resident slot (chunks): latent [32 rows][32], rope [32][8], scales
  // [32][1], padded to whole DMA instructions (21 x 64)
  static constexpr int kF8Lat = 0, kF8Rope = 1024, kF8Scl = 1280, kF8Used = 1312, kF8Slot = 1344;
  static constexpr int SLOT = F8R ? kF8Slot : TR * kChunksMax;   // slot stride (chunks)
  // S exchange buffers and the query rows (chunk offsets in lds_ring): above
  // the ring; F8R: the exchange after the last slot, the query rows from the
  // last key-group's third slot (not in the first fill) on
  static constexpr int kXsChunk = F8R ? KW * NST * SLOT : kRingRows * kChunksMax;
  static constexpr int kQChunk = F8R ? (KW - 1) * NST * SLOT + (NST - 1) * SLOT : kQRow0 * kChunksMax;
  static constexpr int CH = D / 8;                          // 16-byte chunks per bf16 row
  static constexpr int KS = D / 32;                         // QK^T k-steps
  // k-steps of one wave. fp8 rows: S is summed per 128-channel scale group
  // (4 k-steps) and each group's sum scaled in fp32, so a channel split
  // follows the groups: half 0 takes groups 0-1 and the two rope k-steps,
  // half 1 groups 2-3 and two k-steps of zero Q (10 each).
  static constexpr int KSQ = QS && !KSP ? (F8R ? 9 : KVF ? 10 : KS / 2) : KS;
  static constexpr int NLG = QS ? 2 : 4;                    // fp8: scale groups per wave
  static constexpr int GT = WK * 64;                        // threads per key-group
  static constexpr int NI = F8R ? kF8Slot / 64 : TR * CH / 64;   // DMA instructions per step
  static constexpr int OPS = (NI + WK - 1) / WK;            // most DMA ops per wave per step
  static constexpr int ROWB = KVF ? kRow656 : D * 2;
  // fp8 register staging: 40 work chunks per row (32 latent x 16 values, 8 rope)
  static constexpr int FCPR = 40;
  static constexpr int FOPS = (TR * FCPR + GT - 1) / GT;
  static_assert(F8R || TR * CH % 64 == 0, "whole DMA instructions");
  static_assert(!KVF || (KS == 18 && CH == kChunksMax), "fp8 rows: 512 latent + 64 rope channels");
  static_assert(!F8R || (QS && Q2 && KW == 2 && NW == 8 && kF8Slot % 64 == 0 && TR == 32),
                "fp8-resident slots: the 8-wave, two-key-group, paired-QK^T plan");
  static_assert(!F8R || (kXsChunk + NW * 64 * MT <= kLdsRows * kChunksMax &&
                         kQChunk + 16 * HW * CH <= kLdsRows * kChunksMax),
                "fp8-resident ring, S exchange and query rows fit");
  static_assert(NST >= 2 && NST <= 4, "ring depth");
  static_assert((NST - 1) * OPS < 64, "vmcnt range");
  static_assert(F8R || KW * NST * SLOT <= kRingRows * kChunksMax, "ring fits");
  static_assert(F8R || !QS || (KS % 2 == 0 && NW * 64 * MT * 4 * 4 <= (kLdsRows - kRingRows) * kChunksMax * 16),
                "S exchange fits above the ring");
  static_assert(!KSP || kXsChunk + 2 * NW * 96 <= kLdsRows * kChunksMax, "key-split P exchange fits above the ring");
  // the last key-group's first fill (slots 0 .. NST - 2) ends at or before the query rows
  static_assert(!QL || (NW == 8 && (KW - 1) * NST * SLOT + (NST - 1) * SLOT <= kQChunk),
                "query rows clear of the first fill");
};

template <int HW, int NW, int D, typename QT, int KVF>
struct Fwd {
  using C = Cfg<HW, NW, D, QT, KVF>;
  const FwdParams& p;
  const int lane, c16, g, kw, hw, cs, jw, gt, nops;
  int rbeg;            // this key-group's first row in lds_rows
  int ring;           // chunk offset of this key-group's NST slots in lds_ring
  int nrows;           // rows this key-group owns
  int nsteps, nsteps_max;
  uint4 qf[C::NQ][C::KSQ];   // Q^T operand of the wave's QK^T head tiles
  float m_run, l_run;
  f32x4 acc[C::NTL];
  uint4 fbuf[KVF == 1 ? C::FOPS : 1];
  float fsc[KVF == 1 ? C::FOPS : 1];

  // wave = kw * WK + jw, jw = cs * HW + hw; wave jw of a key-group issues the
  // DMA instructions i = jw, jw + WK, ... of every step (nops of them)
  __device__ Fwd(const FwdParams& p_, int lane_, int wave)
      : p(p_), lane(lane_), c16(lane_ & 15), g(lane_ >> 4), kw(wave / C::WK), hw(wave % HW),
        cs((wave % C::WK) / HW), jw(wave % C::WK), gt((wave % C::WK) * 64 + lane_),
        nops((C::NI - wave % C::WK + C::WK - 1) / C::WK) {}

  __device__ __forceinline__ int slot(int j) const { return ring + j * C::SLOT; }
  // QK^T k-steps: this wave's first one, and the one its local k-step ks
  // computes (fp8 channel halves: local k-steps 8 and 9 are the rope k-steps
  // 16 and 17, with zero Q in half 1)
  __device__ __forceinline__ int kbase() const { return C::QS && !C::KSP ? (KVF ? cs * 8 : cs * C::KSQ) : 0; }
  // (fp8-resident: channel half cs takes latent groups 2 cs, 2 cs + 1 and
  // rope k-step 16 + cs, nine k-steps each)
  __device__ __forceinline__ int kglob(int ks) const {
    return (KVF && C::QS && ks >= 8) ? (C::F8R ? 16 + cs : ks + 8) : kbase() + ks;
  }

  // -- bf16 / fp16 rows: DMA one step into slot j ------------------------------
  // Lane `lane` of the wave's o-th instruction of a step moves row drow(o) of
  // the step, logical chunk pc ^ swz(row) (byte offset dcol(o)) to slot chunk
  // (o * WK + jw) * 64 + lane. The row addresses are read from LDS for all of
  // the wave's instructions first, so one LDS wait covers them (the DMA asm
  // is a memory barrier to the compiler). Rows past the end of the last step
  // repeat its last row: they are masked out of the softmax, and a real row
  // keeps P.V finite.
  __device__ __forceinline__ int drow(int o) const { return ((o * C::WK + jw) * 64 + lane) / C::CH; }
  __device__ __forceinline__ uint32_t dcol(int o) const {
    const int P = (o * C::WK + jw) * 64 + lane, r = P / C::CH;
    return (uint32_t)(((P - r * C::CH) ^ swz<C::CH>(r)) * 16);
  }
  // -- fp8-resident slots (F8R) ----------------------------------------------
  // Slot chunk position P of a step (0 .. kF8Slot): latent chunk (P & 31) ^
  // swz8l(row) of row P >> 5 below kF8Rope; rope chunk (q & 7) ^ swz8r(row) of
  // row q >> 3, q = P - kF8Rope, below kF8Scl; the scale chunk of row P -
  // kF8Scl below kF8Used; past it row 0, chunk 0 (padding, never read).
  // swz8l is a bijection of the 32 rows onto the 32 latent chunk columns
  // (even for rows 0-15, odd for 16-31), so a 16-row K read (two chunks per
  // row) and the 32-row transposed V read (one chunk per row) each touch 32
  // distinct columns.
  static __device__ __forceinline__ int swz8l(int r) { return ((r << 1) | (r >> 4)) & 31; }
  static __device__ __forceinline__ int swz8r(int r) { return (r >> 1) & 7; }
  __device__ __forceinline__ int drow8(int o) const {
    const int P = (o * C::WK + jw) * 64 + lane;
    return P < C::kF8Rope ? P >> 5 : P < C::kF8Scl ? (P - C::kF8Rope) >> 3 : P < C::kF8Used ? P - C::kF8Scl : 0;
  }
  __device__ __forceinline__ uint32_t dcol8(int o) const {
    const int P = (o * C::WK + jw) * 64 + lane;
    if (P < C::kF8Rope) return (uint32_t)(((P & 31) ^ swz8l(P >> 5)) * 16);
    if (P < C::kF8Scl) {
      const int q = P - C::kF8Rope;
      return 528u + (uint32_t)(((q & 7) ^ swz8r(q >> 3)) * 16);
    }
    return P < C::kF8Used ? 512u : 0u;
  }
  struct Dma {
    uint64_t ra[C::OPS];   // row address of each of the wave's instructions
    uint32_t lds;          // LDS byte address of the slot
  };
  __device__ __forceinline__ void prep(Dma& d, int j, int step) const {
    const int rp = rbeg + step * C::TR;
    if constexpr (C::QL) {
      // lds_rows holds kRowPad copies of the last row past the compacted
      // ones, and a step's rows end within them: no clamp
      // the step's first entry as one scalar LDS address, so each lookup
      // is one add to the lane's constant offset
      const uint32_t rb = __builtin_amdgcn_readfirstlane(lds_addr_of(lds_rows + rp));
#pragma unroll
      for (int o = 0; o < C::OPS; ++o)
        d.ra[o] = *reinterpret_cast<const LDS_AS uint64_t*>((size_t)(rb + 8u * (uint32_t)(C::F8R ? drow8(o) : drow(o))));
    } else {
      const int last = rp + min(C::TR, nrows - step * C::TR) - 1;   // nk >= 1 for every issued step
#pragma unroll
      for (int o = 0; o < C::OPS; ++o) d.ra[o] = lds_rows[min(rp + drow(o), last)];
    }
    d.lds = lds_addr_of(&lds_ring[slot(j)]);
  }
  __device__ __forceinline__ void fire(const Dma& d, int o) const {
    if (C::NI % C::WK && o * C::WK + jw >= C::NI) return;   // wave-uniform
    dma16(reinterpret_cast<const void*>(d.ra[o] + (C::F8R ? dcol8(o) : dcol(o))),
          __builtin_amdgcn_readfirstlane(d.lds + (o * C::WK + jw) * 64 * 16));
  }
  __device__ __forceinline__ void issue(int j, int step) {
    Dma d;
    prep(d, j, step);
#pragma unroll
    for (int o = 0; o < C::OPS; ++o) fire(d, o);
  }

  // -- query rows via LDS (QL) -----------------------------------------------
  // Waves 4-7 DMA the workgroup's 16 HW query rows (head h of the group at
  // LDS row kQRow0 + h, chunk c at c ^ swz(h)); after the caller's wait and
  // barrier every wave reads its Q^T fragments like K-operand fragments.
  __device__ __forceinline__ void q_dma(const Tok& k, int wave) const {
    constexpr int NIQ = 16 * HW * C::CH / 64;   // DMA instructions
    static_assert(NIQ * 64 == 16 * HW * C::CH, "whole instructions");
    const uint8_t* qb = p.q + ((size_t)k.t * p.H + k.hg * 16 * HW) * D * 2;
    const uint32_t lb = lds_addr_of(&lds_ring[C::kQChunk]);
    for (int i = wave - 4; i < NIQ; i += 4) {   // wave-uniform
      const int P = i * 64 + lane, r = P / C::CH, pc = P - r * C::CH;
      dma16(qb + (size_t)r * D * 2 + (pc ^ swz<C::CH>(r)) * 16, __builtin_amdgcn_readfirstlane(lb + i * 64 * 16));
    }
  }
  __device__ __forceinline__ void q_from_lds() {
    constexpr int SG = kSwzGroup<C::CH>;
#pragma unroll
    for (int n = 0; n < C::NQ; ++n) {
      const int h = (C::Q2 ? (hw & ~1) + n : hw) * 16 + c16;   // head in the group
      const int hsw = swz<C::CH>(h);
      const uint4* qr = &lds_ring[C::kQChunk + h * C::CH];
#pragma unroll
      for (int ks = 0; ks < C::KSQ; ++ks) {
        const int L = 4 * kglob(ks) + g;
        qf[n][ks] = qr[(L & -SG) | ((L & (SG - 1)) ^ hsw)];
        if (KVF == 1 && C::QS && ks >= 8 && cs == 1) qf[n][ks] = make_uint4(0, 0, 0, 0);
      }
    }
  }

  // -- fp8 rows: global -> registers, dequantised into a slot on store -------
  // Every lane issues the same two loads whatever its chunk (latent or rope,
  // inside the step or not): a 16-byte load at a per-lane offset and the
  // scale of its latent group. (Loads into the same registers under
  // divergent latent / rope branches made the compiler wait for every load
  // in flight between the branches, s_waitcnt vmcnt(0), so a step's fetch
  // took several round trips.) Lanes past the step's rows repeat its last
  // row (masked out of the softmax; a real row keeps P.V finite), lanes past
  // the step's chunks load its first row and store nothing.
  __device__ __forceinline__ void fload(int step) {
    const int rp = rbeg + step * C::TR;
    const int nk = min(C::TR, nrows - step * C::TR);   // >= 1 for every loaded step
#pragma unroll
    for (int k = 0; k < C::FOPS; ++k) {
      const int e = gt + k * C::GT;
      const int r = e / C::FCPR, c = e - r * C::FCPR;
      const uint64_t src = lds_rows[rp + (e < C::TR * C::FCPR ? min(r, nk - 1) : 0)];
      fbuf[k] = gld16(src + (c < 32 ? c * 16 : 528 + (c - 32) * 16));
      fsc[k] = gldf(src + 512 + 4 * ((c & 31) >> 3));
    }
  }
  __device__ __forceinline__ void fstore(int j) {
    const int sl = slot(j);
#pragma unroll
    for (int k = 0; k < C::FOPS; ++k) {
      const int e = gt + k * C::GT;
      if (e >= C::TR * C::FCPR) continue;
      const int r = e / C::FCPR, c = e - r * C::FCPR;
      uint4* row = &lds_ring[sl + r * C::CH];
      const int sw = swz<C::CH>(r);
      if (c < 32) {
        // the e4m3 values unscaled (exact in bf16); the group's scale goes to
        // the scale table, applied to S and P in fp32 (qk, pv)
        const uint32_t w[4] = {fbuf[k].x, fbuf[k].y, fbuf[k].z, fbuf[k].w};
        uint32_t o[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) e4m3x4_to_bf16(w[i], o[2 * i], o[2 * i + 1]);
        row[(2 * c) ^ sw] = make_uint4(o[0], o[1], o[2], o[3]);
        row[(2 * c + 1) ^ sw] = make_uint4(o[4], o[5], o[6], o[7]);
        if ((c & 7) == 0) lds_fsc[c >> 3][sl / C::CH + r] = fsc[k];
      } else {
        row[(64 + c - 32) ^ sw] = fbuf[k];
      }
    }
  }

  // -- one step of attention (TR keys) for this wave's 16 heads --------------
  // qk: S^T of the step in slot sl as two accumulation chains (even / odd
  // k-steps). dma(o), o < OPS, issues the wave's o-th DMA instruction of a
  // later step; the calls are spread over the k-steps so the vector memory
  // pipe works while the MFMAs run.
  // mid(ks), with kMid set, puts VALU work of another step between the
  // k-steps (the MFMAs of this step overlap it).
  template <bool kMid = false, typename DmaFn, typename MidFn = void (*)(int)>
  __device__ __forceinline__ void qk(int sl, f32x4 (&sacc)[C::MT], f32x4 (&sodd)[C::MT], DmaFn&& dma,
                                     MidFn&& mid = [](int) {}) {
    constexpr int MT = C::MT;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) { sacc[mt] = f32x4{0.f, 0.f, 0.f, 0.f}; sodd[mt] = sacc[mt]; }
    // K operand: rows c16 and 16 + c16 share the swizzle; logical chunk
    // 4ks + g lies in XOR group ks / KPG at offset qo[ks % KPG], the group
    // base being an immediate offset. Reads run kPfK k-steps ahead of the
    // MFMAs that consume them.
    // This wave's k-steps are cs * KSQ + ks, ks < KSQ; logical chunk L sits
    // at (L & -SG) | ((L & (SG - 1)) ^ swz), and k-step ks + KPG one group
    // (SG chunks) after k-step ks.
    constexpr int SG = kSwzGroup<C::CH>, KPG = SG / 4;
    const int ksw = swz<C::CH>(c16);
    // Q2: one 16-row tile (rows 16 (hw & 1) + c16, same swizzle as c16), the
    // two head tiles of the pair as the two accumulators sacc[0..1]
    const uint4* qrow = &lds_ring[sl + ((C::Q2 ? (hw & 1) * 16 : 0) + c16) * C::CH];
    int qo[KPG];
#pragma unroll
    for (int j = 0; j < KPG; ++j) {
      const int L = 4 * (kbase() + j) + g;
      qo[j] = (L & -SG) | ((L & (SG - 1)) ^ ksw);
    }
    auto kfrag = [&](int ks, int mt) {
      return qrow[mt * 16 * C::CH + (ks / KPG) * SG + qo[ks % KPG] + (kglob(ks) - kbase() - ks) * 4];
    };
    // fp8 rows: S = sum over the wave's scale groups of scale (per row, fp32)
    // x that group's MFMA chain (unscaled e4m3 values, exact), plus the rope
    // k-steps, which accumulate straight into sacc. Two group chains
    // alternate so one is folded while the next runs. fs: the scales of the
    // lane's four rows 4g..4g+3 of each row tile.
    constexpr int NG8 = KVF ? C::NLG : 1, SRT = C::Q2 ? 1 : MT;
    f32x4 gacc[2][MT], fs[NG8][SRT];
    if constexpr (KVF) {
      const int rr = sl / C::CH + (C::Q2 ? (hw & 1) * 16 : 0) + 4 * g;
      const int g0 = C::QS ? 2 * cs : 0;
#pragma unroll
      for (int lg = 0; lg < NG8; ++lg)
#pragma unroll
        for (int t = 0; t < SRT; ++t) fs[lg][t] = *reinterpret_cast<const f32x4*>(&lds_fsc[g0 + lg][rr + t * 16]);
    }
    constexpr int kPfK = C::PFK;
    constexpr int RT = C::Q2 ? 1 : MT;   // K row tiles read per k-step
    // k-step order: fp8 rows interleave the k-steps of two scale groups
    // (0, 4, 1, 5, 2, 6, 3, 7, then the next pair), so consecutive MFMAs feed
    // the two group chains alternately; else k-step i is the i-th.
    auto kord = [](int i) {
      if (!KVF || i >= 4 * C::NLG) return i;
      const int j = i & 7;
      return (i & ~7) + (j & 1) * 4 + (j >> 1);
    };
    uint4 af[kPfK][RT];
#pragma unroll
    for (int i = 0; i < kPfK; ++i)
#pragma unroll
      for (int mt = 0; mt < RT; ++mt) af[i][mt] = kfrag(kord(i), mt);
    // even / odd k-steps accumulate separately: 2 MT independent MFMA chains
#pragma unroll
    for (int i = 0; i < C::KSQ; ++i) {
      const int ks = kord(i);
      uint4 a[RT];
#pragma unroll
      for (int mt = 0; mt < RT; ++mt) a[mt] = af[i % kPfK][mt];
      if (i + kPfK < C::KSQ) {
#pragma unroll
        for (int mt = 0; mt < RT; ++mt) af[i % kPfK][mt] = kfrag(kord(i + kPfK), mt);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 am = a[C::Q2 ? 0 : mt];
        const uint4 bq = qf[C::Q2 ? mt : 0][ks];
        if constexpr (KVF) {
          if (ks < 4 * C::NLG) {
            f32x4& ga = gacc[(ks / 4) & 1][mt];
            ga = mfma32k<QT>(am, bq, ks % 4 == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : ga);
          } else {
            sacc[mt] = mfma32k<QT>(am, bq, sacc[mt]);
          }
        } else if (C::CH2 && (ks & 1)) {
          sodd[mt] = mfma32k<QT>(am, bq, sodd[mt]);
        } else {
          sacc[mt] = mfma32k<QT>(am, bq, sacc[mt]);
        }
      }
      if constexpr (KVF) {
        // a pair of groups complete: fold both into S
        if (i < 4 * C::NLG && i % 8 == 7) {
          const int lg = i / 4 - 1;   // the pair's first group
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            sacc[mt] += fs[lg][C::Q2 ? 0 : mt] * gacc[0][mt] + fs[lg + 1][C::Q2 ? 0 : mt] * gacc[1][mt];
        }
      }
      if ((i & 1) && i / 2 < C::OPS) dma(i / 2);
      if constexpr (kMid) mid(i);
    }
    // schedule: the prefetch reads first, then per k-step MT MFMAs + RT reads
    // (+ a share of the other step's VALU work). Placed before the remaining
    // DMA issues: a wave-dependent guard there starts a new basic block, and
    // these groups order only the instructions of their own block. (fp8
    // rows: the compiler's own order around the scale reads and folds.)
    if constexpr (!KVF) __builtin_amdgcn_sched_group_barrier(0x100, RT * kPfK, 0);
#pragma unroll
    for (int ks = 0; ks < (KVF ? 0 : C::KSQ); ++ks) {
      __builtin_amdgcn_sched_group_barrier(0x008, MT, 0);
      if (ks + kPfK < C::KSQ) __builtin_amdgcn_sched_group_barrier(0x100, RT, 0);
      if constexpr (kMid) __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
#pragma unroll
    for (int o = C::KSQ / 2; o < C::OPS; ++o) dma(o);
  }

  // smax: mask, scale and sink-seeded online softmax of a finished S^T; P
  // rounded to the query dtype in the PV B-operand layout (pk), O and l
  // rescaled when the reference max moves.
  // smax_a: scaled, masked scores sv and the rescale; smax_b(e) for e in
  // [0, MT * 4 + 2): exp of score e, then the packing of P, then the sum.
  // kChains: S still in two accumulation chains (sacc + sodd).
  template <bool kChains = C::CH2>
  __device__ __forceinline__ void smax_a(f32x4 (&sacc)[C::MT], const f32x4 (&sodd)[C::MT], int step,
                                         float (&sv)[C::MT][4]) {
    constexpr int MT = C::MT;
    const int nk = min(C::TR, nrows - step * C::TR);
    if constexpr (kChains) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) sacc[mt] += sodd[mt];
    }
    float mloc = -INFINITY;
    if (nk >= C::TR) {   // a full step: no key to mask
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sv[mt][j] = sacc[mt][j] * p.scale_log2;
          mloc = fmaxf(mloc, sv[mt][j]);
        }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = mt * 16 + g * 4 + j;
          const float x = key < nk ? sacc[mt][j] * p.scale_log2 : -INFINITY;
          sv[mt][j] = x;
          mloc = fmaxf(mloc, x);
        }
    }
    mloc = rows_max(mloc);
    // Lazy rescale: m_run is a reference max, moved (and O, l rescaled) only
    // when some head's max rises more than kLazyLog2 above it, so P <= 2^8.
    // out = acc / l and lse = m_run + log2 l are exact for any reference.
    if (__ballot(mloc > m_run + kLazyLog2)) {
      const float m_new = fmaxf(m_run, mloc);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int i = 0; i < C::NTL; ++i) acc[i] *= alpha;
    }
  }
  // smax_a for the pipelined 8-wave loop, written without branches so it can
  // sit between the next step's QK^T MFMAs: every key goes through the mask,
  // and the reference max and l move by alpha = exp2(m_run - m_new) (1 when
  // no head rises past the lazy threshold). Returns whether O must be scaled
  // by alpha before the step's P.V (the caller does it after the MFMAs).
  // kFull: the caller knows the step is full (every step but the last), so
  // no key is masked.
  template <bool kFull = false>
  __device__ __forceinline__ bool smax_front(const f32x4 (&sacc)[C::MT], int step, float (&sv)[C::MT][4],
                                             float& alpha) {
    constexpr int MT = C::MT;
    const int nk = kFull ? C::TR : min(C::TR, nrows - step * C::TR);
    float mloc = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = mt * 16 + g * 4 + j;
        const float x = kFull || key < nk ? sacc[mt][j] * p.scale_log2 : -INFINITY;
        sv[mt][j] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = rows_max(mloc);
    const bool r = __ballot(mloc > m_run + kLazyLog2) != 0;
    const float m_new = r ? fmaxf(m_run, mloc) : m_run;
    alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
    m_run = m_new;
    return r;
  }
  static constexpr int kSmaxB = C::MT * 4 + 2;
  __device__ __forceinline__ void smax_b(int e, float (&sv)[C::MT][4], float& lsum, uint32_t (&pk)[2 * C::MT]) {
    constexpr int MT = C::MT;
    if (e < MT * 4) {
      float& x = sv[e / 4][e % 4];
      // v_exp_f32: results below 2^-126 flush to zero (against a row sum >= 1)
      x = __builtin_amdgcn_exp2f(x - m_run);
      lsum = e == 0 ? x : lsum + x;
    } else if (e == MT * 4) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        pk[mt * 2 + 0] = pack2<QT>(sv[mt][0], sv[mt][1]);
        pk[mt * 2 + 1] = pack2<QT>(sv[mt][2], sv[mt][3]);
      }
    } else {
      l_run += rows_sum(lsum);
    }
  }
  __device__ __forceinline__ void smax(f32x4 (&sacc)[C::MT], const f32x4 (&sodd)[C::MT], int step,
                                       uint32_t (&pk)[2 * C::MT]) {
    float sv[C::MT][4], lsum = 0.f;
    smax_a(sacc, sodd, step, sv);
#pragma unroll
    for (int e = 0; e < kSmaxB; ++e) smax_b(e, sv, lsum, pk);
  }

  // pv: O^T += V^T . P^T for the step in slot sl; dma(o) as in qk, spread
  // over the channel tiles.
  template <typename DmaFn>
  __device__ __forceinline__ void pv(int sl, const uint32_t (&pk)[2 * C::MT], DmaFn&& dma) {
    constexpr int MT = C::MT;
    // V^T operand by transposed reads: lanes of group g address rows
    // 4g + c16/4 (and +16), channels mt*16 + 4*(c16&3); each lane receives
    // 4 keys of channel mt*16 + c16. Reads run kPfV channel tiles ahead.
    // This wave's O tiles are channel tiles cs * NTL + mt, mt < NTL (their
    // chunks start cs * NTL * 2 chunks into the row).
    const int vr = 4 * g + (c16 >> 2);
    const int vsw = swz<C::CH>(vr);
    const int vb = (c16 & 3) >> 1;
    const char* vbase = reinterpret_cast<const char*>(&lds_ring[sl + vr * C::CH]) + (c16 & 1) * 8 +
                        cs * C::NTL * 32;
    // logical chunk 2mt + vb lies in XOR group mt / TPG at voff[mt % TPG]
    constexpr int TPG = kSwzGroup<C::CH> / 2;
    int voff[TPG];
#pragma unroll
    for (int q = 0; q < TPG; ++q) voff[q] = ((2 * q + vb) ^ vsw) * 16;
    constexpr int kPfV = C::PFV;
    // fp8 rows: V holds the unscaled e4m3 values, so channel tile mt of scale
    // group G takes the B operand P x scale[G] (P as rounded to the query
    // dtype, times the key's fp32 scale, rounded once more); the lane's keys
    // are rows 4g..4g+3 (+16) of the step, as in S^T.
    constexpr int NG8 = KVF ? C::NLG : 1, TPL = C::NTL / NG8;   // channel tiles per group
    uint32_t pks[NG8][2 * MT];
    if constexpr (KVF) {
      const int rr = sl / C::CH + 4 * g;
      const int g0 = C::QS ? 2 * cs : 0;
#pragma unroll
      for (int lg = 0; lg < NG8; ++lg)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x4 f = *reinterpret_cast<const f32x4*>(&lds_fsc[g0 + lg][rr + mt * 16]);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t w = pk[mt * 2 + h];
            pks[lg][mt * 2 + h] = pack2<QT>(__uint_as_float(w << 16) * f[2 * h],
                                            __uint_as_float(w & 0xffff0000u) * f[2 * h + 1]);
          }
        }
    }
    if constexpr (MT == 2) {
      auto vfrag = [&](int mt) {
        const char* a0 = vbase + (mt / TPG) * TPG * 32 + voff[mt % TPG];
        const i16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4*)(a0));
        const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4*)(a0 + 16 * C::CH * 16));
        const uint2 u0 = __builtin_bit_cast(uint2, v0), u1 = __builtin_bit_cast(uint2, v1);
        return make_uint4(u0.x, u0.y, u1.x, u1.y);
      };
      const uint4 pfrag = make_uint4(pk[0], pk[1], pk[2], pk[3]);
      uint4 vf[kPfV];
#pragma unroll
      for (int i = 0; i < kPfV; ++i) vf[i] = vfrag(i);
#pragma unroll
      for (int mt = 0; mt < C::NTL; ++mt) {
        const uint4 a = vf[mt % kPfV];
        if (mt + kPfV < C::NTL) vf[mt % kPfV] = vfrag(mt + kPfV);
        const int lg = mt / TPL;
        acc[mt] = mfma32k<QT>(a, KVF ? make_uint4(pks[lg][0], pks[lg][1], pks[lg][2], pks[lg][3]) : pfrag, acc[mt]);
        if (mt % 3 == 2 && mt / 3 < C::OPS) dma(mt / 3);
      }
#pragma unroll
      for (int o = C::NTL / 3; o < C::OPS; ++o) dma(o);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * kPfV, 1);
#pragma unroll
      for (int mt = 0; mt < C::NTL; ++mt) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        if (mt + kPfV < C::NTL) __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
      }
    } else {
      // 16 keys: one transposed read per 16-channel tile, 16x16x16 MFMA whose
      // B operand (keys 4g..4g+3 of head c16) is exactly this lane's P
      auto vfrag = [&](int mt) {
        const char* a0 = vbase + (mt / TPG) * TPG * 32 + voff[mt % TPG];
        return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4*)(a0)));
      };
      const uint2 pfrag = make_uint2(pk[0], pk[1]);
      constexpr int kPf = C::PFV;
      uint2 vf[kPf];
#pragma unroll
      for (int i = 0; i < kPf; ++i) vf[i] = vfrag(i);
#pragma unroll
      for (int mt = 0; mt < C::NTL; ++mt) {
        const uint2 a = vf[mt % kPf];
        if (mt + kPf < C::NTL) vf[mt % kPf] = vfrag(mt + kPf);
        const int lg = mt / TPL;
        acc[mt] = mfma16k<QT>(a, KVF ? make_uint2(pks[lg][0], pks[lg][1]) : pfrag, acc[mt]);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, kPf, 1);
#pragma unroll
      for (int mt = 0; mt < C::NTL; ++mt) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        if (mt + kPf < C::NTL) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
      }
#pragma unroll
      for (int o = 0; o < C::OPS; ++o) dma(o);
    }
  }


  // -- fp8-resident QK^T (F8R) -------------------------------------------------
  // Paired head tiles, as qk with Q2: this wave's 16-row half (hw & 1) of the
  // step against both head tiles of its pair, over its channel half's nine
  // k-steps (scale groups 2 cs and 2 cs + 1, then rope k-step 16 + cs). A
  // latent k-step's K fragment is 8 fp8 bytes of the lane's row
  // (ds_read_b64), read kPfK k-steps ahead and converted to bf16 (exact,
  // unscaled) just before its two MFMAs; each group's four-k-step chain is
  // folded into S with the rows' fp32 scale of that group, as in qk. The
  // rope fragment is bf16 already.
  template <typename DmaFn>
  __device__ __forceinline__ void qk8(int sl, f32x4 (&sacc)[C::MT], DmaFn&& dma) {
    static_assert(C::Q2 && C::MT == 2 && C::KSQ == 9 && C::NLG == 2, "fp8-resident QK^T layout");
    constexpr int MT = C::MT;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sacc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int r = (hw & 1) * 16 + c16;
    const uint32_t lat = lds_addr_of(&lds_ring[sl + C::kF8Lat + r * 32]) + 8u * (uint32_t)(g & 1);
    const uint32_t rop = lds_addr_of(&lds_ring[sl + C::kF8Rope + r * 8]);
    const int sw = swz8l(r), swr = swz8r(r);
    // scale of group 2 cs + lg of key row k: float 4 k + 2 cs + lg of the scale chunks
    const float* sc = reinterpret_cast<const float*>(&lds_ring[sl + C::kF8Scl]) + 2 * cs;
    auto kraw = [&](int ks) -> uint4 {
      typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
      if (ks < 8) {
        const int c = 2 * (cs * 8 + ks) + (g >> 1);   // latent chunk of channels 32 k + 8 g ..
        const u32x2 v = *reinterpret_cast<const LDS_AS u32x2*>((size_t)(lat + (uint32_t)((c ^ sw) * 16)));
        return make_uint4(v.x, v.y, 0u, 0u);
      }
      const int c = 4 * cs + g;                       // rope chunk of channels 512 + 32 cs + 8 g ..
      const u32x4 v = *reinterpret_cast<const LDS_AS u32x4*>((size_t)(rop + (uint32_t)((c ^ swr) * 16)));
      return make_uint4(v.x, v.y, v.z, v.w);
    };
    constexpr int kPfK = C::PFK;
    uint4 af[kPfK];
#pragma unroll
    for (int i = 0; i < kPfK; ++i) af[i] = kraw(i);
    f32x4 gacc[MT];
#pragma unroll
    for (int ks = 0; ks < C::KSQ; ++ks) {
      const uint4 raw = af[ks % kPfK];
      if (ks + kPfK < C::KSQ) af[ks % kPfK] = kraw(ks + kPfK);
      uint4 a = raw;
      if (ks < 8) {
        uint32_t o0, o1, o2, o3;
        e4m3x4_to_bf16(raw.x, o0, o1);
        e4m3x4_to_bf16(raw.y, o2, o3);
        a = make_uint4(o0, o1, o2, o3);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (ks < 8) gacc[mt] = mfma32k<QT>(a, qf[mt][ks], ks % 4 == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : gacc[mt]);
        else sacc[mt] = mfma32k<QT>(a, qf[mt][ks], sacc[mt]);
      }
      if (ks == 3 || ks == 7) {
        const int lg = ks / 4, k0 = (hw & 1) * 16 + 4 * g;
        const f32x4 f = {sc[4 * k0 + lg], sc[4 * (k0 + 1) + lg], sc[4 * (k0 + 2) + lg], sc[4 * (k0 + 3) + lg]};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) sacc[mt] += f * gacc[mt];
      }
      if ((ks & 1) && ks / 2 < C::OPS) dma(ks / 2);
    }
#pragma unroll
    for (int o = C::KSQ / 2; o < C::OPS; ++o) dma(o);
  }

  // -- fp8-resident P.V (F8R) --------------------------------------------------
  // O^T += V^T . P^T over the step's 32 keys, one 16x16x32 MFMA per 16-channel
  // tile of the wave's channel half. The lane's P holds keys kappa(g, s) =
  // 4 g + s (s < 4) and 16 + 4 g + s - 4 (s >= 4) of head c16; the V^T
  // fragment must hold the same keys of channel c16 of the tile. The 8-bit
  // transposed read gives lane j of each 16-lane group byte j % 8 of the
  // addresses of lanes 2 s + (j >= 8), s = 0 .. 7: so lane (g, c16) points
  // at key row kappa(g, c16 >> 1), bytes 8 (c16 & 1) .. of the tile's chunk,
  // and receives channel c16 of its group's eight keys in kappa order. The
  // fp8 values are converted at use; P is scaled per group as in pv.
  __device__ __forceinline__ void pv8(int sl, const uint32_t (&pk)[2 * C::MT]) {
    static_assert(C::MT == 2 && C::NLG == 2 && C::NTL == 16, "fp8-resident P.V layout");
    typedef int v2i __attribute__((ext_vector_type(2)));
    const int s = c16 >> 1;
    const int kr = s < 4 ? 4 * g + s : 12 + 4 * g + s;
    const uint32_t vrow = lds_addr_of(&lds_ring[sl + C::kF8Lat + kr * 32]) + 8u * (uint32_t)(c16 & 1);
    const int sw = swz8l(kr);
    // P x scale of group 2 cs + lg for the lane's keys (4 g + i, 16 + 4 g + i)
    uint32_t pks[2][4];
    {
      // scale of group 2 cs + lg of key row k: float 4 k + 2 cs + lg of the scale chunks
      const float* sc = reinterpret_cast<const float*>(&lds_ring[sl + C::kF8Scl]) + 2 * cs;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int lg = 0; lg < 2; ++lg)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int k0 = mt * 16 + 4 * g + 2 * h;
            const uint32_t w = pk[mt * 2 + h];
            pks[lg][mt * 2 + h] = pack2<QT>(__uint_as_float(w << 16) * sc[4 * k0 + lg],
                                            __uint_as_float(w & 0xffff0000u) * sc[4 * (k0 + 1) + lg]);
          }
    }
    auto vraw = [&](int mt) -> v2i {
      const int c = cs * 16 + mt;   // latent chunk of channels 16 c .. 16 c + 15
      return __builtin_amdgcn_ds_read_tr8_b64_v2i32((LDS_AS v2i*)(size_t)(vrow + (uint32_t)((c ^ sw) * 16)));
    };
    constexpr int kPfV = C::PFV;
    v2i vf[kPfV];
#pragma unroll
    for (int i = 0; i < kPfV; ++i) vf[i] = vraw(i);
#pragma unroll
    for (int mt = 0; mt < C::NTL; ++mt) {
      const v2i raw = vf[mt % kPfV];
      if (mt + kPfV < C::NTL) vf[mt % kPfV] = vraw(mt + kPfV);
      uint32_t o0, o1, o2, o3;
      e4m3x4_to_bf16((uint32_t)raw.x, o0, o1);
      e4m3x4_to_bf16((uint32_t)raw.y, o2, o3);
      const int lg = mt / 8;
      acc[mt] = mfma32k<QT>(make_uint4(o0, o1, o2, o3), make_uint4(pks[lg][0], pks[lg][1], pks[lg][2], pks[lg][3]),
                            acc[mt]);
    }
  }

  // One step. With QS the two halves of S meet in LDS (one barrier, taken by
  // every wave of the workgroup whether or not its key-group has the step).
  template <typename DmaFn>
  __device__ __forceinline__ void compute(int sl, int step, DmaFn&& dma) {
    f32x4 sacc[C::MT], sodd[C::MT];
    uint32_t pk[2 * C::MT];
    const bool live = C::KW == 1 || step < nsteps;   // one key-group: every step is live
    if constexpr (C::F8R) {
      if (live) qk8(sl, sacc, dma);
    } else {
      if (live) qk(sl, sacc, sodd, dma);
    }
    if constexpr (C::QS) {
      f32x4* xs = reinterpret_cast<f32x4*>(lds_ring + C::kXsChunk);
      const int wave = kw * C::WK + jw;
      const int other = wave ^ HW;   // same heads, other channel half
      // Q2 piece (head tile ht, row tile rt, channel half c) of this key-group
      auto piece = [&](int ht, int rt, int c) { return (((kw * HW + ht) * 2 + rt) * 2 + c) * 64 + lane; };
      if (live) {
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt) {
          if constexpr (C::CH2) sacc[mt] += sodd[mt];
          if constexpr (C::Q2) xs[piece((hw & ~1) + mt, hw & 1, cs)] = sacc[mt];
          else xs[(wave * C::MT + mt) * 64 + lane] = sacc[mt];
        }
      }
      lds_barrier();
      if (live) {
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt) {
          if constexpr (C::Q2) sacc[mt] = xs[piece(hw, mt, 0)] + xs[piece(hw, mt, 1)];
          else sacc[mt] += xs[(other * C::MT + mt) * 64 + lane];
        }
        float sv[C::MT][4], lsum = 0.f;
        smax_a<false>(sacc, sodd, step, sv);
#pragma unroll
        for (int e = 0; e < kSmaxB; ++e) smax_b(e, sv, lsum, pk);
        if constexpr (C::F8R) pv8(sl, pk);
        else pv(sl, pk, [](int) {});
      }
      return;
    }
    if (live) {
      smax(sacc, sodd, step, pk);
      pv(sl, pk, [](int) {});
    }
  }

  // Step sync. WK > 1: the key-group's waves share slots, so a workgroup
  // barrier; WK = 1: the wave reads only slots it filled itself, and its own
  // LDS-DMA writes are complete once vmcnt has drained past them.
  __device__ __forceinline__ void step_sync() {
    if constexpr (C::WK > 1) lds_barrier();
    else wait_lgkm0();
  }

  // -- the step loop of this key-group ----------------------------------------
  template <int J>
  __device__ __forceinline__ void step_j(int it0) {
    const int it = it0 + J;
    if (it >= nsteps_max) return;   // uniform over the workgroup (HW > 1) / wave
    if constexpr (KVF != 1) {
      // Steps up to it + NST - 2 have been issued. My DMA for step `it` done
      // (the later ones may still stream), then all waves: every wave has
      // finished step it - 1, so its slot (J + NST - 1) % NST takes step
      // it + NST - 1 while step it computes.
      const int after = it < nsteps ? min(C::NST - 2, nsteps - 1 - it) : 0;
      wait_steps(after);
      step_sync();
      if (it < nsteps || C::QS) {
        const bool more = it + C::NST - 1 < nsteps;
        Dma d;
        if (more) prep(d, (J + C::NST - 1) % C::NST, it + C::NST - 1);
        compute(slot(J), it, [&](int o) { if (more) fire(d, o); });
      }
    } else {
      // fp8: registers hold step it+1; slot J holds step it (with QS every
      // wave takes the S exchange barrier of every step)
      step_sync();
      if (it < nsteps || C::QS) compute(slot(J), it, [](int) {});
      if (it + 1 < nsteps) fstore((J + 1) % C::NST);
      if (it + 2 < nsteps) fload(it + 2);
    }
  }

  // -- software-pipelined step loop (one key-group, 4-slot ring) -------------
  // Iteration it runs QK^T of step it + 1 and the softmax of step it, which
  // are independent (the MFMAs of the one overlap the VALU work of the
  // other), then P.V of step it with the DMA of step it + 3 going into the
  // slot that step it - 1 freed. Steps up to it + 2 have been issued when
  // iteration it starts.
  static constexpr bool kPipe = !KVF && C::NST == 4 && C::KW == 1 && NW == 4;
  // My DMAs of all but the n newest steps (n <= NST - 2) have landed. A wave
  // issues OPS or OPS - 1 instructions per step (nops, wave-uniform), so the
  // vmcnt immediate is one of a few compile-time values.
  template <int M>
  __device__ __forceinline__ void wait_ops(int n) {
    static_assert(2 * M < 64, "vmcnt range");
    if (n <= 0) wait_vm<0>();
    else if (n == 1 || C::NST <= 3) wait_vm<M>();
    else wait_vm<2 * M>();
  }
  __device__ __forceinline__ void wait_steps(int n) {
    if constexpr (C::NI % C::WK) {
      if (nops == C::OPS) wait_ops<C::OPS>(n);
      else wait_ops<C::OPS - 1>(n);
    } else {
      wait_ops<C::OPS>(n);
    }
  }
  template <int J>
  __device__ __forceinline__ void pipe_j(int it0, f32x4 (&se)[C::MT], f32x4 (&so)[C::MT]) {
    const int it = it0 + J;
    if (it >= nsteps) return;   // uniform: one key-group
    constexpr int Jn = (J + 1) % 4, Jf = (J + 3) % 4;
    const bool nxt = it + 1 < nsteps;
    if (nxt) wait_steps(it + 2 < nsteps ? 1 : 0);
    step_sync();
    uint32_t pk[2 * C::MT];
    float sv[C::MT][4], lsum = 0.f;
    smax_a(se, so, it, sv);
    f32x4 ne[C::MT], no[C::MT];
    if (nxt) {
      qk<true>(slot(Jn), ne, no, [](int) {}, [&](int ks) {
        if (ks < kSmaxB) smax_b(ks, sv, lsum, pk);
      });
#pragma unroll
      for (int e = C::KSQ; e < kSmaxB; ++e) smax_b(e, sv, lsum, pk);
    } else {
#pragma unroll
      for (int e = 0; e < kSmaxB; ++e) smax_b(e, sv, lsum, pk);
    }
    const bool more = it + 3 < nsteps;
    Dma d;
    if (more) prep(d, Jf, it + 3);
    pv(slot(J), pk, [&](int o) { if (more) fire(d, o); });
    if (nxt) {
#pragma unroll
      for (int mt = 0; mt < C::MT; ++mt) { se[mt] = ne[mt]; so[mt] = no[mt]; }
    }
  }
  __device__ __forceinline__ void run_pipe() {
#pragma unroll
    for (int j = 0; j < 3; ++j)
      if (j < nsteps) issue(j, j);
    if (nsteps <= 0) return;
    wait_steps(min(2, nsteps - 1));
    step_sync();
    f32x4 se[C::MT], so[C::MT];
    qk(slot(0), se, so, [](int) {});
    for (int it0 = 0; it0 < nsteps; it0 += 4) {
      pipe_j<0>(it0, se, so);
      pipe_j<1>(it0, se, so);
      pipe_j<2>(it0, se, so);
      pipe_j<3>(it0, se, so);
    }
  }

  // -- exact-window schedule (4 waves, at most kLdsRows rows, one split) -----
  // Every key-group's rows fit its NST slots (KW x NST x TR = kLdsRows), so
  // the whole row set is gathered at once and stays resident. QK^T runs
  // twice over it: first for each head's maximum over all rows and the sink
  // (key-groups exchange theirs through LDS), then for P, which is thus
  // rounded against the final maximum of the tile, as golden rounds its
  // single window tile (golden.py:178-195) and as the reference kernel runs
  // a 128-row window as one chunk (kernel.py:83, 97-100, 1743). Used for the
  // window-only scenario, whose key set is that one tile.
  __device__ __forceinline__ void run_exact(int wave, float sink_log2) {
    static_assert(NW == 4 && C::KW * C::NST * C::TR == kLdsRows, "exact schedule: the ring holds every row");
    if constexpr (!KVF) {
#pragma unroll
      for (int j = 0; j < C::NST; ++j)
        if (j < nsteps) issue(j, j);
      wait_vm<0>();
    } else {
#pragma unroll
      for (int j = 0; j < C::NST; ++j)
        if (j < nsteps) { fload(j); fstore(j); }
    }
    lds_barrier();
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < C::NST; ++j) {
      if (j >= nsteps) break;   // uniform over the key-group's waves
      f32x4 sacc[C::MT], sodd[C::MT];
      qk(slot(j), sacc, sodd, [](int) {});
      const int nk = min(C::TR, nrows - j * C::TR);
#pragma unroll
      for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (mt * 16 + g * 4 + i < nk) mloc = fmaxf(mloc, (sacc[mt][i] + sodd[mt][i]) * p.scale_log2);
    }
    mloc = rows_max(mloc);
    if constexpr (C::KW > 1) {
      if (g == 0) lds_ml[wave][0][c16] = mloc;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < C::KW; ++j) mloc = fmaxf(mloc, lds_ml[j * C::WK + jw][0][c16]);
      __syncthreads();   // read before the epilogue reuses lds_ml
    }
    // every key-group rounds against M = max(sink, all rows); the sink's
    // (1 at its own maximum) term is counted once, by key-group 0. A split
    // of several (sink_log2 = -inf) leaves the sink to the merge.
    m_run = fmaxf(mloc, sink_log2);
    l_run = kw == 0 && sink_log2 > -INFINITY ? __builtin_amdgcn_exp2f(sink_log2 - m_run) : 0.f;
#pragma unroll
    for (int j = 0; j < C::NST; ++j) {
      if (j >= nsteps) break;
      f32x4 sacc[C::MT], sodd[C::MT];
      uint32_t pk[2 * C::MT];
      qk(slot(j), sacc, sodd, [](int) {});
      smax(sacc, sodd, j, pk);
      pv(slot(j), pk, [](int) {});
    }
  }

  // -- software-pipelined loop of the 8-wave channel-split kernel -----------
  // (64-head workgroups, one key-group, built with SAS_KSPLIT=0; the default
  // for this configuration is the key-split loop, run_pipe8k.) The two
  // waves of a 16-head pair each sum S over half of D and exchange their
  // halves through LDS. Iteration it, after one workgroup barrier, reads the
  // exchanged S of step it, then runs the QK^T MFMAs of step it + 1 with the
  // softmax of step it interleaved between them (independent work: the
  // matrix pipe and the VALU overlap), writes its S half of step it + 1 to
  // the other exchange buffer, and runs P.V of step it. Steps it + 1 and it
  // use two ring slots; the third, freed by P.V of step it - 1 before the
  // barrier, receives the DMA of step it + 2. One barrier per step instead of
  // two (step + exchange).
  static constexpr bool kPipe8 = !KVF && C::Q2 && C::KW == 1 && C::NST == 3 && NW == 8;
  __device__ __forceinline__ f32x4* xs_buf(int b) const {
    return reinterpret_cast<f32x4*>(lds_ring + C::kXsChunk) + b * (NW * C::MT * 64);
  }
  // Q2 piece (head tile ht, row tile rt, channel half c)
  __device__ __forceinline__ int piece(int ht, int rt, int c) const { return ((ht * 2 + rt) * 2 + c) * 64 + lane; }
  __device__ __forceinline__ void xs_write(int b, const f32x4 (&sacc)[C::MT]) const {
    f32x4* xs = xs_buf(b);
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) xs[piece((hw & ~1) + mt, hw & 1, cs)] = sacc[mt];
  }
  __device__ __forceinline__ void xs_read(int b, f32x4 (&sacc)[C::MT]) const {
    const f32x4* xs = xs_buf(b);
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) sacc[mt] = xs[piece(hw, mt, 0)] + xs[piece(hw, mt, 1)];
  }
  template <int J>
  __device__ __forceinline__ void pipe8_j(int it0) {
    const int it = it0 + J;
    if (it >= nsteps) return;   // uniform: one key-group
    constexpr int Jn = (J + 1) % 3, Jf = (J + 2) % 3;
    const bool nxt = it + 1 < nsteps;
    // my DMA of step it + 1 (the only one in flight) has landed; after the
    // barrier every wave's has, every S half of step it is written, and
    // every wave has finished P.V of step it - 1 (slot Jf is free)
    wait_vm<0>();
    lds_barrier();
    f32x4 sc[C::MT];
    xs_read(it & 1, sc);
    float sv[C::MT][4], lsum = 0.f, alpha = 1.f;
    uint32_t pk[2 * C::MT];
    bool resc;
    if (nxt) {
      // The DMA of step it + 2 goes out unconditionally: past the last step
      // it re-reads the last row into slot Jf, which no later step reads (the
      // last iteration waits for it), so the QK^T loop has no branch. The
      // softmax front of step it (S read back above, max, reference move)
      // runs between the first MFMAs. (Its exps and packing, which the
      // compiler places after the MFMAs, measured slower when forced between
      // them: the other wave on the SIMD overlaps them already.)
      Dma d;
      prep(d, Jf, it + 2);
      f32x4 sn[C::MT], so[C::MT];
      qk<true>(slot(Jn), sn, so, [&](int o) { fire(d, o); }, [&](int ks) {
        if (ks == 0) resc = smax_front<true>(sc, it, sv, alpha);   // step it < nsteps - 1: full
        else if (ks - 1 < kSmaxB) smax_b(ks - 1, sv, lsum, pk);
      });
#pragma unroll
      for (int e = C::KSQ - 1; e < kSmaxB; ++e) smax_b(e, sv, lsum, pk);
      xs_write((it + 1) & 1, sn);
    } else {
      // (an empty asm on the scores keeps the compiler from hoisting this
      // copy of the softmax above the branch)
#pragma unroll
      for (int mt = 0; mt < C::MT; ++mt) asm volatile("" : "+v"(sc[mt]));
      resc = smax_front(sc, it, sv, alpha);
#pragma unroll
      for (int e = 0; e < kSmaxB; ++e) smax_b(e, sv, lsum, pk);
    }
    if (resc) {
#pragma unroll
      for (int i = 0; i < C::NTL; ++i) acc[i] *= alpha;
    }
    pv(slot(J), pk, [](int) {});
  }

  template <typename QFn>
  __device__ __forceinline__ void run_pipe8(QFn&& qload) {
    if (nsteps <= 0) return;   // uniform over the workgroup
    issue(0, 0);
    if (nsteps > 1) issue(1, 1);
    qload();
    wait_steps(nsteps > 1 ? 1 : 0);   // my part of step 0
    lds_barrier();
    f32x4 s0[C::MT], so[C::MT];
    qk(slot(0), s0, so, [](int) {});
    xs_write(0, s0);
    for (int it0 = 0; it0 < nsteps; it0 += 3) {
      pipe8_j<0>(it0);
      pipe8_j<1>(it0);
      pipe8_j<2>(it0);
    }
  }

  // -- key-split 8-wave loop (KSP: 64-head workgroups, one key-group) -------
  // Wave (hw, cs) computes S^T for keys 16 cs .. 16 cs + 15 of a step against
  // head tile hw over all D channels (two chains, even / odd k-steps), the
  // softmax of those 16 keys, and P.V over all 32 keys for its channel half,
  // with the other 16 keys' P from its partner (same heads, other half)
  // through LDS. Iteration it, after one workgroup barrier: read the
  // partner's P of step it and its reference max, QK^T of step it + 1, join
  // the two references and round both halves' P to the query dtype, the
  // softmax of step it + 1, P.V of step it, and write P of step it + 1. The
  // ring and its DMA schedule are run_pipe8's; the last step's P.V follows
  // the loop. (This pair split replaces the channel-split loop's exchange of
  // S halves, 6 KB per wave and step, by 1.5 KB of P, and halves each
  // wave's softmax; each wave reads K for all D channels of its 16 keys.)
  //
  // The pair starts from one reference: the max over both halves of step 0
  // (exchanged once, before the loop), as the channel-split loop's first
  // step sets it. Later each wave runs the lazy rescale over its own keys
  // (its reference moves to its own max when one of its keys rises more
  // than 2^8 above the common one, r0); the pair then joins at the
  // exchange: if either moved, both take, head by head, the max of r0 and
  // both halves' maxima of the step, which is where the channel-split loop
  // moves the reference, and O, l and each P are scaled by 2^(its
  // reference - the joined one). P is exchanged in fp32 and rounded only
  // after the join, once, so every P equals exp2(s - reference) as in the
  // channel-split loop, up to fp32 rounding.
  static constexpr bool kPipe8K = C::KSP && C::KW == 1 && C::NST == 3;
  __device__ __forceinline__ int partner() const { return (1 - cs) * HW + hw; }
  // P in fp32 (this lane's keys 4g .. 4g + 3 of its key half, head c16),
  // the reference it was computed against and the half's max of the step
  __device__ __forceinline__ f32x4* kx_p(int b) const {
    return reinterpret_cast<f32x4*>(lds_ring + C::kXsChunk) + b * (NW * 96);
  }
  __device__ __forceinline__ void kx_write(int b, const f32x4& pf, float mloc) const {
    f32x4* xs = kx_p(b);
    xs[(cs * HW + hw) * 64 + lane] = pf;
    reinterpret_cast<float2*>(xs + NW * 64)[(cs * HW + hw) * 64 + lane] = make_float2(m_run, mloc);
  }
  __device__ __forceinline__ void kx_read(int b, f32x4& pp, float2& mp) const {
    const f32x4* xs = kx_p(b);
    pp = xs[partner() * 64 + lane];
    mp = reinterpret_cast<const float2*>(xs + NW * 64)[partner() * 64 + lane];
  }
  // 2^(a - b) for a <= b (0 for a = -inf)
  static __device__ __forceinline__ float ref_factor(float a, float b) {
    return a == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(a - b);
  }
  // the P.V operand of step it: own P (po, half max mo) and the partner's
  // (pp; its reference and half max in mp) on one reference, rounded to the
  // query dtype; r0 is the pair's reference before step it's softmax. O and
  // l follow the reference when it moves.
  __device__ __forceinline__ void kx_join(f32x4 pp, float2 mp, f32x4 po, float mo, float r0, uint32_t (&pk)[4]) {
    if (__ballot(m_run != r0 || mp.x != r0)) {   // rare: a lazy move in either half
      const float M = fmaxf(r0, fmaxf(mo, mp.y));
      const float a = m_run < M ? ref_factor(m_run, M) : 1.f;
      const float b = mp.x < M ? ref_factor(mp.x, M) : 1.f;
      // in place (as inline asm): scaled copies of acc made the compiler
      // copy all of acc on the path that does not scale it
#pragma unroll
      for (int i = 0; i < C::NTL; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(acc[i][j]) : "v"(a));
      l_run *= a;
      po *= a;
      pp *= b;
      m_run = M;
    }
    // key tile 0 is half 0's keys, tile 1 half 1's
    const f32x4 p0 = cs == 0 ? po : pp, p1 = cs == 0 ? pp : po;
    pk[0] = pack2<QT>(p0[0], p0[1]);
    pk[1] = pack2<QT>(p0[2], p0[3]);
    pk[2] = pack2<QT>(p1[0], p1[1]);
    pk[3] = pack2<QT>(p1[2], p1[3]);
  }
  template <typename DmaFn>
  __device__ __forceinline__ void qk_ks(int sl, f32x4& se, f32x4& so, DmaFn&& dma) {
    constexpr int SG = kSwzGroup<C::CH>, KPG = SG / 4, KS = C::KS;
    const int ksw = swz<C::CH>(c16);   // rows c16 and 16 + c16 share the swizzle
    const uint4* krow = &lds_ring[sl + (cs * 16 + c16) * C::CH];
    int qo[KPG];
#pragma unroll
    for (int j = 0; j < KPG; ++j) qo[j] = (4 * j + g) ^ ksw;
    auto kfrag = [&](int ks) { return krow[(ks / KPG) * SG + qo[ks % KPG]]; };
    se = f32x4{0.f, 0.f, 0.f, 0.f};
    so = se;
    constexpr int kPfK = C::PFK;
    uint4 af[kPfK];
#pragma unroll
    for (int i = 0; i < kPfK; ++i) af[i] = kfrag(i);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint4 a = af[ks % kPfK];
      if (ks + kPfK < KS) af[ks % kPfK] = kfrag(ks + kPfK);
      if (ks & 1) so = mfma32k<QT>(a, qf[0][ks], so);
      else se = mfma32k<QT>(a, qf[0][ks], se);
      if ((ks & 1) && ks / 2 < C::OPS) dma(ks / 2);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, kPfK, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (ks + kPfK < KS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int o = KS / 2; o < C::OPS; ++o) dma(o);
  }
  // softmax of this wave's 16 keys of a step (S^T = se + so): e = 0 the
  // mask, max and reference move (returns through resc / alpha whether O
  // must be scaled after the P.V in flight), e = 1..4 the exps (P in fp32,
  // pf), 5 the sum
  static constexpr int kKsB = 6;
  __device__ __forceinline__ void ks_smax(int e, const f32x4& se, const f32x4& so, int step, f32x4& pf,
                                          float& mloc, float& lsum, bool& resc, float& alpha) {
    if (e == 0) {
      const int nk = min(C::TR, nrows - step * C::TR) - cs * 16;   // my valid keys (may be <= 0)
      mloc = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x = g * 4 + j < nk ? (se[j] + so[j]) * p.scale_log2 : -INFINITY;
        pf[j] = x;
        mloc = fmaxf(mloc, x);
      }
      mloc = rows_max(mloc);
      resc = __ballot(mloc > m_run + kLazyLog2) != 0;
      const float m_new = resc ? fmaxf(m_run, mloc) : m_run;
      alpha = resc ? ref_factor(m_run, m_new) : 1.f;
      l_run *= alpha;
      m_run = m_new;
    } else if (e <= 4) {
      // (with m_run = -inf every key of this half so far is masked: P = 0)
      const float x = __builtin_amdgcn_exp2f(pf[e - 1] - fmaxf(m_run, -3.0e38f));
      pf[e - 1] = x;
      lsum = e == 1 ? x : lsum + x;
    } else {
      l_run += rows_sum(lsum);
    }
  }
  template <int J>
  __device__ __forceinline__ void pipe8k_j(int it0, f32x4& pown, float& mown, float& r0) {
    const int it = it0 + J;
    if (it >= nsteps - 1) return;   // uniform: one key-group; the last step follows the loop
    constexpr int Jn = (J + 1) % 3, Jf = (J + 2) % 3;
    // my DMA of step it + 1 has landed; after the barrier every wave's has,
    // every P of step it is written, and slot Jf is free (as in pipe8_j)
    wait_vm<0>();
    lds_barrier();
    f32x4 pp;
    float2 mp;
    kx_read(it & 1, pp, mp);
    // The DMA goes out unconditionally: in the loop's last iteration it
    // re-reads step nsteps (rows within the padded row list) into slot Jf,
    // which no step reads; the wait after the loop drains it.
    Dma d;
    prep(d, Jf, min(it + 2, nsteps));
    f32x4 se, so;
    qk_ks(slot(Jn), se, so, [&](int o) { fire(d, o); });
    uint32_t pk[4];
    kx_join(pp, mp, pown, mown, r0, pk);
    float lsum = 0.f, alpha = 1.f;
    bool resc = false;
    r0 = m_run;
#pragma unroll
    for (int e = 0; e < kKsB; ++e) ks_smax(e, se, so, it + 1, pown, mown, lsum, resc, alpha);
    pv(slot(J), pk, [](int) {});
    if (resc) {
#pragma unroll
      for (int i = 0; i < C::NTL; ++i) acc[i] *= alpha;
    }
    kx_write((it + 1) & 1, pown, mown);
  }
  template <typename QFn>
  __device__ __forceinline__ void run_pipe8k(QFn&& qload) {
    if (nsteps > 0) {   // uniform over the workgroup
      issue(0, 0);
      if (nsteps > 1) issue(1, 1);
      qload();
      wait_steps(nsteps > 1 ? 1 : 0);   // my part of step 0
      lds_barrier();
      f32x4 se, so;
      qk_ks(slot(0), se, so, [](int) {});
      {
        // the pair's common first reference: the lazy move over both halves
        // of step 0 (the softmax below then finds no key above it)
        const int nk = min(C::TR, nrows) - cs * 16;
        float mloc = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (g * 4 + j < nk) mloc = fmaxf(mloc, (se[j] + so[j]) * p.scale_log2);
        mloc = rows_max(mloc);
        if (g == 0) lds_ml[cs * HW + hw][0][c16] = mloc;
        lds_barrier();
        mloc = fmaxf(mloc, lds_ml[partner()][0][c16]);
        if (__ballot(mloc > m_run + kLazyLog2)) {
          const float m_new = fmaxf(m_run, mloc);
          l_run *= ref_factor(m_run, m_new);
          m_run = m_new;
        }
      }
      f32x4 pown;
      float mown, r0 = m_run;
      {
        float lsum = 0.f, alpha = 1.f;
        bool resc = false;
#pragma unroll
        for (int e = 0; e < kKsB; ++e) ks_smax(e, se, so, 0, pown, mown, lsum, resc, alpha);
        // (O is still zero: nothing to rescale)
      }
      kx_write(0, pown, mown);
      for (int it0 = 0; it0 < nsteps - 1; it0 += 3) {
        pipe8k_j<0>(it0, pown, mown, r0);
        pipe8k_j<1>(it0, pown, mown, r0);
        pipe8k_j<2>(it0, pown, mown, r0);
      }
      // the last step: its P exchange and P.V only (the wait also drains
      // the loop's re-read of step nsteps before the ring is reused)
      const int it = nsteps - 1;
      wait_vm<0>();
      lds_barrier();
      f32x4 pp;
      float2 mp;
      kx_read(it & 1, pp, mp);
      uint32_t pk[4];
      kx_join(pp, mp, pown, mown, r0, pk);
      pv(slot(it % 3), pk, [](int) {});
    }
    // the pair's references agree here (joined at the last step); l is the
    // sum of both halves' sums
    if (g == 0) lds_ml[cs * HW + hw][1][c16] = l_run;
    lds_barrier();
    l_run += lds_ml[partner()][1][c16];
  }

  // qload(): the wave's Q^T fragments from the LDS query rows (8-wave
  // kernels), run after the first steps' row DMA is issued (the rows lie
  // outside its slots), so the query reads overlap the rows' round trip
  // instead of delaying its issue
  template <typename QFn>
  __device__ __forceinline__ void run(QFn&& qload) {
    if constexpr (kPipe) {
      run_pipe();
      return;
    }
    if constexpr (kPipe8) {
      run_pipe8(qload);
      return;
    }
    if constexpr (kPipe8K) {
      run_pipe8k(qload);
      return;
    }
    if constexpr (KVF != 1) {
#pragma unroll
      for (int j = 0; j < C::NST - 1; ++j)
        if (j < nsteps) issue(j, j);
    } else {
      if (nsteps > 0) { fload(0); fstore(0); }
      if (nsteps > 1) fload(1);
    }
    qload();
    for (int it0 = 0; it0 < nsteps_max; it0 += C::NST) {
      step_j<0>(it0);
      step_j<1>(it0);
      if constexpr (C::NST > 2) step_j<2>(it0);
      if constexpr (C::NST > 3) step_j<3>(it0);
    }
  }
};

// ---------------------------------------------------------------------------
// shared epilogue
// ---------------------------------------------------------------------------

constexpr int kObufStride = kDV + 4;   // floats per staged head row (bank spread)
constexpr int kObufChunks = 16 * kObufStride / 4;   // one wave's 16 staged head rows
static_assert(kMaxWaves / 2 * kObufChunks <= kLdsRows * kChunksMax, "epilogue staging fits");

// Store 16 staged head rows (kCph 16-byte chunks each, kRowB bytes apart in
// LDS) to global rows kDstB bytes apart; with nt, non-temporal buffer stores
// (a plain store loop under the same branch would be merged with the other
// one, dropping the hint; the range covers the 16 rows, dword 3 is gfx9's
// raw 32-bit buffer format).
template <int kCph, int kRowB, int kDstB>
__device__ __forceinline__ void store_rows(const uint8_t* sb, uint8_t* dst, int nt, int lane) {
  static_assert(16 * kCph % 64 == 0, "whole store instructions");
  if (nt) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(dst, 0, 16 * kDstB, 0x00020000);
#pragma unroll
    for (int i = 0; i < 16 * kCph / 64; ++i) {
      const int q = i * 64 + lane, h = q / kCph, c = (q - h * kCph) * 16;
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
      __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4*>(sb + h * kRowB + c), rs,
                                             h * kDstB + c, 0, 2 /* nt */);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16 * kCph / 64; ++i) {
      const int q = i * 64 + lane, h = q / kCph, c = (q - h * kCph) * 16;
      *reinterpret_cast<uint4*>(dst + (size_t)h * kDstB + c) = *reinterpret_cast<const uint4*>(sb + h * kRowB + c);
    }
  }
}

// After the step loop every wave holds (m, l, acc) of its 16 heads over its
// key-group's rows. The KW key-groups of each head-wave are rescaled to a
// common max and summed pairwise through LDS (a tree: half of the remaining
// waves stage their O, the other half add it), then the key-group-0 waves
// write the output (one split) or the split's fp32 partial (merged by the
// split-KV combine kernel).
template <int HW, int NW, int CS, typename QT>
__device__ __forceinline__ void epilogue(const FwdParams& p, const Tok& k, int tid, int wave, int lane,
                                         float m_run, float l_run, f32x4 (&acc)[kDV / 16 / CS]) {
  constexpr int WK = HW * CS, KW = NW / WK, NTL = kDV / 16 / CS;
  const int c16 = lane & 15, g = lane >> 4, kw = wave / WK, jw = wave % WK, hw = jw % HW, cs = jw / HW;
  const int ch0 = cs * NTL * 16;   // this wave's first O channel
  const int nhead_wg = 16 * HW;
  const int hq = k.hg * nhead_wg + hw * 16 + c16;
  const bool split = p.nsplit > 1;
  const int t = k.t;
  float M = m_run, L = l_run;
#if SAS_KG2_SPLIT_MERGE
  if constexpr (KW == 2 && CS == 2) {
    // Two key-groups, channel-split waves (the 32-head decode workgroup):
    // the two waves holding the same 16 heads x 256 channels (one per
    // key-group) each own half of those channels. Each passes the other
    // its scaled O for the other half through LDS, adds what it receives
    // (same sum as one wave adding both: own + other is commutative), and
    // stores its half, so the merge, the staging and the stores run on all
    // eight waves.
    constexpr int HT = NTL / 2;                      // tiles per owned half
    constexpr int XS = 16 * (HT * 16 + 4);           // floats per passed half (+4 pad per head)
    static_assert(NW * XS * 4 <= kLdsRows * kChunksMax * 16, "merge buffers fit");
    if (g == 0) { lds_ml[wave][0][c16] = m_run; lds_ml[wave][1][c16] = l_run; }
    __syncthreads();
    const int pw = (1 - kw) * WK + jw;               // the partner wave
    const float m0 = lds_ml[jw][0][c16], m1 = lds_ml[WK + jw][0][c16];
    M = fmaxf(m0, m1);
    const float w0 = m0 == -INFINITY ? 0.f : exp2f(m0 - M), w1 = m1 == -INFINITY ? 0.f : exp2f(m1 - M);
    L = w0 * lds_ml[jw][1][c16] + w1 * lds_ml[WK + jw][1][c16];
    const float w_self = kw == 0 ? w0 : w1;
    // o: the owned half (tiles HT kw ..), selected without indexing acc by a
    // runtime value (which would move acc to scratch memory)
    f32x4 o[HT];
    {
      float* xb = reinterpret_cast<float*>(lds_ring) + pw * XS;
#pragma unroll
      for (int i = 0; i < HT; ++i) {
        const f32x4 lo = acc[i] * w_self, hi = acc[HT + i] * w_self;
        o[i] = kw == 0 ? lo : hi;
        *reinterpret_cast<f32x4*>(xb + c16 * (HT * 16 + 4) + i * 16 + g * 4) = kw == 0 ? hi : lo;
      }
    }
    __syncthreads();
    {
      const float* xb = reinterpret_cast<const float*>(lds_ring) + wave * XS;
#pragma unroll
      for (int i = 0; i < HT; ++i) o[i] += *reinterpret_cast<const f32x4*>(xb + c16 * (HT * 16 + 4) + i * 16 + g * 4);
    }
    const int chw = ch0 + kw * HT * 16;              // this wave's first stored channel
    const int h0 = k.hg * nhead_wg + hw * 16;
    constexpr int PES = sizeof(PartT<QT>);
    int e2 = 0;
    if (split && PES == 2) {
      // one exponent per (head, 256-channel half): the max over both owners
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < HT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) a = fmaxf(a, fabsf(o[i][j]));
      a = rows_max(a);
      if (g == 0) lds_ml[wave][0][c16] = a;          // lds_ml was last read before the barrier above
      __syncthreads();
      a = fmaxf(a, lds_ml[pw][0][c16]);
      if (a > 0.f && a <= 3.0e38f) { (void)frexpf(a, &e2); e2 = 15 - e2; }   // a < 2^(15 - e2)
    }
    __syncthreads();   // every passed half read before the staging reuses the buffers
    uint8_t* sb0 = reinterpret_cast<uint8_t*>(lds_ring);
    if (!split) {
      constexpr int kRowB = HT * 16 * 2 + 32;
      constexpr int kCph = HT * 16 * 2 / 16;
      uint8_t* sb = sb0 + (size_t)wave * 16 * kRowB;
      const float inv = k.padded ? 0.f : 1.f / L;
#pragma unroll
      for (int i = 0; i < HT; ++i)
        *reinterpret_cast<uint2*>(sb + c16 * kRowB + (i * 16 + g * 4) * 2) =
            make_uint2(pack2<QT>(o[i][0] * inv, o[i][1] * inv),
                       pack2<QT>(o[i][2] * inv, o[i][3] * inv));
      uint8_t* ob = p.out + (((size_t)t * p.H + h0) * kDV + chw) * 2;
      store_rows<kCph, kRowB, kDV * 2>(sb, ob, p.out_nt, lane);
      if (g == 0 && cs == 0 && kw == 0) p.lse[(size_t)t * p.H + hq] = k.padded ? 0.f : M * kLn2 + logf(L);
    } else {
      constexpr int kRowB = HT * 16 * PES + (PES == 2 ? 32 : 16);
      constexpr int kCph = HT * 16 * PES / 16;
      uint8_t* sb = sb0 + (size_t)wave * 16 * kRowB;
      if constexpr (PES == 2) {
#pragma unroll
        for (int i = 0; i < HT; ++i)
          *reinterpret_cast<uint2*>(sb + c16 * kRowB + (i * 16 + g * 4) * 2) =
              make_uint2(pack2<_Float16>(ldexpf(o[i][0], e2), ldexpf(o[i][1], e2)),
                         pack2<_Float16>(ldexpf(o[i][2], e2), ldexpf(o[i][3], e2)));
      } else {
#pragma unroll
        for (int i = 0; i < HT; ++i)
          *reinterpret_cast<f32x4*>(sb + c16 * kRowB + (i * 16 + g * 4) * 4) = o[i];
      }
      const size_t row0 = ((size_t)t * p.nsplit + k.sp) * p.H + h0;
      uint8_t* ob = p.part_o + (row0 * kDV + chw) * PES;
      store_rows<kCph, kRowB, kDV * PES>(sb, ob, p.part_nt, lane);
      if (g == 0 && kw == 0) {
        float* pm = p.part_ml + (row0 + c16) * 4;   // (m, l, e_lo, e_hi); l < 0 marks a padded token
        if (cs == 0) *reinterpret_cast<float2*>(pm) = make_float2(M, k.padded ? -1.f : L);
        pm[2 + cs] = (float)e2;
      }
    }
    return;
  }
#endif
  if constexpr (KW > 1) {
    if (g == 0) { lds_ml[wave][0][c16] = m_run; lds_ml[wave][1][c16] = l_run; }
    __syncthreads();
    M = -INFINITY;
#pragma unroll
    for (int j = 0; j < KW; ++j) M = fmaxf(M, lds_ml[j * WK + jw][0][c16]);
    L = 0.f;
    float w_self = 0.f;
#pragma unroll
    for (int j = 0; j < KW; ++j) {
      const float mk = lds_ml[j * WK + jw][0][c16];
      const float wk = mk == -INFINITY ? 0.f : exp2f(mk - M);
      L += wk * lds_ml[j * WK + jw][1][c16];
      if (j == kw) w_self = wk;
    }
#pragma unroll
    for (int mt = 0; mt < NTL; ++mt) acc[mt] *= w_self;
#pragma unroll
    for (int half = KW / 2; half >= 1; half >>= 1) {
      if (kw >= half && kw < 2 * half) {
        float* ob = reinterpret_cast<float*>(lds_ring + ((kw - half) * WK + jw) * kObufChunks);
#pragma unroll
        for (int mt = 0; mt < NTL; ++mt)
          *reinterpret_cast<f32x4*>(ob + c16 * kObufStride + mt * 16 + g * 4) = acc[mt];
      }
      __syncthreads();
      if (kw < half) {
        const float* ob = reinterpret_cast<const float*>(lds_ring + (kw * WK + jw) * kObufChunks);
#pragma unroll
        for (int mt = 0; mt < NTL; ++mt)
          acc[mt] += *reinterpret_cast<const f32x4*>(ob + c16 * kObufStride + mt * 16 + g * 4);
      }
      __syncthreads();
    }
  }
  // The key-group-0 waves write their 16 heads x NTL * 16 channels: staged
  // through LDS (one region per wave, its own writes then reads, in order)
  // so every store instruction covers whole runs of a head's row instead of
  // 16 short pieces of 16 rows. The ring is free: every wave has left the
  // step loop (the key-group merge ends with a barrier; one key-group takes
  // one here).
  if constexpr (KW == 1) __syncthreads();
  if (kw == 0) {
    const int h0 = k.hg * nhead_wg + hw * 16;   // first head of this wave
    // Rows staged in LDS, then stored: the output in the query dtype (one
    // split), or the split's unnormalised partial (PartT<QT>: fp16 for bf16
    // outputs, scaled by 2^e with one e per head and 256-channel half chosen
    // so the half's largest |value| lies in [2^14, 2^15): exact power-of-two
    // scaling, no overflow, 8x finer than the output's rounding; fp32 for
    // fp16 outputs, e = 0).
    constexpr int PES = sizeof(PartT<QT>);
    constexpr int NH = NTL / 16;              // channel halves this wave holds
    uint8_t* sb0 = reinterpret_cast<uint8_t*>(lds_ring);
    int ex[NH];
    for (int hh = 0; hh < NH; ++hh) ex[hh] = 0;
    if (!split) {
      constexpr int kRowB = NTL * 16 * 2 + 32;   // staged row bytes (32 B pad)
      constexpr int kCph = NTL * 16 * 2 / 16;    // 16-byte chunks per head
      static_assert(NW * 16 * kRowB <= kLdsRows * kChunksMax * 16, "output staging fits");
      uint8_t* sb = sb0 + (size_t)jw * 16 * kRowB;
      const float inv = k.padded ? 0.f : 1.f / L;
#pragma unroll
      for (int mt = 0; mt < NTL; ++mt)
        *reinterpret_cast<uint2*>(sb + c16 * kRowB + (mt * 16 + g * 4) * 2) =
            make_uint2(pack2<QT>(acc[mt][0] * inv, acc[mt][1] * inv), pack2<QT>(acc[mt][2] * inv, acc[mt][3] * inv));
      uint8_t* ob = p.out + (((size_t)t * p.H + h0) * kDV + ch0) * 2;
      store_rows<kCph, kRowB, kDV * 2>(sb, ob, p.out_nt, lane);
      if (g == 0 && cs == 0) p.lse[(size_t)t * p.H + hq] = k.padded ? 0.f : M * kLn2 + logf(L);
    } else {
      constexpr int kRowB = NTL * 16 * PES + (PES == 2 ? 32 : 16);
      constexpr int kCph = NTL * 16 * PES / 16;
      static_assert(NW * 16 * kRowB <= kLdsRows * kChunksMax * 16, "partial staging fits");
      uint8_t* sb = sb0 + (size_t)jw * 16 * kRowB;
      if constexpr (PES == 2) {
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
          float a = 0.f;
#pragma unroll
          for (int mt = hh * 16; mt < hh * 16 + 16; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j) a = fmaxf(a, fabsf(acc[mt][j]));
          a = rows_max(a);   // over the head's four lane groups
          int e2 = 0;
          if (a > 0.f && a <= 3.0e38f) { (void)frexpf(a, &e2); e2 = 15 - e2; }   // a < 2^(15 - e2)
          ex[hh] = e2;
        }
#pragma unroll
        for (int mt = 0; mt < NTL; ++mt) {
          const int e2 = ex[mt / 16];
          *reinterpret_cast<uint2*>(sb + c16 * kRowB + (mt * 16 + g * 4) * 2) =
              make_uint2(pack2<_Float16>(ldexpf(acc[mt][0], e2), ldexpf(acc[mt][1], e2)),
                         pack2<_Float16>(ldexpf(acc[mt][2], e2), ldexpf(acc[mt][3], e2)));
        }
      } else {
#pragma unroll
        for (int mt = 0; mt < NTL; ++mt)
          *reinterpret_cast<f32x4*>(sb + c16 * kRowB + (mt * 16 + g * 4) * 4) = acc[mt];
      }
      const size_t row0 = ((size_t)t * p.nsplit + k.sp) * p.H + h0;
      uint8_t* ob = p.part_o + (row0 * kDV + ch0) * PES;
      store_rows<kCph, kRowB, kDV * PES>(sb, ob, p.part_nt, lane);
      if (g == 0) {
        // (m, l, e_lo, e_hi); l < 0 marks a padded token
        float* pm = p.part_ml + (row0 + c16) * 4;
        if constexpr (NH == 2) {
          *reinterpret_cast<float4*>(pm) = make_float4(M, k.padded ? -1.f : L, (float)ex[0], (float)ex[1]);
        } else {
          if (cs == 0) *reinterpret_cast<float2*>(pm) = make_float2(M, k.padded ? -1.f : L);
          pm[2 + cs] = (float)ex[0];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// forward kernel, head-waves sharing LDS tiles (HW = 2, 4)
// ---------------------------------------------------------------------------

// EXW: the exact-window schedule (Fwd::run_exact) instead of the streaming loop
template <int HW, int NW, int D, typename QT, int KVF, bool EXW>
__global__ void __launch_bounds__(NW * 64)
sas_fwd_kernel(const FwdParams p) {
  using C = Cfg<HW, NW, D, QT, KVF>;
  // the wave index and every count derived from it are wave-uniform: kept
  // in scalar registers, the step loop's bounds and DMA guards become scalar
  // branches instead of exec-mask updates
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int item = item_index(p);
  if (item < 0) return;
  Tok k = item_of(p, item);
  Fwd<HW, NW, D, QT, KVF> f(p, lane, wave);
  const int hq = k.hg * (16 * HW) + f.hw * 16 + f.c16;
  // Q^T operand in registers (head hq, channels ks*32 + 8g .. +8): with QL
  // through LDS (DMA by the waves that do no slot resolution, at once), else
  // loaded behind the block-table reads of the slot resolution
  // QL: the query rows depend on the token index only, so waves 4-7 (which
  // do no slot resolution) issue their DMA before anything else, under the
  // latency of the index round trip, and are done issuing by the time the
  // compaction barrier waits for them
  if constexpr (C::QL) {
    if (wave >= 4) f.q_dma(k, wave);
  }
  resolve<256, C::ROWB>(p, k, tid, lane, wave, [&] {
    if constexpr (C::QL) return;
    const uint4* qp = reinterpret_cast<const uint4*>(p.q + ((size_t)k.t * p.H + hq) * D * 2);
#pragma unroll
    for (int n = 0; n < C::NQ; ++n) {
      // head tile hw, or with Q2 the pair's tiles (hw & ~1) + n
      const int dh = C::Q2 ? ((f.hw & ~1) + n - f.hw) * 16 : 0;
#pragma unroll
      for (int ks = 0; ks < C::KSQ; ++ks)
        f.qf[n][ks] = qp[(long long)dh * (D / 8) + ((C::QS ? f.cs * C::KSQ : 0) + ks) * 4 + f.g];
    }
  });
  const int nvalid = __builtin_amdgcn_readfirstlane(k.nvalid);
  // QL kernels: pad lds_rows with copies of the last row (read after the
  // query barrier below; with no rows no step is issued)
  if constexpr (C::QL && KVF != 1) {
    static_assert(2 * C::TR <= kRowPad, "a step past the last reaches at most 2 TR entries beyond it");
    if (tid < kRowPad) lds_rows[nvalid + tid] = lds_rows[nvalid > 0 ? nvalid - 1 : 0];
  }

  // key-group shares: whole steps, group 0 first
  const int per = ((nvalid + C::KW * C::TR - 1) / (C::KW * C::TR)) * C::TR;
  const int gbeg = min(nvalid, f.kw * per);
  f.rbeg = gbeg;
  f.ring = f.kw * C::NST * C::SLOT;
  f.nrows = min(nvalid, gbeg + per) - gbeg;
  f.nsteps = (f.nrows + C::TR - 1) / C::TR;
  f.nsteps_max = per / C::TR;

  // retire every load the compiler tracks (Q, tables, indices, sink) before
  // the DMA ring starts, so none of its own vmcnt waits lands inside the loop
  const bool seed_sink = p.nsplit == 1 && f.kw == 0;
  const float sink = (seed_sink || EXW) ? p.sinks[hq] : 0.f;
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (C::QL) __syncthreads();   // every wave's query DMA has landed
  f.m_run = seed_sink ? sink * kLog2e : -INFINITY;
  f.l_run = seed_sink ? 1.f : 0.f;
  if constexpr (C::KSP) f.l_run = seed_sink && f.cs == 0 ? 1.f : 0.f;   // the sink's term: half 0's sum
#pragma unroll
  for (int i = 0; i < C::NTL; ++i) f.acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (EXW) f.run_exact(wave, p.nsplit == 1 ? sink * kLog2e : -INFINITY);
  // (the query rows are read before the first step barrier, ahead of any
  // write to them)
  else f.run([&] { if constexpr (C::QL) f.q_from_lds(); });
  epilogue<HW, NW, C::CS, QT>(p, k, tid, wave, lane, f.m_run, f.l_run, f.acc);
}

// ---------------------------------------------------------------------------
// decode kernel: every wave streams its own rows through registers (HW = 1)
// ---------------------------------------------------------------------------
//
// A wave owns 16 heads and a contiguous share of the workgroup's rows, in
// steps of 16 rows. Each lane loads its part of a step's rows straight into
// the QK^T A-operand layout (row c16, channels 8(4ks+g) .. +8 for k-step
// ks: one 16-byte load per k-step), NP steps ahead, so up to NP x 18 KB per
// wave are in flight with no LDS staging; the QK^T MFMAs read those
// registers. Only the V half (channels 0..511) passes through LDS, written
// from the same registers into a per-wave tile that the PV operand reads
// transposed. (fp8 rows take the LDS kernels.)

template <int D, typename QT, int KVF>
struct Dec {
  static constexpr int KS = D / 32;          // k-steps per row (chunks per lane)
  static constexpr int NP = 3;               // steps in flight per wave
  static constexpr int VCH = kDV / 8;        // chunks per V row
  // V tile row stride: 72 chunks, so the 8-chunk-group swizzle applies (a
  // 16-chunk-group one costs the kernel its registers)
  static constexpr int VRS = VCH + 8;
  static constexpr int VT = 16 * VRS;        // chunks per V tile
  static constexpr int ROWB = D * 2;
  // fp8 rows take the LDS kernels, which apply the scales per 128-channel
  // group to S and P in fp32
  static_assert(!KVF, "cache rows in the query dtype only");
  static_assert(4 * VT <= kLdsRows * kChunksMax, "V tiles fit");

  struct Stage {
    uint4 k[KS];   // the row's chunks 4ks + g
  };

  const FwdParams& p;
  const int lane, c16, g;
  int rbeg, nrows, nsteps, vt;
  uint64_t dummy;
  uint4 qf[KS];
  float m_run, l_run;
  f32x4 acc[kDV / 16];

  __device__ Dec(const FwdParams& p_, int lane_) : p(p_), lane(lane_), c16(lane_ & 15), g(lane_ >> 4) {}


  // Step `step` of this wave into a stage. Loads are issued for every stage
  // unconditionally, so the compiler's vmcnt bookkeeping sees the same load
  // sequence on every path and waits exactly for the stage in use; a step
  // past the end parks all lanes on one address (one cache line per load).
  __device__ __forceinline__ void load(Stage& st, int step) const {
    const int i = step * 16 + c16;
    const bool live = step < nsteps;
    const uint64_t ra = lds_rows[rbeg + min(i, max(nrows - 1, 0))];
    const uint64_t src = live && i < nrows ? ra : dummy;
    const int gm = live ? g : 0, lm = live ? 1 : 0;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) st.k[ks] = gld16(src + lm * (4 * ks + gm) * 16);
  }

  // A-operand chunk 4ks + g of the lane's row
  __device__ __forceinline__ uint4 kchunk(const Stage& st, int ks) const { return st.k[ks]; }

  template <int J, bool REFILL>
  __device__ __forceinline__ void step(Stage (&st)[NP], int it0) {
    const int it = it0 + J;
    const int nk = min(16, nrows - it * 16);
    uint4 kf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = kchunk(st[J], ks);
    // V half -> this wave's LDS tile (row c16, chunk 4ks + g, swizzled)
    const int vsw_w = swz<VRS>(c16);
#pragma unroll
    for (int ks = 0; ks < VCH / 4; ++ks) lds_ring[vt + c16 * VRS + (((4 * ks + g) & ~7) | (((4 * ks + g) & 7) ^ vsw_w))] = kf[ks];
    // S^T[16 keys x 16 heads] = K . Q^T, even / odd k-steps in two chains
    f32x4 se = f32x4{0.f, 0.f, 0.f, 0.f}, so = se;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks & 1) so = mfma32k<QT>(kf[ks], qf[ks], so);
      else se = mfma32k<QT>(kf[ks], qf[ks], se);
    }
    // the stage's registers are consumed: refill them NP steps ahead
    if constexpr (REFILL) load(st[J], it + NP);
    se += so;
    float sv[4];
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float x = g * 4 + j < nk ? se[j] * p.scale_log2 : -INFINITY;
      sv[j] = x;
      mloc = fmaxf(mloc, x);
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    // lazy rescale (see Fwd::compute)
    if (__ballot(mloc > m_run + kLazyLog2)) {
      const float m_new = fmaxf(m_run, mloc);
      const float alpha = exp2f(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int i = 0; i < kDV / 16; ++i) acc[i] *= alpha;
    }
    float pv[4], lsum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pv[j] = __builtin_amdgcn_exp2f(sv[j] - m_run);
      lsum += pv[j];
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    l_run += lsum;
    const uint2 pfrag = make_uint2(pack2<QT>(pv[0], pv[1]), pack2<QT>(pv[2], pv[3]));
    // O^T[512 x 16] += V^T . P^T: one transposed read per 16-channel tile
    // (rows 4g + c16/4, channels mt*16 + 4*(c16&3)), 16x16x16 MFMA
    const int vr = 4 * g + (c16 >> 2);
    const int vsw = swz<VRS>(vr);
    const int vb = (c16 & 3) >> 1;
    const char* vbase = reinterpret_cast<const char*>(&lds_ring[vt + vr * VRS]) + (c16 & 1) * 8;
    constexpr int TPG = kSwzGroup<VRS> / 2;
    int voff[TPG];
#pragma unroll
    for (int q = 0; q < TPG; ++q) voff[q] = ((2 * q + vb) ^ vsw) * 16;
    auto vfrag = [&](int mt) {
      const char* a0 = vbase + (mt / TPG) * TPG * 32 + voff[mt % TPG];
      return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS i16x4*)(a0)));
    };
    constexpr int kPf = 8;
    uint2 vf[kPf];
#pragma unroll
    for (int i = 0; i < kPf; ++i) vf[i] = vfrag(i);
#pragma unroll
    for (int mt = 0; mt < kDV / 16; ++mt) {
      const uint2 a = vf[mt % kPf];
      if (mt + kPf < kDV / 16) vf[mt % kPf] = vfrag(mt + kPf);
      acc[mt] = mfma16k<QT>(a, pfrag, acc[mt]);
    }
  }

  // Whole groups of NP steps in the loop (every step refills its stage),
  // the remaining 0..NP-1 steps after it (no refills).
  __device__ __forceinline__ void run() {
    Stage st[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) load(st[j], j);
    int it0 = 0;
    for (; it0 + NP <= nsteps; it0 += NP) {
      step<0, true>(st, it0);
      step<1, true>(st, it0);
      step<2, true>(st, it0);
    }
    const int r = nsteps - it0;
    if (r > 0) step<0, false>(st, it0);
    if (r > 1) step<1, false>(st, it0);
  }
};

template <int D, typename QT, int KVF>
__global__ void __launch_bounds__(256)
sas_dec_kernel(const FwdParams p) {
  using C = Dec<D, QT, KVF>;
  // the wave index and every count derived from it are wave-uniform: kept
  // in scalar registers, the step loop's bounds and DMA guards become scalar
  // branches instead of exec-mask updates
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int item = item_index(p);
  if (item < 0) return;
  Tok k = item_of(p, item);
  C f(p, lane);
  resolve<256, C::ROWB>(p, k, tid, lane, wave, [] {});
  const int nvalid = __builtin_amdgcn_readfirstlane(k.nvalid);
  const int hq = k.hg * 16 + f.c16;
  // key-group share of wave `wave`: whole 16-row steps, wave 0 first
  const int per = ((nvalid + 63) >> 6) << 4;
  const int gbeg = min(nvalid, wave * per);
  f.rbeg = gbeg;
  f.nrows = min(nvalid, gbeg + per) - gbeg;
  f.nsteps = (f.nrows + 15) >> 4;
  f.dummy = nvalid > 0 ? lds_rows[0] : reinterpret_cast<uint64_t>(p.ori_kv);
  f.vt = wave * C::VT;
  // Q^T operand in registers (head hq, channels ks*32 + 8g .. +8), ahead of
  // the first K loads
  {
    const uint4* qp = reinterpret_cast<const uint4*>(p.q + ((size_t)k.t * p.H + hq) * D * 2);
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) f.qf[ks] = qp[ks * 4 + f.g];
  }
  const bool seed_sink = p.nsplit == 1 && wave == 0;
  f.m_run = seed_sink ? p.sinks[hq] * kLog2e : -INFINITY;
  f.l_run = seed_sink ? 1.f : 0.f;
#pragma unroll
  for (int i = 0; i < kDV / 16; ++i) f.acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (f.nsteps > 0) f.run();
  epilogue<1, 4, 1, QT>(p, k, tid, wave, lane, f.m_run, f.l_run, f.acc);
}

// ---------------------------------------------------------------------------
// split-KV combine (separate launch; used with SAS_FWD_NO_COMBINE)
// ---------------------------------------------------------------------------

#ifndef SAS_COMBINE_THREADS
#define SAS_COMBINE_THREADS 256
#endif
constexpr int kCombineThreads = SAS_COMBINE_THREADS;
// Split counts: the planner's own choice fills the CUs with at most
// kMaxAutoSplits; a token with more key slots than kMaxAutoSplits x kMaxSlots
// (long CFA rows, wide windows), or an explicit count, takes up to
// kMaxSplits. The combine merges any count, kB splits' loads at a time.
constexpr int kMaxAutoSplits = 64;
constexpr int kMaxSplits = 1 << 16;
constexpr long long kMaxTokenSlots = (long long)kMaxSplits * kMaxSlots;

// One workgroup per (token, 4 heads), thread = (head, 8 channels): 16-byte
// fp16 partial loads (C2 call 19.95 -> 19.7 us against 4 channels).
template <typename QT>
__global__ void __launch_bounds__(kCombineThreads)
sas_combine_kernel(const FwdParams p) {
  constexpr int kHeads = kCombineThreads / (kDV / kCombineCpt);   // heads per workgroup
  const int nhb = (p.H + kHeads - 1) / kHeads;
  // token t's workgroups go to the XCD its split workgroups ran on
  // (item_index's dealing), whose L2 still holds the partials they wrote
  // (measured: C2 call 24.3 -> 23.7 µs)
  const unsigned nx = (unsigned)p.nxcd;
  const int x = (int)(blockIdx.x % nx), l = (int)(blockIdx.x / nx);
  const int t = p.T - 1 - ((l / nhb) * p.nxcd + x);
  if (t < 0) return;
  const int h0 = (l % nhb) * kHeads;
  merge_partials<QT>(p, t, h0, min(kHeads, p.H - h0), threadIdx.x, kCombineThreads);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// bytes per split-partial O element: fp16 (scaled) for bf16 outputs, fp32 for fp16 outputs
int part_bytes(int q_dtype) { return q_dtype == SAS_DT_FP16 ? 4 : 2; }

struct Plan {
  int hw, nw, nhg, nslots, nsplit, sps;
  bool exact;   // exact-window schedule (Fwd::run_exact)
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
  if (a->win_left < 0) return sas::set_error(SAS_EINVAL, "win_left out of range");
  if (a->scenario >= SAS_CFA && (a->cmp_ratio < 1 || a->K < 0)) return sas::set_error(SAS_EINVAL, "bad cmp_ratio/K");
  const long long nslots_ll = (long long)a->win_left + 1 + (a->scenario >= SAS_CFA ? a->K : 0);
  if (nslots_ll > kMaxTokenSlots)
    return sas::set_error(SAS_EINVAL, "%lld key slots per token (win_left + 1 + K) beyond %lld", nslots_ll,
                          kMaxTokenSlots);
  pl->nslots = (int)nslots_ll;
  const long long T = std::max<long long>(a->T, 1);
  int hw = a->head_waves;
  int ns = a->num_splits;
  // Window-only calls whose window fits the ring run the exact-window
  // schedule: one split, 4 waves, P rounded against the window's final
  // maximum (golden's one window tile). An explicit split count above 1 or
  // 8 waves selects the streaming schedule instead. (16-head groups may take
  // the exact schedule with splits too, below.)
  pl->exact = a->scenario == SAS_SWA && pl->nslots <= kLdsRows && ns <= 1 && (a->waves == 0 || a->waves == 4);
  const bool fp8 = a->kv_dtype == SAS_DT_FP8_E4M3_ROW656;
  // Every workgroup of a token runs on the token's XCD (item_index deals
  // tokens round-robin over the XCDs, blockIdx % XCDs): with one workgroup
  // per CU, a grid fills the chip in one round when each XCD's share,
  // ceil(T / XCDs) tokens x head groups x splits, fits its CUs. A second round
  // roughly doubles a decode call (31-token, 128-head decode with 5 splits
  // of 64 heads: 43.8 µs, 4 splits: 28.7 µs).
  const int cus = sas::device_cus();
  const int xcds = sas::device_xcds();
  const long long cus_x = std::max(1, cus / xcds);
  const long long tpx = (T + xcds - 1) / xcds;
  auto one_round_splits = [&](int h) { return std::max<long long>(1, cus_x / (tpx * (a->H / (16 * h)))); };
  if (hw <= 0) {
    // Heads sharing one gathered tile inside a workgroup (16 per wave); each
    // row crosses L2 -> CU once per head group. With many tokens every
    // workgroup holds 64 heads. With few, 32-head groups (2 head-waves x 2
    // key-groups, 8 waves) while they still allow 4 splits in one round:
    // half the rows per split at equal grid size, and fewer partials to
    // merge (32-token, 64-head decode: 18.4 µs at 32 heads x 4 splits,
    // 21.1 µs at 64 heads x 8 splits); else 64-head groups, which leave room
    // for twice the splits (31-token, 128-head decode: 28.7 µs at 64 x 4
    // against 32.4 µs at 32 x 2). fp8 rows take 32-head groups whenever the
    // heads allow: their 8-wave kernel keeps the rows fp8 in LDS, while the
    // 64-head fp8 kernels (4 waves, rows converted through registers) spill
    // (8-token, 128-head fp8 decode: 23.2 µs at 32 heads x 8 waves x 8
    // splits, 26.3 µs at 64 heads x 4 waves x 12 splits; 31-token, 128-head
    // fp8 decode 30.3 against 42.2 µs; 4K-token, 64-head fp8 prefill 686
    // against 880 µs).
    if (fp8 && a->H % 32 == 0) hw = 2;
    else if (a->H % 64 == 0 && T * (a->H / 64) >= 2 * cus) hw = 4;
    else if (a->H % 64 == 0 && one_round_splits(2) < 4) hw = 4;
    else if (a->H % 32 == 0) hw = 2;
    else hw = 1;
  }
  if (hw != 1 && hw != 2 && hw != 4) return sas::set_error(SAS_EINVAL, "head_waves must be 1, 2 or 4");
  while (hw > 1 && a->H % (16 * hw)) hw >>= 1;
  int nw = a->waves;
  // 8 waves: two per SIMD, a pair per 16 heads splitting both the QK^T and
  // the O channels; the second wave on a SIMD overlaps the other's LDS and
  // softmax latencies (measured: 4K prefill 593 vs 650 µs, 32-token decode
  // split kernel 19.3 vs 20.4 µs). With fp8 rows the 64-head 8-wave build
  // spills (the staging registers beside the scale groups): 4 waves there.
  if (nw <= 0) nw = (hw == 2 || (hw == 4 && !fp8)) ? 8 : 4;
  if (nw != 4 && nw != 8) return sas::set_error(SAS_EINVAL, "waves must be 4 or 8");
  if (hw == 1 || pl->exact) nw = 4;
  pl->nw = nw;
  pl->hw = hw;
  pl->nhg = (int)a->H / (16 * hw);
  if (pl->exact) ns = 1;
  if (ns <= 0) {
    // as many splits as fill each XCD's CUs in one round, each split at
    // least min_sps slots (1-token, 16-head decode: 15.5 µs at 4 splits of
    // 48 slots, 16.1 µs at 3 of 64; fp8 rows, which cost the 4-wave kernel
    // more per row to stage: 8-token, 128-head decode 25.6 µs at 12 splits of
    // 96 slots, 26.3 µs at 16 of 72)
    const int min_sps = fp8 ? 96 : hw == 1 ? 48 : 64;
    const int max_by_len = std::max(1, (pl->nslots + min_sps - 1) / min_sps);
    ns = (int)std::min<long long>(one_round_splits(hw), max_by_len);
  }
  ns = std::max(1, std::min(ns, a->num_splits > 0 ? kMaxSplits : kMaxAutoSplits));
  // fp8 rows in the 32-head 8-wave plan: two key-groups of 32-row steps per
  // workgroup. Of the split counts whose workgroups take the same number of
  // steps (the key-group holding the first share of rows sets the time),
  // the fewest: fewer partials to write and merge (C5, 1152 slots: 8 splits
  // give key-groups of 96 + 48 rows, 6 splits 96 + 96; 22.6-22.8 against
  // 23.0 µs with caches flushed, 18.0 against 18.3-18.4 µs warm)
  if (a->num_splits <= 0 && fp8 && hw == 2 && nw == 8 && !pl->exact) {
    auto steps = [&](int n) {
      const int r = (pl->nslots + n - 1) / n;
      return (r + 63) / 64;   // 32-row steps of the first key-group's ceil(r / 64) x 32 rows
    };
    while (ns > 1 && steps(ns - 1) == steps(ns)) --ns;
  }
  // 16-head groups run the exact schedule when a split's rows fit the ring
  // (every row gathered at once, no per-step barriers; 1-token, 16-head
  // decode: 12.7 µs against 15.5 µs for the register-streaming decode
  // kernel), taking the splits that make them fit if one round holds them
  if (!pl->exact && hw == 1 && (a->waves == 0 || a->waves == 4)) {
    const int fit = (pl->nslots + kLdsRows - 1) / kLdsRows;
    if (a->num_splits <= 0 && ns < fit && fit <= std::min<long long>(one_round_splits(1), kMaxAutoSplits)) ns = fit;
    pl->exact = (pl->nslots + ns - 1) / ns <= kLdsRows;
  }
  int sps = (pl->nslots + ns - 1) / ns;
  if (sps > kMaxSlots) {
    ns = (pl->nslots + kMaxSlots - 1) / kMaxSlots;
    if (ns > kMaxSplits) return sas::set_error(SAS_EINVAL, "too many key slots per token");
    sps = (pl->nslots + ns - 1) / ns;
  }
  ns = (pl->nslots + sps - 1) / sps;  // drop empty trailing splits
  pl->nsplit = std::max(ns, 1);
  pl->sps = sps;
  pl->ws = pl->nsplit > 1 ? (size_t)a->T * pl->nsplit * a->H * (kDV * part_bytes(a->q_dtype) + 4 * sizeof(float)) : 0;
  return SAS_OK;
}

template <int HW, int NW, int D, typename QT, int KVF, bool EXW = false>
int launch_fwd(const FwdParams& fp, int nblocks, hipStream_t st) {
  hipLaunchKernelGGL((sas_fwd_kernel<HW, NW, D, QT, KVF, EXW>), dim3(nblocks), dim3(NW * 64), 0, st, fp);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return sas::set_error(SAS_ELAUNCH, "sas_fwd launch: %s", hipGetErrorString(e));
  return SAS_OK;
}

template <int D, typename QT, int KVF>
int launch_dec(const FwdParams& fp, int nblocks, hipStream_t st) {
  hipLaunchKernelGGL((sas_dec_kernel<D, QT, KVF>), dim3(nblocks), dim3(256), 0, st, fp);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return sas::set_error(SAS_ELAUNCH, "sas_dec launch: %s", hipGetErrorString(e));
  return SAS_OK;
}

template <int D, typename QT, int KVF>
int dispatch_hw(int hw, int nw, bool exact, const FwdParams& fp, int nb, hipStream_t st) {
  if (exact) {
    if (hw == 1) return launch_fwd<1, 4, D, QT, KVF, true>(fp, nb, st);
    if (hw == 2) return launch_fwd<2, 4, D, QT, KVF, true>(fp, nb, st);
    if (hw == 4) return launch_fwd<4, 4, D, QT, KVF, true>(fp, nb, st);
    return sas::set_error(SAS_EINVAL, "unsupported head grouping");
  }
  // 16-head groups: the register-streamed decode kernel, or for fp8 rows
  // (whose scales are applied per 128-channel group in the LDS kernels) the
  // 4-wave streaming kernel
  if (hw == 1) {
    if constexpr (KVF) return launch_fwd<1, 4, D, QT, KVF>(fp, nb, st);
    else return launch_dec<D, QT, KVF>(fp, nb, st);
  }
  if (hw == 2 && nw == 4) return launch_fwd<2, 4, D, QT, KVF>(fp, nb, st);
  if (hw == 4 && nw == 4) return launch_fwd<4, 4, D, QT, KVF>(fp, nb, st);
  // fp8 rows in the 32-head 8-wave plan: kept as fp8 in LDS (KVF 2)
  if (hw == 2 && nw == 8) return launch_fwd<2, 8, D, QT, KVF ? SAS_FP8_RESIDENT : 0>(fp, nb, st);
  if (hw == 4 && nw == 8) return launch_fwd<4, 8, D, QT, KVF>(fp, nb, st);
  return sas::set_error(SAS_EINVAL, "unsupported head grouping");
}

int launch_combine(const FwdParams& fp, int out_dtype, hipStream_t st) {
  constexpr int kHeads = kCombineThreads / (kDV / kCombineCpt);
  const long long nx = fp.nxcd;
  const dim3 grid((unsigned)(((fp.T + nx - 1) / nx) * nx * ((fp.H + kHeads - 1) / kHeads)));
  if (out_dtype == SAS_DT_BF16)
    hipLaunchKernelGGL(sas_combine_kernel<__bf16>, grid, dim3(kCombineThreads), 0, st, fp);
  else if (out_dtype == SAS_DT_FP16)
    hipLaunchKernelGGL(sas_combine_kernel<_Float16>, grid, dim3(kCombineThreads), 0, st, fp);
  else
    return sas::set_error(SAS_EINVAL, "combine: bad out dtype");
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return sas::set_error(SAS_ELAUNCH, "sas_combine launch: %s", hipGetErrorString(e));
  return SAS_OK;
}

int combine_impl(const SasCombineArgs* a, hipStream_t st) {
  if (!a || !a->part_o || !a->part_ml || !a->sinks || !a->out || !a->lse)
    return sas::set_error(SAS_EINVAL, "combine: null pointer");
  if (a->DV != kDV || a->S < 1 || a->S > kMaxSplits || a->H < 1 || a->T < 0)
    return sas::set_error(SAS_EINVAL, "combine: bad dims (S must be 1..%d, DV 512)", kMaxSplits);
  if (a->T == 0) return SAS_OK;
  FwdParams fp{};
  fp.part_o = (uint8_t*)const_cast<void*>(a->part_o);
  fp.part_ml = const_cast<float*>(a->part_ml);
  fp.sinks = a->sinks;
  fp.out = (uint8_t*)a->out;
  fp.lse = a->lse;
  fp.T = (int)a->T; fp.H = (int)a->H; fp.nsplit = (int)a->S;
  fp.nxcd = sas::device_xcds();
  return launch_combine(fp, a->out_dtype, st);
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
  if (!a->q || !a->ori_kv || !a->ori_block_table || !a->q_prefix || !a->act_kv ||
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

  FwdParams fp{};
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
  if (pl.nsplit > 1) {
    fp.part_o = (uint8_t*)a->workspace;
    fp.part_ml = (float*)((uint8_t*)a->workspace + (size_t)a->T * pl.nsplit * a->H * kDV * part_bytes(a->q_dtype));
  }
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
  // item_index(): ceil(T / XCDs) tokens per XCD, nhg * nsplit workgroups each
  fp.nxcd = sas::device_xcds();
  const long long nblocks_ll = (long long)((a->T + fp.nxcd - 1) / fp.nxcd) * pl.nhg * pl.nsplit * fp.nxcd;
  if (nblocks_ll > INT_MAX)
    return sas::set_error(SAS_EINVAL, "%lld workgroups (tokens x head groups x splits) beyond one launch",
                          nblocks_ll);
  const int nblocks = (int)nblocks_ll;
  // Large partials of a grid that is resident all at once stream out during
  // the kernel instead of leaving the L2 dirty for the writeback at its end
  // (C2 decode: 22.7 -> 22.0 µs); with a second wave of workgroups, or small
  // partials, the L2 copy the combine reads is worth more (C4, C1 slower).
  fp.part_nt = pl.nsplit > 1 && nblocks <= sas::device_cus() && pl.ws >= (size_t(4) << 20);
  // An output far beyond the L2s (4K prefill: 268 MB) streams out instead of
  // evicting the cache rows the next tokens gather (C3: 586 -> 571 µs).
  fp.out_nt = pl.nsplit == 1 && (size_t)a->T * a->H * kDV * 2 >= (size_t(16) << 20);
  hipStream_t st = (hipStream_t)stream;

  if (fp8) rc = dispatch_hw<576, __bf16, 1>(pl.hw, pl.nw, pl.exact, fp, nblocks, st);
  else if (a->q_dtype == SAS_DT_BF16)
    rc = a->D == 576 ? dispatch_hw<576, __bf16, 0>(pl.hw, pl.nw, pl.exact, fp, nblocks, st)
                     : dispatch_hw<512, __bf16, 0>(pl.hw, pl.nw, pl.exact, fp, nblocks, st);
  else
    rc = a->D == 576 ? dispatch_hw<576, _Float16, 0>(pl.hw, pl.nw, pl.exact, fp, nblocks, st)
                     : dispatch_hw<512, _Float16, 0>(pl.hw, pl.nw, pl.exact, fp, nblocks, st);
  if (rc || pl.nsplit == 1 || (a->flags & SAS_FWD_NO_COMBINE)) return rc;
  return launch_combine(fp, a->q_dtype, st);
}

// ---------------------------------------------------------------------------
// no-allocation forward: split partials in a file-scope device array
// ---------------------------------------------------------------------------

namespace {

constexpr size_t kScratchBytes = size_t(16) << 20;   // split partials of one call, at most
constexpr int kMaxDevices = 64;

// Each device holds its own copy once the library's code object is loaded
// there. Host code never uses this name as an address: the device address
// comes from hipGetSymbolAddress, once per device (scratch_ptr below).
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the stream's device, which must be the
// current device; looked up on the first call per device.
int scratch_ptr(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(SAS_ELAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (st) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess) return set_error(SAS_ELAUNCH, "hipStreamGetDevice: %s", hipGetErrorString(e));
    if (sdev != dev)
      return set_error(SAS_EINVAL, "no-alloc forward: the stream is on device %d, the current device is %d",
                       (int)sdev, dev);
  }
  if (dev < 0 || dev >= kMaxDevices) return set_error(SAS_EINVAL, "device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(SAS_ELAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SAS_OK;
}

}  // namespace

extern "C" int sas_fwd_noalloc_v1(const SasFwdArgs* a, void* stream) {
  sas::clear_error();
  Plan pl;
  const int rc = make_plan(a, &pl);
  if (rc) return rc;
  if (a->flags & SAS_FWD_NO_COMBINE)
    return sas::set_error(SAS_EINVAL, "no-alloc forward: SAS_FWD_NO_COMBINE would leave the partials in the "
                                      "library's scratch; use sas_fwd_v1 with a workspace");
  if (pl.ws > kScratchBytes)
    return sas::set_error(SAS_ENOWS, "no-alloc forward: %zu bytes of split partials needed, beyond the %zu-byte "
                                     "scratch (use sas_fwd_v1 with a workspace, or fewer tokens per call)",
                          pl.ws, kScratchBytes);
  if (a->T == 0) return SAS_OK;
  SasFwdArgs b = *a;
  b.workspace = nullptr;
  b.workspace_bytes = 0;
  if (pl.ws) {
    void* ptr = nullptr;
    const int r2 = scratch_ptr((hipStream_t)stream, &ptr);
    if (r2) return r2;
    b.workspace = ptr;
    b.workspace_bytes = kScratchBytes;
  }
  return sas_fwd_v1(&b, stream);
}

extern "C" int sas_combine_v1(const SasCombineArgs* a, void* stream) {
  sas::clear_error();
  return combine_impl(a, (hipStream_t)stream);
}

}  // namespace sas
