// The fused 2/4-bit quantized split kernel (gfx950) and its launcher.
// Included by quant_split_k*v*.hip, which instantiate the launcher for one
// K/V bit-width pair each.
#pragma once

#include "decode_common.h"

namespace tkv {

// ===========================================================================
// Fused quantized split kernel.
//
// Every chunk (32 tokens) of K codes, V codes and the four metadata tensors is
// copied by direct-to-LDS buffer loads (buffer_load_dword{,x4} ... lds) into a
// per-wave ring of NSTAGE stages, NSTAGE-1 chunks ahead of the compute.  Each
// load instruction moves whole 16-byte lanes of a contiguous range, so every
// line of the cache is fetched once with the non-temporal policy, and the
// prefetch depth costs LDS instead of VGPRs.  The MFMA operands are then
// gathered from LDS:
//   K, V codes  blocks of 16 tokens, each block [16-byte unit][token]: every
//               DMA instruction still copies one contiguous kilobyte, and the
//               16 rows of an MFMA tile read from one unit are 16 consecutive
//               entries, so the operand reads spread over the banks;
//   metadata    the global layout [t][g] of each tensor, one dword DMA per
//               lane; pairs of tokens are gathered with v_perm_b32.
// Scores, softmax and PV follow the design notes at the top of this file.
// ===========================================================================
template <int D, int KNB, int VNB, int GS>
struct StageGeom {
  using KL = KLayout<D, KNB, GS>;
  using VL = VLayout<D, VNB, GS>;
  static constexpr int NG = D / GS;
  // fp16 slots per token row of a staged metadata tensor: the global row of NG
  // values, except NG == 1: a chunk whose rows all lie before the split's last
  // token is copied as whole dwords (fp16 pairs of tokens 2i, 2i + 1, MROW_PAIRS
  // = 1), the chunk holding the last token one fp16 per dword (MROW = 2: a dword
  // copy could straddle the end of the buffer range there).
  static constexpr int MROW = NG >= 2 ? NG : 2;
  static constexpr int MROW_PAIRS = NG >= 2 ? NG : 1;
  static constexpr int KB = kChunk * KL::DP;    // K code bytes per chunk
  static constexpr int VB = kChunk * VL::DP;    // V code bytes per chunk
  static constexpr int MB = kChunk * MROW * 2;  // bytes of one staged metadata tensor
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = K_OFF + KB;
  static constexpr int M_OFF = V_OFF + VB;    // ks, kz, vs, vz at M_OFF + t * MB
  // MB bytes of fp16 1.0 pairs behind vz: the ones row of the V zero-point
  // MFMA reads them through the same offsets as the zero points (written
  // once per launch; no DMA touches them).
  static constexpr int ONES_OFF = M_OFF + 4 * MB;
  // One group per row: MB zero bytes behind the ones, read by the rows past
  // the ones row of that MFMA when the chunk's pairs are read whole (the
  // matrix cores then multiply zeros there).
  static constexpr int ZERO_OFF = ONES_OFF + MB;
  static constexpr int BYTES = ZERO_OFF + (NG == 1 ? MB : 0);
  static constexpr int NKI = (KB + 1023) / 1024;  // 16-byte-lane DMA instructions for K
  static constexpr int NVI = (VB + 1023) / 1024;
  static constexpr int NMI = (MB + 255) / 256;    // dword-lane DMA instructions per tensor
  static constexpr int NINSTR = NKI + NVI + 4 * NMI;
  static_assert(KB % 512 == 0 && VB % 512 == 0 && MB % 64 == 0, "chunk sizes");

  // Staged K/V code layout: blocks of 16 tokens, each block [unit][token]:
  // 16-byte unit u of token t sits at position
  //   (t / 16) * 16 * NU + 16 * u + (t + 4u) % 16    (NU = DP / 16 units per row)
  // so a block is one contiguous 16 * DP bytes of the cache, and the 16 rows an
  // MFMA tile reads from one unit are 16 consecutive 16-byte entries.  The
  // token rotation by 4 per unit puts the same token's consecutive units 320
  // bytes apart instead of 256 (one full bank cycle), so V operand reads of
  // two units no longer land on the same banks (LDS bank-conflict cycles
  // 11% -> 7% of the 4-bit kernel's time).
  template <int DP>
  __device__ static constexpr int pos_of(int t, int u) {
    return (t >> 4) * 16 * (DP / 16) + 16 * u + ((t + 4 * u) & 15);
  }
  template <int DP>
  __device__ static constexpr int token_of(int pos) {
    return 16 * (pos / (16 * (DP / 16))) +
           (((pos & 15) - 4 * ((pos % (16 * (DP / 16))) >> 4)) & 15);
  }
  template <int DP>
  __device__ static constexpr int unit_of(int pos) {
    return (pos % (16 * (DP / 16))) >> 4;
  }
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ lds_ptr_t to_lds(void* p) {
  return (lds_ptr_t)(uintptr_t)(uint32_t)(uintptr_t)p;
}

// Direct-to-LDS buffer loads of 16 / 4 bytes per lane (lane L writes
// lds + L * size).  Plain functions per cache policy: the builtin is device-only.
__device__ __forceinline__ void dma16_default(rsrc_t r, lds_ptr_t lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, off, 0, 0, kPolicyDefault);
}
__device__ __forceinline__ void dma16_nt(rsrc_t r, lds_ptr_t lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, off, 0, 0, kPolicyNT);
}
__device__ __forceinline__ void dma4_default(rsrc_t r, lds_ptr_t lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 4, off, 0, 0, kPolicyDefault);
}
__device__ __forceinline__ void dma4_nt(rsrc_t r, lds_ptr_t lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 4, off, 0, 0, kPolicyNT);
}
// 2 bytes per lane, zero-extended into a dword at lds + 4 * L.
__device__ __forceinline__ void dma2_default(rsrc_t r, lds_ptr_t lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 2, off, 0, 0, kPolicyDefault);
}
__device__ __forceinline__ void dma2_nt(rsrc_t r, lds_ptr_t lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 2, off, 0, 0, kPolicyNT);
}
template <int POL>
__device__ __forceinline__ void dma16(rsrc_t r, lds_ptr_t lds, uint32_t off) {
  if constexpr (POL == kPolicyNT) dma16_nt(r, lds, off);
  else dma16_default(r, lds, off);
}
template <int POL>
__device__ __forceinline__ void dma4(rsrc_t r, lds_ptr_t lds, uint32_t off) {
  if constexpr (POL == kPolicyNT) dma4_nt(r, lds, off);
  else dma4_default(r, lds, off);
}
template <int POL>
__device__ __forceinline__ void dma2(rsrc_t r, lds_ptr_t lds, uint32_t off) {
  if constexpr (POL == kPolicyNT) dma2_nt(r, lds, off);
  else dma2_default(r, lds, off);
}

// f(std::integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// vmcnt-only wait (gfx9 encoding: vmcnt[3:0] | expcnt 7 | lgkmcnt 15 | vmcnt[5:4]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
}

// Issue the DMA of one chunk into a stage.  `valid` false turns every lane's
// offset out of the buffer range, so the instructions still retire (keeping
// the vmcnt arithmetic static) but read nothing and write zeros.  `pairs`
// (wave-uniform; one group per row only): the chunk ends before the split's
// last token, and its metadata rows go in as whole dwords (StageGeom::MROW_PAIRS).
template <int D, int KNB, int VNB, int GS, bool KCH = false>
__device__ __forceinline__ void issue_chunk(uint8_t* stage, const rsrc_t& rk, const rsrc_t& rv,
                                            const rsrc_t (&rm)[4], int cb, bool valid, int lane,
                                            bool pairs) {
  // cb: index, within the resources, of the chunk's first row
  using SG = StageGeom<D, KNB, VNB, GS>;
  using KL = typename SG::KL;
  using VL = typename SG::VL;
  constexpr uint32_t kOut = 0x80000000u;
  // K / V: instruction q copies the contiguous kilobyte [1024q, 1024q + 1024)
  // of the chunk (whole lines).  Lane L takes the 16-byte unit that belongs at
  // stage position 64q + L of the layout described at the top of this kernel.
#pragma unroll
  for (int q = 0; q < SG::NKI; ++q) {
    const int t = SG::template token_of<KL::DP>(64 * q + lane);
    const int u = SG::template unit_of<KL::DP>(64 * q + lane);
    const uint32_t off = valid ? (uint32_t)(cb + t) * KL::DP + 16 * u : kOut;
    if (SG::KB >= 1024 || lane < SG::KB / 16)
      dma16<kPolDma>(rk, to_lds(stage + SG::K_OFF + 1024 * q), off);
  }
#pragma unroll
  for (int q = 0; q < SG::NVI; ++q) {
    const int t = SG::template token_of<VL::DP>(64 * q + lane);
    const int u = SG::template unit_of<VL::DP>(64 * q + lane);
    const uint32_t off = valid ? (uint32_t)(cb + t) * VL::DP + 16 * u : kOut;
    if (SG::VB >= 1024 || lane < SG::VB / 16)
      dma16<kPolDma>(rv, to_lds(stage + SG::V_OFF + 1024 * q), off);
  }
  // metadata: the chunk's [t][g] rows are contiguous; lane L copies dword L
  // (NG == 1: below).  Per-channel keys: the K
  // scale and zero tensors hold one row of D fp16 per 32-token block, the
  // chunk's block; its 2D bytes go to the front of the tensor's MB bytes
  // (MB >= 2D for the group sizes that allow them); further instructions read
  // nothing, keeping the instruction count of the vmcnt arithmetic.
  if constexpr (SG::NG == 1 && !KCH) {
    // One branch for the four tensors (one instruction each either way: the
    // vmcnt arithmetic counts instructions).
    if (pairs) {
      const uint32_t off = valid ? (uint32_t)(cb + 2 * lane) * 2 : kOut;
      if (lane < kChunk / 2) {
#pragma unroll
        for (int tsr = 0; tsr < 4; ++tsr) dma4<kPolDma>(rm[tsr], to_lds(stage + SG::M_OFF + tsr * SG::MB), off);
      }
    } else {
      const uint32_t off = valid ? (uint32_t)(cb + lane) * 2 : kOut;
      if (lane < kChunk) {
#pragma unroll
        for (int tsr = 0; tsr < 4; ++tsr) dma2<kPolDma>(rm[tsr], to_lds(stage + SG::M_OFF + tsr * SG::MB), off);
      }
    }
    return;
  }
#pragma unroll
  for (int tsr = 0; tsr < 4; ++tsr)
#pragma unroll
    for (int q = 0; q < SG::NMI; ++q) {
      uint8_t* dst = stage + SG::M_OFF + tsr * SG::MB + 256 * q;
      if (KCH && tsr < 2) {
        static_assert(!KCH || SG::MB >= 2 * D, "per-channel key row must fit the K metadata slot");
        const uint32_t off = valid && q == 0 ? (uint32_t)(cb / kChunk) * D * 2 + 4 * lane : kOut;
        if (lane < D / 2) dma4<kPolDma>(rm[tsr], to_lds(dst), off);
      } else {
        const uint32_t off = valid ? (uint32_t)cb * SG::NG * 2 + 4 * (64 * q + lane) : kOut;
        if (SG::MB >= 256 || lane < SG::MB / 4) dma4<kPolDma>(rm[tsr], to_lds(dst), off);
      }
    }
}

// ---------------------------------------------------------------------------
// Paired tiles, for GQA groups of at most 8 query heads.
//
// A 16x16 MFMA has 16 columns.  With G <= 8 heads per group, half or more of
// them would carry padding heads, and every per-score instruction after the
// score MFMAs (scale fold, softmax, exponentials) would spend that share of its
// lanes on them.  Instead the two 16-token tiles of a chunk share one set of
// MFMAs: column c = 8 * tile + head, and the K dimension is split between the
// tiles (a block-diagonal B operand): lane groups j = 0, 1 carry tile 0's
// codes, j = 2, 3 tile 1's, and their B entries hold q for columns of their
// own tile and zero for the other.  Each MFMA covers 16 dims of both tiles
// (D / 16 MFMAs, as many as two tiles x D / 32), and each lane ends up with
// the 4 scores of one tile for one head: half the fold and softmax work.
// The PV product keeps its layout: lane (j, c < 8) needs the probabilities of
// head c for both tiles, which are its own and those of lane c + 8.
// ---------------------------------------------------------------------------
template <int D, int KNB, int GS>
struct QOperandsPT {
  static constexpr int P = 8 / KNB;
  static constexpr int DP = D / P;
  static constexpr int NU = DP / 16;  // 16-byte units per packed row
  static constexpr int NB = D / 16;   // 16-dim blocks: block p * NU + u = unit u of slice p
  u4 qb[NB];
  u4 qzb;  // zero-point MFMA (K = 32): slots 8j + g hold hi (j even) or lo (j odd) of sum q_g
  float qsum;  // one group per row: sum q of this lane's head (its zero term by one FMA per score)
  int eh;  // this lane's head's prescale exponent (as QOperands::eh)
};

// Column col carries head (col & 7) % HC of tile col >> 3 (HC = 8, or 4 when
// the PV products give every head several columns).
template <int D, int KNB, int GS, int HC>
__device__ __forceinline__ void load_q_operands_pt(const SplitParams& prm, int b, int h0, int col,
                                                   int nh, int j, QOperandsPT<D, KNB, GS>& qo) {
  using QO = QOperandsPT<D, KNB, GS>;
  constexpr int NG = D / GS;
  static_assert(HC == 8 || HC == 4, "head columns per tile");
  // q stays in fp16 pairs, as in load_q_operands: integer max of the
  // magnitude bits, one packed prescale multiply per operand dword, and the
  // other tile's k-slots (and heads past nh) cleared with one AND.
  const int h = col & (HC - 1);
  const bool hv = h < nh;
  const bool own = (col >> 3) == (j >> 1);  // these k-slots belong to this column's tile
  const uint32_t hvm = hv ? 0xFFFFFFFFu : 0u;
  const uint32_t opm = (hv && own) ? 0xFFFFFFFFu : 0u;
  const int64_t qrow = ((int64_t)b * prm.HQ + h0 + (hv ? h : 0)) * D;
  // natural-order pairs of the lane's 8 dims of block bi: dims
  // (bi / NU) * DP + 16 * (bi % NU) + 8 * (j & 1) .. + 7
  uint32_t qh[QO::NB][4];
  if (prm.q_fp32) {
    const float* qp = static_cast<const float*>(prm.q) + qrow + 8 * (j & 1);
#pragma unroll
    for (int bi = 0; bi < QO::NB; ++bi) {
      const int d0 = (bi / QO::NU) * QO::DP + 16 * (bi % QO::NU);
      const f4 a = *reinterpret_cast<const f4*>(qp + d0);
      const f4 c = *reinterpret_cast<const f4*>(qp + d0 + 4);
      qh[bi][0] = pack_h2(a[0], a[1]);
      qh[bi][1] = pack_h2(a[2], a[3]);
      qh[bi][2] = pack_h2(c[0], c[1]);
      qh[bi][3] = pack_h2(c[2], c[3]);
    }
  } else {
    const _Float16* qp = static_cast<const _Float16*>(prm.q) + qrow + 8 * (j & 1);
#pragma unroll
    for (int bi = 0; bi < QO::NB; ++bi) {
      const int d0 = (bi / QO::NU) * QO::DP + 16 * (bi % QO::NU);
      const u4 v = *reinterpret_cast<const u4*>(qp + d0);
#pragma unroll
      for (int e = 0; e < 4; ++e) qh[bi][e] = v[e];
    }
  }
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  us2 mag = us2{0, 0};
#pragma unroll
  for (int bi = 0; bi < QO::NB; ++bi)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      mag = __builtin_elementwise_max(mag, __builtin_bit_cast(us2, qh[bi][e] & 0x7FFF7FFFu));
  const uint32_t mbits = mag[0] > mag[1] ? mag[0] : mag[1];
  const float amax = hv ? (float)__builtin_bit_cast(_Float16, (unsigned short)mbits) : 0.0f;
  // lanes j and j ^ 1 hold the two halves of each 16-dim block of the head
  qo.eh = q_prescale_exp(max_xor16(amax), (QO::P - 1) * KNB);
  float qz[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) qz[g] = 0.0f;
  const h2 ones = h2{(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
  for (int p = 0; p < QO::P; ++p) {
    // 2^(eh - p * KNB) as an fp16 pair (a normal number: eh >= -1, p * KNB <= 6)
    const uint32_t pe = (uint32_t)(qo.eh - p * KNB + 15) << 10;
    const uint32_t pre = pe | (pe << 16);
#pragma unroll
    for (int u = 0; u < QO::NU; ++u) {
      const int bi = p * QO::NU + u;
      const int g = (p * QO::DP + 16 * u) / GS;
      // slot order: pairs of dims (0,2) (1,3) (4,6) (5,7)
      const uint32_t sl[4] = {perm(qh[bi][1], qh[bi][0], 0x05040100u), perm(qh[bi][1], qh[bi][0], 0x07060302u),
                              perm(qh[bi][3], qh[bi][2], 0x05040100u), perm(qh[bi][3], qh[bi][2], 0x07060302u)};
      qo.qb[bi] = u4{pk_mul(sl[0], pre) & opm, pk_mul(sl[1], pre) & opm, pk_mul(sl[2], pre) & opm,
                     pk_mul(sl[3], pre) & opm};
      float zs = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        zs = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qh[bi][e] & hvm), ones, zs, false);
      qz[g] += zs;
    }
  }
  // lanes j and j ^ 1 hold the two halves of every 16-dim block (j ^ 2 repeats them)
#pragma unroll
  for (int g = 0; g < NG; ++g) qz[g] = sum_xor16(qz[g]);
  float hl[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    float v = 0.0f;
    if (g < NG && own) {
      const float hi16 = (float)(_Float16)qz[g < NG ? g : 0];
      v = (j & 1) ? qz[g < NG ? g : 0] - hi16 : hi16;
    }
    hl[g] = v;
  }
  qo.qzb = u4{pack_h2(hl[0], hl[1]), pack_h2(hl[2], hl[3]), pack_h2(hl[4], hl[5]),
              pack_h2(hl[6], hl[7])};
  qo.qsum = qz[0];
}

// Online-softmax step of a paired-tile chunk: 4 scores per lane (one tile, one
// head); the head's 32 tokens span lanes c and c ^ 8 of all four lane groups.
// Returns whether any running max moved; ph holds the lane's fp16 pairs.
// As softmax_chunk: the lane's own max decides whether any head moved, and
// the cross-lane max runs only when one did.
__device__ __forceinline__ bool softmax_chunk_pt(const float (&x)[4], float lscale, float& m,
                                                 float& alpha, uint32_t (&ph)[2], float (&p)[4]) {
  const float lm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])) * lscale;  // this lane's max
  const bool any_moved = __builtin_amdgcn_ballot_w64(lm > m) != 0;
  alpha = 1.0f;
  if (any_moved) {
    const float mn = vmax(m, xor_max16_32(vmax(lm, lane_xor8(lm))));
    alpha = safe_exp2_diff(m, mn);
    m = mn;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(x[i], lscale, -m));
  ph[0] = pack_h2(p[0], p[1]);
  ph[1] = pack_h2(p[2], p[3]);
  return any_moved;
}

template <int D, int KNB, int VNB, int GS, int NW, int NSTAGE>
struct LdsKernelSmem {
  using SG = StageGeom<D, KNB, VNB, GS>;
  static constexpr int RING = NSTAGE * SG::BYTES;
  // After the loop the ring holds the wave's partial (and, in wave 0, the
  // workgroup's combine ticket flag right behind it).
  static constexpr int OUT = (int)sizeof(WavePartial<D>) + 16;
  static constexpr int WAVE = ((RING > OUT ? RING : OUT) + 15) / 16 * 16;
  // Fused append: the new token's row in staged form (K bytes, V bytes, then
  // the fp16 scale/zero of K and V, NG each), behind the waves' rings.
  static constexpr int PATCH_META = SG::KL::DP + SG::VL::DP;
  static constexpr int PATCH = (PATCH_META + 4 * SG::NG * 2 + 15) / 16 * 16;
  // Unpaired tiles: the q operands one wave builds for the workgroup (qf, qn,
  // qzb, eh: 8 * NKM + 3 dwords per lane), behind the patch.
  static constexpr int QOP = (8 * SG::KL::NKM + 3) * 4 * 64;
};

// 12-wave workgroups: three waves per SIMD (VGPRs <= 168) in one workgroup
// per CU, for the formats whose kernel is bound by issue rather than by its
// loads (more waves to interleave), measured at the Llama-3-8B shape (one
// workgroup per CU, 32768 tokens each): 2-bit gs32 -7%, per-channel 2-bit
// keys -5%, 2-bit gs128 -4%, 4-bit gs128 -3%, while 4-bit gs32 (at the read
// pattern's ceiling) was 1% slower.  Only formats whose 12-wave kernels
// compile without spills are listed (several others spill at 168 VGPRs); the
// workgroup's rings, patch and shared q operands must also fit the 160 KB of
// LDS.  A 12-wave request for any other kernel runs 8 waves.
template <int D, int KNB, int VNB, int GS, int HS, bool PT>
constexpr bool kTwelveWaves =
    D == 128 &&
    ((KNB == 2 && VNB == 2 && GS == 32 && HS == 4) || (KNB == VNB && GS == 128)) &&
    12 * LdsKernelSmem<D, KNB, VNB, GS, 12, 2>::WAVE + LdsKernelSmem<D, KNB, VNB, GS, 12, 2>::PATCH +
            (PT ? 0 : LdsKernelSmem<D, KNB, VNB, GS, 12, 2>::QOP) <= 160 * 1024;

// Probabilities enter the PV products as fp16 (B operands of the MFMAs), as
// they do in the reference's tl.dot.  Their rounding reaches the output as
// about 2^-11 * |v| / sqrt(L) for a row of L tokens, whichever chunk it falls
// in, so rows of at most kHiLoMaxLen tokens take them as hi/lo fp16 pairs in
// every chunk -- P = pb + pbl and P * s_g = pg + pgl to about 22 bits, one
// more MFMA per product.  Measured with x8 outliers (2-bit codes): 33 tokens
// 2.1e-3 -> 1.5e-4 max-abs; 2-5 tokens up to 2^-10 * max|v| -> 5e-5.  Longer
// rows keep fp16 P: at 256 tokens the estimate is already about 8e-4 at the
// same values, and the pairs cost 0.15-0.4 us per latency-bound Qwen-shape
// step and 9-18% at the DRAM-bound Llama-3-8B shape.
constexpr int kHiLoMaxLen = 256;

// Longer rows keep fp16 P, but the products P * s_g can be carried with their
// exact remainders (one pk_fma per pair and one more MFMA per V product).
// The rounding of an fp16 P * s reaches the output as up to 2^-12 * |c * s|
// per token, and |c * s| spans the V group's whole range: with 2-bit codes
// and 128-dim groups (one group per row, so every group holds a key's
// outlier channels) that range is largest.  Measured on the Llama-3-8B shape
// with x8 outlier channels, whole batch against the binary64-sum oracle:
// 2.07e-3 max-abs with fp16 P * s, 1.42e-3 with the remainders (for 7% more
// time: 118.6 -> 126.9 us); 2-bit gs32 is 0.98e-3 without them.
template <int VNB, int NG>
constexpr bool kPsRemainder = VNB == 2 && NG == 1;


// Dims split (VS workgroups per output row): part `part` computes the V
// MFMAs [part * NVM / VS, (part + 1) * NVM / VS), whole (slice, window) blocks
// of NE MFMAs in (slice, window) order, i.e. the dims [part * D / VS,
// (part + 1) * D / VS).  Whether V MFMA mv, window wi, and P' operand v (of
// S-slot head columns) are used by that part.
template <class VL, int VS>
__device__ constexpr bool v_mfma_in_part(int mv, int part) {
  return mv / (VL::NVM / VS) == part;
}
template <class VL, int VS>
__device__ constexpr bool v_window_in_part(int wi, int part) {
  for (int p = 0; p < VL::P; ++p)
    for (int e = 0; e < VL::NE; ++e)
      if (v_mfma_in_part<VL, VS>(VL::mfma_index(p, wi, e), part)) return true;
  return false;
}
template <class VL, int VS, int S>
__device__ constexpr bool v_operand_in_part(int v, int part) {
  for (int mv = 0; mv < VL::NVM; ++mv)
    if (v_mfma_in_part<VL, VS>(mv, part) && VL::group_of(mv) / S == v) return true;
  return false;
}

// ORD: the launch carries a dispatch order (prm.order).  A separate
// instantiation, because a run-time test of the pointer ahead of everything
// else made the compiler fetch the cache pointers in a second, serial round
// trip to the argument block: 0.1-0.3 us on every Qwen2.5-1.5B-shape call.
//
// SMALL (with VS > 1): the grid holds fewer than 8 (unit, split, head block)
// tuples and takes the small-grid layout below.  A separate instantiation:
// a run-time choice of layout ahead of the first DMA cost 0.2-0.25 us on
// every cold Qwen2.5-1.5B-shape step that did not take it.
//
// VS: workgroups that share one (unit, split, block of heads) by splitting
// the head dim of the output.  Workgroup z % VS computes every score (the K
// side, the softmax) but only the V products, the partial and the merge of
// dims [part * D / VS, (part + 1) * D / VS): less work per chunk and VS times
// the workgroups when a launch has far fewer workgroups than the GPU has CUs.
template <int D, int KNB, int VNB, int GS, int NW, int NSTAGE, bool PAGED, bool PT, bool KCH, int HS,
          bool ORD, int VS, bool SMALL>
__global__ void __launch_bounds__(NW * 64)
quant_split_lds_kernel(SplitParams prm) {
  using SG = StageGeom<D, KNB, VNB, GS>;
  using KL = typename SG::KL;
  using VL = typename SG::VL;
  using SM = LdsKernelSmem<D, KNB, VNB, GS, NW, NSTAGE>;
  constexpr int NG = SG::NG;
  constexpr int NKM = KL::NKM;
  constexpr int NVM = VL::NVM;
  constexpr int NI = SG::NINSTR;
  static_assert(2 * NG <= 16, "zero-point MFMA holds hi/lo of at most 8 groups");
  static_assert((NSTAGE - 1) * NI < 64, "vmcnt range");
  static_assert(!KCH || (!PAGED && !PT && GS <= 32), "per-channel keys: contiguous, one-tile path");
  // Head columns of the PV products.  Column c of every PV MFMA carries query
  // head c % HS.  With HS < 16 (GQA groups of at most HS heads) the 16 / HS
  // copies of a head take different V groups: column c holds P * s_g for
  // group g = v * S + c / HS in the v-th of NPG P' operands, so one packed
  // multiply per token pair serves S groups where it used to serve one (the
  // other columns carried padding heads).  A V MFMA over dims of group g then
  // accumulates the true products in the columns of slot g % S only, and
  // those are the ones written out.
  static_assert(HS == 16 || (HS == 8 || HS == 4), "head columns");
  static_assert(HS == 16 || NG >= 2, "one V group: nothing to share");
  constexpr int S = 16 / HS;             // V-group slots per head
  constexpr int NPG = (NG + S - 1) / S;  // P' operands per chunk

  __shared__ __attribute__((aligned(16))) uint8_t smem[NW * SM::WAVE + SM::PATCH + (PT ? 0 : SM::QOP)];

  // x fastest: consecutive workgroups (which the dispatcher deals to the 8 XCDs
  // in turn) take other units.  A ragged batch may pass a longest-first order.
  int unit_ = blockIdx.x, split_ = blockIdx.y, hb_ = blockIdx.z, part_ = 0, L_ = 0;
  if constexpr (ORD) {
    const int2 e = reinterpret_cast<const int2*>(prm.order)[blockIdx.y * gridDim.x + blockIdx.x];
    unit_ = e.x % (int)gridDim.x;
    split_ = e.x / (int)gridDim.x;
    L_ = e.y;
  }
  if constexpr (VS > 1) {
    // Dims split.  The parts of one (unit, split, head block) tuple run on one
    // XCD, whose L2 then serves the rows they all load: the dispatcher deals
    // workgroups to the 8 XCDs in turn, so parts 8k workgroups apart share one.
    if constexpr (!SMALL) {
      // T >= 8 tuples, T % 8 == 0 in the common cases: z = head block * VS +
      // part, and the parts of a tuple are T workgroups apart.
      part_ = (int)blockIdx.z % VS;
      hb_ = (int)blockIdx.z / VS;
    } else {
      // T < 8 tuples: grid (8 * VS); workgroup x takes part x / 8 of tuple
      // x % 8, and the workgroups past the last tuple leave at once.
      const int units = prm.xcd_units;
      const int tuples = units * prm.num_splits * ((prm.G + 15) / 16);
      const int t = (int)blockIdx.x % 8;
      if (t >= tuples) return;
      part_ = (int)blockIdx.x / 8;
      unit_ = t % units;
      split_ = (t / units) % prm.num_splits;
      hb_ = t / (units * prm.num_splits);
    }
  }
  const int unit = __builtin_amdgcn_readfirstlane(unit_);
  const int split = __builtin_amdgcn_readfirstlane(split_);
  const int b = unit / prm.HKV, hk = unit % prm.HKV;
  const int vpart = __builtin_amdgcn_readfirstlane(part_);  // dims part (VS > 1)
  const int hb0 = __builtin_amdgcn_readfirstlane(hb_) * 16;
  const int nh = min(16, prm.G - hb0);
  const int h0 = hk * prm.G + hb0;
  const int L = ORD ? __builtin_amdgcn_readfirstlane(L_)
                    : (prm.seq_lens ? min(prm.seq_lens[b], prm.S) : prm.S);
  const int lo = split * prm.split_size;
  const int hi = min(lo + prm.split_size, L);
  const int last = hi - 1;

  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r = lane & 15, j = lane >> 4;
  const int n = r;
  const int slot = r / HS;  // V-group slot of this lane's column
  // An empty split (a row of a ragged batch that ends before the split
  // starts) writes the empty partial -- max -inf, sum 0, output 0 -- and
  // leaves, with no q operands, DMA or merge.  With counters (the
  // last-workgroup merge counts every split's ticket) it takes the full path.
  if (lo >= L && prm.ns_total > 1 && prm.counters == nullptr) {
    constexpr int DNV = D / VS;  // this workgroup's dims
    for (int idx = tid; idx < nh * DNV; idx += NW * 64) {
      const int hn = idx / DNV, d = vpart * DNV + idx % DNV;
      const int64_t pr = ((int64_t)b * prm.HQ + h0 + hn) * prm.ns_total + prm.split_base + split;
      prm.acc[pr * D + d] = 0.0f;
      if (d == 0) {
        prm.maxs[pr] = -INFINITY;
        prm.sums[pr] = 0.0f;
      }
    }
    return;
  }
  // Where a chunk's rows live.  Contiguous caches: one buffer resource per
  // tensor over this (b, kv head) block, chunk rows at token index cb.  Paged
  // caches: resources over the (pool page, kv head) slab holding the chunk
  // (chunks never straddle a page: page_size % 32 == 0), rows at cb % page.
  // Either way the hardware range check returns zeros past the resource.
  struct ChunkSrc {
    rsrc_t k, v, m[4];
    int row;
  };
  auto slab_src = [&](int64_t slab, int rows, int row) -> ChunkSrc {
    return ChunkSrc{make_rsrc(prm.k + slab * rows * KL::DP, (uint32_t)rows * KL::DP),
                    make_rsrc(prm.v + slab * rows * VL::DP, (uint32_t)rows * VL::DP),
                    {make_rsrc(prm.ks + slab * rows * NG, (uint32_t)rows * NG * 2),
                     make_rsrc(prm.kz + slab * rows * NG, (uint32_t)rows * NG * 2),
                     make_rsrc(prm.vs + slab * rows * NG, (uint32_t)rows * NG * 2),
                     make_rsrc(prm.vz + slab * rows * NG, (uint32_t)rows * NG * 2)},
                    row};
  };
  ChunkSrc unit_src = slab_src(PAGED ? 0 : (int64_t)unit, PAGED ? prm.page_size : prm.S, 0);
  if constexpr (KCH) {  // K scale / zero: (S/32, D) per (b, kv head)
    const int64_t nblk = prm.S / kChunk;
    unit_src.m[0] = make_rsrc(prm.ks + (int64_t)unit * nblk * D, (uint32_t)(nblk * D * 2));
    unit_src.m[1] = make_rsrc(prm.kz + (int64_t)unit * nblk * D, (uint32_t)(nblk * D * 2));
  }
  auto chunk_src = [&](int cb, int page) -> ChunkSrc {
    if constexpr (PAGED)
      return slab_src((int64_t)page * prm.HKV + hk, prm.page_size,
                      (int)((uint32_t)cb % (uint32_t)prm.page_size));
    else
      return ChunkSrc{unit_src.k, unit_src.v, {unit_src.m[0], unit_src.m[1], unit_src.m[2], unit_src.m[3]}, cb};
  };
  // Paged: block-table entries are read with vector loads, each issued right
  // behind a chunk's DMA for the chunk two steps ahead, so it retires with
  // the next step's wait and no lookup ever stalls the stream.  Entries of
  // chunks at or past the end of the split are never read (their offset is
  // out of range and reads 0), and every entry is clamped into the pool, so a
  // bad entry can only select another page, never leave the pool.
  const rsrc_t rtab = make_rsrc(prm.block_table + (PAGED ? (int64_t)b * prm.bt_stride : 0),
                                PAGED ? (uint32_t)prm.bt_stride * 4u : 0u);
  auto tab_entry = [&](int c) -> uint32_t {
    return buf_u32<kPolicyDefault>(
        rtab, c < hi ? (uint32_t)c / (uint32_t)prm.page_size * 4u : 0x80000000u);
  };
  auto to_page = [&](uint32_t e) -> int {
    return min(max((int)__builtin_amdgcn_readfirstlane(e), 0), prm.num_pages - 1);
  };
  uint8_t* ring = smem + w * SM::WAVE;
#pragma unroll
  for (int s = 0; s < NSTAGE; ++s)
    for (int i = lane; i < SG::MB / 4; i += 64) {
      reinterpret_cast<uint32_t*>(ring + s * SG::BYTES + SG::ONES_OFF)[i] = 0x3C003C00u;
      if constexpr (NG == 1) reinterpret_cast<uint32_t*>(ring + s * SG::BYTES + SG::ZERO_OFF)[i] = 0u;
    }

  // Chunk k of this wave starts at token lo + 32 * (w + NW * k).
  const int cb0 = lo + kChunk * w;
  const int cstride = kChunk * NW;
  static_assert(NSTAGE >= 2 && (!PAGED || NSTAGE == 2), "ring depth");
  // Paged: page_next is the pool page of the chunk whose DMA is issued next;
  // tab_pending the (in-flight) table entry of the chunk after that.
  int page_next = 0;
  uint32_t tab_pending = 0;
  if constexpr (PAGED) {
    const uint32_t e0 = tab_entry(cb0), e1 = tab_entry(cb0 + cstride);
    const int page0 = to_page(e0);
    page_next = to_page(e1);
    const ChunkSrc src = chunk_src(cb0, page0);
    issue_chunk<D, KNB, VNB, GS, KCH>(ring, src.k, src.v, src.m, src.row, cb0 < hi, lane,
                                      cb0 + kChunk < hi);
    tab_pending = tab_entry(cb0 + 2 * cstride);
  } else {
    // the first NSTAGE - 1 chunks into stages 0 .. NSTAGE - 2
    static_for<NSTAGE - 1>([&](auto s) __attribute__((always_inline)) {
      constexpr int SS = decltype(s)::value;
      const int c = cb0 + SS * cstride;
      const ChunkSrc src = chunk_src(c, 0);
      issue_chunk<D, KNB, VNB, GS, KCH>(ring + SS * SG::BYTES, src.k, src.v, src.m, src.row, c < hi, lane,
                                        c + kChunk < hi);
    });
  }


  using QP = QOperandsPT<D, KNB, GS>;
  // Per-lane set-up, ahead of the q operands: the waves that wait for wave 0
  // to build them do it meanwhile.
  uint32_t vsel[VL::NE];
#pragma unroll
  for (int e = 0; e < VL::NE; ++e) vsel[e] = VL::perm_sel(VL::byte_in_dword(e, r));
  uint32_t kmask[NKM];
#pragma unroll
  for (int m = 0; m < NKM; ++m) kmask[m] = slice_mask<KNB>(KL::slice_of(m, j));

  constexpr bool kVChain = NPG == 1;  // every V MFMA takes the same P' operand
  static_assert(!SMALL || VS > 1, "small-grid layout: dims-split kernels only");
  static_assert(VS == 1 || ((VS == 2 || VS == 4) && !PT && !KCH && !PAGED && !ORD && !kVChain &&
                             NVM % (VS * VL::NE) == 0),
                "dims split: unpaired, per-token keys, contiguous, grid order, no slice chain, "
                "whole (slice, window) blocks per part");

  // Per-lane LDS byte offsets inside a stage.
  // K operand of tile a, load Lh: row 16a + r, byte load_offset(Lh, j).
  uint32_t koff[KL::NLOAD];
#pragma unroll
  for (int Lh = 0; Lh < KL::NLOAD; ++Lh) {
    const int ob = KL::load_offset(Lh, j);
    koff[Lh] = SG::K_OFF + SG::template pos_of<KL::DP>(r, ob >> 4) * 16 + (ob & 15);
  }
  // Paired tiles: unit u of token 16 * (j >> 1) + r, bytes 8 * (j & 1) .. + 7.
  uint32_t koffp[QP::NU];
#pragma unroll
  for (int u = 0; u < QP::NU; ++u)
    koffp[u] = SG::K_OFF + SG::template pos_of<KL::DP>(16 * (j >> 1) + r, u) * 16 + 8 * (j & 1);
  const int tile_pt = 16 * (r >> 3);  // paired tiles: the tile of this lane's scores
  // Paired tiles: columns of padding heads (head >= nh; 8 head slots per tile
  // at 16 head columns) carry p = 0 into the PV products, so the matrix cores
  // multiply zeros there instead of a padding head's probabilities of 1
  // (less switching under the power cap: 2-bit gs128 2% faster on one box,
  // 0.5% on another).
  const uint32_t pcol = ((r & ((HS < 8 ? HS : 8) - 1)) < nh) ? 0xFFFFFFFFu : 0u;
  // V operand of slot i, window wi: token slot_token(j, i), dword dword_offset(wi, r).
  uint32_t voff[VL::NWIN];
#pragma unroll
  for (int wi = 0; wi < VL::NWIN; ++wi) {
    const int ob = VL::dword_offset(wi, r);
    voff[wi] = SG::V_OFF + SG::template pos_of<VL::DP>(4 * j, ob >> 4) * 16 + (ob & 15);
  }
  // P' operand v of this lane: the V scales of group v * S + slot (clamped:
  // a slot past the last group computes a copy nobody reads); dword offset of
  // its fp16 pair in a staged [t][MROW] row and the v_perm selector of its half.
  uint32_t soff[NPG], ssel[NPG];
#pragma unroll
  for (int v = 0; v < NPG; ++v) {
    const int g = min(v * S + slot, NG - 1);
    soff[v] = 2 * (g & ~1);
    ssel[v] = (g & 1) ? 0x07060302u : 0x05040100u;
  }
  // A operand of the V zero-point MFMA: row r < NG holds group r's zero
  // points, gathered for two tokens into one fp16 pair with a single v_perm
  // (low or high half of each token's dword); row NG is all ones (fp16 1.0
  // pairs, read from the stage's ones area through the same offsets), so the
  // same MFMA also accumulates sum_t p_t, the softmax denominator, from the
  // very fp16 probabilities the PV products use; rows r > NG are zero (their
  // selector yields constant zero bytes; pairs read whole: the zero area).
  int zoff = r < NG ? 2 * (r & ~1) : (r == NG || NG > 1 ? SG::MB : 2 * SG::MB);
  uint32_t zsel = r < NG ? ((r & 1) ? 0x07060302u : 0x05040100u)
                         : (r == NG ? 0x05040100u : 0x0C0C0C0Cu);
  if constexpr (!PT) {
    // Materialise them here: otherwise the compiler sinks this arithmetic
    // past the barrier below, onto every wave's path to its first chunk.
    auto pin = [](auto& x) __attribute__((always_inline)) { asm volatile("" : "+v"(x)); };
#pragma unroll
    for (int e = 0; e < VL::NE; ++e) pin(vsel[e]);
#pragma unroll
    for (int m = 0; m < NKM; ++m) pin(kmask[m]);
#pragma unroll
    for (int Lh = 0; Lh < KL::NLOAD; ++Lh) pin(koff[Lh]);
#pragma unroll
    for (int wi = 0; wi < VL::NWIN; ++wi) pin(voff[wi]);
#pragma unroll
    for (int v = 0; v < NPG; ++v) {
      pin(soff[v]);
      pin(ssel[v]);
    }
    pin(zoff);
    pin(zsel);
  }

  // q operands: one per MFMA step of a tile, or (paired tiles, G <= 8) one
  // block-diagonal operand per 16-dim block of both tiles.
  QOperands<D, KNB, GS> qo;
  QP qpt;
  // Per-channel keys multiply q by the chunk's channel scales in fp16 (q * s
  // as hi/lo pairs), so their q keeps eh = 0: a larger prescale could
  // overflow there.
  if constexpr (PT) {
    load_q_operands_pt<D, KNB, GS, HS < 8 ? HS : 8>(prm, b, h0, r, nh, j, qpt);
  } else {
    // Every wave of the workgroup serves the same query heads, so wave 0
    // alone builds the q operands and the others read them from LDS: on a
    // short row the build (q loads, then ~300 VALU) would otherwise be
    // repeated by the second wave of every SIMD ahead of its first chunk.
    uint32_t* const qop = reinterpret_cast<uint32_t*>(smem + NW * SM::WAVE + SM::PATCH) + lane;
    constexpr int QN = 4 * NKM;  // dword slots of qn (used by per-channel keys)
    if (w == 0) {
      load_q_operands<D, KNB, GS, KCH ? 0 : (KL::P - 1) * KNB, KCH>(prm, b, h0, n % HS, nh, j, qo);
#pragma unroll
      for (int m = 0; m < NKM; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qop[64 * (4 * m + e)] = qo.qf[m][e];
          if constexpr (KCH) qop[64 * (QN + 4 * m + e)] = qo.qn[m][e];
        }
      qop[64 * (2 * QN)] = qo.qzb[0];
      qop[64 * (2 * QN + 1)] = qo.qzb[1];
      qop[64 * (2 * QN + 2)] = (uint32_t)qo.eh;
    }
    __syncthreads();
    if (w != 0) {
#pragma unroll
      for (int m = 0; m < NKM; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qo.qf[m][e] = qop[64 * (4 * m + e)];
          if constexpr (KCH) qo.qn[m][e] = qop[64 * (QN + 4 * m + e)];
        }
      qo.qzb = u2{qop[64 * (2 * QN)], qop[64 * (2 * QN + 1)]};
      qo.eh = (int)qop[64 * (2 * QN + 2)];
    }
  }
  const int eh = PT ? qpt.eh : qo.eh;
  const float zsc = __builtin_ldexpf(1.0f, eh - 24);  // code-dot units per score unit
  const u4* qf = qo.qf;
  const u2 qzb = qo.qzb;
  // Per-channel keys with replicated head columns (HS < 16): column c carries
  // the hi part of head c % HS's q * s when c & HS is clear, the lo part when
  // it is set, so one MFMA per step serves both and the score of a column is
  // its own sum plus that of column c ^ HS (a DPP row rotation by HS).  qlo
  // is q in the lo columns and zero in the hi ones, so q * s - fp16(qlo * s),
  // one packed multiply and one packed FMA as before, is fp16(q * s) in a hi
  // column and the exact remainder q * s - fp16(q * s) in a lo column.
  constexpr bool KCOL = KCH && HS < 16;
  u4 qlo[KCOL ? NKM : 1];
  if constexpr (KCOL) {
    const bool lo_col = (n & HS) != 0;
#pragma unroll
    for (int m = 0; m < NKM; ++m)
#pragma unroll
      for (int e = 0; e < 4; ++e) qlo[m][e] = lo_col ? qf[m][e] : 0u;
  }
  // ... and when the NR = 16 / HS copies of a head cover the NKM steps
  // (HS = 4 at D = 128, HS = 8 at D = 64), the zero term sum_d z_d q_d takes
  // one MFMA for all steps: copy k = n / HS of column n carries q of step k,
  // A row r the zero points of step r % NR, so lane (j, n), which holds rows
  // 4j..4j+3, finds its step's partial in accumulator k, and row rotations by
  // HS, 2 HS, .. add the copies' partials.
  constexpr int NR = 16 / HS;
  constexpr bool KZ1 = KCOL && KL::CB == 8 && NKM == NR;
  u4 qz1 = u4{0u, 0u, 0u, 0u};
  int zoff1 = 0;
  if constexpr (KZ1) {
#pragma unroll
    for (int m = 0; m < NKM; ++m)
      if (n / HS == m) qz1 = qo.qn[m];
    zoff1 = 2 * ((r % NR) * KL::KSTEP + KL::CB * j);
  }

  // ---- fused append ----------------------------------------------------------
  // The token at L - 1 comes from k_new / v_new.  The wave whose chunk holds it
  // quantizes the row here (quantize_row, the append kernel's own code), keeps
  // the row in the workgroup's patch area and, in the first block of query
  // heads, stores it into the cache.  Once that chunk's DMA has landed the wave
  // overwrites the chunk's row with the patch, so the step never depends on
  // when the store becomes visible to its own loads.
  uint8_t* const patch = smem + NW * SM::WAVE;
  int cb_new = -1;  // first token of the chunk this wave patches, or -1
  int t_new = 0;    // the new token's row within that chunk
  if (prm.k_new && L - 1 >= lo && L - 1 < hi && ((L - 1 - lo) / kChunk) % NW == w) {
    const int tn = L - 1;
    int64_t row = (int64_t)unit * prm.S + tn;
    bool use = true;
    if constexpr (PAGED) {
      const int e = prm.block_table[(int64_t)b * prm.bt_stride + tn / prm.page_size];
      use = e >= 0 && e < prm.num_pages;  // as the append kernel: such a token is not stored
      row = ((int64_t)e * prm.HKV + hk) * prm.page_size + tn % prm.page_size;
    }
    if (use) {
      cb_new = lo + kChunk * ((tn - lo) / kChunk);
      t_new = tn - cb_new;
      const int64_t xoff = (int64_t)unit * D * (prm.new_fp32 ? 4 : 2);
      float xk[KL::P], xv[VL::P];
      load_row_for_quant<D, KNB>(static_cast<const uint8_t*>(prm.k_new) + xoff, prm.new_fp32, lane, xk);
      load_row_for_quant<D, VNB>(static_cast<const uint8_t*>(prm.v_new) + xoff, prm.new_fp32, lane, xv);
      const RowQuant<D, KNB, GS> rk = quantize_row<D, KNB, GS>(xk, lane);
      const RowQuant<D, VNB, GS> rv = quantize_row<D, VNB, GS>(xv, lane);
      uint16_t* pmeta = reinterpret_cast<uint16_t*>(patch + SM::PATCH_META);
      if (lane < KL::DP) patch[lane] = (uint8_t)rk.byte;
      if (lane < VL::DP) patch[KL::DP + lane] = (uint8_t)rv.byte;
      if (lane < NG) {
        pmeta[lane] = (uint16_t)(rk.meta & 0xFFFFu);
        pmeta[NG + lane] = (uint16_t)(rk.meta >> 16);
        pmeta[2 * NG + lane] = (uint16_t)(rv.meta & 0xFFFFu);
        pmeta[3 * NG + lane] = (uint16_t)(rv.meta >> 16);
      }
      if (hb0 == 0 && vpart == 0) {
        if (lane < KL::DP) const_cast<uint8_t*>(prm.k)[row * KL::DP + lane] = (uint8_t)rk.byte;
        if (lane < VL::DP) const_cast<uint8_t*>(prm.v)[row * VL::DP + lane] = (uint8_t)rv.byte;
        if (lane < NG) {
          const_cast<uint16_t*>(prm.ks)[row * NG + lane] = (uint16_t)(rk.meta & 0xFFFFu);
          const_cast<uint16_t*>(prm.kz)[row * NG + lane] = (uint16_t)(rk.meta >> 16);
          const_cast<uint16_t*>(prm.vs)[row * NG + lane] = (uint16_t)(rv.meta & 0xFFFFu);
          const_cast<uint16_t*>(prm.vz)[row * NG + lane] = (uint16_t)(rv.meta >> 16);
        }
      }
    }
  }

  f4 accv[NVM];
#pragma unroll
  for (int mv = 0; mv < NVM; ++mv) accv[mv] = f4{0.f, 0.f, 0.f, 0.f};
  f4 oz = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  // Whether this wave has run a chunk: before its first one the accumulators
  // are zero, and a move of the running max needs no rescale.
  bool live = false;
  float zero_v = 0.0f;  // an opaque zero (see the one-group score fold)
  asm volatile("" : "+v"(zero_v));
  const float lscale = prm.qk_scale * __builtin_ldexpf(1.0f, 24 - eh);  // per lane (its head)

  // In the tail chunk, rows past the sequence hold whatever the cache holds
  // there (possibly NaN/Inf bit patterns in scale/zero): their V scale and
  // zero-point pairs are cleared, since p = 0 alone would not cancel them.
  auto tail_pair_mask = [&](int tok0, int tok1) -> uint32_t {
    return (tok0 <= last ? 0x0000FFFFu : 0u) | (tok1 <= last ? 0xFFFF0000u : 0u);
  };
  auto half_at = [&](const uint8_t* base, int idx) -> uint32_t {  // fp16 bits of element idx
    return *reinterpret_cast<const uint16_t*>(base + 2 * idx);
  };
  // The dword holding element (t, g) of a staged [t][MROW] metadata tensor.
  auto dword_at = [&](const uint8_t* base, int t, int g) -> uint32_t {
    return *reinterpret_cast<const uint32_t*>(base + 2 * (t * SG::MROW + (g & ~1)));
  };

  // Chunk k of the wave uses stage k % NSTAGE; the loop below is unrolled by
  // NSTAGE so every stage offset is a compile-time constant.
  auto step = [&](int cb, auto tail, auto stage, auto pmode, auto part) __attribute__((always_inline)) {
    constexpr bool TAIL = decltype(tail)::value;
    constexpr int SK = decltype(stage)::value;
    constexpr int PART = decltype(part)::value;  // dims part (VS > 1)
    // hi/lo probabilities in the PV products (see kHiLoMaxLen)
    // Precision of the PV products (see kHiLoMaxLen and kPsRemainder): 0 fp16
    // P and P * s; 1 adds the exact remainder of each fp16 product P * s;
    // 2 (HILO) also carries P itself as hi/lo fp16 pairs.
    constexpr int PMODE = decltype(pmode)::value;
    constexpr bool HILO = PMODE == 2;
    constexpr bool PSREM = PMODE >= 1;
    // Paired tiles with 16 head columns (one V group per row: no head columns)
    // leave columns 8-15 without a head of their own (G <= 8).  With the
    // P * s remainders those columns carry them -- column 8 + c the
    // remainders of head c, which lane 8 + c holds anyway (both tiles, in
    // order) -- so one V MFMA per product serves both, and the epilogue adds
    // column 8 + c into column c.
    constexpr bool FOLD = PMODE == 1 && PT && HS == 16;
    // fp16 slots per staged metadata row in this chunk (see StageGeom::MROW)
    constexpr int MR = TAIL ? SG::MROW : SG::MROW_PAIRS;
    // refill the stage consumed by the previous chunk, NSTAGE-1 chunks ahead
    {
      const int cn = cb + (NSTAGE - 1) * cstride;
      wait_lgkmcnt0();  // the previous chunk's LDS reads of that stage are done
      asm volatile("" ::: "memory");
      const bool valid = !TAIL && cn < hi;
      const ChunkSrc src = chunk_src(cn, page_next);
      issue_chunk<D, KNB, VNB, GS, KCH>(ring + ((SK + NSTAGE - 1) % NSTAGE) * SG::BYTES, src.k, src.v,
                                   src.m, src.row, valid, lane, cn + kChunk < hi);
    }
    // Paged: one more vector load in flight, behind the DMA just issued.
    uint32_t tab_new = 0;
    if constexpr (PAGED) tab_new = tab_entry(cb + 3 * cstride);
    wait_vmcnt<(NSTAGE - 1) * NI + (PAGED ? 1 : 0)>();
    asm volatile("" ::: "memory");  // no LDS read of this stage above the wait
    if constexpr (PAGED) {  // retired with the wait above: issued a step ago
      page_next = to_page(tab_pending);
      tab_pending = tab_new;
    }
    // Fused append: the new token is the split's last (L - 1 = hi - 1), so its
    // chunk is always a TAIL step; its row replaces what the DMA read.
    if (TAIL && cb == cb_new) {
      uint8_t* sw = ring + SK * SG::BYTES;
      const uint16_t* pmeta = reinterpret_cast<const uint16_t*>(patch + SM::PATCH_META);
      if (lane < KL::DP)
        sw[SG::K_OFF + SG::template pos_of<KL::DP>(t_new, lane >> 4) * 16 + (lane & 15)] = patch[lane];
      if (lane < VL::DP)
        sw[SG::V_OFF + SG::template pos_of<VL::DP>(t_new, lane >> 4) * 16 + (lane & 15)] =
            patch[KL::DP + lane];
      if (lane < 4 * NG)
        *reinterpret_cast<uint16_t*>(sw + SG::M_OFF + (lane / NG) * SG::MB +
                                     2 * (t_new * SG::MROW + lane % NG)) = pmeta[lane];
    }
    const uint8_t* st = ring + SK * SG::BYTES;
    const uint8_t* mks = st + SG::M_OFF;
    const uint8_t* mkz = mks + SG::MB;
    const uint8_t* mvs = mkz + SG::MB;
    const uint8_t* mvz = mvs + SG::MB;

    u4 pb;  // P^T in the PV MFMA's B layout: lane (j, c) holds tokens slot_token(j, .) of head c
    u4 pbl = u4{0u, 0u, 0u, 0u};  // HILO: the fp16 remainders P - pb, same layout
    if constexpr (PT) {
      // ---- scores: both tiles in one set of MFMAs (paired tiles) ----------
      float x[4];  // tokens 16 * tile + 4j + i of head c & 7, tile = c >> 3
      {
        f4 c[NG];
#pragma unroll
        for (int g = 0; g < NG; ++g) c[g] = f4{0.f, 0.f, 0.f, 0.f};
        u2 kx[QP::NU];
#pragma unroll
        for (int u = 0; u < QP::NU; ++u) kx[u] = *reinterpret_cast<const u2*>(st + koffp[u]);
#pragma unroll
        for (int p = 0; p < QP::P; ++p)
#pragma unroll
          for (int u = 0; u < QP::NU; ++u) {
            const int g = (p * QP::DP + 16 * u) / GS;
            c[g] = mfma_k32(k_extract8(kx[u], slice_mask<KNB>(p)), qpt.qb[p * QP::NU + u], c[g]);
          }
        if constexpr (NG == 1) {
          // One group per row: the zero term z_t * sum q by one FMA per score
          // instead of an MFMA (rows past the sequence get -inf below,
          // whatever their z).
          const float qz = qpt.qsum * zsc;
          if constexpr (MR == 1) {
            // The lane's 4 tokens are consecutive: two fp16 pairs per tensor.
            // z * qz is an FMA with a zero the compiler cannot see (a literal
            // zero would become a separate convert and multiply).
            const int t0 = tile_pt + 4 * j;
            const u2 zz = *reinterpret_cast<const u2*>(mkz + 2 * t0);
            const u2 ss = *reinterpret_cast<const u2*>(mks + 2 * t0);
            x[0] = fma_mix_h<false>(ss[0], c[0][0], fma_mix_h<false>(zz[0], qz, zero_v));
            x[1] = fma_mix_h<true>(ss[0], c[0][1], fma_mix_h<true>(zz[0], qz, zero_v));
            x[2] = fma_mix_h<false>(ss[1], c[0][2], fma_mix_h<false>(zz[1], qz, zero_v));
            x[3] = fma_mix_h<true>(ss[1], c[0][3], fma_mix_h<true>(zz[1], qz, zero_v));
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int t = tile_pt + 4 * j + i;
              const float zv = (float)__builtin_bit_cast(_Float16, (uint16_t)half_at(mkz, t * MR));
              const float sv = (float)__builtin_bit_cast(_Float16, (uint16_t)half_at(mks, t * MR));
              x[i] = fmaf(sv, c[0][i], zv * qz);
            }
          }
        } else {
        // zero-point part: A row = token 16 * (j >> 1) + r, k-slots 8j + g = its zero points
        u4 za;
        {
          const uint8_t* zrow = mkz + (16 * (j >> 1) + r) * MR * 2;
          if constexpr (NG == 8) {
            za = *reinterpret_cast<const u4*>(zrow);
          } else if constexpr (NG == 4) {
            const u2 z4 = *reinterpret_cast<const u2*>(zrow);
            za = u4{z4[0], z4[1], 0u, 0u};
          } else if constexpr (NG == 2) {
            za = u4{*reinterpret_cast<const uint32_t*>(zrow), 0u, 0u, 0u};
          } else {
            za = u4{(uint32_t)*reinterpret_cast<const uint16_t*>(zrow), 0u, 0u, 0u};
          }
          // A row r mixes both tiles' token r, and 0 * NaN is NaN: zero points of
          // rows past the sequence (whatever the cache holds there) are cleared
          // so they cannot reach the other tile's columns.
          if constexpr (TAIL)
            if (cb + 16 * (j >> 1) + r > last) za = u4{0u, 0u, 0u, 0u};
        }
        const f4 yz = mfma_k32(za, qpt.qzb, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = tile_pt + 4 * j + i;
          float sc = yz[i] * zsc;
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const float sv =
                (float)__builtin_bit_cast(_Float16, (uint16_t)half_at(mks, t * MR + g));
            sc = fmaf(sv, c[g][i], sc);
          }
          x[i] = sc;
        }
        }  // NG > 1
      }
      if constexpr (TAIL) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (cb + tile_pt + 4 * j + i > last) x[i] = -INFINITY;
      }
      // ---- online softmax ---------------------------------------------------
      float alpha;
      uint32_t ph[2];
      float pf[4];
      if (softmax_chunk_pt(x, lscale, m_run, alpha, ph, pf) && live) {
#pragma unroll
        for (int mv = 0; mv < NVM; ++mv)
          if (v_mfma_in_part<VL, VS>(mv, PART)) accv[mv] *= alpha;
        oz *= alpha;

      }
      // The PV operand of column c needs tile 0 then tile 1 of head c % HS:
      // lane c holds tile c >> 3 of it and lane c ^ 8 the other tile.  (With
      // HS = 16 the columns c >= 8 are padding heads and take any order.)
      const bool swap = (HS < 16 || FOLD) && r >= 8;
      auto tiles = [&](uint32_t a0, uint32_t a1) -> u4 {
        const uint32_t o0 = lane_xor8(a0), o1 = lane_xor8(a1);
        return swap ? u4{o0, o1, a0, a1} : u4{a0, a1, o0, o1};
      };
      pb = tiles(ph[0] & pcol, ph[1] & pcol);
      if constexpr (HILO)
        pbl = tiles(pack_h2_rem(pf[0], pf[1], ph[0]) & pcol, pack_h2_rem(pf[2], pf[3], ph[1]) & pcol);
    } else {
      // ---- scores S^T for the two 16-token tiles ---------------------------
      float x[8];
      float kbias = 0.0f;  // KCOL: the chunk's zero term in logit units
      if constexpr (KCH) {
        // Per-channel keys: score = sum_d (q_d s_d) c_d + sum_d q_d z_d with
        // the chunk's (block's) scale and zero of channel d.  The B operands
        // become q * s for the chunk, in the slot order of qf, as two fp16
        // parts: hi = fp16(q s) and lo = q s - hi, exact by one fused
        // multiply-add (the error of an fp16 product is an fp16 number), so
        // the products see q s to about 22 bits -- a single fp16 product
        // alone put the scores of keys with large channels off by up to
        // 2^-12 of each term.  Two MFMAs per step, or one with the parts in
        // separate head columns (KCOL).
        u4 qs[NKM], ql[KCOL ? 1 : NKM];
        f4 cz = f4{0.f, 0.f, 0.f, 0.f};  // the zero term, in every token row of head n
#pragma unroll
        for (int m = 0; m < NKM; ++m) {
          const int d0 = m * KL::KSTEP + KL::CB * j;
          u4 sn, zn;
          if constexpr (KL::CB == 8) {
            sn = *reinterpret_cast<const u4*>(mks + 2 * d0);
            zn = *reinterpret_cast<const u4*>(mkz + 2 * d0);
          } else {
            const u2 s2 = *reinterpret_cast<const u2*>(mks + 2 * d0);
            const u2 z2 = *reinterpret_cast<const u2*>(mkz + 2 * d0);
            sn = u4{s2[0], s2[1], 0u, 0u};
            zn = u4{z2[0], z2[1], 0u, 0u};
          }
          // natural order, as qf and the codes of this path
          const uint32_t ss[4] = {sn[0], sn[1], sn[2], sn[3]};
          if constexpr (KCOL) {
            // hi columns: fp16(q s) - 0; lo columns: q s - fp16(q s), exact
#pragma unroll
            for (int e = 0; e < 4; ++e)
              qs[m][e] = (KL::CB == 8 || e < 2) ? pk_fma_rem(qf[m][e], ss[e], pk_mul(qlo[m][e], ss[e])) : 0u;
          } else {
            qs[m] = u4{pk_mul(qf[m][0], ss[0]), pk_mul(qf[m][1], ss[1]),
                       KL::CB == 8 ? pk_mul(qf[m][2], ss[2]) : 0u,
                       KL::CB == 8 ? pk_mul(qf[m][3], ss[3]) : 0u};
            ql[m] = u4{pk_fma_rem(qf[m][0], ss[0], qs[m][0]), pk_fma_rem(qf[m][1], ss[1], qs[m][1]),
                       KL::CB == 8 ? pk_fma_rem(qf[m][2], ss[2], qs[m][2]) : 0u,
                       KL::CB == 8 ? pk_fma_rem(qf[m][3], ss[3], qs[m][3]) : 0u};
          }
          // zero term by MFMA: every A row is the step's zero points (natural
          // order), B is q of the same dims (natural order, unscaled), so each
          // output row holds sum_d z_d q_{n,d} over the step: exact fp16
          // products, fp32 sums, no cross-lane reduction.
          if constexpr (KZ1) {
          } else if constexpr (KL::CB == 8) {
            cz = mfma_k32(zn, qo.qn[m], cz);
          } else {
            cz = mfma_k16(u2{zn[0], zn[1]}, u2{qo.qn[m][0], qo.qn[m][1]}, cz);
          }
        }
        float zt = cz[0];
        if constexpr (KZ1) {
          cz = mfma_k32(*reinterpret_cast<const u4*>(mkz + zoff1), qz1, cz);
          // accumulator k = n / HS by selects (a chain of equality tests
          // became divergent branches)
          const int k = n / HS;
          const float t0 = (k & 1) ? cz[1] : cz[0];
          const float t1 = (k & 1) ? cz[3] : cz[2];
          zt = (NR == 4 && (k & 2)) ? t1 : t0;
          if constexpr (NR == 4) zt += lane_ror<4>(zt);
          zt += lane_ror<8>(zt);
        }
        // KCOL: the zero term enters the softmax as a logit offset
        const float bias24 = zt * (KCOL ? zsc * lscale : zsc);
        if constexpr (KCOL) kbias = bias24;
  #pragma unroll
        for (int a = 0; a < 2; ++a) {
          f4 c = f4{0.f, 0.f, 0.f, 0.f};
          typename std::conditional<KL::CB == 8, u2, uint32_t>::type kx[KL::NLOAD];
  #pragma unroll
          for (int Lh = 0; Lh < KL::NLOAD; ++Lh) {
            constexpr int kTile = 16 * (KL::DP / 16) * 16;
            if constexpr (KL::CB == 8) kx[Lh] = *reinterpret_cast<const u2*>(st + koff[Lh] + kTile * a);
            else kx[Lh] = *reinterpret_cast<const uint32_t*>(st + koff[Lh] + kTile * a);
          }
  #pragma unroll
          for (int m = 0; m < NKM; ++m) {
            if constexpr (KL::CB == 8) {
              const u4 a8 = k_extract8_nat(kx[KL::load_of_step(m)], kmask[m]);
              c = mfma_k32(a8, qs[m], c);
              if constexpr (!KCOL) c = mfma_k32(a8, ql[m], c);
            } else {
              const u2 a4 = k_extract4_nat(kx[KL::load_of_step(m)], kmask[m]);
              c = mfma_k16(a4, u2{qs[m][0], qs[m][1]}, c);
              if constexpr (!KCOL) c = mfma_k16(a4, u2{ql[m][0], ql[m][1]}, c);
            }
          }
  #pragma unroll
          for (int i = 0; i < 4; ++i)
            x[4 * a + i] = KCOL ? c[i] + lane_ror<HS < 16 ? HS : 8>(c[i]) : c[i] + bias24;
        }
      } else {
  #pragma unroll
      for (int a = 0; a < 2; ++a) {
        f4 c[NG];
  #pragma unroll
        for (int g = 0; g < NG; ++g) c[g] = f4{0.f, 0.f, 0.f, 0.f};
        typename std::conditional<KL::CB == 8, u2, uint32_t>::type kx[KL::NLOAD];
  #pragma unroll
        for (int Lh = 0; Lh < KL::NLOAD; ++Lh) {
          // tile a = rows 16a.. = block a: 16 * NU entries further
          constexpr int kTile = 16 * (KL::DP / 16) * 16;
          if constexpr (KL::CB == 8) kx[Lh] = *reinterpret_cast<const u2*>(st + koff[Lh] + kTile * a);
          else kx[Lh] = *reinterpret_cast<const uint32_t*>(st + koff[Lh] + kTile * a);
        }
  #pragma unroll
        for (int m = 0; m < NKM; ++m) {
          const int g = KL::group_of_step(m);
          if constexpr (KL::CB == 8)
            c[g] = mfma_k32(k_extract8(kx[KL::load_of_step(m)], kmask[m]), qf[m], c[g]);
          else
            c[g] = mfma_k16(k_extract4(kx[KL::load_of_step(m)], kmask[m]), u2{qf[m][0], qf[m][1]}, c[g]);
        }
        // zero-point part: A row = token 16a + r, k-slots = its NG zero points
        u2 za;
        {
          const uint8_t* zr = mkz + (16 * a + r) * MR * 2;
          if constexpr (NG == 8) {
            const u4 z8 = *reinterpret_cast<const u4*>(zr);
            za = (j & 1) ? u2{z8[2], z8[3]} : u2{z8[0], z8[1]};
          } else if constexpr (NG == 4) {
            za = *reinterpret_cast<const u2*>(zr);
          } else if constexpr (NG == 2) {
            const uint32_t z2 = *reinterpret_cast<const uint32_t*>(zr);
            za = u2{z2, z2};
          } else {
            const uint32_t z1 = *reinterpret_cast<const uint16_t*>(zr);
            za = u2{z1 | (z1 << 16), 0u};
          }
        }
        const f4 yz = mfma_k16(za, qzb, f4{0.f, 0.f, 0.f, 0.f});
  #pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * a + 4 * j + i;
          float sc = yz[i] * zsc;
  #pragma unroll
          for (int g = 0; g < NG; ++g) {
            const float sv = (float)__builtin_bit_cast(_Float16, (uint16_t)half_at(mks, t * MR + g));
            sc = fmaf(sv, c[g][i], sc);
          }
          x[4 * a + i] = sc;
        }
      }
      }  // per-token key groups
      if constexpr (TAIL) {
  #pragma unroll
        for (int a = 0; a < 2; ++a)
  #pragma unroll
          for (int i = 0; i < 4; ++i)
            if (cb + 16 * a + 4 * j + i > last) x[4 * a + i] = -INFINITY;
      }

      // ---- online softmax ---------------------------------------------------
      float alpha;
      ChunkProbs pr;
      if (softmax_chunk<false, KCOL>(x, lscale, m_run, l_run, alpha, pr, kbias) && live) {
  #pragma unroll
        for (int mv = 0; mv < NVM; ++mv)
          if (v_mfma_in_part<VL, VS>(mv, PART)) accv[mv] *= alpha;
        oz *= alpha;

      }
      pb = u4{pr.ph[0], pr.ph[1], pr.ph[2], pr.ph[3]};
      if constexpr (HILO) {
#pragma unroll
        for (int i = 0; i < 4; ++i) pbl[i] = pack_h2_rem(pr.p[2 * i], pr.p[2 * i + 1], pr.ph[i]);
      }
    }

    live = true;
    // ---- V zero point: oz += Z^T P (A rows = groups, k = the lane's 8 tokens)
    {
      uint32_t zp[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t0 = slot_token(j, 2 * q), t1 = slot_token(j, 2 * q + 1);
        if constexpr (MR == 1) {
          // fp16 pairs staged whole (t1 = t0 + 1): row 0 the zero points, row 1
          // the ones, rows > 1 the zero area.
          zp[q] = *reinterpret_cast<const uint32_t*>(mvz + zoff + 2 * t0);
        } else {
          zp[q] = perm(*reinterpret_cast<const uint32_t*>(mvz + zoff + 2 * t1 * MR),
                       *reinterpret_cast<const uint32_t*>(mvz + zoff + 2 * t0 * MR), zsel);
        }
        if constexpr (TAIL) zp[q] &= tail_pair_mask(cb + t0, cb + t1);
      }
      oz = mfma_k32(u4{zp[0], zp[1], zp[2], zp[3]}, pb, oz);
      if constexpr (HILO) oz = mfma_k32(u4{zp[0], zp[1], zp[2], zp[3]}, pbl, oz);
    }
    // ---- P' = P * s_g, g = v * S + slot ----------------------------------------
    u4 pg[NPG];
    u4 pgl[PSREM ? NPG : 1];
#pragma unroll
    for (int v = 0; v < NPG; ++v) {
      if (!v_operand_in_part<VL, VS, S>(v, PART)) continue;  // another part's groups
      uint32_t sp[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t0 = slot_token(j, 2 * q), t1 = slot_token(j, 2 * q + 1);
        if constexpr (MR == 1) {
          sp[q] = *reinterpret_cast<const uint32_t*>(mvs + 2 * t0);  // the pair (t0, t1 = t0 + 1)
        } else {
          const uint32_t d0 = *reinterpret_cast<const uint32_t*>(mvs + 2 * t0 * MR + soff[v]);
          const uint32_t d1 = *reinterpret_cast<const uint32_t*>(mvs + 2 * t1 * MR + soff[v]);
          sp[q] = perm(d1, d0, ssel[v]);
        }
        if constexpr (TAIL) sp[q] &= tail_pair_mask(cb + t0, cb + t1);
      }
      pg[v] = u4{pk_mul(pb[0], sp[0]), pk_mul(pb[1], sp[1]), pk_mul(pb[2], sp[2]), pk_mul(pb[3], sp[3])};
      if constexpr (HILO) {
        // P * s = pg + (pb * s - pg) + pbl * s: the exact remainder of the
        // fp16 product plus the low part's product, summed in fp16
#pragma unroll
        for (int q = 0; q < 4; ++q)
          pgl[v][q] = pk_add(pk_fma_rem(pb[q], sp[q], pg[v][q]), pk_mul(pbl[q], sp[q]));
      } else if constexpr (PSREM) {
#pragma unroll
        for (int q = 0; q < 4; ++q) pgl[v][q] = pk_fma_rem(pb[q], sp[q], pg[v][q]);
      }
      if constexpr (FOLD) {
#pragma unroll
        for (int q = 0; q < 4; ++q) pg[v][q] = r >= 8 ? pgl[v][q] : pg[v][q];
      }
    }

    // ---- O^T += V^T P'^T ---------------------------------------------------
#pragma unroll
    for (int wi = 0; wi < VL::NWIN; ++wi) {
      if (!v_window_in_part<VL, VS>(wi, PART)) continue;  // another part's dims
      uint32_t vx[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        // slot i: token 4j + i (block 0) or 16 + 4j + i - 4 (block 1)
        vx[i] = *reinterpret_cast<const uint32_t*>(
            st + voff[wi] + (i < 4 ? 0 : 16 * (VL::DP / 16) * 16) + 16 * (i & 3));
#pragma unroll
      for (int e = 0; e < VL::NE; ++e) {
        uint32_t pm[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pm[i] = perm(vx[2 * i + 1], vx[2 * i], vsel[e]);
        // When every V MFMA takes the same P' operand (one V group, or head
        // columns that give each group columns of its own: NPG == 1), every
        // slice of a byte meets the same P' in each column, so slice p's MFMA
        // may take the byte with only the slices above p cleared (the top
        // slice: the raw byte): its accumulator holds the codes of slices
        // <= p at their bit positions, and slice p alone is recovered after
        // the loop as acc[p] - acc[p - 1] -- one AND fewer per byte pair.  Slices below p weigh less than slice p's own code
        // (c * 2^(p*VNB) against at most 2^(p*VNB) - 1), so that difference
        // loses at most about one bit of the accumulators' precision.  (The
        // other direction, clearing the slices below p and subtracting
        // acc[p + 1], leaves slice 0 as the small difference of two sums of
        // whole bytes: up to ~85x the rounding at 2 bits, measured 2.8e-3
        // max-abs on the Llama-3-8B shape with outlier channels.)  Otherwise
        // each slice is isolated by its own mask.  (A dims part, VS > 1,
        // takes its own MFMAs and never runs the chain.)
#pragma unroll
        for (int p = 0; p < VL::P; ++p) {
          const int mv = VL::mfma_index(p, wi, e);
          if (!v_mfma_in_part<VL, VS>(mv, PART)) continue;  // another part's dims
          const uint32_t msk = kVChain ? lo_slices_mask<VNB>(p) : slice_mask<VNB>(p);
          const u4 av = (kVChain && p == VL::P - 1) ? u4{pm[0], pm[1], pm[2], pm[3]}
                                                    : u4{pm[0] & msk, pm[1] & msk, pm[2] & msk, pm[3] & msk};
          accv[mv] = mfma_k32(av, pg[VL::group_of(mv) / S], accv[mv]);
          if constexpr (PSREM && !FOLD) accv[mv] = mfma_k32(av, pgl[VL::group_of(mv) / S], accv[mv]);
        }
      }
    }
  };

  // Runs of NSTAGE chunks that end before the split's last token (stages
  // 0 .. NSTAGE-1), then what is left: at most NSTAGE - 1 such chunks and the
  // chunk holding the last token, which always runs as the TAIL step (even
  // when it is full).  A single loop exit keeps the accumulators in place
  // across the unrolled copies.
  auto stream = [&](auto pmode, auto part) __attribute__((always_inline)) {
    int cb = cb0;
    for (; cb + (NSTAGE - 1) * cstride + kChunk < hi; cb += NSTAGE * cstride) {
      static_for<NSTAGE>([&](auto s) __attribute__((always_inline)) {
        step(cb + decltype(s)::value * cstride, std::false_type{}, s, pmode, part);
      });
    }
    bool more = true;
    static_for<NSTAGE>([&](auto s) __attribute__((always_inline)) {
      if (more) {
        if (cb + kChunk < hi) {
          step(cb, std::false_type{}, s, pmode, part);
          cb += cstride;
        } else {
          if (cb < hi) step(cb, std::true_type{}, s, pmode, part);
          more = false;
        }
      }
    });
  };
  // The stream, this wave's partial and the workgroup merge, for dims part
  // PART (VS > 1; one part otherwise): each part is its own straight-line
  // copy of the loop, so a part's accumulators are all it carries.
  auto run = [&](auto part) __attribute__((always_inline)) {
    constexpr int PART = decltype(part)::value;
    // Short rows take hi/lo probabilities in every chunk (see kHiLoMaxLen);
    // longer ones the remainders of P * s where kPsRemainder asks for them.
    if (L <= kHiLoMaxLen) stream(std::integral_constant<int, 2>{}, part);
    else stream(std::integral_constant<int, kPsRemainder<VNB, NG> ? 1 : 0>{}, part);
    wait_vmcnt<0>();  // retire the trailing (out-of-range) prefetches
    wave_lds_fence();
    // whether the V accumulators of columns 8-15 hold the P * s remainders of
    // columns 0-7 (the stream ran with FOLD)
    const bool folded = PT && HS == 16 && kPsRemainder<VNB, NG> && L > kHiLoMaxLen;

    // ---- this wave's partial into its own ring region -----------------------
    WavePartial<D>& wp = *reinterpret_cast<WavePartial<D>*>(ring);
    {
      // Row g of the V zero-point MFMA (group g; row NG: the ones row, sum p)
      // sits in lane 16 * (g / 4) + n, element g % 4: broadcast to every lane
      // of column n.
      const float lt = row_bcast(oz[NG % 4], NG / 4);
      float ozg[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) ozg[g] = row_bcast(oz[g % 4], g / 4);
#pragma unroll
      for (int mv = 0; mv < NVM; ++mv) {
        if (!v_mfma_in_part<VL, VS>(mv, PART)) continue;
        const int p = VL::slice_of(mv);
        const float fac = kTwo24 * __builtin_ldexpf(1.0f, -p * VNB);
        const float zv = ozg[VL::group_of(mv)];
        f4 a = accv[mv];
        if (kVChain && p > 0) a -= accv[VL::mfma_index(p - 1, VL::window_of(mv), VL::e_of(mv))];
        if (folded) {
#pragma unroll
          for (int i = 0; i < 4; ++i) a[i] += lane_xor8(a[i]);
        }
        if (S == 1 || VL::group_of(mv) % S == slot) {  // this column's products are group mv's
#pragma unroll
          for (int i = 0; i < 4; ++i) wp.o[n % HS][VL::dim_of(mv, 4 * j + i)] = fmaf(a[i], fac, zv);
        }
      }
      if (j == 0) {
        wp.m[n] = m_run;
        wp.l[n] = lt;
      }
    }
    WavePartial<D>& wp0 = *reinterpret_cast<WavePartial<D>*>(smem);
    const MergeView view{&wp0.o[0][0], &wp0.m[0], &wp0.l[0], SM::WAVE / 4,
                         reinterpret_cast<int*>(smem + sizeof(WavePartial<D>))};
    // part PART holds the dims of slices [P0, P0 + P / VS): [PART * D / VS, ...)
    merge_and_store<D, NW, D / VS>(prm, view, b, h0, nh, split, PART * (D / VS));
  };
  if constexpr (VS == 1) {
    run(std::integral_constant<int, 0>{});
  } else if constexpr (VS == 2) {
    if (vpart == 0) run(std::integral_constant<int, 0>{});
    else run(std::integral_constant<int, 1>{});
  } else {
    static_assert(VS == 4, "two or four dims parts");
    if (vpart == 0) run(std::integral_constant<int, 0>{});
    else if (vpart == 1) run(std::integral_constant<int, 1>{});
    else if (vpart == 2) run(std::integral_constant<int, 2>{});
    else run(std::integral_constant<int, 3>{});
  }
}

// Ring depth per wave of the quantized split kernel.  8-wave workgroups run
// one per CU (VGPRs), so their LDS could hold three stages, but a third stage
// measured slightly slower at the Llama-3-8B shape (208 vs 206 us): one chunk
// in flight per wave already saturates what this access pattern streams.
// Paged caches use two stages.
constexpr int kStages8 = 2;  // also the ring depth of 12-wave workgroups
static_assert(kStages8 == 2, "kTwelveWaves sizes two-stage rings");
constexpr int kStages4 = 2;

// Compute units of the current device (cached per device; 0 if unknown).
inline int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) cus[dev] = n;
  }
  return cus[dev];
}

// Formats with dims-split kernels: head dim 128, equal K/V bits, groups of
// 32 and 8 head columns (GQA groups of 5-8 heads, as Qwen2.5-1.5B's small
// grids).  There every V group has P' operands of its own (no slice chain),
// so each part's V products, partial and merge are the very operations of
// the one-workgroup kernel: the output is bitwise the same.  With 4 head
// columns the slices of a byte share one chain (acc[p] - acc[p - 1]), which
// a part that starts past slice 0 would have to restart: different bits.
template <int D, int KNB, int VNB, int GS, int HS>
constexpr bool kDimsSplit = D == 128 && KNB == VNB && GS == 32 && HS == 8;

template <int D, int KNB, int VNB, int GS, bool PT, int HS, bool ORD>
void launch_quant_pto(const SplitParams& p, dim3 grid, int waves, hipStream_t st) {
  const bool paged = p.page_size > 0;
  // A grid of at most a quarter (a half) as many workgroups as the GPU has
  // CUs runs each (unit, split, head block) as four (two) workgroups, each
  // over a quarter (a half) of the head dim.
  if constexpr (!PT && !ORD && kDimsSplit<D, KNB, VNB, GS, HS>) {
    const unsigned long long wgs = 1ull * grid.x * grid.y * grid.z;
    const unsigned long long cus = (unsigned long long)device_cus();
    if (!paged && p.counters == nullptr && p.key_block == 0 && waves != 12 && 2 * wgs <= cus) {
      // fewer than 8 tuples: grid (8 * VS), xcd_units set and the small-grid
      // layout; else VS times the z axis (see the kernel's dims-split mapping)
      auto go = [&](auto vs, auto sg) {
        constexpr int V = decltype(vs)::value;
        constexpr bool SGL = decltype(sg)::value;
        SplitParams q = p;
        if (SGL) q.xcd_units = (int)grid.x;
        const dim3 g = SGL ? dim3(8 * V) : dim3(grid.x, grid.y, grid.z * V);
        if (waves >= 8)
          quant_split_lds_kernel<D, KNB, VNB, GS, 8, kStages8, false, false, false, HS, false, V, SGL>
              <<<g, dim3(8 * 64), 0, st>>>(q);
        else
          quant_split_lds_kernel<D, KNB, VNB, GS, 4, kStages4, false, false, false, HS, false, V, SGL>
              <<<g, dim3(4 * 64), 0, st>>>(q);
      };
      using I2 = std::integral_constant<int, 2>;
      using I4 = std::integral_constant<int, 4>;
      if (4 * wgs <= cus) {
        if (wgs < 8) go(I4{}, std::true_type{});
        else go(I4{}, std::false_type{});
      } else {
        if (wgs < 8) go(I2{}, std::true_type{});
        else go(I2{}, std::false_type{});
      }
      return;
    }
  }
  if constexpr (kTwelveWaves<D, KNB, VNB, GS, HS, PT>) {
    if (waves == 12 && !paged) {
      quant_split_lds_kernel<D, KNB, VNB, GS, 12, kStages8, false, PT, false, HS, ORD, 1, false>
          <<<grid, dim3(12 * 64), 0, st>>>(p);
      return;
    }
  }
  if (waves >= 8) {
    if (paged)
      quant_split_lds_kernel<D, KNB, VNB, GS, 8, 2, true, PT, false, HS, ORD, 1, false><<<grid, dim3(8 * 64), 0, st>>>(p);
    else
      quant_split_lds_kernel<D, KNB, VNB, GS, 8, kStages8, false, PT, false, HS, ORD, 1, false><<<grid, dim3(8 * 64), 0, st>>>(p);
  } else {
    if (paged)
      quant_split_lds_kernel<D, KNB, VNB, GS, 4, 2, true, PT, false, HS, ORD, 1, false><<<grid, dim3(4 * 64), 0, st>>>(p);
    else
      quant_split_lds_kernel<D, KNB, VNB, GS, 4, kStages4, false, PT, false, HS, ORD, 1, false><<<grid, dim3(4 * 64), 0, st>>>(p);
  }
}

// Kernels that read a dispatch order exist for head dim 128 only (the host
// refuses an order elsewhere, before anything is launched).
template <int D, int KNB, int VNB, int GS, bool PT, int HS>
void launch_quant_pt(const SplitParams& p, dim3 grid, int waves, hipStream_t st) {
  if constexpr (D == 128) {
    if (p.order) return launch_quant_pto<D, KNB, VNB, GS, PT, HS, true>(p, grid, waves, st);
  }
  launch_quant_pto<D, KNB, VNB, GS, PT, HS, false>(p, grid, waves, st);
}

// Paired tiles when the GQA group has at most 8 query heads and every
// workgroup streams a long history.  They cost about 1 us more per workgroup
// (twice the q operands to build, three more cross-lane moves per chunk), so
// they pay only over many chunks per wave: measured 4-6% faster at 32768 tokens
// per workgroup (2-bit, K4/V2), equal at 4096, 5-10% slower at 512-1024.
constexpr int kPairedTilesMinSplit = 8192;

// ===========================================================================
// Read-ceiling probe: what the split kernel's access pattern streams with no
// arithmetic behind it.  Same grid, waves, 32-token chunk order, two-stage
// per-wave ring and direct-to-LDS instructions (issue_chunk) over the same
// contiguous caches; each chunk is consumed by one LDS read per lane, so the
// loads stay live.  The measurement counterpart, for this kernel's read
// pattern, of a device-copy bandwidth probe.
// ===========================================================================
template <int D, int KNB, int VNB, int GS, int NW>
__global__ void __launch_bounds__(NW * 64) read_probe_kernel(SplitParams prm) {
  using SG = StageGeom<D, KNB, VNB, GS>;
  constexpr int NG = SG::NG;
  constexpr int NI = SG::NINSTR;
  __shared__ __attribute__((aligned(16))) uint8_t smem[NW * 2 * SG::BYTES];
  int unit_ = blockIdx.x, split_ = blockIdx.y, L_ = 0;
  if (prm.order) {  // the split kernel's dispatch order
    const int2 e = reinterpret_cast<const int2*>(prm.order)[blockIdx.y * gridDim.x + blockIdx.x];
    unit_ = e.x % (int)gridDim.x;
    split_ = e.x / (int)gridDim.x;
    L_ = e.y;
  }
  const int unit = __builtin_amdgcn_readfirstlane(unit_);
  const int split = __builtin_amdgcn_readfirstlane(split_);
  const int b = unit / prm.HKV;
  const int L = prm.order ? __builtin_amdgcn_readfirstlane(L_)
                          : (prm.seq_lens ? min(prm.seq_lens[b], prm.S) : prm.S);
  const int lo = split * prm.split_size;
  const int hi = min(lo + prm.split_size, L);
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t slab = unit;
  const uint32_t rows = (uint32_t)prm.S;
  const rsrc_t rk = make_rsrc(prm.k + slab * rows * SG::KL::DP, rows * SG::KL::DP);
  const rsrc_t rv = make_rsrc(prm.v + slab * rows * SG::VL::DP, rows * SG::VL::DP);
  const rsrc_t rm[4] = {make_rsrc(prm.ks + slab * rows * NG, rows * NG * 2),
                        make_rsrc(prm.kz + slab * rows * NG, rows * NG * 2),
                        make_rsrc(prm.vs + slab * rows * NG, rows * NG * 2),
                        make_rsrc(prm.vz + slab * rows * NG, rows * NG * 2)};
  uint8_t* ring = smem + w * 2 * SG::BYTES;
  const int cstride = kChunk * NW;
  const int cb0 = lo + kChunk * w;
  issue_chunk<D, KNB, VNB, GS>(ring, rk, rv, rm, cb0, cb0 < hi, lane, cb0 + kChunk < hi);
  float acc = 0.0f;
  int s = 0;
  for (int cb = cb0; cb < hi; cb += cstride) {
    wait_lgkmcnt0();  // the previous read of the stage refilled next is done
    asm volatile("" ::: "memory");
    const int cn = cb + cstride;
    issue_chunk<D, KNB, VNB, GS>(ring + (s ^ 1) * SG::BYTES, rk, rv, rm, cn, cn < hi, lane, cn + kChunk < hi);
    wait_vmcnt<NI>();
    asm volatile("" ::: "memory");
    acc += reinterpret_cast<const float*>(ring + s * SG::BYTES)[lane];
    s ^= 1;
  }
  wait_vmcnt<0>();
  if (acc == 1.2345678e-30f) prm.out[blockIdx.x] = acc;  // data-dependent: the loads cannot be dropped
}

template <int D, int KNB, int VNB, int GS>
void launch_read_probe(const SplitParams& p, dim3 grid, int waves, hipStream_t st) {
  // The same workgroup size as the kernel it probes (whose 12-wave form at
  // G <= 4 has head columns of width 4 and, at GS = 128, width 16).
  if constexpr (kTwelveWaves<D, KNB, VNB, GS, GS == 128 ? 16 : 4, true>) {
    if (waves == 12 && (GS == 128 || p.G <= 4)) {
      read_probe_kernel<D, KNB, VNB, GS, 12><<<grid, dim3(12 * 64), 0, st>>>(p);
      return;
    }
  }
  if (waves >= 8) read_probe_kernel<D, KNB, VNB, GS, 8><<<grid, dim3(8 * 64), 0, st>>>(p);
  else read_probe_kernel<D, KNB, VNB, GS, 4><<<grid, dim3(4 * 64), 0, st>>>(p);
}

// One head-column width HS (the kernels of one width are instantiated in a
// translation unit of their own, quant_split_k*v*[_h*].hip).
template <int D, int KNB, int VNB, int GS, int HS>
void launch_quant_hs(const SplitParams& p, dim3 grid, int waves, hipStream_t st) {
  if constexpr (GS <= 32) {
    if (p.key_block) {  // per-channel keys (the host checked: contiguous, no fused append)
      if constexpr (kTwelveWaves<D, KNB, VNB, GS, HS, false>) {
        if (waves == 12) {
          quant_split_lds_kernel<D, KNB, VNB, GS, 12, kStages8, false, false, true, HS, false, 1, false>
              <<<grid, dim3(12 * 64), 0, st>>>(p);
          return;
        }
      }
      if (waves >= 8)
        quant_split_lds_kernel<D, KNB, VNB, GS, 8, kStages8, false, false, true, HS, false, 1, false>
            <<<grid, dim3(8 * 64), 0, st>>>(p);
      else
        quant_split_lds_kernel<D, KNB, VNB, GS, 4, kStages4, false, false, true, HS, false, 1, false>
            <<<grid, dim3(4 * 64), 0, st>>>(p);
      return;
    }
  }
  if (p.G <= 8 && p.split_size >= kPairedTilesMinSplit)
    launch_quant_pt<D, KNB, VNB, GS, true, HS>(p, grid, waves, st);
  else launch_quant_pt<D, KNB, VNB, GS, false, HS>(p, grid, waves, st);
}

// Head-column width of a launch: the narrowest of 4, 8, 16 that holds the GQA
// group, when there are V groups to share the columns (D / GS >= 2).
template <int D, int GS>
constexpr bool kHeadColumns = D / GS >= 2;

template <int D, int KNB, int VNB, int GS>
void launch_quant(const SplitParams& p, dim3 grid, int waves, hipStream_t st) {
  if constexpr (kHeadColumns<D, GS>) {
    if (p.G <= 4) return launch_quant_hs<D, KNB, VNB, GS, 4>(p, grid, waves, st);
    if (p.G <= 8) return launch_quant_hs<D, KNB, VNB, GS, 8>(p, grid, waves, st);
  }
  launch_quant_hs<D, KNB, VNB, GS, 16>(p, grid, waves, st);
}

}  // namespace tkv
