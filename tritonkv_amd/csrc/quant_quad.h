// Quad-tile kernel of the fused quantized decode (gfx950): 2-bit K and V
// codes, one scale/zero group per row (group size = head dim 128), GQA groups
// of at most 4 query heads, contiguous caches.  Included by quant_split.h,
// after the split kernel whose staging, DMA ring and PV products it shares,
// inside namespace tkv.
#pragma once

// ---------------------------------------------------------------------------
// Quad tiles.  With at most 4 heads per group, paired tiles (8 head columns
// per tile) still spend half the score columns -- and half the fold and
// softmax instructions after the score MFMAs -- on padding heads.  Here each
// step takes two chunks of the wave (four 16-token tiles) through one set of
// score MFMAs: column c is head c & 3 of tile c >> 2, lane group j carries
// tile j's codes (a block-diagonal B operand over four tiles: 8 dims of every
// tile per MFMA, D / 8 MFMAs per step, as many per token as paired tiles),
// and each lane ends with the 4 scores of one tile for one head.  No column
// holds a padding head: half the fold, exponentials and conversions per token.
//
// The PV products keep the split kernel's layout per chunk (column c < 4
// carries head c's P * s, columns 4-7 its remainders): the probabilities of a
// chunk's two tiles move to the columns of their head with DPP row shifts
// written into 4-lane banks.  The score operands (D / 8 of them, 64 VGPRs
// per lane) stay in LDS, built once per workgroup by wave 0, and the ring
// holds four stages per wave: the two chunks of a step and the two in flight.
// ---------------------------------------------------------------------------
template <int NW>
struct QuadSmem {
  using SG = StageGeom<128, 2, 2, 128>;
  static constexpr int RING = 4 * SG::BYTES;
  static constexpr int OUT = (int)sizeof(WavePartial<128>) + 16;
  static constexpr int WAVE = ((RING > OUT ? RING : OUT) + 15) / 16 * 16;
  static constexpr int NQ = 16;                // score MFMAs per step
  static constexpr int QOP = NQ * 64 * 16;     // their B operands, [mfma][lane] u4
  static constexpr int QEX = 2 * 64 * 4;       // per lane: eh, sum q
  // Fused append: the new token's row in staged form (as the split kernel's).
  static constexpr int PATCH_META = SG::KL::DP + SG::VL::DP;
  static constexpr int PATCH = (PATCH_META + 4 * SG::NG * 2 + 15) / 16 * 16;
  static constexpr int TOTAL = NW * WAVE + QOP + QEX + PATCH;
  static_assert(TOTAL <= 160 * 1024, "quad-tile LDS");
};

// DPP move of src within 16-lane rows (CTRL: 0x100 + n row_shl:n, lane i takes
// lane i + n; 0x110 + n row_shr:n, lane i takes lane i - n), written only into
// the 4-lane banks set in BM; every other lane keeps old.
template <int CTRL, int BM>
__device__ __forceinline__ uint32_t dpp_banks(uint32_t old, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, CTRL, 0xF, BM, false);
}
template <int N>
__device__ __forceinline__ float row_ror(float v) {  // lane i takes lane (i - N) mod 16 of its row
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x120 + N, 0xF,
                                                            0xF, true));
}

// PV operand of one chunk for the lane's column (banks 0 and 1: head c & 3):
// its head's fp16 probability pairs v0, v1 (tokens 4j..4j+3) of the chunk's
// first tile, then of its second.  Chunk 0's tiles sit in banks 0 and 1,
// chunk 1's in banks 2 and 3 of the score layout.  Banks 2 and 3 of the
// result are not read.
template <int X>
__device__ __forceinline__ u4 quad_pv_operand(uint32_t v0, uint32_t v1) {
  if constexpr (X == 0) {
    return u4{dpp_banks<0x114, 0x2>(v0, v0), dpp_banks<0x114, 0x2>(v1, v1),
              dpp_banks<0x104, 0x1>(v0, v0), dpp_banks<0x104, 0x1>(v1, v1)};
  } else {
    return u4{dpp_banks<0x104, 0x2>(dpp_banks<0x108, 0x1>(v0, v0), v0),
              dpp_banks<0x104, 0x2>(dpp_banks<0x108, 0x1>(v1, v1), v1),
              dpp_banks<0x108, 0x2>(dpp_banks<0x10C, 0x1>(v0, v0), v0),
              dpp_banks<0x108, 0x2>(dpp_banks<0x10C, 0x1>(v1, v1), v1)};
  }
}

// Score operands of lane (c, j) into LDS: operand mi = p * 4 + o holds, when
// lane group j carries the column's tile (c >> 2 == j) and head c & 3 < nh,
// that head's q at dims 32p + 8o .. + 7 in the slot order of k_extract8
// (pairs (0,2) (1,3) (4,6) (5,7)), scaled by 2^(eh - 2p); zeros otherwise.
// Behind them: the lane's prescale exponent eh and its head's sum of q (the
// zero term).  Every lane holds its head's whole row, so neither needs a
// cross-lane step.
__device__ __forceinline__ void build_quad_q(const SplitParams& prm, int b, int h0, int nh, int lane,
                                             uint32_t* qop) {
  constexpr int D = 128, KNB = 2, P = 4;
  const int c = lane & 15, j = lane >> 4, h = c & 3;
  const bool hv = h < nh;
  const uint32_t hvm = hv ? 0xFFFFFFFFu : 0u;
  const uint32_t opm = (hv && (c >> 2) == j) ? 0xFFFFFFFFu : 0u;
  const int64_t qrow = ((int64_t)b * prm.HQ + h0 + (hv ? h : 0)) * D;
  uint32_t qh[D / 8][4];  // natural fp16 pairs: qh[k][e] = dims 8k + 2e, 8k + 2e + 1
  if (prm.q_fp32) {
    const float* qp = static_cast<const float*>(prm.q) + qrow;
#pragma unroll
    for (int k = 0; k < D / 8; ++k) {
      const f4 a = *reinterpret_cast<const f4*>(qp + 8 * k);
      const f4 e = *reinterpret_cast<const f4*>(qp + 8 * k + 4);
      qh[k][0] = pack_h2(a[0], a[1]);
      qh[k][1] = pack_h2(a[2], a[3]);
      qh[k][2] = pack_h2(e[0], e[1]);
      qh[k][3] = pack_h2(e[2], e[3]);
    }
  } else {
    const _Float16* qp = static_cast<const _Float16*>(prm.q) + qrow;
#pragma unroll
    for (int k = 0; k < D / 8; ++k) {
      const u4 v = *reinterpret_cast<const u4*>(qp + 8 * k);
#pragma unroll
      for (int e = 0; e < 4; ++e) qh[k][e] = v[e] & hvm;
    }
  }
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  us2 mag = us2{0, 0};
  float qsum = 0.0f;
  const h2 ones = h2{(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
  for (int k = 0; k < D / 8; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qh[k][e] &= hvm;
      mag = __builtin_elementwise_max(mag, __builtin_bit_cast(us2, qh[k][e] & 0x7FFF7FFFu));
      qsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qh[k][e]), ones, qsum, false);
    }
  const uint32_t mbits = mag[0] > mag[1] ? mag[0] : mag[1];
  const float amax = (float)__builtin_bit_cast(_Float16, (unsigned short)mbits);
  const int eh = q_prescale_exp(amax, (P - 1) * KNB);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    // 2^(eh - 2p) as an fp16 pair (a normal number: eh >= -1, 2p <= 6)
    const uint32_t pe = (uint32_t)(eh - p * KNB + 15) << 10;
    const uint32_t pre = pe | (pe << 16);
#pragma unroll
    for (int o = 0; o < 4; ++o) {
      const uint32_t* v = qh[4 * p + o];
      const uint32_t sl[4] = {perm(v[1], v[0], 0x05040100u), perm(v[1], v[0], 0x07060302u),
                              perm(v[3], v[2], 0x05040100u), perm(v[3], v[2], 0x07060302u)};
      uint32_t* dst = qop + ((p * 4 + o) * 64 + lane) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e] = pk_mul(sl[e], pre) & opm;
    }
  }
  qop[QuadSmem<1>::QOP / 4 + lane] = (uint32_t)eh;
  qop[QuadSmem<1>::QOP / 4 + 64 + lane] = __builtin_bit_cast(uint32_t, qsum);
}

// ORD: the launch carries a dispatch order (as the split kernel's ORD).
template <int NW, bool ORD>
__global__ void __launch_bounds__(NW * 64) quant_quad_kernel(SplitParams prm) {
  constexpr int D = 128, KNB = 2, VNB = 2, GS = 128;
  using SG = StageGeom<D, KNB, VNB, GS>;
  using KL = typename SG::KL;
  using VL = typename SG::VL;
  using SM = QuadSmem<NW>;
  constexpr int NVM = VL::NVM;
  constexpr int NI = SG::NINSTR;
  constexpr int P = 8 / KNB;       // slices per byte
  constexpr int NO = KL::DP / 8;   // byte octets per row
  static_assert(P * NO == SM::NQ && SG::NG == 1 && VL::NWIN == 1 && kPsRemainder<VNB, 1>,
                "quad-tile geometry: 2-bit codes, one group per row");
  static_assert(2 * NI < 64, "vmcnt range");
  constexpr bool kVChain = true;  // one V group: every V MFMA takes the same P' operand

  __shared__ __attribute__((aligned(16))) uint8_t smem[SM::TOTAL];

  int unit_ = blockIdx.x, split_ = blockIdx.y, L_ = 0;
  if constexpr (ORD) {
    const int2 e = reinterpret_cast<const int2*>(prm.order)[blockIdx.y * gridDim.x + blockIdx.x];
    unit_ = e.x % (int)gridDim.x;
    split_ = e.x / (int)gridDim.x;
    L_ = e.y;
  }
  const int unit = __builtin_amdgcn_readfirstlane(unit_);
  const int split = __builtin_amdgcn_readfirstlane(split_);
  const int hb0 = __builtin_amdgcn_readfirstlane((int)blockIdx.z) * 16;
  const int b = unit / prm.HKV, hk = unit % prm.HKV;
  const int nh = min(16, prm.G - hb0);
  const int h0 = hk * prm.G + hb0;
  const int L = ORD ? __builtin_amdgcn_readfirstlane(L_)
                    : (prm.seq_lens ? min(prm.seq_lens[b], prm.S) : prm.S);
  const int lo = split * prm.split_size;
  const int hi = min(lo + prm.split_size, L);
  const int last = hi - 1;
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r = lane & 15, j = lane >> 4;
  // An empty split writes the empty partial and leaves (as the split kernel).
  if (lo >= L && prm.ns_total > 1 && prm.counters == nullptr) {
    for (int idx = tid; idx < nh * D; idx += NW * 64) {
      const int hn = idx / D, d = idx % D;
      const int64_t pr = ((int64_t)b * prm.HQ + h0 + hn) * prm.ns_total + prm.split_base + split;
      prm.acc[pr * D + d] = 0.0f;
      if (d == 0) {
        prm.maxs[pr] = -INFINITY;
        prm.sums[pr] = 0.0f;
      }
    }
    return;
  }
  // One resource per tensor over this (b, kv head) block (the hardware range
  // check returns zeros past it).
  const int64_t slab = unit;
  const uint32_t rows = (uint32_t)prm.S;
  const rsrc_t rk = make_rsrc(prm.k + slab * rows * KL::DP, rows * KL::DP);
  const rsrc_t rv = make_rsrc(prm.v + slab * rows * VL::DP, rows * VL::DP);
  const rsrc_t rm[4] = {make_rsrc(prm.ks + slab * rows, rows * 2), make_rsrc(prm.kz + slab * rows, rows * 2),
                        make_rsrc(prm.vs + slab * rows, rows * 2), make_rsrc(prm.vz + slab * rows, rows * 2)};
  uint8_t* ring = smem + w * SM::WAVE;
#pragma unroll
  for (int s = 0; s < 4; ++s)
    for (int i = lane; i < SG::MB / 4; i += 64)
      reinterpret_cast<uint32_t*>(ring + s * SG::BYTES + SG::ONES_OFF)[i] = 0x3C003C00u;

  // Step i of this wave takes chunks cb0 + 2i * cstride (A, stage 2i % 4) and
  // one cstride further (B, the next stage).  A step's metadata goes in as
  // fp16 pairs when the step ends before the split's last token (both chunks
  // full), else one fp16 per dword (the step that runs as TAIL).
  const int cb0 = lo + kChunk * w;
  const int cstride = kChunk * NW;
  {
    const bool pr = cb0 + cstride + kChunk < hi;
    issue_chunk<D, KNB, VNB, GS>(ring, rk, rv, rm, cb0, cb0 < hi, lane, pr);
    issue_chunk<D, KNB, VNB, GS>(ring + SG::BYTES, rk, rv, rm, cb0 + cstride, cb0 + cstride < hi, lane, pr);
  }

  // Per-lane set-up, while wave 0 builds the score operands.
  // Score MFMAs: lane (r, j) carries token 16 * (j & 1) + r of chunk j >> 1;
  // its two 16-byte units hold the four octets of its codes.
  uint32_t koff[2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
    koff[u] = (j >> 1) * SG::BYTES + SG::K_OFF + SG::template pos_of<KL::DP>(16 * (j & 1) + r, u) * 16;
  // Its scores: tokens 16 * ((r >> 2) & 1) + 4j + i of chunk r >> 3, head r & 3.
  const int sc_tok = 16 * ((r >> 2) & 1) + 4 * j;
  const int sc_chunk = r >> 3;
  const uint32_t moff = sc_chunk * SG::BYTES + SG::M_OFF;
  // PV products (per chunk, as the split kernel): V operand rows = dims.
  uint32_t vsel[VL::NE];
#pragma unroll
  for (int e = 0; e < VL::NE; ++e) vsel[e] = VL::perm_sel(VL::byte_in_dword(e, r));
  const int ob = VL::dword_offset(0, r);
  const uint32_t voff = SG::V_OFF + SG::template pos_of<VL::DP>(4 * j, ob >> 4) * 16 + (ob & 15);
  // V zero-point MFMA rows: 0 the zero points, 1 the ones (the sum of p);
  // rows past 1 read the ones as well and feed output rows nobody reads.
  const int zoff = r == 0 ? 0 : SG::MB;
  const uint32_t zsel = r <= 1 ? 0x05040100u : 0x0C0C0C0Cu;
  const bool rem_col = (r >> 2) == 1;  // columns 4-7: the P * s remainders of head r & 3

  uint32_t* const qop = reinterpret_cast<uint32_t*>(smem + NW * SM::WAVE);
  if (w == 0) build_quad_q(prm, b, h0, nh, lane, qop);
  __syncthreads();
  const uint32_t* const qlane = qop + lane * 4;
  // 8-wave workgroups (256 VGPRs per lane) keep the score operands in registers.
  constexpr bool QREG = NW <= 8;
  u4 qreg[QREG ? SM::NQ : 1];
  if constexpr (QREG) {
#pragma unroll
    for (int mi = 0; mi < SM::NQ; ++mi) qreg[mi] = *reinterpret_cast<const u4*>(qlane + mi * 256);
  }
  const int eh = (int)qop[SM::QOP / 4 + lane];
  const float qsum = __builtin_bit_cast(float, qop[SM::QOP / 4 + 64 + lane]);
  const float zsc = __builtin_ldexpf(1.0f, eh - 24);  // code-dot units per score unit
  const float qz = qsum * zsc;
  const float lscale = prm.qk_scale * __builtin_ldexpf(1.0f, 24 - eh);

  // ---- fused append (as the split kernel's) --------------------------------
  // The wave whose chunk holds token L - 1 quantizes the new row into the
  // patch area and, in the first block of query heads, into the cache; its
  // TAIL step (the step that holds the split's last token) then overwrites the
  // staged row with the patch.
  uint8_t* const patch = smem + NW * SM::WAVE + SM::QOP + SM::QEX;
  int cb_new = -1;  // first token of the chunk this wave patches, or -1
  int t_new = 0;    // the new token's row within that chunk
  if (prm.k_new && L - 1 >= lo && L - 1 < hi && ((L - 1 - lo) / kChunk) % NW == w) {
    const int tn = L - 1;
    const int64_t row = (int64_t)unit * prm.S + tn;
    cb_new = lo + kChunk * ((tn - lo) / kChunk);
    t_new = tn - cb_new;
    const int64_t xoff = (int64_t)unit * D * (prm.new_fp32 ? 4 : 2);
    float xk[KL::P], xv[VL::P];
    load_row_for_quant<D, KNB>(static_cast<const uint8_t*>(prm.k_new) + xoff, prm.new_fp32, lane, xk);
    load_row_for_quant<D, VNB>(static_cast<const uint8_t*>(prm.v_new) + xoff, prm.new_fp32, lane, xv);
    const RowQuant<D, KNB, GS> rk_ = quantize_row<D, KNB, GS>(xk, lane);
    const RowQuant<D, VNB, GS> rv_ = quantize_row<D, VNB, GS>(xv, lane);
    uint16_t* pmeta = reinterpret_cast<uint16_t*>(patch + SM::PATCH_META);
    if (lane < KL::DP) patch[lane] = (uint8_t)rk_.byte;
    if (lane < VL::DP) patch[KL::DP + lane] = (uint8_t)rv_.byte;
    if (lane == 0) {
      pmeta[0] = (uint16_t)(rk_.meta & 0xFFFFu);
      pmeta[1] = (uint16_t)(rk_.meta >> 16);
      pmeta[2] = (uint16_t)(rv_.meta & 0xFFFFu);
      pmeta[3] = (uint16_t)(rv_.meta >> 16);
    }
    if (hb0 == 0) {
      if (lane < KL::DP) const_cast<uint8_t*>(prm.k)[row * KL::DP + lane] = (uint8_t)rk_.byte;
      if (lane < VL::DP) const_cast<uint8_t*>(prm.v)[row * VL::DP + lane] = (uint8_t)rv_.byte;
      if (lane == 0) {
        const_cast<uint16_t*>(prm.ks)[row] = (uint16_t)(rk_.meta & 0xFFFFu);
        const_cast<uint16_t*>(prm.kz)[row] = (uint16_t)(rk_.meta >> 16);
        const_cast<uint16_t*>(prm.vs)[row] = (uint16_t)(rv_.meta & 0xFFFFu);
        const_cast<uint16_t*>(prm.vz)[row] = (uint16_t)(rv_.meta >> 16);
      }
    }
  }
  // The new token's row replaces what the DMA read into the staged chunk at sw
  // (one fp16 per dword: the TAIL step's metadata layout).
  auto apply_patch = [&](uint8_t* sw) __attribute__((always_inline)) {
    const uint16_t* pmeta = reinterpret_cast<const uint16_t*>(patch + SM::PATCH_META);
    if (lane < KL::DP)
      sw[SG::K_OFF + SG::template pos_of<KL::DP>(t_new, lane >> 4) * 16 + (lane & 15)] = patch[lane];
    if (lane < VL::DP)
      sw[SG::V_OFF + SG::template pos_of<VL::DP>(t_new, lane >> 4) * 16 + (lane & 15)] = patch[KL::DP + lane];
    if (lane < 4)
      *reinterpret_cast<uint16_t*>(sw + SG::M_OFF + lane * SG::MB + 2 * (t_new * SG::MROW)) = pmeta[lane];
  };
  float zero_v = 0.0f;  // an opaque zero (see the score fold)
  asm volatile("" : "+v"(zero_v));

  f4 accv[NVM];
#pragma unroll
  for (int mv = 0; mv < NVM; ++mv) accv[mv] = f4{0.f, 0.f, 0.f, 0.f};
  f4 oz = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  bool live = false;

  auto tail_pair_mask = [&](int tok0, int tok1) -> uint32_t {
    return (tok0 <= last ? 0x0000FFFFu : 0u) | (tok1 <= last ? 0xFFFF0000u : 0u);
  };
  auto half_at = [&](const uint8_t* base, int idx) -> uint32_t {
    return *reinterpret_cast<const uint16_t*>(base + 2 * idx);
  };

  auto step = [&](int cb, auto tail, auto stage, auto pmode) __attribute__((always_inline)) {
    constexpr bool TAIL = decltype(tail)::value;
    constexpr int SK = decltype(stage)::value;  // stage of chunk A (0 or 2)
    constexpr int PMODE = decltype(pmode)::value;
    constexpr bool HILO = PMODE == 2;
    constexpr bool FOLD = PMODE == 1;
    constexpr int MR = TAIL ? SG::MROW : SG::MROW_PAIRS;
    // refill the previous step's two stages with the next step's chunks
    {
      const int cn = cb + 2 * cstride;
      wait_lgkmcnt0();  // the previous step's LDS reads of those stages are done
      asm volatile("" ::: "memory");
      const bool pr = cn + cstride + kChunk < hi;
      uint8_t* sn = ring + ((SK + 2) % 4) * SG::BYTES;
      issue_chunk<D, KNB, VNB, GS>(sn, rk, rv, rm, cn, !TAIL && cn < hi, lane, pr);
      issue_chunk<D, KNB, VNB, GS>(sn + SG::BYTES, rk, rv, rm, cn + cstride, !TAIL && cn + cstride < hi, lane, pr);
    }
    wait_vmcnt<2 * NI>();
    asm volatile("" ::: "memory");  // no LDS read of this step's stages above the wait
    if constexpr (TAIL) {  // fused append: the new token is the split's last
      if (cb_new == cb) apply_patch(ring + SK * SG::BYTES);
      else if (cb_new == cb + cstride) apply_patch(ring + (SK + 1) * SG::BYTES);
    }
    const uint8_t* st = ring + SK * SG::BYTES;

    // ---- scores: four tiles in one set of MFMAs ----------------------------
    float x[4];
    {
      const u4 ku0 = *reinterpret_cast<const u4*>(st + koff[0]);
      const u4 ku1 = *reinterpret_cast<const u4*>(st + koff[1]);
      const u2 kx[NO] = {u2{ku0[0], ku0[1]}, u2{ku0[2], ku0[3]}, u2{ku1[0], ku1[1]}, u2{ku1[2], ku1[3]}};
      f4 c = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int o = 0; o < NO; ++o) {
          const u4 qb = QREG ? qreg[p * NO + o] : *reinterpret_cast<const u4*>(qlane + (p * NO + o) * 256);
          c = mfma_k32(k_extract8(kx[o], slice_mask<KNB>(p)), qb, c);
        }
      const uint8_t* ms = st + moff;       // K scales of the lane's chunk
      const uint8_t* mz = ms + SG::MB;     // K zero points
      if constexpr (MR == 1) {
        const u2 zz = *reinterpret_cast<const u2*>(mz + 2 * sc_tok);
        const u2 ss = *reinterpret_cast<const u2*>(ms + 2 * sc_tok);
        x[0] = fma_mix_h<false>(ss[0], c[0], fma_mix_h<false>(zz[0], qz, zero_v));
        x[1] = fma_mix_h<true>(ss[0], c[1], fma_mix_h<true>(zz[0], qz, zero_v));
        x[2] = fma_mix_h<false>(ss[1], c[2], fma_mix_h<false>(zz[1], qz, zero_v));
        x[3] = fma_mix_h<true>(ss[1], c[3], fma_mix_h<true>(zz[1], qz, zero_v));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float zv = (float)__builtin_bit_cast(_Float16, (uint16_t)half_at(mz, (sc_tok + i) * MR));
          const float sv = (float)__builtin_bit_cast(_Float16, (uint16_t)half_at(ms, (sc_tok + i) * MR));
          x[i] = fmaf(sv, c[i], zv * qz);
        }
      }
    }
    if constexpr (TAIL) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (cb + sc_chunk * cstride + sc_tok + i > last) x[i] = -INFINITY;
    }
    // ---- online softmax (16 lanes per head: 4 tiles x 4 lane groups) -------
    float pf[4];
    uint32_t ph[2];
    {
      const float lm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])) * lscale;  // this lane's max
      if (__builtin_amdgcn_ballot_w64(lm > m_run) != 0) {
        float mx = vmax(lm, row_ror<4>(lm));
        mx = vmax(mx, row_ror<8>(mx));
        const float mn = vmax(m_run, xor_max16_32(mx));
        const float alpha = safe_exp2_diff(m_run, mn);
        m_run = mn;
        if (live) {
#pragma unroll
          for (int mv = 0; mv < NVM; ++mv) accv[mv] *= alpha;
          oz *= alpha;
        }
      }
      live = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) pf[i] = __builtin_amdgcn_exp2f(fmaf(x[i], lscale, -m_run));
      ph[0] = pack_h2(pf[0], pf[1]);
      ph[1] = pack_h2(pf[2], pf[3]);
    }
    uint32_t phl[2] = {0u, 0u};  // HILO: the fp16 remainders of p
    if constexpr (HILO) {
      phl[0] = pack_h2_rem(pf[0], pf[1], ph[0]);
      phl[1] = pack_h2_rem(pf[2], pf[3], ph[1]);
    }

    // ---- PV products, chunk by chunk ----------------------------------------
    auto pv = [&](auto chunk) __attribute__((always_inline)) {
      constexpr int X = decltype(chunk)::value;
      const uint8_t* sx = st + X * SG::BYTES;
      const int cbx = cb + X * cstride;
      const uint8_t* mvs = sx + SG::M_OFF + 2 * SG::MB;
      const uint8_t* mvz = mvs + SG::MB;
      const u4 pb = quad_pv_operand<X>(ph[0], ph[1]);
      u4 pbl = u4{0u, 0u, 0u, 0u};
      if constexpr (HILO) pbl = quad_pv_operand<X>(phl[0], phl[1]);
      // V zero point and sum of p: oz += Z^T P
      {
        uint32_t zp[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int t0 = slot_token(j, 2 * q), t1 = slot_token(j, 2 * q + 1);
          if constexpr (MR == 1) {
            zp[q] = *reinterpret_cast<const uint32_t*>(mvz + zoff + 2 * t0);
          } else {
            zp[q] = perm(*reinterpret_cast<const uint32_t*>(mvz + zoff + 2 * t1 * MR),
                         *reinterpret_cast<const uint32_t*>(mvz + zoff + 2 * t0 * MR), zsel);
            if constexpr (TAIL) zp[q] &= tail_pair_mask(cbx + t0, cbx + t1);
          }
        }
        oz = mfma_k32(u4{zp[0], zp[1], zp[2], zp[3]}, pb, oz);
        if constexpr (HILO) oz = mfma_k32(u4{zp[0], zp[1], zp[2], zp[3]}, pbl, oz);
      }
      // P' = P * s, with the exact remainders (FOLD: in columns 4-7)
      u4 pg, pgl;
      {
        uint32_t sp[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int t0 = slot_token(j, 2 * q), t1 = slot_token(j, 2 * q + 1);
          if constexpr (MR == 1) {
            sp[q] = *reinterpret_cast<const uint32_t*>(mvs + 2 * t0);
          } else {
            sp[q] = perm(*reinterpret_cast<const uint32_t*>(mvs + 2 * t1 * MR),
                         *reinterpret_cast<const uint32_t*>(mvs + 2 * t0 * MR), 0x05040100u);
            if constexpr (TAIL) sp[q] &= tail_pair_mask(cbx + t0, cbx + t1);
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          pg[q] = pk_mul(pb[q], sp[q]);
          if constexpr (HILO) pgl[q] = pk_add(pk_fma_rem(pb[q], sp[q], pg[q]), pk_mul(pbl[q], sp[q]));
          else pgl[q] = pk_fma_rem(pb[q], sp[q], pg[q]);
          if constexpr (FOLD) pg[q] = rem_col ? pgl[q] : pg[q];
        }
      }
      // O^T += V^T P'^T
      uint32_t vx[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        vx[i] = *reinterpret_cast<const uint32_t*>(sx + voff + (i < 4 ? 0 : 16 * (VL::DP / 16) * 16) +
                                                   16 * (i & 3));
#pragma unroll
      for (int e = 0; e < VL::NE; ++e) {
        uint32_t pm[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pm[i] = perm(vx[2 * i + 1], vx[2 * i], vsel[e]);
#pragma unroll
        for (int p = 0; p < VL::P; ++p) {
          const int mv = VL::mfma_index(p, 0, e);
          const uint32_t msk = lo_slices_mask<VNB>(p);
          const u4 av = (p == VL::P - 1) ? u4{pm[0], pm[1], pm[2], pm[3]}
                                         : u4{pm[0] & msk, pm[1] & msk, pm[2] & msk, pm[3] & msk};
          accv[mv] = mfma_k32(av, pg, accv[mv]);
          if constexpr (!FOLD) accv[mv] = mfma_k32(av, pgl, accv[mv]);
        }
      }
    };
    pv(std::integral_constant<int, 0>{});
    pv(std::integral_constant<int, 1>{});
  };

  // Pairs of steps (stages 0-1, then 2-3) that end before the split's last
  // token, then at most two more: a full one and the TAIL step (the step
  // whose chunk B does not end before the last token).
  auto stream = [&](auto pmode) __attribute__((always_inline)) {
    int cb = cb0;
    for (; cb + 3 * cstride + kChunk < hi; cb += 4 * cstride) {
      step(cb, std::false_type{}, std::integral_constant<int, 0>{}, pmode);
      step(cb + 2 * cstride, std::false_type{}, std::integral_constant<int, 2>{}, pmode);
    }
    bool more = true;
    static_for<2>([&](auto s) __attribute__((always_inline)) {
      constexpr int SK = 2 * decltype(s)::value;
      if (more) {
        if (cb + cstride + kChunk < hi) {
          step(cb, std::false_type{}, std::integral_constant<int, SK>{}, pmode);
          cb += 2 * cstride;
        } else {
          if (cb < hi) step(cb, std::true_type{}, std::integral_constant<int, SK>{}, pmode);
          more = false;
        }
      }
    });
  };
  // Short rows: hi/lo probabilities (kHiLoMaxLen); longer ones the P * s
  // remainders in columns 4-7.
  if (L <= kHiLoMaxLen) stream(std::integral_constant<int, 2>{});
  else stream(std::integral_constant<int, 1>{});
  wait_vmcnt<0>();  // retire the trailing (out-of-range) prefetches
  wave_lds_fence();
  const bool folded = L > kHiLoMaxLen;

  // ---- this wave's partial into its own ring region -------------------------
  WavePartial<D>& wp = *reinterpret_cast<WavePartial<D>*>(ring);
  {
    const float lt = row_bcast(oz[1], 0);   // row 1: the sum of p
    const float zv = row_bcast(oz[0], 0);   // row 0: the V zero-point term
#pragma unroll
    for (int mv = 0; mv < NVM; ++mv) {
      const int p = VL::slice_of(mv);
      const float fac = kTwo24 * __builtin_ldexpf(1.0f, -p * VNB);
      f4 a = accv[mv];
      if (kVChain && p > 0) a -= accv[VL::mfma_index(p - 1, VL::window_of(mv), VL::e_of(mv))];
      if (folded) {
#pragma unroll
        for (int i = 0; i < 4; ++i)  // column c < 4 adds column c + 4 (its remainders)
          a[i] += __builtin_bit_cast(float, dpp_banks<0x104, 0x1>(0u, __builtin_bit_cast(uint32_t, a[i])));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) wp.o[r][VL::dim_of(mv, 4 * j + i)] = fmaf(a[i], fac, zv);
    }
    if (j == 0) {
      wp.m[r] = m_run;
      wp.l[r] = lt;
    }
  }
  WavePartial<D>& wp0 = *reinterpret_cast<WavePartial<D>*>(smem);
  const MergeView view{&wp0.o[0][0], &wp0.m[0], &wp0.l[0], SM::WAVE / 4,
                       reinterpret_cast<int*>(smem + sizeof(WavePartial<D>))};
  merge_and_store<D, NW>(prm, view, b, h0, nh, split);
}
