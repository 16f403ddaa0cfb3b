// Flash-decoding split kernels (fused 2/4-bit and fp16 control) and the
// log-sum-exp combine kernel, for gfx950.
//
// Reference behaviour being reproduced:
//   _fused_decode_attn_split   kernels/fused_decode_attn.py:155-353
//   _fp16_decode_attn_split    kernels/fp16_decode_attn.py:47-135
//   _combine_splits            kernels/fused_decode_attn.py:355-395
//
// Design (MI355X-first, not a translation of the Triton program):
//   * One workgroup = one (split, batch row, kv head, block of <=16 query heads)
//     with NW waves.  All query heads of a GQA group share one pass over the
//     packed K/V, so the unpack is paid once per group.
//   * Each wave walks 32-token chunks of the split.  Scores come from
//     v_mfma_f32_16x16x{32,16}_f16 with tokens as rows and query heads as
//     columns (S^T = K Q^T); the quantized K codes enter the MFMA raw, as exact
//     fp16 subnormals, and each group's fp16 scale/zero is applied to the
//     group's partial dot product afterwards:
//         q.k = sum_g  s_g * (q_g . c_g)  +  z_g * sum(q_g)
//   * The output is accumulated as O^T = V^T P^T: the MFMA's C layout of S^T
//     is exactly the B layout P^T needs, so probabilities never leave
//     registers.  V codes again enter raw; the V scale is folded into P per
//     group (P'_g = P * s_g, packed fp16 multiply) and the V zero point
//     contributes sum_t z_tg p_t, accumulated in fp32.
//   * Online softmax in base 2 (logit = score * sm_scale * log2 e), wave-level
//     max via cross-lane shuffles; the rescale of the accumulators is skipped
//     when no head's running max moved.
//   * Per-token scale/zero rows of each chunk are staged in LDS by one
//     coalesced load per lane; the partial (m, l, acc) of the NW waves is
//     merged in LDS and written once per workgroup.
#include "tkv_codec.h"
#include "../../include/tkv.h"

namespace tkv {

struct SplitParams {
  const void* q;
  const uint8_t* k;
  const uint16_t* ks;
  const uint16_t* kz;
  const uint8_t* v;
  const uint16_t* vs;
  const uint16_t* vz;
  const int32_t* seq_lens;
  float* acc;
  float* maxs;
  float* sums;
  float* out;
  int HQ, HKV, S, G, num_splits, split_size, q_fp32;
  float qk_scale;  // sm_scale * log2(e)
};

constexpr int kChunk = 32;  // tokens per wave iteration (two 16-row MFMA tiles)

// Token of k-slot i (0..7) of lane-group j within a chunk: the rows 4j..4j+3
// of tile 0 followed by those of tile 1 -- the order in which the S^T
// accumulators of the two tiles hand P^T to the V MFMA without any shuffle.
__device__ __forceinline__ int slot_token(int j, int i) { return (i < 4 ? 0 : 12) + 4 * j + i; }

__device__ __forceinline__ float load_q(const SplitParams& p, int64_t idx) {
  return p.q_fp32 ? static_cast<const float*>(p.q)[idx]
                  : (float)static_cast<const _Float16*>(p.q)[idx];
}

// ---------------------------------------------------------------------------
// Online softmax over one chunk.  x[8]: scores of this lane's 8 tokens for
// its head, already -inf where masked; logit = x * lscale.  Updates m (shared
// by the four lanes of a head) and the lane's partial l; returns alpha, the
// factor the accumulators must be multiplied by (1 if no head moved), and the
// probabilities as 4 fp16 pairs in slot order plus fp32 values.
// ---------------------------------------------------------------------------
struct ChunkProbs {
  uint32_t ph[4];
  float p[8];
};

__device__ __forceinline__ bool softmax_chunk(const float (&x)[8], float lscale, float& m,
                                              float& l, float& alpha, ChunkProbs& out) {
  float mx = x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) mx = fmaxf(mx, x[i]);
  mx = xor_max16_32(mx) * lscale;
  const bool moved = mx > m;
  const bool any_moved = __builtin_amdgcn_ballot_w64(moved) != 0;
  alpha = 1.0f;
  if (any_moved) {
    const float mn = fmaxf(m, mx);
    alpha = safe_exp2_diff(m, mn);
    m = mn;
    l *= alpha;
  }
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    out.p[i] = __builtin_amdgcn_exp2f(fmaf(x[i], lscale, -m));
    sum += out.p[i];
  }
  l += sum;
#pragma unroll
  for (int i = 0; i < 4; ++i) out.ph[i] = pack_h2(out.p[2 * i], out.p[2 * i + 1]);
  return any_moved;
}

// ---------------------------------------------------------------------------
// Workgroup merge of the NW waves' (m, l, O) and the final store.
// o_lds[w][n][d] holds each wave's unnormalised output for head n.
// ---------------------------------------------------------------------------
template <int D, int NW>
struct MergeLds {
  float m[NW][16];
  float l[NW][16];
  float o[NW][16][D + 1];
};

template <int D, int NW>
__device__ void merge_and_store(const SplitParams& prm, MergeLds<D, NW>& lds, int b, int h0,
                                int nh, int split) {
  __syncthreads();
  const int tid = threadIdx.x;
  for (int idx = tid; idx < nh * D; idx += NW * 64) {
    const int n = idx / D, d = idx % D;
    float mstar = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mstar = fmaxf(mstar, lds.m[w][n]);
    float o = 0.0f, l = 0.0f;
    if (mstar != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = safe_exp2_diff(lds.m[w][n], mstar);
        o = fmaf(f, lds.o[w][n][d], o);
        l = fmaf(f, lds.l[w][n], l);
      }
    }
    const int64_t row = (int64_t)b * prm.HQ + h0 + n;
    if (prm.num_splits == 1) {
      prm.out[row * D + d] = o / l;
    } else {
      const int64_t pr = row * prm.num_splits + split;
      prm.acc[pr * D + d] = o;
      if (d == 0) {
        prm.maxs[pr] = mstar;
        prm.sums[pr] = l;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Per-wave LDS staging of the chunk's scale/zero rows: 4 tensors (K scale,
// K zero, V scale, V zero) x 32 tokens x NG fp16, one coalesced load per lane
// and tensor.  Token rows past the split end are clamped to its last token
// (their scores are masked, but their metadata must stay finite).
// ---------------------------------------------------------------------------
template <int NG>
struct MetaLds {
  uint32_t t[4][kChunk * NG / 2 > 0 ? kChunk * NG / 2 : 1];
};

template <int NG>
__device__ __forceinline__ void stage_meta(MetaLds<NG>& ml, const uint16_t* const (&src)[4],
                                           int64_t row0, int cb, int hi, int lane) {
  if constexpr (NG >= 2) {
    constexpr int DW = NG / 2;  // dwords per token row
#pragma unroll
    for (int idx = lane; idx < kChunk * DW; idx += 64) {
      const int tok = idx / DW, dw = idx % DW;
      const int row = min(cb + tok, hi - 1);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        ml.t[t][idx] = reinterpret_cast<const uint32_t*>(src[t] + (row0 + row) * NG)[dw];
    }
  } else {
    uint16_t* h = reinterpret_cast<uint16_t*>(&ml.t[0][0]);
    if (lane < kChunk) {
      const int row = min(cb + lane, hi - 1);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        reinterpret_cast<uint16_t*>(&ml.t[t][0])[lane] = src[t][row0 + row];
    }
    (void)h;
  }
}

// fp16 value of group g of token `tok` in tensor t.
template <int NG>
__device__ __forceinline__ float meta_val(const MetaLds<NG>& ml, int t, int tok, int g) {
  const uint16_t bits = reinterpret_cast<const uint16_t*>(&ml.t[t][0])[tok * NG + g];
  return (float)__builtin_bit_cast(_Float16, bits);
}
// fp16 pair (token tok, group g) and (token tok+1, group g) of tensor t.
template <int NG>
__device__ __forceinline__ uint32_t meta_pair(const MetaLds<NG>& ml, int t, int tok, int g) {
  const uint16_t* h = reinterpret_cast<const uint16_t*>(&ml.t[t][0]);
  return (uint32_t)h[tok * NG + g] | ((uint32_t)h[(tok + 1) * NG + g] << 16);
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ===========================================================================
// Fused quantized split kernel.
// ===========================================================================
template <int D, int KNB, int VNB, int GS, int NW>
__global__ void __launch_bounds__(NW * 64)
quant_split_kernel(SplitParams prm) {
  using KL = KLayout<D, KNB, GS>;
  using VL = VLayout<D, VNB, GS>;
  constexpr int NG = D / GS;
  constexpr int NKM = KL::NKM;
  constexpr int NVM = VL::NVM;

  __shared__ MergeLds<D, NW> mlds;
  __shared__ MetaLds<NG> meta[NW];

  const int split = blockIdx.x;
  const int unit = blockIdx.y;
  const int b = unit / prm.HKV, hk = unit % prm.HKV;
  const int hb0 = blockIdx.z * 16;
  const int nh = min(16, prm.G - hb0);
  const int h0 = hk * prm.G + hb0;
  const int L = prm.seq_lens ? min(prm.seq_lens[b], prm.S) : prm.S;
  const int lo = split * prm.split_size;
  const int hi = min(lo + prm.split_size, L);

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int r = lane & 15, j = lane >> 4;  // MFMA row/col index and lane-group
  const int n = r;                         // query head (column) of this lane
  const int64_t row0 = (int64_t)unit * prm.S;  // first cache row of this (b, kv head)

  // ---- Q^T operand in K slot order, pre-scaled by 2^-(slice*KNB) ---------
  u4 qf[NKM];
  float qz[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) qz[g] = 0.0f;
  {
    const bool hv = n < nh;
    const int64_t qrow = ((int64_t)b * prm.HQ + h0 + (hv ? n : 0)) * D;
#pragma unroll
    for (int m = 0; m < NKM; ++m) {
      const int p = KL::slice_of(m, j);
      const float pre = __builtin_ldexpf(1.0f, -p * KNB);
      uint32_t wv[4] = {0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < KL::CB; s += 2) {
        float q0 = 0.0f, q1 = 0.0f;
        if (hv) {
          q0 = (float)(_Float16)load_q(prm, qrow + KL::dim_of(m, j, s));
          q1 = (float)(_Float16)load_q(prm, qrow + KL::dim_of(m, j, s + 1));
        }
        qz[KL::group_of_step(m)] += q0 + q1;
        wv[s / 2] = pack_h2(q0 * pre, q1 * pre);
      }
      qf[m] = u4{wv[0], wv[1], wv[2], wv[3]};
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) qz[g] = xor_sum16_32(qz[g]) * kTwoM24;
  }

  // ---- per-lane constants of the V unpack -------------------------------
  uint32_t vsel[VL::NE];
#pragma unroll
  for (int e = 0; e < VL::NE; ++e) vsel[e] = VL::perm_sel(VL::byte_in_dword(e, r));
  uint32_t kmask[NKM];
#pragma unroll
  for (int m = 0; m < NKM; ++m) kmask[m] = slice_mask<KNB>(KL::slice_of(m, j));

  f4 accv[NVM];
#pragma unroll
  for (int mv = 0; mv < NVM; ++mv) accv[mv] = f4{0.f, 0.f, 0.f, 0.f};
  float ozp[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) ozp[g] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const float lscale = prm.qk_scale * kTwo24;

  const uint8_t* kbase = prm.k + row0 * KL::DP;
  const uint8_t* vbase = prm.v + row0 * VL::DP;
  const uint16_t* const msrc[4] = {prm.ks, prm.kz, prm.vs, prm.vz};
  MetaLds<NG>& ml = meta[w];

  for (int cb = lo + kChunk * w; cb < hi; cb += kChunk * NW) {
    // ---- issue loads -------------------------------------------------------
    wave_lds_fence();
    stage_meta<NG>(ml, msrc, row0, cb, hi, lane);

    typename std::conditional<KL::CB == 8, u2, uint32_t>::type kx[2][KL::NLOAD];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int tr = min(cb + 16 * a + r, hi - 1);
#pragma unroll
      for (int Lh = 0; Lh < KL::NLOAD; ++Lh) {
        const uint8_t* src = kbase + (int64_t)tr * KL::DP + KL::load_offset(Lh, j);
        if constexpr (KL::CB == 8) kx[a][Lh] = ld_u2(src);
        else kx[a][Lh] = ld_u32(src);
      }
    }
    uint32_t vx[8][VL::NWIN];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int tr = min(cb + slot_token(j, i), hi - 1);
#pragma unroll
      for (int wi = 0; wi < VL::NWIN; ++wi)
        vx[i][wi] = ld_u32(vbase + (int64_t)tr * VL::DP + VL::dword_offset(wi, r));
    }
    wave_lds_fence();

    // ---- scores S^T for the two 16-token tiles -----------------------------
    float x[8];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      f4 c[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) c[g] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < NKM; ++m) {
        const int g = KL::group_of_step(m);
        if constexpr (KL::CB == 8)
          c[g] = mfma_k32(k_extract8(kx[a][KL::load_of_step(m)], kmask[m]), qf[m], c[g]);
        else
          c[g] = mfma_k16(k_extract4(kx[a][KL::load_of_step(m)], kmask[m]),
                          u2{qf[m][0], qf[m][1]}, c[g]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = 16 * a + 4 * j + i;
        float sc = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          sc = fmaf(meta_val<NG>(ml, 0, tok, g), c[g][i], sc);
          sc = fmaf(meta_val<NG>(ml, 1, tok, g), qz[g], sc);
        }
        x[4 * a + i] = (cb + tok < hi) ? sc : -INFINITY;
      }
    }

    // ---- online softmax ----------------------------------------------------
    float alpha;
    ChunkProbs pr;
    if (softmax_chunk(x, lscale, m_run, l_run, alpha, pr)) {
#pragma unroll
      for (int mv = 0; mv < NVM; ++mv) accv[mv] *= alpha;
#pragma unroll
      for (int g = 0; g < NG; ++g) ozp[g] *= alpha;
    }

    // ---- V: zero-point term and P'_g = P * s_g -----------------------------
    u4 pg[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float oz = ozp[g];
#pragma unroll
      for (int i = 0; i < 8; ++i) oz = fmaf(meta_val<NG>(ml, 3, slot_token(j, i), g), pr.p[i], oz);
      ozp[g] = oz;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pg[g][i] = pk_mul(pr.ph[i], meta_pair<NG>(ml, 2, slot_token(j, 2 * i), g));
    }

    // ---- O^T += V^T P'^T ---------------------------------------------------
#pragma unroll
    for (int wi = 0; wi < VL::NWIN; ++wi) {
#pragma unroll
      for (int e = 0; e < VL::NE; ++e) {
        uint32_t pm[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pm[i] = perm(vx[2 * i + 1][wi], vx[2 * i][wi], vsel[e]);
#pragma unroll
        for (int p = 0; p < VL::P; ++p) {
          const int mv = VL::mfma_index(p, wi, e);
          const uint32_t msk = slice_mask<VNB>(p);
          const u4 av = u4{pm[0] & msk, pm[1] & msk, pm[2] & msk, pm[3] & msk};
          accv[mv] = mfma_k32(av, pg[VL::group_of(mv)], accv[mv]);
        }
      }
    }
  }

  // ---- this wave's partial into LDS ---------------------------------------
  {
    float ozt[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) ozt[g] = xor_sum16_32(ozp[g]);
    const float lt = xor_sum16_32(l_run);
#pragma unroll
    for (int mv = 0; mv < NVM; ++mv) {
      const float fac = kTwo24 * __builtin_ldexpf(1.0f, -VL::slice_of(mv) * VNB);
      const float oz = ozt[VL::group_of(mv)];
#pragma unroll
      for (int i = 0; i < 4; ++i) mlds.o[w][n][VL::dim_of(mv, 4 * j + i)] = fmaf(accv[mv][i], fac, oz);
    }
    if (j == 0) {
      mlds.m[w][n] = m_run;
      mlds.l[w][n] = lt;
    }
  }
  merge_and_store<D, NW>(prm, mlds, b, h0, nh, split);
}

// ===========================================================================
// fp16 control split kernel: same split, softmax, GQA grouping, merge and
// combine; K/V read as fp16 (kernels/fp16_decode_attn.py:16-22 -- the control
// differs from the fused kernel only in how K/V are read).
// ===========================================================================
template <int D, int NW>
__global__ void __launch_bounds__(NW * 64)
fp16_split_kernel(SplitParams prm) {
  constexpr int NKM = D / 32;   // 16x16x32 steps over the head dim
  constexpr int EPL = D / 16;   // V dims per lane (and V MFMAs)
  __shared__ MergeLds<D, NW> mlds;

  const int split = blockIdx.x;
  const int unit = blockIdx.y;
  const int b = unit / prm.HKV, hk = unit % prm.HKV;
  const int hb0 = blockIdx.z * 16;
  const int nh = min(16, prm.G - hb0);
  const int h0 = hk * prm.G + hb0;
  const int L = prm.seq_lens ? min(prm.seq_lens[b], prm.S) : prm.S;
  const int lo = split * prm.split_size;
  const int hi = min(lo + prm.split_size, L);

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int r = lane & 15, j = lane >> 4;
  const int n = r;
  const int64_t row0 = (int64_t)unit * prm.S;

  u4 qf[NKM];
  {
    const bool hv = n < nh;
    const int64_t qrow = ((int64_t)b * prm.HQ + h0 + (hv ? n : 0)) * D;
#pragma unroll
    for (int m = 0; m < NKM; ++m) {
      uint32_t wv[4];
#pragma unroll
      for (int s = 0; s < 8; s += 2) {
        float q0 = 0.0f, q1 = 0.0f;
        if (hv) {
          q0 = load_q(prm, qrow + 32 * m + 8 * j + s);
          q1 = load_q(prm, qrow + 32 * m + 8 * j + s + 1);
        }
        wv[s / 2] = pack_h2(q0, q1);
      }
      qf[m] = u4{wv[0], wv[1], wv[2], wv[3]};
    }
  }

  f4 accv[EPL];
#pragma unroll
  for (int mv = 0; mv < EPL; ++mv) accv[mv] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  const float lscale = prm.qk_scale;
  const _Float16* kbase = reinterpret_cast<const _Float16*>(prm.k) + row0 * D;
  const _Float16* vbase = reinterpret_cast<const _Float16*>(prm.v) + row0 * D;

  for (int cb = lo + kChunk * w; cb < hi; cb += kChunk * NW) {
    u4 kx[2][NKM];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int tr = min(cb + 16 * a + r, hi - 1);
#pragma unroll
      for (int m = 0; m < NKM; ++m)
        kx[a][m] = *reinterpret_cast<const u4*>(kbase + (int64_t)tr * D + 32 * m + 8 * j);
    }
    uint32_t vx[8][EPL / 2];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int tr = min(cb + slot_token(j, i), hi - 1);
      const uint32_t* src = reinterpret_cast<const uint32_t*>(vbase + (int64_t)tr * D + EPL * r);
#pragma unroll
      for (int q = 0; q < EPL / 2; ++q) vx[i][q] = src[q];
    }

    float x[8];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      f4 c = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < NKM; ++m) c = mfma_k32(kx[a][m], qf[m], c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = 16 * a + 4 * j + i;
        x[4 * a + i] = (cb + tok < hi) ? c[i] : -INFINITY;
      }
    }

    float alpha;
    ChunkProbs pr;
    if (softmax_chunk(x, lscale, m_run, l_run, alpha, pr)) {
#pragma unroll
      for (int mv = 0; mv < EPL; ++mv) accv[mv] *= alpha;
    }
    const u4 pb = u4{pr.ph[0], pr.ph[1], pr.ph[2], pr.ph[3]};
#pragma unroll
    for (int mv = 0; mv < EPL; ++mv) {
      const uint32_t sel = (mv & 1) ? 0x07060302u : 0x05040100u;
      u4 av;
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = perm(vx[2 * i + 1][mv / 2], vx[2 * i][mv / 2], sel);
      accv[mv] = mfma_k32(av, pb, accv[mv]);
    }
  }

  {
    const float lt = xor_sum16_32(l_run);
#pragma unroll
    for (int mv = 0; mv < EPL; ++mv)
#pragma unroll
      for (int i = 0; i < 4; ++i) mlds.o[w][n][EPL * (4 * j + i) + mv] = accv[mv][i];
    if (j == 0) {
      mlds.m[w][n] = m_run;
      mlds.l[w][n] = lt;
    }
  }
  merge_and_store<D, NW>(prm, mlds, b, h0, nh, split);
}

// ===========================================================================
// Combine: out[b,h,:] = sum_s 2^(m_s - m*) acc_s / sum_s 2^(m_s - m*) l_s.
// One 256-thread workgroup per (b, h).  Thread (sg, dq) owns float4 column dq
// of the splits s = sg, sg + SG, ...: it streams them with an online
// log-sum-exp merge (all loads of an iteration are independent of the
// previous one, so they stay in flight together), then the SG split groups
// are merged through LDS.  Empty splits (m_s = -inf, only possible with
// per-row lengths) contribute nothing.
// ===========================================================================
template <int D>
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ acc,
                                                      const float* __restrict__ maxs,
                                                      const float* __restrict__ sums,
                                                      float* __restrict__ out, int ns) {
  constexpr int DQ = D / 4;     // float4 columns of a split row
  constexpr int SG = 256 / DQ;  // split groups
  __shared__ float sm_m[SG], sm_l[SG];
  __shared__ f4 sm_a[SG][DQ];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, dq = t % DQ, sg = t / DQ;
  float m = -INFINITY, l = 0.0f;
  f4 a = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int s = sg; s < ns; s += SG) {
    const int64_t ps = row * ns + s;
    const float ms = maxs[ps];
    const float ls = sums[ps];
    const f4 as = reinterpret_cast<const f4*>(acc + ps * D)[dq];
    if (ms == -INFINITY) continue;
    const float mn = fmaxf(m, ms);
    const float al = safe_exp2_diff(m, mn);
    const float be = __builtin_amdgcn_exp2f(ms - mn);
    a = a * al + as * be;
    l = l * al + ls * be;
    m = mn;
  }
  if (dq == 0) {
    sm_m[sg] = m;
    sm_l[sg] = l;
  }
  sm_a[sg][dq] = a;
  __syncthreads();
  if (sg == 0) {
    float mstar = -INFINITY;
#pragma unroll
    for (int g = 0; g < SG; ++g) mstar = fmaxf(mstar, sm_m[g]);
    f4 o = f4{0.f, 0.f, 0.f, 0.f};
    float lt = 0.0f;
#pragma unroll
    for (int g = 0; g < SG; ++g) {
      const float f = safe_exp2_diff(sm_m[g], mstar);
      o += sm_a[g][dq] * f;
      lt += sm_l[g] * f;
    }
    reinterpret_cast<f4*>(out + row * D)[dq] = o / lt;
  }
}

// ===========================================================================
// Host side: validation and dispatch.
// ===========================================================================
constexpr int kWaves = 4;

static int validate_common(const tkv_decode_args* a) {
  if (!a || !a->q || !a->k || !a->v || !a->out) return TKV_EINVAL;
  if (a->B <= 0 || a->HQ <= 0 || a->HKV <= 0 || a->S <= 0 || a->D <= 0) return TKV_EINVAL;
  if (a->HQ % a->HKV) return TKV_EINVAL;
  if (a->split_size <= 0 || a->num_splits <= 0) return TKV_EINVAL;
  if ((int64_t)a->split_size * (a->num_splits - 1) >= a->S) return TKV_EINVAL;  // empty split
  if ((int64_t)a->split_size * a->num_splits < a->S) return TKV_EINVAL;        // uncovered
  if (a->num_splits > 1 && (!a->acc || !a->maxs || !a->sums)) return TKV_EINVAL;
  // Vector loads: caches 16-byte aligned, metadata 4-byte, partials 8-byte.
  if (((uintptr_t)a->k | (uintptr_t)a->v) & 15) return TKV_EINVAL;
  if (((uintptr_t)a->k_scale | (uintptr_t)a->k_zero | (uintptr_t)a->v_scale |
       (uintptr_t)a->v_zero | (uintptr_t)a->q) & 3)
    return TKV_EINVAL;
  if (((uintptr_t)a->acc | (uintptr_t)a->out) & 15) return TKV_EINVAL;  // float4 rows
  if (a->D != 64 && a->D != 128) return TKV_EUNSUPPORTED;
  return TKV_OK;
}

static SplitParams make_params(const tkv_decode_args* a) {
  SplitParams p;
  p.q = a->q;
  p.k = static_cast<const uint8_t*>(a->k);
  p.ks = static_cast<const uint16_t*>(a->k_scale);
  p.kz = static_cast<const uint16_t*>(a->k_zero);
  p.v = static_cast<const uint8_t*>(a->v);
  p.vs = static_cast<const uint16_t*>(a->v_scale);
  p.vz = static_cast<const uint16_t*>(a->v_zero);
  p.seq_lens = a->seq_lens;
  p.acc = a->acc;
  p.maxs = a->maxs;
  p.sums = a->sums;
  p.out = a->out;
  p.HQ = a->HQ;
  p.HKV = a->HKV;
  p.S = a->S;
  p.G = a->HQ / a->HKV;
  p.num_splits = a->num_splits;
  p.split_size = a->split_size;
  p.q_fp32 = a->q_is_fp32 ? 1 : 0;
  p.qk_scale = a->sm_scale * kLog2e;
  return p;
}

static dim3 split_grid(const tkv_decode_args* a) {
  const int G = a->HQ / a->HKV;
  return dim3((unsigned)a->num_splits, (unsigned)(a->B * a->HKV), (unsigned)((G + 15) / 16));
}

template <int D, int KNB, int VNB, int GS>
static void launch_quant(const SplitParams& p, dim3 grid, hipStream_t st) {
  quant_split_kernel<D, KNB, VNB, GS, kWaves><<<grid, dim3(kWaves * 64), 0, st>>>(p);
}

template <int D, int KNB, int VNB>
static int dispatch_gs(const SplitParams& p, dim3 grid, int gs, hipStream_t st) {
  switch (gs) {
    case 16: launch_quant<D, KNB, VNB, 16>(p, grid, st); return TKV_OK;
    case 32: launch_quant<D, KNB, VNB, 32>(p, grid, st); return TKV_OK;
    case 64: launch_quant<D, KNB, VNB, 64>(p, grid, st); return TKV_OK;
    case 128:
      if constexpr (D >= 128) {
        launch_quant<D, KNB, VNB, 128>(p, grid, st);
        return TKV_OK;
      }
      return TKV_EUNSUPPORTED;
    default: return TKV_EUNSUPPORTED;
  }
}

template <int D>
static int dispatch_bits(const SplitParams& p, dim3 grid, int knb, int vnb, int gs, hipStream_t st) {
  if (knb == 4 && vnb == 4) return dispatch_gs<D, 4, 4>(p, grid, gs, st);
  if (knb == 2 && vnb == 2) return dispatch_gs<D, 2, 2>(p, grid, gs, st);
  if (knb == 4 && vnb == 2) return dispatch_gs<D, 4, 2>(p, grid, gs, st);
  if (knb == 2 && vnb == 4) return dispatch_gs<D, 2, 4>(p, grid, gs, st);
  return TKV_EUNSUPPORTED;
}

static int launch_combine(const float* acc, const float* maxs, const float* sums, float* out,
                          int B, int HQ, int ns, int D, hipStream_t st) {
  const dim3 grid((unsigned)(B * HQ));
  if (D == 128)
    combine_kernel<128><<<grid, dim3(256), 0, st>>>(acc, maxs, sums, out, ns);
  else if (D == 64)
    combine_kernel<64><<<grid, dim3(256), 0, st>>>(acc, maxs, sums, out, ns);
  else
    return TKV_EUNSUPPORTED;
  return TKV_OK;
}

static int status_of_launch() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TKV_OK : (int)e;
}

}  // namespace tkv

namespace tkv {

static int launch_fused_split(const tkv_decode_args* a, hipStream_t st) {
  int rc = validate_common(a);
  if (rc) return rc;
  if (!a->k_scale || !a->k_zero || !a->v_scale || !a->v_zero) return TKV_EINVAL;
  const int gs = a->group_size;
  if (gs <= 0 || gs > a->D || a->D % gs) return TKV_EINVAL;
  if ((a->k_nbits != 2 && a->k_nbits != 4) || (a->v_nbits != 2 && a->v_nbits != 4))
    return TKV_EINVAL;
  const SplitParams p = make_params(a);
  const dim3 grid = split_grid(a);
  (void)hipGetLastError();
  rc = a->D == 128 ? dispatch_bits<128>(p, grid, a->k_nbits, a->v_nbits, gs, st)
                   : dispatch_bits<64>(p, grid, a->k_nbits, a->v_nbits, gs, st);
  if (rc) return rc;
  return status_of_launch();
}

static int launch_fp16_split(const tkv_decode_args* a, hipStream_t st) {
  const int rc = validate_common(a);
  if (rc) return rc;
  const SplitParams p = make_params(a);
  const dim3 grid = split_grid(a);
  (void)hipGetLastError();
  if (a->D == 128)
    fp16_split_kernel<128, kWaves><<<grid, dim3(kWaves * 64), 0, st>>>(p);
  else
    fp16_split_kernel<64, kWaves><<<grid, dim3(kWaves * 64), 0, st>>>(p);
  return status_of_launch();
}

static int finish_combine(const tkv_decode_args* a, hipStream_t st) {
  if (a->num_splits <= 1) return TKV_OK;
  (void)hipGetLastError();
  launch_combine(a->acc, a->maxs, a->sums, a->out, a->B, a->HQ, a->num_splits, a->D, st);
  return status_of_launch();
}

}  // namespace tkv

extern "C" int tkv_fused_decode_split(const tkv_decode_args* a, tkv_stream_t stream) {
  return tkv::launch_fused_split(a, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int tkv_fp16_decode_split(const tkv_decode_args* a, tkv_stream_t stream) {
  return tkv::launch_fp16_split(a, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int tkv_fused_decode_attention(const tkv_decode_args* a, tkv_stream_t stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int rc = tkv::launch_fused_split(a, st);
  return rc ? rc : tkv::finish_combine(a, st);
}

extern "C" int tkv_fp16_decode_attention(const tkv_decode_args* a, tkv_stream_t stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int rc = tkv::launch_fp16_split(a, st);
  return rc ? rc : tkv::finish_combine(a, st);
}

extern "C" int tkv_combine_splits(const float* acc, const float* maxs, const float* sums,
                                  float* out, int32_t B, int32_t HQ, int32_t num_splits,
                                  int32_t D, tkv_stream_t stream) {
  using namespace tkv;
  if (!acc || !maxs || !sums || !out || B <= 0 || HQ <= 0 || num_splits <= 0) return TKV_EINVAL;
  if (((uintptr_t)acc | (uintptr_t)out) & 15) return TKV_EINVAL;
  if (D != 64 && D != 128) return TKV_EUNSUPPORTED;
  (void)hipGetLastError();
  launch_combine(acc, maxs, sums, out, B, HQ, num_splits, D, reinterpret_cast<hipStream_t>(stream));
  return status_of_launch();
}
