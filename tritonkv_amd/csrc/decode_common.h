// Shared pieces of the flash-decoding split kernels (gfx950): arguments, the
// online-softmax step, the workgroup merge of the waves' partials and the
// q operands of the quantized kernel.
#pragma once

#include <type_traits>
#include <utility>

#include "tkv_codec.h"
#include "tkv_quant.h"
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
  int* counters;  // fused-combine tickets, or null
  // Paged caches (page_size > 0): the K/V tensors are pools of pages laid out
  // (num_pages, HKV, page_size, ...); logical page p of batch row b is pool
  // page block_table[b * bt_stride + p].  S = bt_stride * page_size.
  const int32_t* block_table;
  int bt_stride, page_size, num_pages;
  // Fused append (quantized path): if k_new is set, the token at L_b - 1 of
  // every (b, kv head) is k_new/v_new[b][kv] (fp16, or fp32 if new_fp32),
  // quantized into the cache by the step itself.
  const void* k_new;
  const void* v_new;
  int new_fp32;
  int HQ, HKV, S, G, num_splits, split_size, q_fp32;
  float qk_scale;  // sm_scale * log2(e)
  // Per-channel keys (quantized path): key_block == 32 makes ks/kz
  // (B, HKV, S/32, D), one fp16 scale and zero per (32-token block, channel).
  int key_block;
  // This launch's splits are partial rows split_base + split of ns_total.
  int split_base, ns_total;
  // Dispatch order (quantized path), or null: workgroup i = y * gridDim.x + x
  // of each z slice reads the pair order[2i], order[2i + 1] = (idx, L) and runs
  // (unit, split) = (idx % gridDim.x, idx / gridDim.x) of a row of L tokens
  // (min(seq_lens[b], S), carried here so the prologue's dependent loads stay
  // one deep).  A permutation, so every (unit, split) runs once and writes its
  // own partial row: the result does not depend on it.
  const int32_t* order;
  // Dims-split kernels on fewer than 8 (unit, split, head block) tuples:
  // B * HKV, the units their (8 * VS)-workgroup grid maps onto; 0 for every
  // other launch (a flag in the argument block, which the prologue loads
  // anyway: the grid's own size would be another load).
  int xcd_units;
};

// Longest piece first: the dispatch order ragged_order_kernel writes.  Piece
// (b, s) is tokens [s * ss, min((s + 1) * ss, L_b)) of row b (empty past the
// row's end); pieces are ranked by length, longest first, ties by s * B + b
// (the natural y-major order), and the HKV units of a piece take consecutive
// slots.  The dispatcher starts workgroups in slot order as CUs free up, so
// the short pieces fill the gaps at the end instead of a full piece of a long
// row starting last.  The rank of piece (b, s), of length len, is the sum over
// rows b2 of ragged_rank_term, where row b2 (length clamped to [0, S]) holds
// f2 full pieces and a remainder of r2 tokens (divided once per row, so the
// sum itself needs no division).
__host__ __device__ inline int ragged_rank_term(int len, int s, int b, int ss, int b2, int f2,
                                                int r2) {
  // Selects, not branches: len differs from lane to lane.
  const int n2 = f2 + (r2 > 0 ? 1 : 0);     // non-empty pieces
  const int before = s + (b2 < b ? 1 : 0);  // pieces s2 of row b2 with s2 * B + b2 < s * B + b
  const int longer = (len < ss ? f2 : 0) + (r2 > len ? 1 : 0);  // full pieces, a longer remainder
  const int tie_full = min(f2, before);
  const int tie_rem = (r2 == len && f2 < before) ? 1 : 0;
  const int tie_empty = max(0, before - n2);  // empty pieces s2 in [n2, before)
  return longer + (len == ss ? tie_full : (len > 0 ? tie_rem : tie_empty));
}

template <class Lens>
__host__ __device__ inline int ragged_piece_rank(int b, int s, int B, int ss, Lens lens) {
  const int len = max(0, min(lens(b) - s * ss, ss));
  int rank = 0;
  for (int b2 = 0; b2 < B; ++b2) {
    const int L2 = lens(b2), f2 = L2 / ss;
    rank += ragged_rank_term(len, s, b, ss, b2, f2, L2 - f2 * ss);
  }
  return rank;
}

constexpr int kChunk = 32;  // tokens per wave iteration (two 16-row MFMA tiles)

// Cache policies of the streamed loads.
constexpr int kPolF16 = kPolicyNT;       // fp16 control K and V rows
constexpr int kPolDma = kPolicyNT;       // LDS-staged kernel: K/V code and metadata ranges

// Token of k-slot i (0..7) of lane-group j within a chunk: the rows 4j..4j+3
// of tile 0 followed by those of tile 1 -- the order in which the S^T
// accumulators of the two tiles hand P^T to the V MFMA without any shuffle.
__device__ __forceinline__ int slot_token(int j, int i) { return (i < 4 ? 0 : 12) + 4 * j + i; }


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

// The lane's own max decides first whether any head moved (a head's max rises
// above m exactly when one of its lanes' does); the cross-lane max runs only
// in chunks where one did.  The reference m stays the exact running max: a
// dominant token then enters the PV products as p = 1 exactly, with no fp16
// rounding.  (A lagging reference -- a rescale only when the max rises by
// more than a few units -- rounds that p: 5.6e-3 max-abs instead of 6.6e-5
// on a dominant-token head of 2-bit values.)
// BIAS: the logits are x * lscale + bl, bl the lane's (head's) chunk-wide
// offset, folded into the max and the exponent instead of an add per score.
template <bool TRACK_L = true, bool BIAS = false>
__device__ __forceinline__ bool softmax_chunk(const float (&x)[8], float lscale, float& m,
                                              float& l, float& alpha, ChunkProbs& out,
                                              float bl = 0.0f) {
  float lm = x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) lm = fmaxf(lm, x[i]);
  lm = BIAS ? fmaf(lm, lscale, bl) : lm * lscale;
  const bool any_moved = __builtin_amdgcn_ballot_w64(lm > m) != 0;
  alpha = 1.0f;
  if (any_moved) {
    const float mn = vmax(m, xor_max16_32(lm));
    alpha = safe_exp2_diff(m, mn);
    m = mn;
    if constexpr (TRACK_L) l *= alpha;
  }
  float sum = 0.0f;
  const float off = BIAS ? bl - m : -m;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    out.p[i] = __builtin_amdgcn_exp2f(fmaf(x[i], lscale, off));
    if constexpr (TRACK_L) sum += out.p[i];
  }
  if constexpr (TRACK_L) l += sum;
#pragma unroll
  for (int i = 0; i < 4; ++i) out.ph[i] = pack_h2(out.p[2 * i], out.p[2 * i + 1]);
  return any_moved;
}

// ---------------------------------------------------------------------------
// Workgroup merge of the NW waves' (m, l, O) and the final store.
// o_lds[w][n][d] holds each wave's unnormalised output for head n.
// ---------------------------------------------------------------------------
// Where a kernel keeps each wave's partial in LDS: output row n of wave w at
// o + w * stride + n * (D + 1), its running max and sum at m / l + w * stride + n.
struct MergeView {
  float* o;
  float* m;
  float* l;
  int stride;  // floats between consecutive waves
  int* last;   // this workgroup holds the final ticket of its unit
};

template <int D>
struct WavePartial {
  float o[16][D + 1];
  float m[16];
  float l[16];
};

template <int D, int NW>
struct MergeLds {
  WavePartial<D> wp[NW];
  int last;
  __device__ MergeView view() {
    constexpr int stride = sizeof(WavePartial<D>) / 4;
    return MergeView{&wp[0].o[0][0], &wp[0].m[0], &wp[0].l[0], stride, &last};
  }
};

// Agent-scope relaxed atomic store / load of a float: coherent across XCDs
// without fences (global_store / global_load with sc1 on gfx950).
__device__ __forceinline__ void coherent_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// DN < D: this workgroup holds dims [d0, d0 + DN) of the output (the
// dims-split kernels); the maxima and sums go out with dim 0's workgroup.
// Those kernels never run the fused combine below.
template <int D, int NW, int DN = D>
__device__ void merge_and_store(const SplitParams& prm, const MergeView& mv, int b, int h0,
                                int nh, int split, int d0 = 0) {
  __syncthreads();
  const int tid = threadIdx.x;
  // Each thread merges four consecutive dims of one head: every thread of
  // the workgroup takes at most one item (at most 16 heads x DN / 4), so the
  // two LDS round trips (the waves' maxima, then their partials) are paid
  // once, not once per element.
  constexpr int DQ4 = DN / 4;
  for (int idx = tid; idx < nh * DQ4; idx += NW * 64) {
    const int n = idx / DQ4, d = d0 + 4 * (idx % DQ4);
    float mw[NW];
    float mstar = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      mw[w] = mv.m[w * mv.stride + n];
      mstar = fmaxf(mstar, mw[w]);
    }
    f4 o = f4{0.f, 0.f, 0.f, 0.f};
    float l = 0.0f;
    if (mstar != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = safe_exp2_diff(mw[w], mstar);
        const float* ow = mv.o + w * mv.stride + n * (D + 1) + d;
        o = o + f4{ow[0], ow[1], ow[2], ow[3]} * f;
        l = fmaf(f, mv.l[w * mv.stride + n], l);
      }
    } else {
      // No wave saw a finite score for this head.  Every wave's o and l are
      // then 0 (no tokens), or NaN where its scores were NaN (a NaN key in the
      // cache); the sum keeps the NaN, as the reference's softmax would.
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float* ow = mv.o + w * mv.stride + n * (D + 1) + d;
        o = o + f4{ow[0], ow[1], ow[2], ow[3]};
        l += mv.l[w * mv.stride + n];
      }
    }
    const int64_t row = (int64_t)b * prm.HQ + h0 + n;
    if (prm.ns_total == 1) {
      *reinterpret_cast<f4*>(prm.out + row * D + d) = o / l;
    } else {
      const int64_t pr = row * prm.ns_total + prm.split_base + split;
      if (prm.counters) {  // read back inside this launch: see the fused combine below
#pragma unroll
        for (int e = 0; e < 4; ++e) coherent_store(prm.acc + pr * D + d + e, o[e]);
        if (d == 0) {
          coherent_store(prm.maxs + pr, mstar);
          coherent_store(prm.sums + pr, l);
        }
      } else {
        *reinterpret_cast<f4*>(prm.acc + pr * D + d) = o;
        if (d == 0) {
          prm.maxs[pr] = mstar;
          prm.sums[pr] = l;
        }
      }
    }
  }
  if (prm.ns_total == 1 || prm.counters == nullptr || DN < D) return;  // counters: split_base 0, all splits

  // Fused combine.  Each workgroup publishes its partials and takes a ticket;
  // the one that draws the last ticket reads everyone's partials and merges
  // the splits of its rows, then resets the counter for the next call.  The
  // reader may sit on another XCD, whose L2 is not coherent with this one, so
  // the partials move as agent-scope atomic stores and loads, which the
  // memory model makes coherent across XCDs by themselves: the stores write
  // through the L2 and the loads fetch past it (sc1 on gfx950).  The stores
  // then only have to be complete before the ticket is taken (each thread
  // waits for its own, then the barrier), which is the release sequence of
  // the memory model without its L2 writeback (buffer_wbl2): that writeback
  // is only needed for plain stores, and it made the merge 5 us slower at the
  // Qwen2.5-1.5B shape (ctx 2048, 16 splits: 15.1 us per call with it, 9.8
  // without; a separate combine launch: 7.7).
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  __syncthreads();
  const int cidx = (b * prm.HKV + h0 / prm.G) * ((prm.G + 15) / 16) + (h0 % prm.G) / 16;
  if (tid == 0) {
    const int t = __hip_atomic_fetch_add(prm.counters + cidx, 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    *mv.last = (t == prm.num_splits - 1);
  }
  __syncthreads();
  if (!*mv.last) return;
  constexpr int DQ = D / 4;
  const int ns = prm.num_splits;
  for (int idx = tid; idx < nh * DQ; idx += NW * 64) {
    const int n = idx / DQ, dq = idx % DQ;
    const int64_t row = (int64_t)b * prm.HQ + h0 + n;
    float m = -INFINITY, l = 0.0f;
    f4 a = f4{0.f, 0.f, 0.f, 0.f};
    // Batches of 8 splits: every load of a batch is issued before the first
    // is used (atomic loads are not hoisted over the skip branch).  Indices
    // past the last split are clamped to it and skipped.
    constexpr int NB = 8;
    for (int s0 = 0; s0 < ns; s0 += NB) {
      float ms[NB], ls[NB];
      f4 as[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int64_t ps = row * ns + min(s0 + i, ns - 1);
        ms[i] = coherent_load(prm.maxs + ps);
        ls[i] = coherent_load(prm.sums + ps);
#pragma unroll
        for (int e = 0; e < 4; ++e) as[i][e] = coherent_load(prm.acc + ps * D + 4 * dq + e);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        if (s0 + i >= ns || is_empty_partial(ms[i], ls[i])) continue;
        const float mn = fmaxf(m, ms[i]);
        const float al = safe_exp2_diff(m, mn);
        const float be = __builtin_amdgcn_exp2f(ms[i] - mn);
        a = a * al + as[i] * be;
        l = l * al + ls[i] * be;
        m = mn;
      }
    }
    reinterpret_cast<f4*>(prm.out + row * D)[dq] = a / l;
  }
  if (tid == 0) __hip_atomic_store(prm.counters + cidx, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}


// ---------------------------------------------------------------------------
// Q^T as the B operand of the score MFMAs, in K slot order, plus the B operand
// of the K zero-point MFMA.  Lane-group j's dims of step m are the contiguous
// run [m*KSTEP + CB*j, +CB): one vector load per step, then slot order.  Lanes
// of heads >= nh hold zeros.
//
// Prescale.  Slice p of a packed byte enters the MFMA as the fp16 subnormal
// c * 2^(p*KNB - 24), so q is scaled by 2^(eh - p*KNB) to give every slice the
// same weight 2^(eh - 24).  eh is chosen per head, as large as EMAX and
// max|q| * 2^eh < 2^15 allow: scaling *up* by a power of two is exact, while
// scaling down (eh = 0) pushes |q| < 2^(p*KNB - 14) into fp16's subnormal
// range and costs absolute precision -- at 2 bits, slice 3's q * 2^-6 kept
// only 2^-18 of q, which against scale * code ~ 60 in outlier groups put
// scores 1e-4 off and outputs 2-3e-3 off.  The kernel scales the code dots by
// 2^(24 - eh) (zsc, lsc).
// ---------------------------------------------------------------------------
template <int D, int KNB, int GS>
struct QOperands {
  u4 qf[KLayout<D, KNB, GS>::NKM];
  u2 qzb;
  // The same dims of step m in natural order, unscaled fp16 pairs (CB/2 used):
  // for per-channel keys, whose zero-point term is a dot product with q.
  u4 qn[KLayout<D, KNB, GS>::NKM];
  int eh;  // this lane's head's prescale exponent
};

// Largest exponent e <= emax with amax * 2^e < 2^15 (amax >= 0).
__device__ __forceinline__ int q_prescale_exp(float amax, int emax) {
  return min(emax, 15 - __builtin_amdgcn_frexp_expf(amax));
}

// NAT: the score operands qf in natural dim order (pairs (0,1) (2,3) ...), for
// the per-channel key path, whose codes are extracted in that order so the
// chunk's channel scales need no reordering.
template <int D, int KNB, int GS, int EMAX, bool NAT = false>
__device__ __forceinline__ void load_q_operands(const SplitParams& prm, int b, int h0, int n, int nh,
                                                int j, QOperands<D, KNB, GS>& qo) {
  using KL = KLayout<D, KNB, GS>;
  constexpr int NG = D / GS;
  constexpr int NKM = KL::NKM;
  constexpr int NP = KL::CB / 2;  // fp16 pairs per step and lane
  // q stays in fp16 pairs throughout (an fp32 q is rounded to fp16 first, as
  // the reference's fp16 MFMA operand does): the max |q| is an integer max of
  // the magnitude bits, the prescale one packed multiply by a power of two
  // (the same rounding as scaling in fp32 and rounding once), and a head past
  // nh is cleared with one AND per operand dword.
  const bool hv = n < nh;
  const uint32_t hvm = hv ? 0xFFFFFFFFu : 0u;
  const int64_t qrow = ((int64_t)b * prm.HQ + h0 + (hv ? n : 0)) * D;
  uint32_t qh[NKM][NP];  // natural-order pairs of the lane's CB dims of step m
  if (prm.q_fp32) {
    const float* qp = static_cast<const float*>(prm.q) + qrow;
#pragma unroll
    for (int m = 0; m < NKM; ++m)
#pragma unroll
      for (int c = 0; c < KL::CB; c += 4) {
        const f4 v = *reinterpret_cast<const f4*>(qp + m * KL::KSTEP + KL::CB * j + c);
        qh[m][c / 2] = pack_h2(v[0], v[1]);
        qh[m][c / 2 + 1] = pack_h2(v[2], v[3]);
      }
  } else {
    const _Float16* qp = static_cast<const _Float16*>(prm.q) + qrow;
#pragma unroll
    for (int m = 0; m < NKM; ++m) {
      if constexpr (KL::CB == 8) {
        const u4 v = *reinterpret_cast<const u4*>(qp + m * KL::KSTEP + KL::CB * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) qh[m][e] = v[e];
      } else {
        const u2 v = *reinterpret_cast<const u2*>(qp + m * KL::KSTEP + KL::CB * j);
        qh[m][0] = v[0];
        qh[m][1] = v[1];
      }
    }
  }
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  us2 mag = us2{0, 0};
#pragma unroll
  for (int m = 0; m < NKM; ++m)
#pragma unroll
    for (int e = 0; e < NP; ++e)
      mag = __builtin_elementwise_max(mag, __builtin_bit_cast(us2, qh[m][e] & 0x7FFF7FFFu));
  const uint32_t mbits = mag[0] > mag[1] ? mag[0] : mag[1];
  const float amax = hv ? (float)__builtin_bit_cast(_Float16, (unsigned short)mbits) : 0.0f;
  qo.eh = q_prescale_exp(xor_max16_32(amax), EMAX);
  float qz[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) qz[g] = 0.0f;
  const h2 ones = h2{(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
  for (int m = 0; m < NKM; ++m) {
    // 2^(eh - p * KNB) as an fp16 pair: eh >= -1 and p * KNB <= 6, so the
    // exponent stays in the normal range
    const int p = KL::slice_of(m, j);
    const uint32_t pe = (uint32_t)(qo.eh - p * KNB + 15) << 10;
    const uint32_t pre = pe | (pe << 16);
    // slot order: pairs of dims (0,2) (1,3) (4,6) (5,7) of the step (NAT:
    // natural order)
    uint32_t sl[NP];
#pragma unroll
    for (int e = 0; e < NP; e += 2) {
      sl[e] = NAT ? qh[m][e] : perm(qh[m][e + 1], qh[m][e], 0x05040100u);
      sl[e + 1] = NAT ? qh[m][e + 1] : perm(qh[m][e + 1], qh[m][e], 0x07060302u);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qo.qf[m][e] = e < NP ? pk_mul(sl[e], pre) & hvm : 0u;
      qo.qn[m][e] = e < NP ? qh[m][e] & hvm : 0u;
    }
    float zs = 0.0f;
#pragma unroll
    for (int e = 0; e < NP; ++e)
      zs = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qh[m][e]), ones, zs, false);
    qz[KL::group_of_step(m)] += zs;
  }
#pragma unroll
  for (int g = 0; g < NG; ++g) qz[g] = xor_sum16_32(hv ? qz[g] : 0.0f);
  // B operand of the K zero-point MFMA: k-slot k < NG holds fp16(Qz_k),
  // NG <= k < 2NG the fp16 remainder Qz - fp16(Qz), so the product with the
  // exact fp16 zero points keeps fp32 precision.  Lane group j holds k-slots
  // 4j .. 4j + 3.
  float hiv[NG], lov[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    hiv[g] = (float)(_Float16)qz[g];
    lov[g] = qz[g] - hiv[g];
  }
  float hl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int k = 4 * jj + i;
      if (k < 2 * NG && j == jj) v = k < NG ? hiv[k < NG ? k : 0] : lov[k >= NG && k < 2 * NG ? k - NG : 0];
    }
    hl[i] = v;
  }
  qo.qzb = u2{pack_h2(hl[0], hl[1]), pack_h2(hl[2], hl[3])};
}

}  // namespace tkv
