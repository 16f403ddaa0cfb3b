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
//   * Each chunk's codes and scale/zero rows reach LDS by direct-to-LDS loads
//     (quantized kernel) or registers (fp16 control); the partial (m, l, acc)
//     of the NW waves is merged in LDS and written once per workgroup.
#include <mutex>

#include "decode_common.h"

namespace tkv {

// ===========================================================================
// fp16 control split kernel: same split, softmax, GQA grouping, merge and
// combine; K/V read as fp16 (kernels/fp16_decode_attn.py:16-22 -- the control
// differs from the fused kernel only in how K/V are read).
// ===========================================================================
template <int D>
struct Fp16Tile {
  static constexpr int NKM = D / 32;
  static constexpr int EPL = D / 16;
  u4 kx[2][NKM];
  uint32_t vx[8][EPL / 2];
};

template <int D, int NW>
__global__ void __launch_bounds__(NW * 64)
fp16_split_kernel(SplitParams prm) {
  using Tile = Fp16Tile<D>;
  constexpr int NKM = Tile::NKM;  // 16x16x32 steps over the head dim
  constexpr int EPL = Tile::EPL;  // V dims per lane (and V MFMAs)
  __shared__ MergeLds<D, NW> mlds;

  const int unit = blockIdx.x;   // fastest: consecutive workgroups (which the
  const int split = blockIdx.y;  // dispatcher deals to the 8 XCDs in turn) take other units
  const int b = unit / prm.HKV, hk = unit % prm.HKV;
  const int hb0 = blockIdx.z * 16;
  const int nh = min(16, prm.G - hb0);
  const int h0 = hk * prm.G + hb0;
  const int L = prm.seq_lens ? min(prm.seq_lens[b], prm.S) : prm.S;
  const int lo = split * prm.split_size;
  const int hi = min(lo + prm.split_size, L);
  const int last = hi - 1;

  // The wave index is wave-uniform; saying so lets every chunk address live in
  // SGPRs and the loads use the scalar-base + lane-offset form.
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r = lane & 15, j = lane >> 4;
  const int n = r;
  const int64_t row0 = (int64_t)unit * prm.S;
  // Buffer resources over this (b, kv head) block: tokens >= S read as 0.
  const rsrc_t rk = make_rsrc(reinterpret_cast<const _Float16*>(prm.k) + row0 * D, (uint32_t)prm.S * D * 2);
  const rsrc_t rv = make_rsrc(reinterpret_cast<const _Float16*>(prm.v) + row0 * D, (uint32_t)prm.S * D * 2);
  const uint32_t klane = (r * D + 8 * j) * 2;      // + (16a*D + 32m) * 2
  const uint32_t vlane = (4 * j * D + EPL * r) * 2;  // + slot row * D * 2

  auto load_k = [&](Tile& t, int cb) {
    const uint32_t kb = klane + (uint32_t)cb * D * 2;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int m = 0; m < NKM; ++m) t.kx[a][m] = buf_u4<kPolF16>(rk, kb + (16 * a * D + 32 * m) * 2);
  };
  auto load_v = [&](Tile& t, int cb) {
    const uint32_t vb = vlane + (uint32_t)cb * D * 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t o = vb + ((i < 4 ? 0 : 12) + i) * D * 2;
      if constexpr (EPL == 8) {
        const u4 v4 = buf_u4<kPolF16>(rv, o);
        t.vx[i][0] = v4[0]; t.vx[i][1] = v4[1]; t.vx[i][2] = v4[2]; t.vx[i][3] = v4[3];
      } else {
        const u2 v2 = buf_u2<kPolF16>(rv, o);
        t.vx[i][0] = v2[0]; t.vx[i][1] = v2[1];
      }
    }
  };

  Tile t;
  const int cb0 = lo + kChunk * w;
  if (cb0 < hi) {
    load_k(t, cb0);
    load_v(t, cb0);
  }

  u4 qf[NKM];
  {
    // dims 32m + 8j .. +7 of head n: one vector load per MFMA step
    const bool hv = n < nh;
    const int64_t qrow = ((int64_t)b * prm.HQ + h0 + (hv ? n : 0)) * D;
#pragma unroll
    for (int m = 0; m < NKM; ++m) {
      float qv[8];
      if (prm.q_fp32) {
        const float* qp = static_cast<const float*>(prm.q) + qrow + 32 * m + 8 * j;
        const f4 a0 = *reinterpret_cast<const f4*>(qp);
        const f4 a1 = *reinterpret_cast<const f4*>(qp + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qv[e] = a0[e];
          qv[4 + e] = a1[e];
        }
      } else {
        const h8 v = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(prm.q) + qrow + 32 * m + 8 * j);
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[e] = (float)v[e];
      }
      uint32_t wv[4];
#pragma unroll
      for (int s2 = 0; s2 < 8; s2 += 2) wv[s2 / 2] = hv ? pack_h2(qv[s2], qv[s2 + 1]) : 0u;
      qf[m] = u4{wv[0], wv[1], wv[2], wv[3]};
    }
  }

  f4 accv[EPL];
#pragma unroll
  for (int mv = 0; mv < EPL; ++mv) accv[mv] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  const float lscale = prm.qk_scale;

  auto step = [&](Tile& cur, int cb, auto tail) {
    constexpr bool TAIL = decltype(tail)::value;
    const int cn = cb + kChunk * NW;
    const bool more = !TAIL && cn < hi;
    float x[8];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      f4 c = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < NKM; ++m) c = mfma_k32(cur.kx[a][m], qf[m], c);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[4 * a + i] = c[i];
    }
    if constexpr (TAIL) {
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (cb + 16 * a + 4 * j + i > last) x[4 * a + i] = -INFINITY;
    }
    if (more) load_k(cur, cn);
    float alpha;
    ChunkProbs pr;
    if (softmax_chunk(x, lscale, m_run, l_run, alpha, pr)) {
#pragma unroll
      for (int mv = 0; mv < EPL; ++mv) accv[mv] *= alpha;
    }
    const u4 pb = u4{pr.ph[0], pr.ph[1], pr.ph[2], pr.ph[3]};
    if constexpr (TAIL) {
      // Rows past the sequence are whatever the cache holds there (possibly
      // NaN/Inf bit patterns); p = 0 alone would not cancel them in the MFMA.
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (cb + slot_token(j, i) > last)
#pragma unroll
          for (int e = 0; e < EPL / 2; ++e) cur.vx[i][e] = 0u;
    }
#pragma unroll
    for (int mv = 0; mv < EPL; ++mv) {
      const uint32_t sel = (mv & 1) ? 0x07060302u : 0x05040100u;
      u4 av;
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = perm(cur.vx[2 * i + 1][mv / 2], cur.vx[2 * i][mv / 2], sel);
      accv[mv] = mfma_k32(av, pb, accv[mv]);
    }
    if (more) load_v(cur, cn);
  };

  // Full chunks, then the split's partial last chunk (if any).
  int cb = cb0;
  for (; cb + kChunk <= hi; cb += kChunk * NW) step(t, cb, std::false_type{});
  if (cb < hi) step(t, cb, std::true_type{});

  {
    const float lt = xor_sum16_32(l_run);
#pragma unroll
    for (int mv = 0; mv < EPL; ++mv)
#pragma unroll
      for (int i = 0; i < 4; ++i) mlds.wp[w].o[n][EPL * (4 * j + i) + mv] = accv[mv][i];
    if (j == 0) {
      mlds.wp[w].m[n] = m_run;
      mlds.wp[w].l[n] = lt;
    }
  }
  merge_and_store<D, NW>(prm, mlds.view(), b, h0, nh, split);
}

// ===========================================================================
// Combine: out[b,h,:] = sum_s 2^(m_s - m*) acc_s / sum_s 2^(m_s - m*) l_s.
// One 256-thread workgroup per (b, h).  Thread (sg, dq) owns float4 column dq
// of the splits s = sg, sg + SG, ...: it streams them with an online
// log-sum-exp merge (all loads of an iteration are independent of the
// previous one, so they stay in flight together), then the SG split groups
// are merged through LDS.  Empty splits (m_s = -inf, only possible with
// per-row lengths) contribute nothing.  Partial rows are `stride` apart; the
// first `ns` of them are merged.
//
// WIN: the fp16 residual window of per-channel keys is attended here too, as
// one more split.  Row b's window holds w.lens[b] <= kWinMax tokens of kv head
// h / G.  Lanes 8t .. 8t+7 compute the score of token t (fp32 products of the
// fp16-rounded q and the fp16 keys, as exact as the fp16 kernel's MFMA), the
// scores meet in LDS, and thread (sg, dq) starts its merge state from the
// window tokens sg, sg + SG, ... with the window's maximum.
// ===========================================================================
constexpr int kWinMax = 32;

struct WindowArgs {
  const void* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* lens;  // nullptr: every row's window holds R tokens
  int q_fp32, R, HQ, G;
  float qk_scale;       // sm_scale * log2(e)
};

template <int D, bool WIN>
__device__ __forceinline__ void combine_row(const float* __restrict__ acc,
                                            const float* __restrict__ maxs,
                                            const float* __restrict__ sums,
                                            float* __restrict__ out, int ns, int stride,
                                            const WindowArgs& w) {
  constexpr int DQ = D / 4;     // float4 columns of a split row
  constexpr int SG = 256 / DQ;  // split groups
  __shared__ float sm_m[SG], sm_l[SG];
  __shared__ f4 sm_a[SG][DQ];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, dq = t % DQ, sg = t / DQ;
  float m = -INFINITY, l = 0.0f;
  f4 a = f4{0.f, 0.f, 0.f, 0.f};
  if constexpr (WIN) {
    __shared__ float sm_s[kWinMax];
    constexpr int DD = D / 8;  // dims per lane of a token's score
    const int b = (int)(row / w.HQ), h = (int)(row % w.HQ);
    const int L = w.lens ? min(max(w.lens[b], 0), w.R) : w.R;  // uniform in the workgroup
    if (L > 0) {
      const int64_t base = ((int64_t)b * (w.HQ / w.G) + h / w.G) * w.R;
      const int tok = t >> 3, part = t & 7;
      float dot = 0.0f;
      if (tok < L) {
        const uint16_t* kr = w.k + (base + tok) * D + part * DD;
#pragma unroll
        for (int i = 0; i < DD; i += 8) {
          const h8 kv = *reinterpret_cast<const h8*>(kr + i);
          float qv[8];
          if (w.q_fp32) {
            const float* qp = static_cast<const float*>(w.q) + row * D + part * DD + i;
            const f4 q0 = *reinterpret_cast<const f4*>(qp), q1 = *reinterpret_cast<const f4*>(qp + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              qv[e] = (float)(_Float16)q0[e];
              qv[4 + e] = (float)(_Float16)q1[e];
            }
          } else {
            const h8 qh = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(w.q) + row * D +
                                                       part * DD + i);
#pragma unroll
            for (int e = 0; e < 8; ++e) qv[e] = (float)qh[e];
          }
          const f4 k0 = __builtin_convertvector(kv.lo, f4), k1 = __builtin_convertvector(kv.hi, f4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            dot = fmaf(qv[e], k0[e], dot);
            dot = fmaf(qv[4 + e], k1[e], dot);
          }
        }
      }
      dot += __shfl_xor(dot, 1, 64);
      dot += __shfl_xor(dot, 2, 64);
      dot += __shfl_xor(dot, 4, 64);
      if (part == 0 && tok < kWinMax) sm_s[tok] = dot * w.qk_scale;
      __syncthreads();
      float mw = -INFINITY;
      for (int i = 0; i < L; ++i) mw = fmaxf(mw, sm_s[i]);
      for (int i = sg; i < L; i += SG) {
        const float p = __builtin_amdgcn_exp2f(sm_s[i] - mw);
        const h4 vh = *reinterpret_cast<const h4*>(w.v + (base + i) * D + 4 * dq);
        a += __builtin_convertvector(vh, f4) * p;
        l += p;
      }
      m = mw;
    }
  }
#pragma unroll 4
  for (int s = sg; s < ns; s += SG) {
    const int64_t ps = row * stride + s;
    const float ms = maxs[ps];
    const float ls = sums[ps];
    const f4 as = reinterpret_cast<const f4*>(acc + ps * D)[dq];
    if (is_empty_partial(ms, ls)) continue;
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

// Plain combine: its argument block stays 36 bytes.  With the window's
// arguments in the same kernel (96 bytes) the 12-workgroup Qwen-shape combine
// took 4.45 instead of 3.25 us per call under a rocprofv3 kernel trace.
template <int D>
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ acc,
                                                      const float* __restrict__ maxs,
                                                      const float* __restrict__ sums,
                                                      float* __restrict__ out, int ns) {
  combine_row<D, false>(acc, maxs, sums, out, ns, ns, WindowArgs{});
}

// Few splits (ns <= MAXS <= 64, no window): one wave per row and no LDS.
// Lane (g, dq) merges splits g, g + NGRP, ... of float4 column dq, all its
// loads issued before the first is used; the NGRP groups then meet through
// lane exchanges.  At the Qwen2.5-1.5B shape (12 rows, 16-64 splits) the
// combine is pure latency, and this drops its barrier and LDS round trips.
constexpr int kSmallCombineMaxSplits = 64;

template <int D, int MAXS>
__global__ void __launch_bounds__(64) combine_small_kernel(const float* __restrict__ acc,
                                                           const float* __restrict__ maxs,
                                                           const float* __restrict__ sums,
                                                           float* __restrict__ out, int ns) {
  constexpr int DQ = D / 4;          // float4 columns of a row
  constexpr int NGRP = 64 / DQ;      // split groups
  constexpr int PER = MAXS / NGRP;   // splits per lane at most
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x, dq = lane % DQ, g = lane / DQ;
  float ms[PER], ls[PER];
  f4 as[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t ps = row * ns + min(g + NGRP * i, ns - 1);  // past ns: clamped, skipped
    ms[i] = maxs[ps];
    ls[i] = sums[ps];
    as[i] = reinterpret_cast<const f4*>(acc + ps * D)[dq];
  }
  float m = -INFINITY, l = 0.0f;
  f4 a = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (g + NGRP * i >= ns || is_empty_partial(ms[i], ls[i])) continue;
    const float mn = fmaxf(m, ms[i]);
    const float al = safe_exp2_diff(m, mn);
    const float be = __builtin_amdgcn_exp2f(ms[i] - mn);
    a = a * al + as[i] * be;
    l = l * al + ls[i] * be;
    m = mn;
  }
#pragma unroll
  for (int off = DQ; off < 64; off *= 2) {
    // the partner lane i ^ off (off = 16 or 32) through one lane swap each
    auto partner = [&](float x) { return off == 32 ? lane_partner<true>(x) : lane_partner<false>(x); };
    const float mo = partner(m), lo = partner(l);
    f4 ao;
#pragma unroll
    for (int e = 0; e < 4; ++e) ao[e] = partner(a[e]);
    const float mn = fmaxf(m, mo);
    const float al = safe_exp2_diff(m, mn), be = safe_exp2_diff(mo, mn);
    a = a * al + ao * be;
    l = l * al + lo * be;
    m = mn;
  }
  if (g == 0) reinterpret_cast<f4*>(out + row * D)[dq] = a / l;
}

template <int D>
static void launch_combine_small(const float* acc, const float* maxs, const float* sums,
                                 float* out, dim3 grid, int ns, hipStream_t st) {
  if (ns <= 16)
    combine_small_kernel<D, 16><<<grid, dim3(64), 0, st>>>(acc, maxs, sums, out, ns);
  else if (ns <= 32)
    combine_small_kernel<D, 32><<<grid, dim3(64), 0, st>>>(acc, maxs, sums, out, ns);
  else
    combine_small_kernel<D, 64><<<grid, dim3(64), 0, st>>>(acc, maxs, sums, out, ns);
}

template <int D>
__global__ void __launch_bounds__(256) combine_window_kernel(const float* __restrict__ acc,
                                                             const float* __restrict__ maxs,
                                                             const float* __restrict__ sums,
                                                             float* __restrict__ out, int ns,
                                                             int stride, WindowArgs w) {
  combine_row<D, true>(acc, maxs, sums, out, ns, stride, w);
}

// ---------------------------------------------------------------------------
// Dispatch order of a ragged batch: one thread per piece (b, s), piece index
// s * B + b; writes the HKV (idx, L) pairs of its rank (longest piece first,
// ragged_rank_term), idx = s * B * HKV + unit, L = min(seq_lens[b], S) as the
// split kernel would read it.  The rows pass through LDS 256 at a time as
// (full pieces, remainder), one division per row per workgroup, so each
// thread's O(B) sum is compares and adds.  The ranks of all pieces are
// distinct, so the pairs are a permutation of the B * HKV * ns workgroups of
// the split grid.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
ragged_order_kernel(const int32_t* __restrict__ seq_lens, int B, int S, int HKV, int ns, int ss,
                    int32_t* __restrict__ order) {
  __shared__ int2 rows[256];  // (full pieces, remainder) of each row
  const int p = blockIdx.x * 256 + threadIdx.x;
  const bool live = p < B * ns;
  const int s = live ? p / B : 0, b = live ? p - s * B : 0;
  const int Lb = seq_lens ? min(seq_lens[b], S) : S;
  auto stage = [&](int base) -> int2 {  // this thread's row of the block at base
    int2 r = make_int2(0, 0);
    if (base + (int)threadIdx.x < B) {
      const int L2 = seq_lens ? max(0, min(seq_lens[base + threadIdx.x], S)) : S;
      const int f2 = L2 / ss;
      r = make_int2(f2, L2 - f2 * ss);
    }
    return r;
  };
  int rank = 0;
  // The first block is staged outside the loop, so its load and Lb's share one wait.
  int2 mine = stage(0);
  for (int base = 0; base < B; base += 256) {
    const int n = min(256, B - base);
    if (base) {
      __syncthreads();  // the previous block of rows has been read
      mine = stage(base);
    }
    rows[threadIdx.x] = mine;
    __syncthreads();
    const int len = max(0, min(max(Lb, 0) - s * ss, ss));
    if (live) {
#pragma unroll 4
      for (int j = 0; j < n; ++j) {
        const int2 r = rows[j];
        rank += ragged_rank_term(len, s, b, ss, base + j, r.x, r.y);
      }
    }
  }
  if (!live) return;
  const int BU = B * HKV;
  int2* out = reinterpret_cast<int2*>(order);
  for (int hk = 0; hk < HKV; ++hk) out[(int64_t)rank * HKV + hk] = make_int2(s * BU + b * HKV + hk, Lb);
}

// ===========================================================================
// Host side: validation and dispatch.
// ===========================================================================
static int validate_common(const tkv_decode_args* a) {
  if (!a || !a->q || !a->k || !a->v || !a->out) return TKV_EINVAL;
  if (a->B <= 0 || a->HQ <= 0 || a->HKV <= 0 || a->S <= 0 || a->D <= 0) return TKV_EINVAL;
  if (a->HQ % a->HKV) return TKV_EINVAL;
  if ((int64_t)a->B * a->HQ > INT32_MAX) return TKV_EINVAL;  // grid and row indices are int
  if (a->split_size <= 0 || a->num_splits <= 0 || a->num_splits > 65535) return TKV_EINVAL;
  if ((int64_t)a->split_size * (a->num_splits - 1) >= a->S) return TKV_EINVAL;  // empty split
  if ((int64_t)a->split_size * a->num_splits < a->S) return TKV_EINVAL;        // uncovered
  const int total = a->num_splits_total ? a->num_splits_total : a->num_splits;
  if (a->split_base < 0 || a->num_splits_total < 0 || total > 65535 ||
      a->split_base + a->num_splits > total)
    return TKV_EINVAL;
  if (total > 1 && (!a->acc || !a->maxs || !a->sums)) return TKV_EINVAL;
  if (a->counters && (a->split_base != 0 || total != a->num_splits)) return TKV_EINVAL;
  if (a->key_block != 0 && a->key_block != 32) return TKV_EINVAL;
  if (a->key_block && (a->S % 32 || a->page_size > 0 || a->k_new)) return TKV_EINVAL;
  // Vector loads: caches 16-byte aligned, metadata 4-byte, partials 8-byte.
  if (((uintptr_t)a->k | (uintptr_t)a->v) & 15) return TKV_EINVAL;
  if (((uintptr_t)a->k_scale | (uintptr_t)a->k_zero | (uintptr_t)a->v_scale |
       (uintptr_t)a->v_zero) & 3)
    return TKV_EINVAL;
  if ((uintptr_t)a->q & 15) return TKV_EINVAL;  // vector loads of q rows
  if (((uintptr_t)a->acc | (uintptr_t)a->out) & 15) return TKV_EINVAL;  // float4 rows
  if (a->waves != 0 && a->waves != 4 && a->waves != 8 && a->waves != 12) return TKV_EINVAL;
  if ((uintptr_t)a->counters & 3) return TKV_EINVAL;
  if (a->page_size < 0) return TKV_EINVAL;
  if (a->page_size > 0) {
    if (a->page_size % 32 || !a->block_table || a->block_table_stride <= 0 || a->num_pages <= 0)
      return TKV_EINVAL;
    if ((int64_t)a->block_table_stride * a->page_size != a->S) return TKV_EINVAL;
  }
  if (a->k_new) {
    if (!a->v_new) return TKV_EINVAL;
    if (((uintptr_t)a->k_new | (uintptr_t)a->v_new) & (a->new_is_fp32 ? 3 : 1)) return TKV_EINVAL;
  }
  if (a->work_order) {
    if ((uintptr_t)a->work_order & 7) return TKV_EINVAL;  // int2 pairs
    // slots hold s * B * HKV + unit as int32
    if ((int64_t)a->B * a->HKV * a->num_splits > INT32_MAX) return TKV_EINVAL;
  }
  if (a->D != 64 && a->D != 128) return TKV_EUNSUPPORTED;
  return TKV_OK;
}

// The split kernels open one buffer resource per (b, kv head) block -- or per
// (page, kv head) slab of a paged pool -- and tensor, with a 32-bit byte range
// and 32-bit lane offsets.  A block of `rows` rows of `row_bytes` bytes each
// must therefore span less than 2^32 bytes, or its range would wrap and the
// hardware range check would return zeros for the rows past the wrap.
static bool block_fits_range(int64_t rows, int64_t row_bytes) {
  return rows * row_bytes < (int64_t(1) << 32);
}

// Rows of one buffer range: a page slab for paged pools, else the block's capacity.
static int64_t range_rows(const tkv_decode_args* a) {
  return a->page_size > 0 ? a->page_size : a->S;
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
  p.counters = a->counters;
  p.block_table = a->page_size > 0 ? a->block_table : nullptr;
  p.bt_stride = a->page_size > 0 ? a->block_table_stride : 0;
  p.page_size = a->page_size > 0 ? a->page_size : 0;
  p.num_pages = a->page_size > 0 ? a->num_pages : 0;
  p.k_new = a->k_new;
  p.v_new = a->k_new ? a->v_new : nullptr;
  p.new_fp32 = a->new_is_fp32 ? 1 : 0;
  p.HQ = a->HQ;
  p.HKV = a->HKV;
  p.S = a->S;
  p.G = a->HQ / a->HKV;
  p.num_splits = a->num_splits;
  p.split_size = a->split_size;
  p.q_fp32 = a->q_is_fp32 ? 1 : 0;
  p.qk_scale = a->sm_scale * kLog2e;
  p.key_block = a->key_block;
  p.split_base = a->split_base;
  p.ns_total = a->num_splits_total ? a->num_splits_total : a->num_splits;
  p.order = nullptr;  // set by launch_fused_split once the order is written
  p.xcd_units = 0;   // set by the small-grid dims-split launch
  return p;
}

// x = (b, kv) unit, y = split, z = block of 16 query heads.  Units vary
// fastest: the dispatcher deals consecutive workgroups to the XCDs in turn,
// so every XCD gets a share of each split index.  With splits fastest, XCD k
// would take split k mod 8 of every unit, and in a ragged batch the late
// splits of short rows are empty, leaving some XCDs idle while others still
// stream (measured: 1.4x slower at 8 splits).
static dim3 split_grid(const tkv_decode_args* a) {
  const int G = a->HQ / a->HKV;
  return dim3((unsigned)(a->B * a->HKV), (unsigned)a->num_splits, (unsigned)((G + 15) / 16));
}

// quant_split_lds_kernel launches, compiled in quant_split_k*v*.hip (one
// file per K/V bit-width pair, so the instantiations build in parallel).
template <int D, int KNB, int VNB, int GS>
void launch_quant(const SplitParams& p, dim3 grid, int waves, hipStream_t st);
template <int D, int KNB, int VNB, int GS>
void launch_read_probe(const SplitParams& p, dim3 grid, int waves, hipStream_t st);

// probe: the read-ceiling probe of the same instantiation instead of the kernel
template <int D, int KNB, int VNB, int GS>
static void launch_one(bool probe, const SplitParams& p, dim3 grid, int waves, hipStream_t st) {
  if (probe) launch_read_probe<D, KNB, VNB, GS>(p, grid, waves, st);
  else launch_quant<D, KNB, VNB, GS>(p, grid, waves, st);
}

template <int D, int KNB, int VNB>
static int dispatch_gs(const SplitParams& p, dim3 grid, int gs, int waves, hipStream_t st,
                       bool probe) {
  switch (gs) {
    case 16: launch_one<D, KNB, VNB, 16>(probe, p, grid, waves, st); return TKV_OK;
    case 32: launch_one<D, KNB, VNB, 32>(probe, p, grid, waves, st); return TKV_OK;
    case 64: launch_one<D, KNB, VNB, 64>(probe, p, grid, waves, st); return TKV_OK;
    case 128:
      if constexpr (D >= 128) {
        launch_one<D, KNB, VNB, 128>(probe, p, grid, waves, st);
        return TKV_OK;
      }
      return TKV_EUNSUPPORTED;
    default: return TKV_EUNSUPPORTED;
  }
}

template <int D>
static int dispatch_bits(const SplitParams& p, dim3 grid, int knb, int vnb, int gs, int waves,
                         hipStream_t st, bool probe = false) {
  if (knb == 4 && vnb == 4) return dispatch_gs<D, 4, 4>(p, grid, gs, waves, st, probe);
  if (knb == 2 && vnb == 2) return dispatch_gs<D, 2, 2>(p, grid, gs, waves, st, probe);
  if (knb == 4 && vnb == 2) return dispatch_gs<D, 4, 2>(p, grid, gs, waves, st, probe);
  if (knb == 2 && vnb == 4) return dispatch_gs<D, 2, 4>(p, grid, gs, waves, st, probe);
  return TKV_EUNSUPPORTED;
}

// Merges partial rows 0 .. ns-1, plus the fp16 window when `win` is given;
// the window form reads partials `stride` rows apart (0: ns).
static int launch_combine(const float* acc, const float* maxs, const float* sums, float* out,
                          int B, int HQ, int ns, int D, hipStream_t st, int stride = 0,
                          const WindowArgs* win = nullptr) {
  const dim3 grid((unsigned)(B * HQ));
  const int sd = stride ? stride : ns;
  const bool small = !win && ns <= kSmallCombineMaxSplits;
  if (D == 128) {
    if (win) combine_window_kernel<128><<<grid, dim3(256), 0, st>>>(acc, maxs, sums, out, ns, sd, *win);
    else if (small) launch_combine_small<128>(acc, maxs, sums, out, grid, ns, st);
    else combine_kernel<128><<<grid, dim3(256), 0, st>>>(acc, maxs, sums, out, ns);
  } else if (D == 64) {
    if (win) combine_window_kernel<64><<<grid, dim3(256), 0, st>>>(acc, maxs, sums, out, ns, sd, *win);
    else if (small) launch_combine_small<64>(acc, maxs, sums, out, grid, ns, st);
    else combine_kernel<64><<<grid, dim3(256), 0, st>>>(acc, maxs, sums, out, ns);
  } else {
    return TKV_EUNSUPPORTED;
  }
  return TKV_OK;
}

static int status_of_launch() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TKV_OK : (int)e;
}

}  // namespace tkv

namespace tkv {

// Every argument check of the quantized split launch; nothing touches the GPU.
static int check_fused_split(const tkv_decode_args* a, bool probe) {
  const int rc = validate_common(a);
  if (rc) return rc;
  if (probe && (a->page_size > 0 || a->k_new || a->key_block)) return TKV_EUNSUPPORTED;
  if (!a->k_scale || !a->k_zero || !a->v_scale || !a->v_zero) return TKV_EINVAL;
  const int gs = a->group_size;
  if (gs <= 0 || gs > a->D || a->D % gs) return TKV_EINVAL;
  if ((a->k_nbits != 2 && a->k_nbits != 4) || (a->v_nbits != 2 && a->v_nbits != 4))
    return TKV_EINVAL;
  if (a->key_block && gs > 32) return TKV_EUNSUPPORTED;  // per-channel keys: V groups of 16 or 32
  // ordered launches: head dim 128, per-token keys (the instantiated forms)
  if (a->work_order && (a->D != 128 || a->key_block)) return TKV_EUNSUPPORTED;
  // the instantiated group sizes (dispatch_gs), checked before anything is launched
  if (gs != 16 && gs != 32 && gs != 64 && gs != 128) return TKV_EUNSUPPORTED;
  // codes (K, V) and fp16 scale/zero rows of one buffer range
  const int64_t rows = range_rows(a);
  if (!block_fits_range(rows, (int64_t)a->D * a->k_nbits / 8) ||
      !block_fits_range(rows, (int64_t)a->D * a->v_nbits / 8) ||
      !block_fits_range(rows, (int64_t)(a->D / gs) * 2))
    return TKV_EUNSUPPORTED;
  return TKV_OK;
}

static int launch_fused_split(const tkv_decode_args* a, hipStream_t st, bool probe = false) {
  int rc = check_fused_split(a, probe);
  if (rc) return rc;
  const int gs = a->group_size;
  SplitParams p = make_params(a);
  const dim3 grid = split_grid(a);
  (void)hipGetLastError();
  if (a->work_order) {
    const int pieces = a->B * a->num_splits;
    ragged_order_kernel<<<dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, st>>>(
        a->seq_lens, a->B, a->S, a->HKV, a->num_splits, a->split_size, a->work_order);
    p.order = a->work_order;
  }
  rc = a->D == 128 ? dispatch_bits<128>(p, grid, a->k_nbits, a->v_nbits, gs, a->waves, st, probe)
                   : dispatch_bits<64>(p, grid, a->k_nbits, a->v_nbits, gs, a->waves, st, probe);
  if (rc) return rc;
  return status_of_launch();
}

static int launch_fp16_split(const tkv_decode_args* a, hipStream_t st) {
  const int rc = validate_common(a);
  if (rc) return rc;
  // the fp16 control reads contiguous caches in the natural order and has no fused append
  if (a->page_size > 0 || a->k_new || a->key_block || a->work_order) return TKV_EUNSUPPORTED;
  if (!block_fits_range(a->S, (int64_t)a->D * 2)) return TKV_EUNSUPPORTED;  // fp16 rows
  const SplitParams p = make_params(a);
  const dim3 grid = split_grid(a);
  (void)hipGetLastError();
  if (a->D == 128) {
    if (a->waves >= 8)  // 12 runs 8
      fp16_split_kernel<128, 8><<<grid, dim3(8 * 64), 0, st>>>(p);
    else
      fp16_split_kernel<128, 4><<<grid, dim3(4 * 64), 0, st>>>(p);
  } else {
    if (a->waves >= 8)
      fp16_split_kernel<64, 8><<<grid, dim3(8 * 64), 0, st>>>(p);
    else
      fp16_split_kernel<64, 4><<<grid, dim3(4 * 64), 0, st>>>(p);
  }
  return status_of_launch();
}

static int finish_combine(const tkv_decode_args* a, hipStream_t st) {
  if (a->num_splits <= 1 || a->counters) return TKV_OK;  // counters: merged in the split kernel
  (void)hipGetLastError();
  launch_combine(a->acc, a->maxs, a->sums, a->out, a->B, a->HQ, a->num_splits, a->D, st);
  return status_of_launch();
}

}  // namespace tkv

extern "C" int tkv_fused_decode_split(const tkv_decode_args* a, tkv_stream_t stream) {
  return tkv::launch_fused_split(a, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int tkv_read_probe(const tkv_decode_args* a, tkv_stream_t stream) {
  return tkv::launch_fused_split(a, reinterpret_cast<hipStream_t>(stream), true);
}

extern "C" int tkv_fp16_decode_split(const tkv_decode_args* a, tkv_stream_t stream) {
  return tkv::launch_fp16_split(a, reinterpret_cast<hipStream_t>(stream));
}

// The whole-attention entry points run every split themselves.
static bool own_all_splits(const tkv_decode_args* a) {
  return a && a->split_base == 0 && (a->num_splits_total == 0 || a->num_splits_total == a->num_splits);
}

extern "C" int tkv_fused_decode_attention(const tkv_decode_args* a, tkv_stream_t stream) {
  if (a && !own_all_splits(a)) return TKV_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int rc = tkv::launch_fused_split(a, st);
  return rc ? rc : tkv::finish_combine(a, st);
}

extern "C" int tkv_fp16_decode_attention(const tkv_decode_args* a, tkv_stream_t stream) {
  if (a && !own_all_splits(a)) return TKV_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int rc = tkv::launch_fp16_split(a, st);
  return rc ? rc : tkv::finish_combine(a, st);
}

extern "C" int tkv_channel_decode_attention(const tkv_decode_args* a, const void* k_res,
                                            const void* v_res, const int32_t* res_lens,
                                            int32_t res_cap, tkv_stream_t stream) {
  using namespace tkv;
  if (!a || !k_res || !v_res || res_cap <= 0) return TKV_EINVAL;
  if (a->key_block != 32) return TKV_EINVAL;
  if (((uintptr_t)k_res | (uintptr_t)v_res) & 15) return TKV_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int total = a->num_splits + 1;
  tkv_decode_args qa = *a;  // the quantized history: partial rows 0 .. num_splits - 1
  qa.split_base = 0;
  qa.num_splits_total = total;
  qa.counters = nullptr;
  int rc = launch_fused_split(&qa, st);
  if (rc) return rc;
  if (res_cap <= kWinMax) {  // the window is attended inside the combine
    WindowArgs w;
    w.q = a->q;
    w.k = static_cast<const uint16_t*>(k_res);
    w.v = static_cast<const uint16_t*>(v_res);
    w.lens = res_lens;
    w.q_fp32 = a->q_is_fp32 ? 1 : 0;
    w.R = res_cap;
    w.HQ = a->HQ;
    w.G = a->HQ / a->HKV;
    w.qk_scale = a->sm_scale * kLog2e;
    (void)hipGetLastError();
    launch_combine(a->acc, a->maxs, a->sums, a->out, a->B, a->HQ, a->num_splits, a->D, st,
                   total, &w);
    return status_of_launch();
  }
  tkv_decode_args ra = *a;  // the fp16 window: partial row num_splits
  ra.k = k_res;
  ra.v = v_res;
  ra.k_scale = ra.k_zero = ra.v_scale = ra.v_zero = nullptr;
  ra.seq_lens = res_lens;
  ra.S = res_cap;
  ra.split_size = res_cap;
  ra.num_splits = 1;
  ra.split_base = a->num_splits;
  ra.num_splits_total = total;
  ra.counters = nullptr;
  ra.key_block = 0;
  ra.waves = 4;
  ra.work_order = nullptr;
  rc = launch_fp16_split(&ra, st);
  if (rc) return rc;
  (void)hipGetLastError();
  launch_combine(a->acc, a->maxs, a->sums, a->out, a->B, a->HQ, total, a->D, st);
  return status_of_launch();
}

// ===========================================================================
// The fused decode step without a workspace: the split partials (acc, maxs,
// sums) of a call live in `scratch`, a device array each GPU holds from the
// library's load until the process ends.  In host code `scratch` names a
// host-side stand-in; its device address is taken once per device with
// hipGetSymbolAddress (with that device current) and only that address is
// handed to kernels.  Every split writes its partial rows (an empty split
// writes max -inf, sum 0), so nothing has to be cleared between calls.  All
// calls on one GPU share the array: calls that overlap in time there race.
// ===========================================================================
static __device__ __align__(256) unsigned char scratch[TKV_NOALLOC_SCRATCH_BYTES];

namespace tkv {

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];

// Device address of `scratch` on the current device (looked up once per device).
static int scratch_on_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return TKV_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return TKV_ENODEVICE;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TKV_OK;
}

constexpr uint64_t align256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

}  // namespace tkv

extern "C" int tkv_fused_decode_attention_noalloc(const tkv_decode_args* a, tkv_stream_t stream) {
  using namespace tkv;
  if (!a || !own_all_splits(a)) return TKV_EINVAL;
  if (a->acc || a->maxs || a->sums || a->counters || a->work_order)  // the partials are ours
    return TKV_EINVAL;
  if (a->B <= 0 || a->HQ <= 0 || a->D <= 0 || a->num_splits <= 0) return TKV_EINVAL;
  tkv_decode_args s = *a;
  if (a->num_splits > 1) {
    const uint64_t rows = (uint64_t)a->B * (uint64_t)a->HQ * (uint64_t)a->num_splits;
    const uint64_t acc_bytes = align256(rows * (uint64_t)a->D * 4);
    const uint64_t ml_bytes = align256(rows * 4);
    if (acc_bytes + 2 * ml_bytes > TKV_NOALLOC_SCRATCH_BYTES) return TKV_ESCRATCH;
    // Every argument is checked before the device is touched; any aligned
    // non-null address stands in for the partials, which are not read here.
    s.acc = s.maxs = s.sums = reinterpret_cast<float*>(uintptr_t(256));
    int rc = check_fused_split(&s, false);
    if (rc) return rc;
    void* base = nullptr;
    rc = scratch_on_current_device(&base);
    if (rc) return rc;
    unsigned char* p = static_cast<unsigned char*>(base);
    s.acc = reinterpret_cast<float*>(p);
    s.maxs = reinterpret_cast<float*>(p + acc_bytes);
    s.sums = reinterpret_cast<float*>(p + acc_bytes + ml_bytes);
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int rc = launch_fused_split(&s, st);
  return rc ? rc : finish_combine(&s, st);
}

extern "C" int tkv_combine_splits(const float* acc, const float* maxs, const float* sums,
                                  float* out, int32_t B, int32_t HQ, int32_t num_splits,
                                  int32_t D, tkv_stream_t stream) {
  using namespace tkv;
  if (!acc || !maxs || !sums || !out || B <= 0 || HQ <= 0 || num_splits <= 0) return TKV_EINVAL;
  if ((int64_t)B * HQ > INT32_MAX) return TKV_EINVAL;
  if (((uintptr_t)acc | (uintptr_t)out) & 15) return TKV_EINVAL;
  if (D != 64 && D != 128) return TKV_EUNSUPPORTED;
  (void)hipGetLastError();
  launch_combine(acc, maxs, sums, out, B, HQ, num_splits, D, reinterpret_cast<hipStream_t>(stream));
  return status_of_launch();
}
