// Group-wise asymmetric quantization of one cache row by one wave, produced
// directly in split-P form (reference quantize_groupwise quantize.py:186-236
// and pack_codes :149-169).
//
// Lane l owns packed byte j = l % DP of the row, i.e. the P = 8/NB codes of
// dims j + p*DP (p < P).  Lanes >= DP repeat lanes l - DP, so every shuffle
// reduction can run over aligned runs of lanes without masking.
//
// Per group: min and max of the fp32 values; scale = (max - min) / qmax, or 1
// when that is not positive (a constant group); scale and zero (= min) are
// rounded to fp16 *before* the codes are computed, and
// code = rint((x - zero) / scale) clamped to [0, qmax] with IEEE binary32
// division and ties to even (torch.round).  0/0 (a scale that underflows to
// fp16 zero) gives code 0, as torch's clamp of NaN does.  The file that uses
// this must not be compiled with fast-math.
//
// Non-finite input follows torch's amin / amax (quantize.py:209-210): a NaN
// anywhere in a group makes its min and max NaN, so the group gets scale 1,
// codes 0 and the canonical fp16 NaN 0x7E00 as its zero, whatever the sign or
// payload of the input NaN.  An infinite range gives an infinite scale and
// codes 0; a range or minimum past 65504 rounds to an infinite fp16 scale or
// zero, as Tensor.half() does.
//
// The group min/max reductions run on the VALU (DPP row permutations and the
// gfx950 permlane swaps), not through LDS.  The code's division is taken as a
// product with the reciprocal; the IEEE quotient is computed only for the
// rare value whose product lies too close to a rounding boundary for the two
// to be told apart (bound below), so the codes are those of the division.
//
// Shared by the append kernel and the decode kernel's fused append, so the two
// write the same bits.
#pragma once

#include "tkv_device.h"

namespace tkv {

template <int D, int NB, int GS>
struct RowQuant {
  static constexpr int P = 8 / NB;
  static constexpr int DP = D / P;
  static constexpr int NG = D / GS;
  static constexpr int QMAX = (1 << NB) - 1;
  uint32_t byte;  // this lane's packed byte (bits 0..7)
  uint32_t meta;  // lanes g < NG: group g's fp16 scale (bits 0..15) and zero (16..31)
};

// IEEE 754-2019 minimum / maximum: NaN when either operand is NaN, as torch's
// amin / amax (v_minimum3_f32 / v_maximum3_f32 on gfx950, one instruction
// each).  fminf / fmaxf would drop the NaN and give the group the range of its
// other values.
__device__ __forceinline__ float nan_min(float a, float b) {
  return __builtin_elementwise_minimum(a, b);
}
__device__ __forceinline__ float nan_max(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

// The fp16 bits of a group's zero point (its minimum): torch returns the
// canonical quiet NaN from amin, so a NaN minimum is stored as 0x7E00.
__device__ __forceinline__ uint16_t zero_bits(float mn) {
  return mn != mn ? (uint16_t)0x7E00u : __builtin_bit_cast(uint16_t, (_Float16)mn);
}

// One butterfly step of a min/max reduction: combine with the value DPP
// control CTRL brings from another lane of the same row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ void minmax_dpp(float& mn, float& mx) {
  const float a = __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, mn), CTRL, 0xF, 0xF, false));
  const float b = __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, mx), CTRL, 0xF, 0xF, false));
  mn = nan_min(mn, a);
  mx = nan_max(mx, b);
}


// Combine min/max across the lane pairs a permlane swap exchanges (rows 2k and
// 2k+1 for SWAP32 = false, the two 32-lane halves for true).  Given the same
// value v twice, the swap returns v with each odd part replaced by its even
// partner in one output and each even part by its odd partner in the other,
// so the min (max) of the two outputs is the pair's in every lane.  The
// outputs go through opaque(): this compiler folds a min/max of the two
// outputs of the swap builtin to its first output.
template <bool SWAP32>
__device__ __forceinline__ void minmax_swap(float& mn, float& mx) {
  const uint32_t n = __builtin_bit_cast(uint32_t, mn), x = __builtin_bit_cast(uint32_t, mx);
  const auto sn = SWAP32 ? __builtin_amdgcn_permlane32_swap(n, n, false, false)
                         : __builtin_amdgcn_permlane16_swap(n, n, false, false);
  const auto sx = SWAP32 ? __builtin_amdgcn_permlane32_swap(x, x, false, false)
                         : __builtin_amdgcn_permlane16_swap(x, x, false, false);
  mn = nan_min(__builtin_bit_cast(float, opaque(sn[0])), __builtin_bit_cast(float, opaque(sn[1])));
  mx = nan_max(__builtin_bit_cast(float, opaque(sx[0])), __builtin_bit_cast(float, opaque(sx[1])));
}

// Min and max over aligned runs of W lanes (W a power of two, 1..64); every
// lane of a run ends with the run's min and max.  nan_min/nan_max select one
// of their operands (or give NaN), so the result does not depend on the order
// of the steps.
//   lane^1, lane^2: quad_perm; the other quad of 8 lanes: row_half_mirror
//   (lane 7-i); the other half of a 16-lane row: row_mirror (lane 15-i);
//   rows 2k and 2k+1: v_permlane16_swap; the two 32-lane halves:
//   v_permlane32_swap.
template <int W>
__device__ __forceinline__ void minmax_lanes(float& mn, float& mx) {
  if constexpr (W >= 2) minmax_dpp<0xB1>(mn, mx);   // quad_perm [1,0,3,2]
  if constexpr (W >= 4) minmax_dpp<0x4E>(mn, mx);   // quad_perm [2,3,0,1]
  if constexpr (W >= 8) minmax_dpp<0x141>(mn, mx);  // row_half_mirror
  if constexpr (W >= 16) minmax_dpp<0x140>(mn, mx); // row_mirror
  if constexpr (W >= 32) minmax_swap<false>(mn, mx);
  if constexpr (W >= 64) minmax_swap<true>(mn, mx);
}

// Codes as rint(a / s) in IEEE binary32 with ties to even (s > 0 or s = +0),
// computed as y = a * rcp(s), q = rint(y).  y differs from the rounded
// quotient d = fl(a/s) by at most 2^-22 |a/s| (v_rcp_f32 is accurate to 1 ulp,
// the product adds half an ulp, d half an ulp), i.e. by less than 2^-17 when
// |y| < 32.  So rint(y) == rint(d) unless y lies within 2^-16 of a
// half-integer, or |y| >= 32 (or y is inf or NaN); only then is the quotient
// itself needed.  s = +0 gives the same inf or NaN both ways.
__device__ __forceinline__ bool quotient_unsure(float y, float q) {
  return !(fabsf(y - q) <= 0.5f - 0x1p-16f) || !(fabsf(y) < 32.0f);
}

__device__ __forceinline__ float rint_quotient(float a, float s, float rs) {
  const float y = a * rs;
  float q = rintf(y);
  if (__builtin_expect(quotient_unsure(y, q), 0)) q = rintf(a / s);
  return q;
}

// x[p] = the row's value at dim (lane % DP) + p * DP, already in fp32.
template <int D, int NB, int GS>
__device__ __forceinline__ RowQuant<D, NB, GS> quantize_row(const float (&x)[8 / NB], int lane) {
  using R = RowQuant<D, NB, GS>;
  constexpr int P = R::P, DP = R::DP, QMAX = R::QMAX;
  static_assert(DP <= 64 && GS % 8 == 0 && D % GS == 0, "row shape");
  float mn[P], mx[P];
#pragma unroll
  for (int p = 0; p < P; ++p) mn[p] = mx[p] = x[p];
  if constexpr (GS <= DP) {
    // A group is GS consecutive bytes of one slice: aligned runs of GS lanes.
#pragma unroll
    for (int p = 0; p < P; ++p) minmax_lanes<GS>(mn[p], mx[p]);
  } else {
    // A group is GS/DP whole slices: fold them in the lane, then all DP bytes.
    constexpr int SPG = GS / DP;
#pragma unroll
    for (int p = 0; p < P; p += SPG) {
#pragma unroll
      for (int e = 1; e < SPG; ++e) {
        mn[p] = nan_min(mn[p], mn[p + e]);
        mx[p] = nan_max(mx[p], mx[p + e]);
      }
      minmax_lanes<DP>(mn[p], mx[p]);
#pragma unroll
      for (int e = 1; e < SPG; ++e) {
        mn[p + e] = mn[p];
        mx[p + e] = mx[p];
      }
    }
  }
  uint32_t byte = 0, sz[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    float sc = (mx[p] - mn[p]) / (float)QMAX;
    if (!(sc > 0.0f)) sc = 1.0f;
    const _Float16 s16 = (_Float16)sc;
    const _Float16 z16 = (_Float16)mn[p];
    const float sf = (float)s16, zf = (float)z16;
    float c = rint_quotient(x[p] - zf, sf, __builtin_amdgcn_rcpf(sf));
    if (c != c) c = 0.0f;
    c = fminf(fmaxf(c, 0.0f), (float)QMAX);
    byte |= (uint32_t)c << (p * NB);
    sz[p] = (uint32_t)__builtin_bit_cast(uint16_t, s16) | ((uint32_t)zero_bits(mn[p]) << 16);
  }
  // Group g starts at dim g*GS: byte (g*GS) % DP, slice (g*GS) / DP.
  const int src = (lane * GS) % DP, slice = (lane * GS) / DP;
  uint32_t meta = 0;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const uint32_t v = (uint32_t)__shfl((int)sz[p], src, 64);
    if (slice == p) meta = v;
  }
  return R{byte, meta};
}

// The row's values for quantize_row from an fp16 or fp32 source row.
template <int D, int NB>
__device__ __forceinline__ void load_row_for_quant(const void* row, bool f32, int lane,
                                                   float (&x)[8 / NB]) {
  constexpr int P = 8 / NB, DP = D / P;
  const int j = lane % DP;
#pragma unroll
  for (int p = 0; p < P; ++p)
    x[p] = f32 ? static_cast<const float*>(row)[j + p * DP]
               : (float)static_cast<const _Float16*>(row)[j + p * DP];
}

}  // namespace tkv
