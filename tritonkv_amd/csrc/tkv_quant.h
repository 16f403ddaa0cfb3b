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
    for (int k = 1; k < GS; k <<= 1)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        mn[p] = fminf(mn[p], __shfl_xor(mn[p], k, 64));
        mx[p] = fmaxf(mx[p], __shfl_xor(mx[p], k, 64));
      }
  } else {
    // A group is GS/DP whole slices: fold them in the lane, then all DP bytes.
    constexpr int SPG = GS / DP;
#pragma unroll
    for (int p = 0; p < P; p += SPG) {
#pragma unroll
      for (int e = 1; e < SPG; ++e) {
        mn[p] = fminf(mn[p], mn[p + e]);
        mx[p] = fmaxf(mx[p], mx[p + e]);
      }
#pragma unroll
      for (int k = 1; k < DP; k <<= 1) {
        mn[p] = fminf(mn[p], __shfl_xor(mn[p], k, 64));
        mx[p] = fmaxf(mx[p], __shfl_xor(mx[p], k, 64));
      }
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
    float c = rintf((x[p] - zf) / sf);
    if (c != c) c = 0.0f;
    c = fminf(fmaxf(c, 0.0f), (float)QMAX);
    byte |= (uint32_t)c << (p * NB);
    sz[p] = (uint32_t)__builtin_bit_cast(uint16_t, s16) |
            ((uint32_t)__builtin_bit_cast(uint16_t, z16) << 16);
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
