// Register-level unpack of split-P codes into MFMA operands (gfx950).
//
// Shared by the decode kernel and by the unpack/dequant export kernel, so the
// export proves bit for bit the exact index arithmetic and bit extraction the
// decode kernel feeds to its matrix instructions.
//
// Split-P layout (reference quantize.py:40-54): P = 8/NB codes per byte,
// DP = D/P bytes per row, dim d lives in byte d % DP at bit slice d / DP.
//
// K operand (scores S^T = K * Q^T, one MFMA row per token):
//   An MFMA step covers KSTEP consecutive dims [m*KSTEP, (m+1)*KSTEP); KSTEP is
//   32 (16x16x32 MFMA) or 16 when the group size is 16 (16x16x16 MFMA), so a step
//   never straddles a quantization group and its partial dot products can be
//   scaled by that group's scale/zero afterwards.  Lane-group j of the wave
//   supplies dims d0 = m*KSTEP + CB*j .. d0+CB-1 (CB = KSTEP/4), which are CB
//   consecutive bytes of one bit slice, loaded as one dword or dwordx2 per row.
//   The dims come out in slot order d0 + slot_byte(s); Q^T is built in the same
//   order once per workgroup, pre-scaled by 2^-(slice*NB) to cancel the
//   in-place bit position of the code.
//
// V operand (O^T = V^T * P^T, one MFMA row per dim, K = 32 tokens):
//   Each MFMA uses 16 dims of one slice inside one window of W bytes
//   (W = min(64, GS, DP)), so all 16 rows share a quantization group and the
//   group's scale can be folded into the P operand.  Lanes r = 0..15 read dword
//   r/LPD of the window (LPD = 64/W lanes share a dword) from each of their 8
//   tokens; v_perm_b32 gathers byte (LPD*e + r%LPD) of two tokens into one
//   fp16 pair and an AND isolates the slice.  The 2^(slice*NB) bit position
//   is removed once, when the accumulator is written out.
#pragma once

#include "tkv_device.h"

namespace tkv {

template <int D, int NB, int GS>
struct KLayout {
  static constexpr int P = 8 / NB;
  static constexpr int DP = D / P;
  static constexpr int NG = D / GS;
  static constexpr int KSTEP = GS >= 32 ? 32 : 16;
  static constexpr int CB = KSTEP / 4;                 // bytes per lane-group per step
  static constexpr int NKM = D / KSTEP;                // MFMA steps per 16-token tile
  static constexpr int NLOAD = KSTEP <= DP ? DP / KSTEP : 1;  // distinct loads per row

  // Byte offset of load L for lane-group j.
  __device__ static constexpr int load_offset(int L, int j) {
    return KSTEP <= DP ? L * KSTEP + CB * j : (CB * j) % DP;
  }
  // Which load MFMA step m reads.
  __device__ static constexpr int load_of_step(int m) {
    return KSTEP <= DP ? ((m * KSTEP) % DP) / KSTEP : 0;
  }
  __device__ static constexpr int slice_of(int m, int j) { return (m * KSTEP + CB * j) / DP; }
  __device__ static constexpr int group_of_step(int m) { return (m * KSTEP) / GS; }
  // Head dim of slot s (0..CB-1) of lane-group j in step m.
  __device__ static constexpr int dim_of(int m, int j, int s) {
    return m * KSTEP + CB * j + slot_byte(s);
  }
};

// Extract the CB codes of one lane-group (already loaded) as fp16 subnormals.
__device__ __forceinline__ u4 k_extract8(u2 x, uint32_t mask) {
  u4 a;
  a[0] = x[0] & mask;
  a[1] = (x[0] >> 8) & mask;
  a[2] = x[1] & mask;
  a[3] = (x[1] >> 8) & mask;
  return a;
}
__device__ __forceinline__ u2 k_extract4(uint32_t x, uint32_t mask) {
  u2 a;
  a[0] = x & mask;
  a[1] = (x >> 8) & mask;
  return a;
}
// The same codes in natural order (fp16 slots hold bytes 0,1 | 2,3 | ...):
// bytes spread into the low halves by v_perm, one more instruction per
// source dword than the shift of the slot order (the spread is shared by the
// slices of a byte).
__device__ __forceinline__ u4 k_extract8_nat(u2 x, uint32_t mask) {
  u4 a;
  a[0] = perm(x[0], x[0], 0x0C010C00u) & mask;
  a[1] = perm(x[0], x[0], 0x0C030C02u) & mask;
  a[2] = perm(x[1], x[1], 0x0C010C00u) & mask;
  a[3] = perm(x[1], x[1], 0x0C030C02u) & mask;
  return a;
}
__device__ __forceinline__ u2 k_extract4_nat(uint32_t x, uint32_t mask) {
  u2 a;
  a[0] = perm(x, x, 0x0C010C00u) & mask;
  a[1] = perm(x, x, 0x0C030C02u) & mask;
  return a;
}

template <int D, int NB, int GS>
struct VLayout {
  static constexpr int P = 8 / NB;
  static constexpr int DP = D / P;
  static constexpr int NG = D / GS;
  static constexpr int W0 = GS < DP ? GS : DP;
  static constexpr int W = W0 < 64 ? W0 : 64;          // window bytes: 16, 32 or 64
  static constexpr int LPD = 64 / W;                   // lanes sharing one dword
  static constexpr int NWIN = DP / W;                  // windows per slice
  static constexpr int NE = 4 / LPD;                   // MFMAs per (slice, window)
  static constexpr int NVM = P * NWIN * NE;            // = D / 16
  static_assert(W >= 16, "window must hold 16 dims");
  static_assert(NVM * 16 == D, "V MFMAs must cover the head dim");

  __device__ static constexpr int mfma_index(int p, int wi, int e) { return (p * NWIN + wi) * NE + e; }
  __device__ static constexpr int slice_of(int mv) { return mv / (NWIN * NE); }
  __device__ static constexpr int window_of(int mv) { return (mv / NE) % NWIN; }
  __device__ static constexpr int e_of(int mv) { return mv % NE; }
  __device__ static constexpr int group_of(int mv) {
    return (slice_of(mv) * DP + W * window_of(mv)) / GS;
  }
  // Byte offset (within the row) of the dword lane r reads for window wi.
  __device__ static constexpr int dword_offset(int wi, int r) { return W * wi + 4 * (r / LPD); }
  // Byte of that dword that row r of MFMA sub-index e uses.
  __device__ static constexpr int byte_in_dword(int e, int r) { return LPD * e + (r % LPD); }
  // Head dim of row rr of V MFMA mv.
  __device__ static constexpr int dim_of(int mv, int rr) {
    return slice_of(mv) * DP + W * window_of(mv) + 4 * (rr / LPD) + byte_in_dword(e_of(mv), rr);
  }
  // v_perm selector gathering byte `bs` of two tokens into fp16 lanes (t0, t1).
  __device__ static constexpr uint32_t perm_sel(int bs) {
    return (uint32_t)bs | (0x0Cu << 8) | ((uint32_t)(4 + bs) << 16) | (0x0Cu << 24);
  }
};

// One fp16 pair (token t0 in the low half, t1 in the high half) of V codes.
__device__ __forceinline__ uint32_t v_extract(uint32_t x_t1, uint32_t x_t0, uint32_t sel,
                                              uint32_t mask) {
  return perm(x_t1, x_t0, sel) & mask;
}

}  // namespace tkv
