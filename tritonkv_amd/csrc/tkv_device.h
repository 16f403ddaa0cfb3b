// Device-side building blocks shared by the tritonkv_amd HIP kernels (gfx950).
//
// Everything here is written for CDNA4: 64-wide wavefronts, the
// v_mfma_f32_16x16x{16,32}_f16 matrix instructions, and v_perm_b32 / bitwise
// AND for unpacking split-P codes straight into MFMA operand registers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tkv {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
// MFMA operands carry codes as fp16 *subnormals*: the bit pattern c << s is the
// value c * 2^(s-24), exact.  Products with fp16 q are exact in fp32, so every
// quantized dot product comes out scaled by 2^-24 and is rescaled once in fp32.
constexpr float kTwo24 = 16777216.0f;
constexpr float kTwoM24 = 5.9604644775390625e-08f;

// ---------------------------------------------------------------------------
// MFMA wrappers.  Lane layout (verified on gfx950):
//   A: lane l holds A[l%16][K/4*(l/16) + i]     (i < K/4)
//   B: lane l holds B[K/4*(l/16) + i][l%16]
//   D: lane l holds D[4*(l/16) + i][l%16]        (i < 4)
// ---------------------------------------------------------------------------
__device__ __forceinline__ f4 mfma_k32(u4 a, u4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a),
                                                __builtin_bit_cast(h8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_k16(u2 a, u2 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a),
                                               __builtin_bit_cast(h4, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Split-P code extraction.
//
// Layout (reference quantize.py:40-54): byte j of a packed row holds the codes
// of dims j, j+DP, j+2*DP, ... in bit slices of NBITS bits.  From one dword
// holding bytes (b0,b1,b2,b3) of a row, slice p of bytes b0 and b2 is
//     x & ((m << s) | (m << (16+s)))         s = p*NBITS, m = 2^NBITS-1
// which *is* a pair of fp16 subnormals (b0's code << s, b2's code << s).
// Bytes b1/b3 need one shift by 8 first.  So a dword yields its 4*P codes as
// 2*P fp16 pairs in "slot order" b0,b2,b1,b3.
// ---------------------------------------------------------------------------
template <int NBITS>
__device__ __forceinline__ constexpr uint32_t slice_mask(int p) {
  return ((((1u << NBITS) - 1u) << (p * NBITS)) * 0x00010001u);
}

// Bits of slices 0..p of every byte held in the low byte of each fp16 half.
template <int NBITS>
__device__ __forceinline__ constexpr uint32_t lo_slices_mask(int p) {
  return (((1u << ((p + 1) * NBITS)) - 1u) & 0xFFu) * 0x00010001u;
}

// Slot order of the four bytes of a dword after extraction: slots 0,1 come
// from bytes 0,2 and slots 2,3 from bytes 1,3.
__device__ __forceinline__ constexpr int slot_byte(int s) {
  return (s & ~3) + ((s & 1) << 1) + ((s >> 1) & 1);
}

// Decode a subnormal-encoded fp16 half back to an integer code.
__device__ __forceinline__ uint32_t code_of_half(uint32_t half_bits, int shift) {
  return (half_bits & 0xffffu) >> shift;
}

// ---------------------------------------------------------------------------
// Wave-level helpers.
// ---------------------------------------------------------------------------
// The value unchanged, but opaque to the optimizer (no instruction).
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Cross-lane combines on the VALU (no LDS round trip as with ds_bpermute).
// v_permlane16_swap exchanges lanes i and i ^ 16, v_permlane32_swap lanes i
// and i ^ 32: given the same value twice, one output holds the lane's own
// value and the other its partner's (which is which depends on the lane), so
// a commutative combine of the two outputs is the pair's in every lane.  The
// outputs pass through opaque(): this compiler folds fminf/fmaxf of the two
// outputs of the swap builtin to its first output.
template <bool SWAP32>
__device__ __forceinline__ void swap_pair(float v, float& a, float& b) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto s = SWAP32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                        : __builtin_amdgcn_permlane16_swap(u, u, false, false);
  a = __builtin_bit_cast(float, opaque(s[0]));
  b = __builtin_bit_cast(float, opaque(s[1]));
}
// a_h * b + c in fp32, a_h the fp16 in the low (HI false) or high half of a
// (the conversion is exact): the compiler selects one v_fma_mix_f32.  Plain
// code, not inline asm, so the compiler still sees the operands (b is often
// an MFMA result, whose readers need wait states it inserts).
template <bool HI>
__device__ __forceinline__ float fma_mix_h(uint32_t a, float b, float c) {
  return fmaf((float)__builtin_bit_cast(_Float16, (uint16_t)(HI ? a >> 16 : a)), b, c);
}
// max(a, b) as one v_max_f32.  fmaxf first quiets each operand the compiler
// cannot prove canonical -- every value that comes out of a DPP move or a lane
// swap -- at one more instruction per operand; the operands here are scores
// and running maxima, never signalling NaNs.
__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max_xor16(float v) {
  float a, b;
  swap_pair<false>(v, a, b);
  return vmax(a, b);
}
__device__ __forceinline__ float sum_xor16(float v) {
  float a, b;
  swap_pair<false>(v, a, b);
  return a + b;
}
__device__ __forceinline__ float xor_max16_32(float v) {
  float a, b;
  swap_pair<false>(v, a, b);
  swap_pair<true>(vmax(a, b), a, b);
  return vmax(a, b);
}
__device__ __forceinline__ float xor_sum16_32(float v) {
  float a, b;
  swap_pair<false>(v, a, b);
  swap_pair<true>(a + b, a, b);
  return a + b;
}
// The value of lane i ^ 16 (SWAP32 = false) or i ^ 32 (true): one lane swap.
// The builtins return the first operand with its odd rows (lanes 16-31 and
// 48-63; for the 32-lane swap its upper half) replaced by the second
// operand's even rows (lower half), then the second operand with the
// exchanged rows: given v twice, the first output holds the partner's value
// in odd rows and the second in even rows.
template <bool SWAP32>
__device__ __forceinline__ float lane_partner(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto s = SWAP32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                        : __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const int lane = (int)(threadIdx.x & 63);
  const bool even = SWAP32 ? lane < 32 : (lane & 16) == 0;
  return __builtin_bit_cast(float, even ? s[1] : s[0]);
}
// Row R (lanes 16R .. 16R + 15) of v in every row: lane i gets v of lane
// 16R + i % 16.  The 16-lane swap leaves rows 0 and 2 (first output) or 1
// and 3 (second) in both rows of each pair, and the 32-lane swap then the
// lower (first output) or upper pair in all four rows.  Two VALU swaps, no
// LDS round trip as with ds_bpermute.
__device__ __forceinline__ float row_bcast(float v, int R) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t t = (R & 1) ? a[1] : a[0];
  const auto c = __builtin_amdgcn_permlane32_swap(t, t, false, false);
  return __builtin_bit_cast(float, (R & 2) ? c[1] : c[0]);
}
// The value of lane i ^ 8 (the other half of the lane's 16-lane row): DPP
// row_ror:8.
__device__ __forceinline__ uint32_t lane_xor8(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true);
}
__device__ __forceinline__ float lane_xor8(float v) {
  return __builtin_bit_cast(float, lane_xor8(__builtin_bit_cast(uint32_t, v)));
}
// The value of lane (i - R) mod 16 of the lane's row of 16 (DPP row_ror:R).
template <int R>
__device__ __forceinline__ float lane_ror(float v) {
  static_assert(R > 0 && R < 16, "row rotation by 1..15");
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x120 + R, 0xF,
                                                             0xF, true));
}

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  h2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float half_lo(uint32_t w) {
  return (float)__builtin_bit_cast(h2, w)[0];
}
__device__ __forceinline__ float half_hi(uint32_t w) {
  return (float)__builtin_bit_cast(h2, w)[1];
}
// a * b - p for two fp16 lanes with one rounding (v_pk_fma_f16): with
// p = pk_mul(a, b), the exact rounding error of that product.
__device__ __forceinline__ uint32_t pk_fma_rem(uint32_t a, uint32_t b, uint32_t p) {
  const h2 r = __builtin_elementwise_fma(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b),
                                         -__builtin_bit_cast(h2, p));
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint32_t pk_mul(uint32_t a, uint32_t b) {
  h2 r = __builtin_bit_cast(h2, a) * __builtin_bit_cast(h2, b);
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint32_t pk_add(uint32_t a, uint32_t b) {
  h2 r = __builtin_bit_cast(h2, a) + __builtin_bit_cast(h2, b);
  return __builtin_bit_cast(uint32_t, r);
}
// fp16 pair of the remainders p - fp16(p): with ph = pack_h2(p0, p1), the
// low parts of a hi/lo split (p0 - half_lo(ph) is exact in fp32).
__device__ __forceinline__ uint32_t pack_h2_rem(float p0, float p1, uint32_t ph) {
  h2 v = {(_Float16)(p0 - (float)__builtin_bit_cast(h2, ph)[0]),
          (_Float16)(p1 - (float)__builtin_bit_cast(h2, ph)[1])};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

__device__ __forceinline__ float safe_exp2_diff(float a, float b) {
  // exp2(a - b) with exp2(-inf - x) = 0 and never NaN for a == b == -inf.
  return (a == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(a - b);
}

// A split partial that saw no token: max -inf and sum 0.  A partial whose
// scores were all NaN also keeps max -inf (the max steps drop NaN), but its sum
// is NaN, and it must be merged so that the NaN reaches the output.  A partial
// with any finite score has a sum of at least 1 (its largest score's term).
__device__ __forceinline__ bool is_empty_partial(float m, float l) {
  return m == -INFINITY && l == 0.0f;
}

// ---------------------------------------------------------------------------
// Raw buffer loads.  A buffer resource (base, size) lives in SGPRs; each load
// takes a 32-bit lane offset (VGPR) plus an immediate, so per-chunk addressing
// costs one VALU add per offset family instead of a 64-bit add per load.  The
// hardware range check returns 0 for any offset >= size, so a tile that runs
// past the end of a cache block reads zeros instead of faulting.
// 0x00020000 is the gfx9-family third descriptor dword (32-bit raw data).
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Cache-policy operand of a load (bit 1 = NT, non-temporal, on gfx94x/gfx950).
constexpr int kPolicyDefault = 0;
constexpr int kPolicyNT = 2;

template <int POL = kPolicyDefault>
__device__ __forceinline__ uint32_t buf_u32(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POL);
}
template <int POL = kPolicyDefault>
__device__ __forceinline__ u2 buf_u2(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POL);
}
template <int POL = kPolicyDefault>
__device__ __forceinline__ u4 buf_u4(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL);
}
template <int POL = kPolicyDefault>
__device__ __forceinline__ uint32_t buf_u16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, POL);
}

// Global loads of 4/8/16 bytes through the vector memory path.
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}
__device__ __forceinline__ u2 ld_u2(const uint8_t* p) {
  return *reinterpret_cast<const u2*>(p);
}
__device__ __forceinline__ u4 ld_u4(const uint8_t* p) {
  return *reinterpret_cast<const u4*>(p);
}

}  // namespace tkv
