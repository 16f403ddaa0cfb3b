// GPU quantize/pack (decode-step append and whole-cache setup), split-P pack
// of given codes, and the unpack/dequant export used to prove bit-exactness.
//
// Reference behaviour being reproduced bit for bit:
//   quantize_groupwise  quantize.py:186-236   (fp32 min/max per group,
//       scale = range/qmax or 1 for a degenerate group, scale and zero rounded
//       to fp16 first, code = rint((x - zero)/scale) clamped to [0, qmax])
//   pack_codes          quantize.py:149-169
//   unpack_codes        quantize.py:172-183
//   dequantize_groupwise quantize.py:239-246 (fp32 code*scale + zero; the
//       product is exact since code <= 15 and scale has 11 significant bits,
//       so fmaf gives the same bits as the reference's mul-then-add)
//
// The arithmetic relies on IEEE binary32 division (hipcc's default correctly
// rounded fp32 divide -- this file must not be built with fast-math) and on
// rintf rounding half to even like torch.round.
#include <stdint.h>
#include <type_traits>

#include "tkv_codec.h"
#include "tkv_quant.h"
#include "../../include/tkv.h"

namespace tkv {

// Destination of appended rows in a paged cache (page_size > 0): logical token
// t of batch row b goes to pool page block_table[b * stride + t / page_size],
// slot t % page_size; pools are laid out (num_pages, HKV, page_size, ...).
struct PageMap {
  const int32_t* block_table;
  int stride, page_size, num_pages;
};

// One wave per cache row (token x kv head), quantized by quantize_row: lane j
// owns packed byte j of the row.  Used when the input or the codes are not
// aligned for the wide kernel below.
template <int D, int NB, int GS, bool F32>
__global__ void __launch_bounds__(256)
quantize_pack_kernel(const void* __restrict__ x, int64_t row0, int64_t rows, int HKV, int N,
                     const int32_t* __restrict__ positions, int S_cap, PageMap pm,
                     uint8_t* __restrict__ packed, uint16_t* __restrict__ scale,
                     uint16_t* __restrict__ zero) {
  using R = RowQuant<D, NB, GS>;
  constexpr int P = R::P, DP = R::DP, NG = R::NG;

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t rr = row0 + (int64_t)blockIdx.x * 4 + w;
  if (rr >= rows) return;  // whole wave
  float xv[P];
  load_row_for_quant<D, NB>(static_cast<const uint8_t*>(x) + rr * D * (F32 ? 4 : 2), F32, lane, xv);
  const int64_t bh = rr / N;
  const int t = (int)(rr - bh * N);
  const int b = (int)(bh / HKV), kv = (int)(bh - (int64_t)b * HKV);
  const int64_t dst_t = (int64_t)(positions ? positions[b] : 0) + t;
  bool in_range = dst_t >= 0 && dst_t < S_cap;
  int64_t dst_row = bh * S_cap + dst_t;
  if (pm.page_size > 0 && in_range) {  // S_cap == stride * page_size
    const int e = pm.block_table[(int64_t)b * pm.stride + dst_t / pm.page_size];
    in_range = e >= 0 && e < pm.num_pages;  // rows mapped outside the pool are not written
    dst_row = ((int64_t)e * HKV + kv) * pm.page_size + dst_t % pm.page_size;
  }
  const R q = quantize_row<D, NB, GS>(xv, lane);
  if (!in_range) return;
  if (lane < DP) packed[dst_row * DP + lane] = (uint8_t)q.byte;
  if (lane < NG) {
    scale[dst_row * NG + lane] = (uint16_t)(q.meta & 0xFFFFu);
    zero[dst_row * NG + lane] = (uint16_t)(q.meta >> 16);
  }
}

// Bulk form of the same quantization (the same arithmetic, so the same bits):
// lane (slot r = l / LPR, column c = l % LPR) owns the E = 8 packed bytes
// [8c, 8c + 8) of its row, i.e. the 8P codes of dims 8c + e + p*DP.  It reads
// P runs of 8 consecutive values (16-byte loads) and writes its 8 bytes in one
// store.  Group min/max fold the lane's own 8 values, then run over the GS/8
// lanes of the group (or, when a group spans GS/DP slices, over the row's LPR
// lanes) by DPP.  A wave covers 64/LPR rows per step; with BULK it takes
// STEPS steps of rows, all their loads issued before any arithmetic.
// Requires x 16-byte and packed 8-byte aligned, rows < 2^31.
template <int D, int NB, int GS, bool F32, bool BULK>
__global__ void __launch_bounds__(256)
quantize_pack_wide_kernel(const void* __restrict__ x, int rows, int HKV, int N,
                          const int32_t* __restrict__ positions, int S_cap, PageMap pm,
                          uint8_t* __restrict__ packed, uint16_t* __restrict__ scale,
                          uint16_t* __restrict__ zero) {
  constexpr int P = 8 / NB, DP = D / P, NG = D / GS, QMAX = (1 << NB) - 1, E = 8;
  constexpr int LPR = DP / E, RPS = 64 / LPR;
  constexpr int NV = F32 ? 2 : 1;  // 16-byte loads per run of E values
  constexpr int STEPS = BULK ? (8 / (P * NV) > 0 ? 8 / (P * NV) : 1) : 1;  // ~128 B per lane
  static_assert(DP % E == 0 && LPR >= 2 && LPR <= 16, "row shape");
  static_assert(GS > DP ? GS % DP == 0 : GS % E == 0, "group shape");

  const int lane = threadIdx.x & 63, slot = lane / LPR, c = lane % LPR;
  const int first = ((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)) * STEPS * RPS;
  u4 raw[STEPS][P][NV];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    int rr = first + s * RPS + slot;
    if (rr >= rows) rr = rows - 1;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t off = (int64_t)rr * D + p * DP + c * E;  // elements
#pragma unroll
      for (int k = 0; k < NV; ++k)
        raw[s][p][k] = F32 ? reinterpret_cast<const u4*>(static_cast<const float*>(x) + off)[k]
                           : reinterpret_cast<const u4*>(static_cast<const _Float16*>(x) + off)[k];
    }
  }
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int rr = first + s * RPS + slot;
    float v[P][E], mn[P], mx[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if constexpr (F32) {
        // Whole-vector casts: this compiler folds a min/max over floats cast
        // one by one from the elements of an integer vector to the first one.
        const f4 lo = __builtin_bit_cast(f4, raw[s][p][0]), hi = __builtin_bit_cast(f4, raw[s][p][1]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[p][e] = lo[e], v[p][e + 4] = hi[e];
      } else {
        const h8 h = __builtin_bit_cast(h8, raw[s][p][0]);
#pragma unroll
        for (int e = 0; e < E; ++e) v[p][e] = (float)h[e];
      }
      mn[p] = mx[p] = v[p][0];
#pragma unroll
      for (int e = 1; e < E; ++e) {
        mn[p] = nan_min(mn[p], v[p][e]);
        mx[p] = nan_max(mx[p], v[p][e]);
      }
    }
    if constexpr (GS <= DP) {
#pragma unroll
      for (int p = 0; p < P; ++p) minmax_lanes<GS / E>(mn[p], mx[p]);
    } else {
      constexpr int SPG = GS / DP;
#pragma unroll
      for (int p = 0; p < P; p += SPG) {
#pragma unroll
        for (int e = 1; e < SPG; ++e) {
          mn[p] = nan_min(mn[p], mn[p + e]);
          mx[p] = nan_max(mx[p], mx[p + e]);
        }
        minmax_lanes<LPR>(mn[p], mx[p]);
#pragma unroll
        for (int e = 1; e < SPG; ++e) {
          mn[p + e] = mn[p];
          mx[p + e] = mx[p];
        }
      }
    }
    float sf[P], zf[P], q[P][E];
    uint16_t s16b[P], z16b[P];
    bool unsure = false;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      float sc = (mx[p] - mn[p]) / (float)QMAX;
      if (!(sc > 0.0f)) sc = 1.0f;
      const _Float16 s16 = (_Float16)sc;
      const _Float16 z16 = (_Float16)mn[p];
      sf[p] = (float)s16;
      zf[p] = (float)z16;
      s16b[p] = __builtin_bit_cast(uint16_t, s16);
      z16b[p] = zero_bits(mn[p]);
      const float rs = __builtin_amdgcn_rcpf(sf[p]);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float y = (v[p][e] - zf[p]) * rs;
        q[p][e] = rintf(y);
        unsure |= quotient_unsure(y, q[p][e]);
      }
    }
    if (__builtin_expect(unsure, 0)) {  // rare: redo the lane's codes by division
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int e = 0; e < E; ++e) q[p][e] = rintf((v[p][e] - zf[p]) / sf[p]);
    }
    uint32_t w[2] = {0, 0};
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float c = q[p][e];
        if (c != c) c = 0.0f;
        c = fminf(fmaxf(c, 0.0f), (float)QMAX);
        w[e / 4] |= (uint32_t)c << (8 * (e % 4) + p * NB);
      }
    if (rr >= rows) continue;  // after the cross-lane steps, which need every lane
    const int bh = rr / N, t = rr - bh * N;
    const int b = bh / HKV, kv = bh - b * HKV;
    const int64_t dst_t = (int64_t)(positions ? positions[b] : 0) + t;
    bool in_range = dst_t >= 0 && dst_t < S_cap;
    int64_t dst_row = (int64_t)bh * S_cap + dst_t;
    if (pm.page_size > 0 && in_range) {  // S_cap == stride * page_size
      const int e = pm.block_table[(int64_t)b * pm.stride + dst_t / pm.page_size];
      in_range = e >= 0 && e < pm.num_pages;  // rows mapped outside the pool are not written
      dst_row = ((int64_t)e * HKV + kv) * pm.page_size + dst_t % pm.page_size;
    }
    if (!in_range) continue;
    *reinterpret_cast<u2*>(packed + dst_row * DP + c * E) = u2{w[0], w[1]};
    // Group g's scale and zero are written by the lane holding its first byte.
#pragma unroll
    for (int p = 0; p < P; ++p) {
      bool first_byte;
      if constexpr (GS <= DP) first_byte = (c * E) % GS == 0;
      else first_byte = c == 0 && p % (GS / DP) == 0;
      if (first_byte) {
        const int g = (p * DP + c * E) / GS;
        scale[dst_row * NG + g] = s16b[p];
        zero[dst_row * NG + g] = z16b[p];
      }
    }
  }
}

// Per-channel (KIVI-style) keys.  One wave quantizes one block of 32 tokens
// of one (b, kv head): every channel of the block is one group of 32 values
// (min/max, fp16 scale and zero, codes), the group-wise arithmetic of
// quantize_row applied along the token axis.  Lane j owns byte column j of
// the block's rows, i.e. channels j + p*DP (p < P), so the min/max need no
// cross-lane step and the lane packs each token's byte j itself.  Lanes >= DP
// repeat lanes j - DP and store nothing.
//   src: element index of the block's first row in x (rows D apart);
//   dst_row: the block's first destination row in packed;
//   meta: element index of the block's scale / zero row (D values).
template <int D, int NB, bool F32>
__device__ __forceinline__ void quantize_key_block(const void* __restrict__ x, int64_t src, int lane,
                                                   bool ok, uint8_t* __restrict__ packed,
                                                   int64_t dst_row, uint16_t* __restrict__ scale,
                                                   uint16_t* __restrict__ zero, int64_t meta) {
  constexpr int P = 8 / NB, DP = D / P, QMAX = (1 << NB) - 1, T = 32;
  const int j = lane % DP;
  ok = ok && lane < DP;
  float v[P][T];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t e = src + (int64_t)t * D + j + p * DP;
      v[p][t] = F32 ? static_cast<const float*>(x)[e] : (float)static_cast<const _Float16*>(x)[e];
    }
  uint32_t bytes[T];
#pragma unroll
  for (int t = 0; t < T; ++t) bytes[t] = 0;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    float mn = v[p][0], mx = v[p][0];
#pragma unroll
    for (int t = 1; t < T; ++t) {
      mn = nan_min(mn, v[p][t]);
      mx = nan_max(mx, v[p][t]);
    }
    float sc = (mx - mn) / (float)QMAX;
    if (!(sc > 0.0f)) sc = 1.0f;
    const _Float16 s16 = (_Float16)sc;
    const _Float16 z16 = (_Float16)mn;
    const float sf = (float)s16, zf = (float)z16, rs = __builtin_amdgcn_rcpf(sf);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float c = rint_quotient(v[p][t] - zf, sf, rs);
      if (c != c) c = 0.0f;
      c = fminf(fmaxf(c, 0.0f), (float)QMAX);
      bytes[t] |= (uint32_t)c << (p * NB);
    }
    if (ok) {
      scale[meta + j + p * DP] = __builtin_bit_cast(uint16_t, s16);
      zero[meta + j + p * DP] = zero_bits(mn);
    }
  }
  if (!ok) return;
#pragma unroll
  for (int t = 0; t < T; ++t) packed[(dst_row + t) * DP + j] = (uint8_t)bytes[t];
}

// One wave per block of 32 tokens of one (b, kv head).  A block whose
// destination does not start on a 32-token boundary, or does not fit
// [0, S_cap), is not written.
template <int D, int NB, bool F32>
__global__ void __launch_bounds__(256)
quantize_keys_channel_kernel(const void* __restrict__ x, int64_t blocks, int HKV, int NBLK,
                             const int32_t* __restrict__ positions, int S_cap,
                             uint8_t* __restrict__ packed, uint16_t* __restrict__ scale,
                             uint16_t* __restrict__ zero) {
  constexpr int T = 32;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t blk = (int64_t)blockIdx.x * 4 + w;
  if (blk >= blocks) return;  // whole wave
  const int64_t bh = blk / NBLK;
  const int tb = (int)(blk - bh * NBLK);
  const int b = (int)(bh / HKV);
  const int64_t dst_t = (int64_t)(positions ? positions[b] : 0) + (int64_t)tb * T;
  const bool ok = dst_t >= 0 && dst_t % T == 0 && dst_t + T <= S_cap;
  quantize_key_block<D, NB, F32>(x, (bh * NBLK + tb) * T * D, lane, ok, packed, bh * S_cap + dst_t,
                                 scale, zero, (bh * (S_cap / T) + dst_t / T) * D);
}

// The fp16 window of per-channel keys: K and V windows (B, HKV, 32, D), row b
// holding res_lens[b] tokens after q_lens[b] quantized ones.
//
// Append: one workgroup per batch row writes the new token of every kv head
// at window row res_lens[b] (if it is below 32) and then advances res_lens[b].
__global__ void __launch_bounds__(256)
channel_window_append_kernel(const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
                             int HKV, int D, uint16_t* __restrict__ k_res,
                             uint16_t* __restrict__ v_res, int32_t* __restrict__ res_lens) {
  constexpr int T = 32;
  const int b = blockIdx.x;
  const int r = res_lens[b];
  if (r < 0 || r >= T) return;  // whole workgroup: a full window must be flushed first
  const int n = HKV * D / 8;    // 16-byte vectors per token and tensor
  for (int i = threadIdx.x; i < 2 * n; i += blockDim.x) {
    const int which = i / n, e = (i % n) * 8, kv = e / D, d = e % D;
    const uint16_t* src = (which ? v_new : k_new) + (int64_t)b * HKV * D + e;
    uint16_t* dst = (which ? v_res : k_res) + (((int64_t)b * HKV + kv) * T + r) * D + d;
    *reinterpret_cast<u4*>(dst) = *reinterpret_cast<const u4*>(src);
  }
  __syncthreads();
  if (threadIdx.x == 0) res_lens[b] = r + 1;
}

// Flush: one workgroup per batch row; if its window holds 32 tokens, wave w
// quantizes the blocks of kv heads w, w + 4, ...: keys per channel
// (quantize_key_block), values per token (quantize_row, as the append kernel)
// into the history at q_lens[b]; then q_lens[b] += 32 and res_lens[b] = 0.
// A window that does not fit the history ([q, q + 32) outside [0, S_cap)) is
// not written and the lengths do not move: res_lens[b] becomes 33, the
// overflow mark, which the append kernel treats as full (nothing more is
// appended) and the decode clamps to the 32 tokens the window holds.
template <int D, int KNB, int VNB, int GS>
__global__ void __launch_bounds__(256)
channel_window_flush_kernel(const uint16_t* __restrict__ k_res, const uint16_t* __restrict__ v_res,
                            int HKV, int S_cap, int32_t* __restrict__ q_lens,
                            int32_t* __restrict__ res_lens, uint8_t* __restrict__ kp,
                            uint16_t* __restrict__ ks, uint16_t* __restrict__ kz,
                            uint8_t* __restrict__ vp, uint16_t* __restrict__ vs,
                            uint16_t* __restrict__ vz) {
  using R = RowQuant<D, VNB, GS>;
  constexpr int T = 32, VDP = R::DP, VNG = R::NG;
  const int b = blockIdx.x;
  if (res_lens[b] != T) return;  // whole workgroup
  const int q = q_lens[b];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (!(q >= 0 && q % T == 0 && q + T <= S_cap)) {  // uniform over the workgroup
    if (threadIdx.x == 0) res_lens[b] = T + 1;
    return;
  }
  const bool ok = true;
  for (int kv = w; kv < HKV; kv += 4) {
    const int64_t bh = (int64_t)b * HKV + kv;
    quantize_key_block<D, KNB, false>(k_res, bh * T * D, lane, ok, kp, bh * S_cap + q, ks, kz,
                                      (bh * (S_cap / T) + q / T) * D);
    for (int t = 0; t < T; ++t) {
      float x[R::P];
      load_row_for_quant<D, VNB>(v_res + (bh * T + t) * D, false, lane, x);
      const R r = quantize_row<D, VNB, GS>(x, lane);
      const int64_t row = bh * S_cap + q + t;
      if (lane < VDP) vp[row * VDP + lane] = (uint8_t)r.byte;
      if (lane < VNG) {
        vs[row * VNG + lane] = (uint16_t)(r.meta & 0xFFFFu);
        vz[row * VNG + lane] = (uint16_t)(r.meta >> 16);
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    q_lens[b] = q + T;
    res_lens[b] = 0;
  }
}

// One thread per packed dword (grid-stride: the grid is capped at 2^20 workgroups).
__global__ void __launch_bounds__(256)
pack_codes_kernel(const uint8_t* __restrict__ codes, int64_t rows, int D, int NB,
                  uint8_t* __restrict__ packed) {
  const int P = 8 / NB, DP = D / P, DW = DP / 4;
  const int64_t n = rows * DW, step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
    const int64_t row = i / DW;
    const int q = (int)(i % DW);
    const uint8_t* c = codes + row * D;
    uint32_t word = 0;
    for (int k = 0; k < 4; ++k) {
      const int jb = 4 * q + k;
      uint32_t byte = 0;
      for (int p = 0; p < P; ++p) byte |= (uint32_t)(c[jb + p * DP] & ((1 << NB) - 1)) << (p * NB);
      word |= byte << (8 * k);
    }
    reinterpret_cast<uint32_t*>(packed + row * DP)[q] = word;
  }
}

__device__ __forceinline__ void emit(uint8_t* codes_out, float* values_out,
                                     const uint16_t* scale, const uint16_t* zero, int64_t row,
                                     int D, int GS, int d, uint32_t code) {
  if (codes_out) codes_out[row * D + d] = (uint8_t)code;
  if (values_out) {
    const int NG = D / GS;
    const float s = (float)__builtin_bit_cast(_Float16, scale[row * NG + d / GS]);
    const float z = (float)__builtin_bit_cast(_Float16, zero[row * NG + d / GS]);
    values_out[row * D + d] = fmaf((float)code, s, z);
  }
}

// Path 0: the K-operand extraction of the decode kernel.  One wave per 16 rows;
// lane (r = l%16, j = l/16) plays the MFMA A-operand role for row r.
template <int D, int NB, int GS>
__global__ void __launch_bounds__(64)
unpack_k_kernel(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scale,
                const uint16_t* __restrict__ zero, int64_t rows, uint8_t* codes_out,
                float* values_out) {
  using KL = KLayout<D, NB, GS>;
  const int lane = threadIdx.x, r = lane & 15, j = lane >> 4;
  const int64_t row = (int64_t)blockIdx.x * 16 + r;
  const int64_t lr = row < rows ? row : rows - 1;
  typename std::conditional<KL::CB == 8, u2, uint32_t>::type kx[KL::NLOAD];
#pragma unroll
  for (int Lh = 0; Lh < KL::NLOAD; ++Lh) {
    const uint8_t* src = packed + lr * KL::DP + KL::load_offset(Lh, j);
    if constexpr (KL::CB == 8) kx[Lh] = ld_u2(src);
    else kx[Lh] = ld_u32(src);
  }
  if (row >= rows) return;
#pragma unroll
  for (int m = 0; m < KL::NKM; ++m) {
    const int p = KL::slice_of(m, j);
    const uint32_t mask = slice_mask<NB>(p);
    uint32_t wv[4] = {0, 0, 0, 0};
    if constexpr (KL::CB == 8) {
      const u4 a = k_extract8(kx[KL::load_of_step(m)], mask);
      wv[0] = a[0]; wv[1] = a[1]; wv[2] = a[2]; wv[3] = a[3];
    } else {
      const u2 a = k_extract4(kx[KL::load_of_step(m)], mask);
      wv[0] = a[0]; wv[1] = a[1];
    }
#pragma unroll
    for (int s = 0; s < KL::CB; ++s) {
      const uint32_t half = (s & 1) ? (wv[s / 2] >> 16) : wv[s / 2];
      emit(codes_out, values_out, scale, zero, row, D, GS, KL::dim_of(m, j, s),
           code_of_half(half, p * NB));
    }
  }
}

// Path 1: the transposed V-operand extraction.  One wave per 32 tokens; lane
// (r, j) gathers tokens slot_token(j, 0..7) for A-operand row r.
template <int D, int NB, int GS>
__global__ void __launch_bounds__(64)
unpack_v_kernel(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scale,
                const uint16_t* __restrict__ zero, int64_t rows, uint8_t* codes_out,
                float* values_out) {
  using VL = VLayout<D, NB, GS>;
  const int lane = threadIdx.x, r = lane & 15, j = lane >> 4;
  const int64_t base = (int64_t)blockIdx.x * 32;
  uint32_t vx[8][VL::NWIN];
  int64_t tok[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    tok[i] = base + (i < 4 ? 0 : 12) + 4 * j + i;
    const int64_t lr = tok[i] < rows ? tok[i] : rows - 1;
#pragma unroll
    for (int wi = 0; wi < VL::NWIN; ++wi)
      vx[i][wi] = ld_u32(packed + lr * VL::DP + VL::dword_offset(wi, r));
  }
#pragma unroll
  for (int wi = 0; wi < VL::NWIN; ++wi) {
#pragma unroll
    for (int e = 0; e < VL::NE; ++e) {
      const uint32_t sel = VL::perm_sel(VL::byte_in_dword(e, r));
#pragma unroll
      for (int p = 0; p < VL::P; ++p) {
        const int mv = VL::mfma_index(p, wi, e);
        const int d = VL::dim_of(mv, r);
        const uint32_t mask = slice_mask<NB>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t pr = v_extract(vx[2 * i + 1][wi], vx[2 * i][wi], sel, mask);
          if (tok[2 * i] < rows)
            emit(codes_out, values_out, scale, zero, tok[2 * i], D, GS, d,
                 code_of_half(pr, p * NB));
          if (tok[2 * i + 1] < rows)
            emit(codes_out, values_out, scale, zero, tok[2 * i + 1], D, GS, d,
                 code_of_half(pr >> 16, p * NB));
        }
      }
    }
  }
}

template <int D, int NB, int GS>
static void launch_quantize(const void* x, bool f32, int64_t rows, int HKV, int N,
                            const int32_t* pos, int S_cap, PageMap pm, uint8_t* pk, uint16_t* sc,
                            uint16_t* zr, hipStream_t st) {
  // The wide kernel needs 16-byte aligned input and 8-byte aligned codes;
  // otherwise one wave per row.  Bulk quantization (a whole prompt or cache)
  // takes several steps of rows per wave.
  constexpr int RPS = 64 / (D * NB / 64);  // rows per wave and step: 64 / (DP / 8)
  const bool wide = !((uintptr_t)x & 15) && !((uintptr_t)pk & 7) && rows <= INT32_MAX;
  if (wide) {
    const bool bulk = rows >= 65536;
    const int steps = bulk ? ((8 / ((8 / NB) * (f32 ? 2 : 1))) > 0 ? 8 / ((8 / NB) * (f32 ? 2 : 1)) : 1) : 1;
    const int per_wg = 4 * RPS * steps;
    const dim3 grid((unsigned)((rows + per_wg - 1) / per_wg));
    const int r = (int)rows;
#define TKV_WIDE(F, BK) \
  quantize_pack_wide_kernel<D, NB, GS, F, BK><<<grid, 256, 0, st>>>(x, r, HKV, N, pos, S_cap, pm, pk, sc, zr)
    if (f32) {
      if (bulk) TKV_WIDE(true, true); else TKV_WIDE(true, false);
    } else {
      if (bulk) TKV_WIDE(false, true); else TKV_WIDE(false, false);
    }
#undef TKV_WIDE
  } else {
    // One wave per row, four per workgroup; launched in pieces so that no grid
    // exceeds 2^32 work-items.
    constexpr int64_t kMaxBlocks = (1 << 24) - 1;
    for (int64_t row0 = 0; row0 < rows; row0 += 4 * kMaxBlocks) {
      const int64_t n = rows - row0 < 4 * kMaxBlocks ? rows - row0 : 4 * kMaxBlocks;
      const dim3 grid((unsigned)((n + 3) / 4));
      if (f32)
        quantize_pack_kernel<D, NB, GS, true><<<grid, 256, 0, st>>>(x, row0, rows, HKV, N, pos, S_cap, pm, pk, sc, zr);
      else
        quantize_pack_kernel<D, NB, GS, false><<<grid, 256, 0, st>>>(x, row0, rows, HKV, N, pos, S_cap, pm, pk, sc, zr);
    }
  }
}

template <int D, int NB, int GS>
static void launch_unpack(const uint8_t* pk, const uint16_t* sc, const uint16_t* zr, int64_t rows,
                          int path, uint8_t* co, float* vo, hipStream_t st) {
  if (path == 0)
    unpack_k_kernel<D, NB, GS><<<dim3((unsigned)((rows + 15) / 16)), 64, 0, st>>>(pk, sc, zr, rows, co, vo);
  else
    unpack_v_kernel<D, NB, GS><<<dim3((unsigned)((rows + 31) / 32)), 64, 0, st>>>(pk, sc, zr, rows, co, vo);
}

// Calls F<D, NB, GS>::run(args...) for the compiled (D, nbits, group size) set.
#define TKV_DISPATCH_DNG(D_, NB_, GS_, CALL)                                          \
  do {                                                                               \
    if ((D_) == 128) {                                                               \
      if ((NB_) == 4) {                                                              \
        if ((GS_) == 16) { CALL(128, 4, 16); }                                       \
        else if ((GS_) == 32) { CALL(128, 4, 32); }                                  \
        else if ((GS_) == 64) { CALL(128, 4, 64); }                                  \
        else if ((GS_) == 128) { CALL(128, 4, 128); }                                \
        else return TKV_EUNSUPPORTED;                                                \
      } else {                                                                       \
        if ((GS_) == 16) { CALL(128, 2, 16); }                                       \
        else if ((GS_) == 32) { CALL(128, 2, 32); }                                  \
        else if ((GS_) == 64) { CALL(128, 2, 64); }                                  \
        else if ((GS_) == 128) { CALL(128, 2, 128); }                                \
        else return TKV_EUNSUPPORTED;                                                \
      }                                                                              \
    } else if ((D_) == 64) {                                                         \
      if ((NB_) == 4) {                                                              \
        if ((GS_) == 16) { CALL(64, 4, 16); }                                        \
        else if ((GS_) == 32) { CALL(64, 4, 32); }                                   \
        else if ((GS_) == 64) { CALL(64, 4, 64); }                                   \
        else return TKV_EUNSUPPORTED;                                                \
      } else {                                                                       \
        if ((GS_) == 16) { CALL(64, 2, 16); }                                        \
        else if ((GS_) == 32) { CALL(64, 2, 32); }                                   \
        else if ((GS_) == 64) { CALL(64, 2, 64); }                                   \
        else return TKV_EUNSUPPORTED;                                                \
      }                                                                              \
    } else {                                                                         \
      return TKV_EUNSUPPORTED;                                                       \
    }                                                                                \
  } while (0)

}  // namespace tkv

extern "C" int tkv_quantize_pack(const void* x, int32_t x_is_fp32, int32_t B, int32_t HKV,
                                 int32_t N, int32_t D, int32_t nbits, int32_t group_size,
                                 const int32_t* positions, int32_t S_cap, uint8_t* packed,
                                 uint16_t* scale, uint16_t* zero, tkv_stream_t stream) {
  using namespace tkv;
  if (!x || !packed || !scale || !zero) return TKV_EINVAL;
  if (B <= 0 || HKV <= 0 || N <= 0 || D <= 0 || S_cap <= 0) return TKV_EINVAL;
  if (nbits != 2 && nbits != 4) return TKV_EINVAL;
  if (group_size <= 0 || D % group_size) return TKV_EINVAL;
  if (!positions && N > S_cap) return TKV_EINVAL;
  if (((uintptr_t)packed & 3) || ((uintptr_t)scale & 1) || ((uintptr_t)zero & 1)) return TKV_EINVAL;
  if ((uintptr_t)x & (x_is_fp32 ? 3 : 1)) return TKV_EINVAL;
  const int64_t rows = (int64_t)B * HKV * N;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const PageMap pm{nullptr, 0, 0, 0};
  (void)hipGetLastError();
#define TKV_Q(Dv, NBv, GSv) \
  launch_quantize<Dv, NBv, GSv>(x, x_is_fp32 != 0, rows, HKV, N, positions, S_cap, pm, packed, scale, zero, st)
  TKV_DISPATCH_DNG(D, nbits, group_size, TKV_Q);
#undef TKV_Q
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TKV_OK : (int)e;
}

extern "C" int tkv_paged_quantize_pack(const void* x, int32_t x_is_fp32, int32_t B, int32_t HKV,
                                       int32_t N, int32_t D, int32_t nbits, int32_t group_size,
                                       const int32_t* positions, const int32_t* block_table,
                                       int32_t block_table_stride, int32_t page_size,
                                       int32_t num_pages, uint8_t* packed, uint16_t* scale,
                                       uint16_t* zero, tkv_stream_t stream) {
  using namespace tkv;
  if (!x || !packed || !scale || !zero || !positions || !block_table) return TKV_EINVAL;
  if (B <= 0 || HKV <= 0 || N <= 0 || D <= 0) return TKV_EINVAL;
  if (block_table_stride <= 0 || page_size <= 0 || page_size % 32 || num_pages <= 0)
    return TKV_EINVAL;
  if ((int64_t)block_table_stride * page_size > INT32_MAX) return TKV_EINVAL;
  if (nbits != 2 && nbits != 4) return TKV_EINVAL;
  if (group_size <= 0 || D % group_size) return TKV_EINVAL;
  if (((uintptr_t)packed & 3) || ((uintptr_t)scale & 1) || ((uintptr_t)zero & 1)) return TKV_EINVAL;
  if ((uintptr_t)x & (x_is_fp32 ? 3 : 1)) return TKV_EINVAL;
  const int64_t rows = (int64_t)B * HKV * N;
  const int S_cap = block_table_stride * page_size;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const PageMap pm{block_table, block_table_stride, page_size, num_pages};
  (void)hipGetLastError();
#define TKV_Q(Dv, NBv, GSv) \
  launch_quantize<Dv, NBv, GSv>(x, x_is_fp32 != 0, rows, HKV, N, positions, S_cap, pm, packed, scale, zero, st)
  TKV_DISPATCH_DNG(D, nbits, group_size, TKV_Q);
#undef TKV_Q
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TKV_OK : (int)e;
}

extern "C" int tkv_quantize_keys_channel(const void* x, int32_t x_is_fp32, int32_t B, int32_t HKV,
                                         int32_t N, int32_t D, int32_t nbits,
                                         const int32_t* positions, int32_t S_cap, uint8_t* packed,
                                         uint16_t* scale, uint16_t* zero, tkv_stream_t stream) {
  using namespace tkv;
  constexpr int T = 32;
  if (!x || !packed || !scale || !zero) return TKV_EINVAL;
  if (B <= 0 || HKV <= 0 || N <= 0 || D <= 0 || S_cap <= 0) return TKV_EINVAL;
  if (N % T || S_cap % T) return TKV_EINVAL;
  if (!positions && N > S_cap) return TKV_EINVAL;
  if (nbits != 2 && nbits != 4) return TKV_EINVAL;
  if (((uintptr_t)scale & 1) || ((uintptr_t)zero & 1)) return TKV_EINVAL;
  if ((uintptr_t)x & (x_is_fp32 ? 3 : 1)) return TKV_EINVAL;
  const int64_t blocks = (int64_t)B * HKV * (N / T);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((blocks + 3) / 4));
  const bool f32 = x_is_fp32 != 0;
  (void)hipGetLastError();
#define TKV_KC(Dv, NBv)                                                                       \
  do {                                                                                        \
    if (f32)                                                                                  \
      quantize_keys_channel_kernel<Dv, NBv, true><<<grid, 256, 0, st>>>(                      \
          x, blocks, HKV, N / T, positions, S_cap, packed, scale, zero);                      \
    else                                                                                      \
      quantize_keys_channel_kernel<Dv, NBv, false><<<grid, 256, 0, st>>>(                     \
          x, blocks, HKV, N / T, positions, S_cap, packed, scale, zero);                      \
  } while (0)
  if (D == 128) {
    if (nbits == 4) TKV_KC(128, 4); else TKV_KC(128, 2);
  } else if (D == 64) {
    if (nbits == 4) TKV_KC(64, 4); else TKV_KC(64, 2);
  } else {
    return TKV_EUNSUPPORTED;
  }
#undef TKV_KC
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TKV_OK : (int)e;
}

extern "C" int tkv_channel_window_append(const void* k_new, const void* v_new, int32_t B,
                                         int32_t HKV, int32_t D, void* k_res, void* v_res,
                                         int32_t res_cap, int32_t* res_lens, tkv_stream_t stream) {
  using namespace tkv;
  if (!k_new || !v_new || !k_res || !v_res || !res_lens) return TKV_EINVAL;
  if (B <= 0 || HKV <= 0 || (D != 64 && D != 128)) return TKV_EINVAL;
  if (res_cap != 32) return TKV_EINVAL;
  if (((uintptr_t)k_new | (uintptr_t)v_new | (uintptr_t)k_res | (uintptr_t)v_res) & 15)
    return TKV_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  channel_window_append_kernel<<<dim3((unsigned)B), 256, 0, st>>>(
      static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new), HKV, D,
      static_cast<uint16_t*>(k_res), static_cast<uint16_t*>(v_res), res_lens);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TKV_OK : (int)e;
}

extern "C" int tkv_channel_window_flush(const void* k_res, const void* v_res, int32_t B,
                                        int32_t HKV, int32_t D, int32_t k_nbits, int32_t v_nbits,
                                        int32_t group_size, int32_t res_cap, int32_t* q_lens,
                                        int32_t* res_lens, int32_t S_cap, uint8_t* k_packed,
                                        uint16_t* k_scale, uint16_t* k_zero, uint8_t* v_packed,
                                        uint16_t* v_scale, uint16_t* v_zero, tkv_stream_t stream) {
  using namespace tkv;
  if (!k_res || !v_res || !q_lens || !res_lens || !k_packed || !k_scale || !k_zero || !v_packed ||
      !v_scale || !v_zero)
    return TKV_EINVAL;
  if (B <= 0 || HKV <= 0 || S_cap <= 0 || S_cap % 32 || res_cap != 32) return TKV_EINVAL;
  if ((k_nbits != 2 && k_nbits != 4) || (v_nbits != 2 && v_nbits != 4)) return TKV_EINVAL;
  if (((uintptr_t)k_res | (uintptr_t)v_res) & 1) return TKV_EINVAL;
  if ((((uintptr_t)k_scale | (uintptr_t)k_zero | (uintptr_t)v_scale | (uintptr_t)v_zero) & 1))
    return TKV_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)B);
  const uint16_t* kr = static_cast<const uint16_t*>(k_res);
  const uint16_t* vr = static_cast<const uint16_t*>(v_res);
  (void)hipGetLastError();
#define TKV_FL(Dv, KB, VB, GSv)                                                                  \
  channel_window_flush_kernel<Dv, KB, VB, GSv><<<grid, 256, 0, st>>>(                            \
      kr, vr, HKV, S_cap, q_lens, res_lens, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero)
#define TKV_FL_GS(Dv, KB, VB)                                                                    \
  do {                                                                                           \
    if (group_size == 16) TKV_FL(Dv, KB, VB, 16);                                                \
    else if (group_size == 32) TKV_FL(Dv, KB, VB, 32);                                           \
    else return TKV_EUNSUPPORTED;                                                                \
  } while (0)
#define TKV_FL_V(Dv, KB)                                                                         \
  do {                                                                                           \
    if (v_nbits == 4) TKV_FL_GS(Dv, KB, 4); else TKV_FL_GS(Dv, KB, 2);                          \
  } while (0)
  if (D == 128) {
    if (k_nbits == 4) TKV_FL_V(128, 4); else TKV_FL_V(128, 2);
  } else if (D == 64) {
    if (k_nbits == 4) TKV_FL_V(64, 4); else TKV_FL_V(64, 2);
  } else {
    return TKV_EUNSUPPORTED;
  }
#undef TKV_FL_V
#undef TKV_FL_GS
#undef TKV_FL
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TKV_OK : (int)e;
}

extern "C" int tkv_pack_codes(const uint8_t* codes, int64_t rows, int32_t D, int32_t nbits,
                              uint8_t* packed, tkv_stream_t stream) {
  using namespace tkv;
  if (!codes || !packed || rows <= 0 || D <= 0) return TKV_EINVAL;
  if (nbits != 2 && nbits != 4) return TKV_EINVAL;
  const int P = 8 / nbits;
  if (D % (4 * P)) return TKV_EUNSUPPORTED;  // whole packed dwords per row
  if ((uintptr_t)packed & 3) return TKV_EINVAL;
  const int64_t n = rows * (D / P / 4);
  (void)hipGetLastError();
  const int64_t blocks = (n + 255) / 256 < (1 << 20) ? (n + 255) / 256 : (1 << 20);  // grid-stride beyond
  pack_codes_kernel<<<dim3((unsigned)blocks), 256, 0,
                      reinterpret_cast<hipStream_t>(stream)>>>(codes, rows, D, nbits, packed);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TKV_OK : (int)e;
}

extern "C" int tkv_unpack_dequant(const uint8_t* packed, const uint16_t* scale,
                                  const uint16_t* zero, int64_t rows, int32_t D, int32_t nbits,
                                  int32_t group_size, int32_t path, uint8_t* codes_out,
                                  float* values_out, tkv_stream_t stream) {
  using namespace tkv;
  if (!packed || rows <= 0 || D <= 0) return TKV_EINVAL;
  if (nbits != 2 && nbits != 4) return TKV_EINVAL;
  if (group_size <= 0 || D % group_size) return TKV_EINVAL;
  if (path != 0 && path != 1) return TKV_EINVAL;
  if (values_out && (!scale || !zero)) return TKV_EINVAL;
  if ((uintptr_t)packed & 7) return TKV_EINVAL;  // dwordx2 loads of the K unpack path
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  (void)hipGetLastError();
#define TKV_U(Dv, NBv, GSv) \
  launch_unpack<Dv, NBv, GSv>(packed, scale, zero, rows, path, codes_out, values_out, st)
  TKV_DISPATCH_DNG(D, nbits, group_size, TKV_U);
#undef TKV_U
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? TKV_OK : (int)e;
}
