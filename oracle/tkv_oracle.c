/* Scalar C restatement of tritonkv's quantizer and fp32 decode attention.
 *
 * TEST INFRASTRUCTURE ONLY: this is a checker (and the CPU baseline that
 * bench.py times), never part of the shipped HIP path.  It is written
 * independently of oracle/quant.py so that the two restatements pin each
 * other bit for bit.
 *
 * Follows the reference:
 *   split-P layout            quantize.py:40-54
 *   pack_codes / unpack_codes quantize.py:149-183
 *   quantize_groupwise        quantize.py:186-236
 *   dequantize_groupwise      quantize.py:239-246
 *   reference attention       reference.py:61-88 (scores, softmax, weighted sum; fp32
 *                             inputs, sums accumulated in binary64, see attend_head)
 *
 * Built with plain IEEE binary32 arithmetic (no -ffast-math): division is
 * correctly rounded, rintf() rounds half to even in the default rounding mode,
 * and the fp16 conversions below are written from the IEEE-754 binary16
 * definition (round to nearest, ties to even).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- binary16 <-> binary32 ------------------------------------------- */

float tkvo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else { /* subnormal: m * 2^-24, renormalise */
        int shift = 0;
        while (!(m & 0x400u)) { m <<= 1; ++shift; }
        m &= 0x3ffu;
        bits = sign | ((uint32_t)(127 - 14 - shift) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t tkvo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) /* inf / nan (nan stays quiet) */
        return sign | 0x7c00u | (a > 0x7f800000u ? (uint16_t)(0x200u | ((a >> 13) & 0x3ffu)) : 0);
    if (a >= 0x477ff000u) /* >= 65520 rounds to infinity */
        return sign | 0x7c00u;
    if (a >= 0x38800000u) { /* normal binary16 range, >= 2^-14 */
        uint32_t h = (((a >> 23) - 127 + 15) << 10) | ((a & 0x7fffffu) >> 13);
        uint32_t rem = a & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
        return sign | (uint16_t)h;
    }
    if (a < 0x33000000u) /* < 2^-25 (or exactly 2^-25, a tie to even) -> 0 */
        return sign;
    { /* subnormal binary16: units of 2^-24 */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        int shift = 126 - (int)e; /* value / 2^-24 = m * 2^(e-126) */
        uint32_t h = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) ++h;
        return sign | (uint16_t)h;
    }
}

/* ---- split-P pack / unpack ------------------------------------------- */

void tkvo_pack_row(const uint8_t *codes, int D, int nbits, uint8_t *packed) {
    int P = 8 / nbits, DP = D / P;
    for (int j = 0; j < DP; ++j) {
        unsigned byte = 0;
        for (int p = 0; p < P; ++p) byte |= (unsigned)codes[j + p * DP] << (p * nbits);
        packed[j] = (uint8_t)byte;
    }
}

void tkvo_unpack_row(const uint8_t *packed, int D, int nbits, uint8_t *codes) {
    int P = 8 / nbits, DP = D / P;
    unsigned mask = (1u << nbits) - 1u;
    for (int d = 0; d < D; ++d)
        codes[d] = (uint8_t)((packed[d % DP] >> ((d / DP) * nbits)) & mask);
}

/* ---- quantize / dequantize ------------------------------------------- */

/* x: rows x D fp32 values.  Writes rows x D/P packed bytes and rows x D/gs
 * fp16 bit patterns of scale and zero.  Returns 0, or -1 on bad arguments. */
int tkvo_quantize(const float *x, int64_t rows, int D, int nbits, int gs,
                  uint8_t *packed, uint16_t *scale16, uint16_t *zero16) {
    if ((nbits != 2 && nbits != 4) || gs <= 0 || D % gs || D % (8 / nbits)) return -1;
    int qmax = (1 << nbits) - 1, NG = D / gs, DP = D / (8 / nbits);
    uint8_t *codes = (uint8_t *)malloc((size_t)D);
    if (!codes) return -1;
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * D;
        for (int g = 0; g < NG; ++g) {
            const float *xg = xr + g * gs;
            float lo = xg[0], hi = xg[0];
            int has_nan = 0;
            for (int i = 0; i < gs; ++i) {
                if (xg[i] != xg[i]) has_nan = 1;
                if (xg[i] < lo) lo = xg[i];
                if (xg[i] > hi) hi = xg[i];
            }
            /* torch's amin/amax propagate a NaN and return the canonical quiet
             * NaN, whatever the input NaN's sign and payload: the group gets
             * scale 1 (NaN > 0 is false), zero fp16 0x7E00 and codes 0. */
            if (has_nan) lo = hi = NAN;
            float scale = (hi - lo) / (float)qmax;
            if (!(scale > 0.0f)) scale = 1.0f;
            uint16_t s16 = tkvo_f32_to_f16(scale);
            uint16_t z16 = has_nan ? (uint16_t)0x7e00u : tkvo_f32_to_f16(lo);
            float sf = tkvo_f16_to_f32(s16), zf = tkvo_f16_to_f32(z16);
            scale16[r * NG + g] = s16;
            zero16[r * NG + g] = z16;
            for (int i = 0; i < gs; ++i) {
                float c = rintf((xg[i] - zf) / sf);
                /* torch.clamp keeps NaN; converting NaN to uint8 then gives 0 */
                if (c != c) c = 0.0f;
                if (c < 0.0f) c = 0.0f;
                if (c > (float)qmax) c = (float)qmax;
                codes[g * gs + i] = (uint8_t)c;
            }
        }
        tkvo_pack_row(codes, D, nbits, packed + r * DP);
    }
    free(codes);
    return 0;
}

void tkvo_dequantize(const uint8_t *packed, const uint16_t *scale16, const uint16_t *zero16,
                     int64_t rows, int D, int nbits, int gs, float *out) {
    int NG = D / gs, DP = D / (8 / nbits);
    uint8_t codes[1024];
    for (int64_t r = 0; r < rows; ++r) {
        tkvo_unpack_row(packed + r * DP, D, nbits, codes);
        for (int d = 0; d < D; ++d) {
            float s = tkvo_f16_to_f32(scale16[r * NG + d / gs]);
            float z = tkvo_f16_to_f32(zero16[r * NG + d / gs]);
            float cs = (float)codes[d] * s; /* exact: code <= 15, s has 11 significant bits */
            out[r * D + d] = cs + z;
        }
    }
}

/* ---- fp32 decode attention ------------------------------------------- */

/* Scores, softmax and the weighted sum accumulate in binary64 and the result
 * is rounded to binary32 once.  The reference computes in fp32 on the GPU,
 * where every reduction is a tree; a scalar loop summing tens of thousands of
 * fp32 terms in order (an fp32 accumulator of ~19 taking addends of 1e-5)
 * drifts by up to ~2e-4 relative, more than the kernel's own error, so the
 * checker keeps the sums exact to well below fp32 resolution instead.  The
 * inputs (dequantized K and V, q) are the fp32 values the reference sees. */
static void attend_head(const float *q, const float *krows, const float *vrows, int n, int D,
                        float sm_scale, double *scores, double *acc, float *out) {
    double m = -INFINITY;
    for (int t = 0; t < n; ++t) {
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += (double)q[d] * (double)krows[(int64_t)t * D + d];
        s *= (double)sm_scale;
        scores[t] = s;
        if (s > m) m = s;
    }
    double l = 0.0;
    for (int t = 0; t < n; ++t) {
        scores[t] = exp(scores[t] - m);
        l += scores[t];
    }
    for (int d = 0; d < D; ++d) acc[d] = 0.0;
    for (int t = 0; t < n; ++t) {
        const double p = scores[t];
        for (int d = 0; d < D; ++d) acc[d] += p * (double)vrows[(int64_t)t * D + d];
    }
    for (int d = 0; d < D; ++d) out[d] = (float)(acc[d] / l);
}

/* q (B,HQ,D), k/v (B,HKV,S,D) fp32, seq_lens NULL or B lengths <= S. */
int tkvo_decode_attention(const float *q, const float *k, const float *v, int B, int HQ, int HKV,
                          int S, int D, float sm_scale, const int64_t *seq_lens, float *out) {
    if (HQ % HKV) return -1;
    int G = HQ / HKV;
    double *scores = (double *)malloc(sizeof(double) * (size_t)(S > 0 ? S : 1));
    double *acc = (double *)malloc(sizeof(double) * (size_t)D);
    if (!scores || !acc) { free(scores); free(acc); return -1; }
    for (int b = 0; b < B; ++b) {
        int n = seq_lens ? (int)seq_lens[b] : S;
        for (int h = 0; h < HQ; ++h) {
            int64_t kv = (int64_t)b * HKV + h / G;
            attend_head(q + ((int64_t)b * HQ + h) * D, k + kv * S * D, v + kv * S * D, n, D,
                        sm_scale, scores, acc, out + ((int64_t)b * HQ + h) * D);
        }
    }
    free(scores); free(acc);
    return 0;
}

/* The reference's CPU path in one call: dequantize K and V of one (b, kv-head)
 * to fp32, then attend with its G query heads.  Caches are (B,HKV,S,*). */
int tkvo_quantized_decode_attention(const float *q, const uint8_t *kp, const uint16_t *ks,
                                    const uint16_t *kz, const uint8_t *vp, const uint16_t *vs,
                                    const uint16_t *vz, int B, int HQ, int HKV, int S, int D,
                                    int nbits, int gs, float sm_scale, float *out) {
    if (HQ % HKV) return -1;
    int G = HQ / HKV, NG = D / gs, DP = D / (8 / nbits);
    float *kf = (float *)malloc(sizeof(float) * (size_t)S * D);
    float *vf = (float *)malloc(sizeof(float) * (size_t)S * D);
    double *scores = (double *)malloc(sizeof(double) * (size_t)(S > 0 ? S : 1));
    double *acc = (double *)malloc(sizeof(double) * (size_t)D);
    if (!kf || !vf || !scores || !acc) { free(kf); free(vf); free(scores); free(acc); return -1; }
    for (int b = 0; b < B; ++b)
        for (int hk = 0; hk < HKV; ++hk) {
            int64_t row0 = ((int64_t)b * HKV + hk) * S;
            tkvo_dequantize(kp + row0 * DP, ks + row0 * NG, kz + row0 * NG, S, D, nbits, gs, kf);
            tkvo_dequantize(vp + row0 * DP, vs + row0 * NG, vz + row0 * NG, S, D, nbits, gs, vf);
            for (int j = 0; j < G; ++j) {
                int h = hk * G + j;
                attend_head(q + ((int64_t)b * HQ + h) * D, kf, vf, S, D, sm_scale, scores, acc,
                            out + ((int64_t)b * HQ + h) * D);
            }
        }
    free(kf); free(vf); free(scores); free(acc);
    return 0;
}
