/*
 * CPU oracle for the MoE expert path -- TEST INFRASTRUCTURE ONLY (see
 * moe_oracle.h).  Loaded by tests/, the smoke check and the benchmark's
 * CPU-baseline leg; never by the product path.
 *
 * Built with -ffp-contract=off: every fused multiply-add the reference build
 * performs is written here as an explicit fmaf(), every other fp32 operation
 * is a separately rounded one, in the reference's order.
 *
 * Parity status of each function (how it is pinned) is listed in
 * tests/test_oracle.py; the whole block is compared bit-for-bit with a build of
 * the reference's own src/quant.cpp + src/tier.cpp (oracle/_ref) and with the
 * committed golden vectors in tests/golden/.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;

void jxo_set_threads(int32_t n) { g_threads = n; }

/* ---------------------------------------------------------------- fp16 -- */

/* Truncating fp32 -> fp16 (src/quant.cpp:909-925): the mantissa is cut, not
 * rounded; exponents below the fp16 normal range shift into subnormals, below
 * 2^-25 give a signed zero, and anything at or above 2^16 (incl. inf/NaN)
 * becomes a signed infinity. */
uint16_t jxo_fp32_to_fp16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t e = (int32_t)((b >> 23) & 0xFFu) - 127 + 15;
    uint32_t m = b & 0x007FFFFFu;
    if (e <= 0) {
        if (e < -10) return sign;
        m |= 0x00800000u;
        return (uint16_t)(sign | (uint16_t)(m >> (uint32_t)(14 - e)));
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (uint16_t)(e << 10) | (uint16_t)(m >> 13));
}

/* Exact IEEE binary16 -> binary32 (src/quant.cpp:876-907). */
float jxo_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t out;
    if (e == 0) {
        if (m == 0) {
            out = sign;
        } else {
            int32_t ee = 1;
            while ((m & 0x400u) == 0) { m <<= 1; ee--; }
            m &= 0x3FFu;
            out = sign | ((uint32_t)(ee + 112) << 23) | (m << 13);
        }
    } else if (e == 31) {
        out = sign | 0x7F800000u | (m << 13);
    } else {
        out = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

static inline float ld_f16(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return jxo_fp16_to_fp32(h);
}

int64_t jxo_row_bytes(int32_t type, int64_t cols) {
    switch (type) {
        case JXO_F32: return cols * 4;
        case JXO_F16:
        case JXO_BF16: return cols * 2;
        case JXO_Q4_0: return ((cols + 31) / 32) * 18;
        case JXO_Q8_0: return ((cols + 31) / 32) * 34;
        case JXO_Q4_K: return ((cols + 255) / 256) * 144;
        case JXO_Q5_0: return ((cols + 31) / 32) * 22;
        case JXO_Q5_K: return ((cols + 255) / 256) * 176;
        case JXO_Q6_K: return ((cols + 255) / 256) * 210;
        default: return -1;
    }
}

/* ------------------------------------------------------ Q8_0 quantize -- */

/* quantize_row_q8_0 (src/quant.cpp:1029-1045): per 32-block d = amax/127,
 * id = 1/d (0 when d == 0), q = clamp(round_half_away(x*id), -127, 127); the
 * stored d is the truncated fp16 of d while q uses the fp32 id. */
void jxo_quantize_row_q8_0(const float* x, uint8_t* y, int64_t k) {
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; ++i) {
        const float* xb = x + i * 32;
        uint8_t* yb = y + i * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            float a = fabsf(xb[j]);
            amax = amax > a ? amax : a;
        }
        const float d = amax / 127.0f;
        const float id = (d != 0.0f) ? (1.0f / d) : 0.0f;
        uint16_t dh = jxo_fp32_to_fp16(d);
        memcpy(yb, &dh, 2);
        for (int j = 0; j < 32; ++j) {
            int v = (int)roundf(xb[j] * id);
            v = v < -127 ? -127 : (v > 127 ? 127 : v);
            yb[2 + j] = (uint8_t)(int8_t)v;
        }
    }
}

/* --------------------------------------------------------- dequantize -- */

static inline void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    /* get_scale_min_k4 (src/quant.cpp:1107-1115): 6-bit scale/min j of 8 */
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* dequantize_row_q4_K (src/quant.cpp:1209-1249).  The reference build
 * contracts  d1*q - m1  into one fused multiply-subtract. */
static void dequant_q4_K(const uint8_t* x, float* y, int64_t k) {
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = x + i * 144;
        const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
        const uint8_t* sc = blk + 4;
        const uint8_t* q = blk + 16;
        float* yb = y + i * 256;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t s, m;
            scale_min_k4(is + 0, sc, &s, &m);
            const float d1 = d * (float)s, m1 = dmin * (float)m;
            scale_min_k4(is + 1, sc, &s, &m);
            const float d2 = d * (float)s, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                yb[j + l] = fmaf(d1, (float)(q[l] & 0x0F), -m1);
                yb[j + 32 + l] = fmaf(d2, (float)(q[l] >> 4), -m2);
            }
            q += 32;
            is += 2;
        }
    }
    const int64_t rem = k - nb * 256;
    if (rem > 0) {
        float tmp[256];
        dequant_q4_K(x + nb * 144, tmp, 256);
        memcpy(y + nb * 256, tmp, (size_t)rem * 4);
    }
}

/* dequantize_row_q5_K (src/quant.cpp:1345-1387), block_q5_K (include/quant.h:36-42: d, dmin,
 * scales[12], qh[32], qs[128]): in 64-element chunk c, element l of the low half takes the low
 * nibble of qs[32c + l] and bit 2c of qh[l], element 32 + l the high nibble and bit 2c + 1;
 * value d*sc*q - dmin*m (d*sc*q is exact, so contracting it changes nothing). */
static void dequant_q5_K(const uint8_t* x, float* y, int64_t k) {
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = x + i * 176;
        const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
        const uint8_t* sc = blk + 4;
        const uint8_t* qh = blk + 16;
        const uint8_t* q = blk + 48;
        float* yb = y + i * 256;
        for (int c = 0; c < 4; ++c) {
            uint8_t s, m;
            scale_min_k4(2 * c, sc, &s, &m);
            const float d1 = d * (float)s, m1 = dmin * (float)m;
            scale_min_k4(2 * c + 1, sc, &s, &m);
            const float d2 = d * (float)s, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                const int q0 = (q[32 * c + l] & 0x0F) | (((qh[l] >> (2 * c)) & 1) << 4);
                const int q1 = (q[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4);
                yb[64 * c + l] = fmaf(d1, (float)q0, -m1);
                yb[64 * c + 32 + l] = fmaf(d2, (float)q1, -m2);
            }
        }
    }
    const int64_t rem = k - nb * 256;
    if (rem > 0) {
        float tmp[256];
        dequant_q5_K(x + nb * 176, tmp, 256);
        memcpy(y + nb * 256, tmp, (size_t)rem * 4);
    }
}

/* The 6-bit quant of element e (0..255) of a block_q6_K (include/quant.h:45-50: ql[128],
 * qh[64], scales[16], d) minus 32, in dequantize_row_q6_K's layout (src/quant.cpp:1389-1428):
 * 128-element half n, quarter r = (e % 128) / 32, l = e % 32 -> nibble (r / 2) of
 * ql[64n + 32 (r % 2) + l] and bits 2r..2r+1 of qh[32n + l]. */
static inline int q6_val(const uint8_t* blk, int e) {
    const int n = e >> 7, r = (e >> 5) & 3, l = e & 31;
    const uint8_t lo = blk[64 * n + 32 * (r & 1) + l];
    const int nib = (r >> 1) ? (lo >> 4) : (lo & 0x0F);
    const int hb = (blk[128 + 32 * n + l] >> (2 * r)) & 3;
    return (nib | (hb << 4)) - 32;
}

/* dequantize_row_q6_K (src/quant.cpp:1389-1428): (d * sc) * q, sc = scales[e / 16]; both
 * products are exact (11-bit d, 8-bit sc, 6-bit q). */
static void dequant_q6_K(const uint8_t* x, float* y, int64_t k) {
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = x + i * 210;
        const float d = ld_f16(blk + 208);
        for (int e = 0; e < 256; ++e)
            y[i * 256 + e] = d * (float)(int8_t)blk[192 + e / 16] * (float)q6_val(blk, e);
    }
    const int64_t rem = k - nb * 256;
    if (rem > 0) {
        float tmp[256];
        dequant_q6_K(x + nb * 210, tmp, 256);
        memcpy(y + nb * 256, tmp, (size_t)rem * 4);
    }
}

/* dequantize_row_q5_0 (src/quant.cpp:1585-1600), block_q5_0 (include/quant.h:60-66: d,
 * qh as a little-endian u32, qs[16]): element j < 16 = low nibble of qs[j] with bit j of qh as
 * its fifth bit, element 16 + j = high nibble with bit 16 + j; value (q - 16) * d (exact). */
static void dequant_q5_0(const uint8_t* x, float* y, int64_t nb) {
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* b = x + i * 22;
        const float d = ld_f16(b);
        uint32_t qh;
        memcpy(&qh, b + 2, 4);
        for (int j = 0; j < 16; ++j) {
            const int lo = (b[6 + j] & 0x0F) | (int)(((qh >> j) & 1u) << 4);
            const int hi = (b[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
            y[i * 32 + j] = (float)(lo - 16) * d;
            y[i * 32 + 16 + j] = (float)(hi - 16) * d;
        }
    }
}

void jxo_dequantize_row(int32_t type, const uint8_t* w, float* y, int64_t k) {
    if (type == JXO_Q4_K) { dequant_q4_K(w, y, k); return; }
    if (type == JXO_Q5_K) { dequant_q5_K(w, y, k); return; }
    if (type == JXO_Q6_K) { dequant_q6_K(w, y, k); return; }
    if (type == JXO_Q5_0) { dequant_q5_0(w, y, k / 32); return; }
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; ++i) {
        if (type == JXO_Q4_0) {  /* dequantize_row_q4_0 (quant.cpp:1014-1027) */
            const uint8_t* b = w + i * 18;
            const float d = ld_f16(b);
            for (int j = 0; j < 16; ++j) {
                y[i * 32 + j] = (float)((b[2 + j] & 0x0F) - 8) * d;
                y[i * 32 + 16 + j] = (float)((b[2 + j] >> 4) - 8) * d;
            }
        } else if (type == JXO_Q8_0) {  /* dequantize_row_q8_0 (quant.cpp:1047-1057) */
            const uint8_t* b = w + i * 34;
            const float d = ld_f16(b);
            for (int j = 0; j < 32; ++j) y[i * 32 + j] = (float)(int8_t)b[2 + j] * d;
        }
    }
}

/* ---------------------------------------------------------- fp32 dots -- */

/* vec_dot_f32 (src/quant.cpp:2756-2778), AVX2 order: two 8-lane FMA chains
 * over 16-element steps, lane-wise add, one more 8-lane FMA pass over an
 * 8-element remainder, a sequential sum of the 8 lanes, then a scalar
 * (contracted) tail. */
float jxo_vec_dot_f32(const float* a, const float* b, int64_t k) {
    float acc0[8] = {0}, acc1[8] = {0};
    int64_t i = 0;
    for (; i + 16 <= k; i += 16) {
        for (int j = 0; j < 8; ++j) {
            acc0[j] = fmaf(a[i + j], b[i + j], acc0[j]);
            acc1[j] = fmaf(a[i + 8 + j], b[i + 8 + j], acc1[j]);
        }
    }
    for (int j = 0; j < 8; ++j) acc0[j] = acc0[j] + acc1[j];
    for (; i + 8 <= k; i += 8)
        for (int j = 0; j < 8; ++j) acc0[j] = fmaf(a[i + j], b[i + j], acc0[j]);
    float sum = 0.0f;
    for (int j = 0; j < 8; ++j) sum += acc0[j];
    for (; i < k; ++i) sum = fmaf(a[i], b[i], sum);
    return sum;
}

/* vec_dot_q4_K_f32 (src/quant.cpp:2910-3013), AVX2 order, including the
 * dequantize-and-vec_dot_f32 treatment of a final partial super-block. */
float jxo_vec_dot_q4_K_f32(const uint8_t* x, const float* y, int64_t k) {
    const int64_t nb = k / 256;
    float acc[8] = {0};
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = x + i * 144;
        const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
        const uint8_t* scs = blk + 4;
        const uint8_t* q = blk + 16;
        const float* yb = y + i * 256;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t s, m;
            scale_min_k4(is + 0, scs, &s, &m);
            const float d1 = d * (float)s, m1 = dmin * (float)m;
            scale_min_k4(is + 1, scs, &s, &m);
            const float d2 = d * (float)s, m2 = dmin * (float)m;
            float qs1[8] = {0}, qs2[8] = {0}, ys1[8] = {0}, ys2[8] = {0};
            for (int h = 0; h < 2; ++h) {
                const uint8_t* qb = q + h * 16;
                const float* y1 = yb + j + h * 16;
                const float* y2 = yb + j + 32 + h * 16;
                for (int t = 0; t < 8; ++t) {
                    ys1[t] = ys1[t] + (y1[t] + y1[8 + t]);
                    ys2[t] = ys2[t] + (y2[t] + y2[8 + t]);
                }
                for (int t = 0; t < 8; ++t) {
                    qs1[t] = fmaf((float)(qb[t] & 0x0F), y1[t], qs1[t]);
                    qs1[t] = fmaf((float)(qb[8 + t] & 0x0F), y1[8 + t], qs1[t]);
                    qs2[t] = fmaf((float)(qb[t] >> 4), y2[t], qs2[t]);
                    qs2[t] = fmaf((float)(qb[8 + t] >> 4), y2[8 + t], qs2[t]);
                }
            }
            for (int t = 0; t < 8; ++t) {
                const float pos = fmaf(d1, qs1[t], d2 * qs2[t]);
                const float neg = fmaf(m1, ys1[t], m2 * ys2[t]);
                acc[t] = acc[t] + (pos - neg);
            }
            q += 32;
            is += 2;
        }
    }
    float total = 0.0f;
    for (int t = 0; t < 8; ++t) total += acc[t];
    const int64_t rem = k - nb * 256;
    if (rem > 0) {
        float deq[256];
        dequant_q4_K(x + nb * 144, deq, 256);
        total += jxo_vec_dot_f32(deq, y + nb * 256, rem);
    }
    return total;
}

/* vec_dot_q4_0_f32 (src/quant.cpp:2780-2827) and vec_dot_q8_0_f32 (2829-2862), AVX2 order:
 * per 32-block an 8-lane sum bsum (Q4_0: lane t = ((lo[t] * y[t] + lo[8+t] * y[8+t]) +
 * hi[t] * y[16+t]) + hi[8+t] * y[24+t] as one multiply and three fmas, weights q - 8; Q8_0:
 * four fmas from zero over 8-element chunks), acc_t = fma(d, bsum_t, acc_t), the 8 lanes
 * summed in order.  Whole blocks only (k / 32). */
static float dot_q4_0_f32(const uint8_t* x, const float* y, int64_t k) {
    float acc[8] = {0};
    for (int64_t i = 0; i < k / 32; ++i) {
        const uint8_t* b = x + i * 18;
        const float d = ld_f16(b);
        const float* yb = y + i * 32;
        for (int t = 0; t < 8; ++t) {
            float bs = (float)((b[2 + t] & 0x0F) - 8) * yb[t];
            bs = fmaf((float)((b[2 + 8 + t] & 0x0F) - 8), yb[8 + t], bs);
            bs = fmaf((float)((b[2 + t] >> 4) - 8), yb[16 + t], bs);
            bs = fmaf((float)((b[2 + 8 + t] >> 4) - 8), yb[24 + t], bs);
            acc[t] = fmaf(d, bs, acc[t]);
        }
    }
    float total = 0.0f;
    for (int t = 0; t < 8; ++t) total += acc[t];
    return total;
}

static float dot_q8_0_f32(const uint8_t* x, const float* y, int64_t k) {
    float acc[8] = {0};
    for (int64_t i = 0; i < k / 32; ++i) {
        const uint8_t* b = x + i * 34;
        const float d = ld_f16(b);
        for (int t = 0; t < 8; ++t) {
            float bs = 0.0f;
            for (int c = 0; c < 4; ++c) bs = fmaf((float)(int8_t)b[2 + 8 * c + t], y[i * 32 + 8 * c + t], bs);
            acc[t] = fmaf(d, bs, acc[t]);
        }
    }
    float total = 0.0f;
    for (int t = 0; t < 8; ++t) total += acc[t];
    return total;
}

/* vec_dot_deq_f32 (src/quant.cpp:3208-3229) as vec_dot_q5_0_f32 uses it (3232-3234), and
 * vec_dot_q5_K_f32 (3069-3085): each block dequantized, vec_dot_f32 over it, the block dots
 * added in order; a partial last block is dequantized whole and dotted over its valid
 * elements. */
static float dot_deq_f32(int32_t type, const uint8_t* x, const float* y, int64_t k) {
    const int blk = type == JXO_Q5_0 ? 32 : 256;
    const int64_t bytes = jxo_row_bytes(type, blk);
    const int64_t nb = k / blk, rem = k - nb * blk;
    float deq[256];
    float sum = 0.0f;
    for (int64_t i = 0; i < nb; ++i) {
        jxo_dequantize_row(type, x + i * bytes, deq, blk);
        sum += jxo_vec_dot_f32(deq, y + i * blk, blk);
    }
    if (rem > 0) {
        jxo_dequantize_row(type, x + nb * bytes, deq, blk);
        sum += jxo_vec_dot_f32(deq, y + nb * blk, rem);
    }
    return sum;
}

/* vec_dot_q6_K_f32 (src/quant.cpp:3087-3165), AVX2 order: per 128-element half and 16-element
 * step is (0, 1), for the four quarters r in order an 8-lane product p_t = fma(q[8+t], y[8+t],
 * q[t] * y[t]) over elements 32 r + 16 is .. + 15 of the half, then acc_t = fma(d * sc, p_t,
 * acc_t) with sc = scales[8 n + 2 r + is]; the 8 lanes summed in order; a partial last block
 * dequantized and dotted with vec_dot_f32. */
static float dot_q6_K_f32(const uint8_t* x, const float* y, int64_t k) {
    const int64_t nb = k / 256;
    float acc[8] = {0};
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = x + i * 210;
        const float d = ld_f16(blk + 208);
        for (int n = 0; n < 2; ++n)
            for (int is = 0; is < 2; ++is)
                for (int r = 0; r < 4; ++r) {
                    const int e0 = 128 * n + 32 * r + 16 * is;
                    const float* yb = y + i * 256 + e0;
                    const float ds = d * (float)(int8_t)blk[192 + 8 * n + 2 * r + is];
                    for (int t = 0; t < 8; ++t) {
                        const float p = fmaf((float)q6_val(blk, e0 + 8 + t), yb[8 + t], (float)q6_val(blk, e0 + t) * yb[t]);
                        acc[t] = fmaf(ds, p, acc[t]);
                    }
                }
    }
    float total = 0.0f;
    for (int t = 0; t < 8; ++t) total += acc[t];
    const int64_t rem = k - nb * 256;
    if (rem > 0) {
        float deq[256];
        dequant_q6_K(x + nb * 210, deq, 256);
        total += jxo_vec_dot_f32(deq, y + nb * 256, rem);
    }
    return total;
}

/* vec_dot_f16_f32 / vec_dot_bf16_f32 (src/quant.cpp:3015-3055), AVX2 order: one 8-lane accumulator
 * over 8-element steps, acc_j = fma(w[i + j], y[i + j], acc_j) with the weight widened exactly
 * (fp16_to_fp32 / bf16_to_fp32, src/quant.cpp:876-932), the 8 lanes summed in order from zero, then
 * the scalar tail contracted like vec_dot_f32's. */
static float h16_to_f32(int32_t type, uint16_t h) {
    if (type == JXO_F16) return jxo_fp16_to_fp32(h);
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float jxo_vec_dot_h16_f32(int32_t type, const uint16_t* w, const float* y, int64_t k) {
    float acc[8] = {0};
    int64_t i = 0;
    for (; i + 8 <= k; i += 8)
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(h16_to_f32(type, w[i + j]), y[i + j], acc[j]);
    float total = 0.0f;
    for (int j = 0; j < 8; ++j) total += acc[j];
    for (; i < k; ++i) total = fmaf(h16_to_f32(type, w[i]), y[i], total);
    return total;
}

/* One router row's logit (matmul_quant_f32(lw.router_gate->type, ...), transformer.cpp:2591: with
 * E < 8 rows or a non-Q8 type, vec_dot_quant_f32 of the row). */
static float router_dot(const jxo_moe_desc* L, int32_t e, const float* x) {
    const int64_t d = L->d_model;
    if (L->router_type == JXO_F16 || L->router_type == JXO_BF16)
        return jxo_vec_dot_h16_f32(L->router_type, (const uint16_t*)L->router + e * d, x, d);
    return jxo_vec_dot_f32((const float*)L->router + e * d, x, d);
}

float jxo_vec_dot_quant_f32(int32_t type, const uint8_t* w, const float* y, int64_t k) {
    switch (type) {
        case JXO_F32: return jxo_vec_dot_f32((const float*)(const void*)w, y, k);
        case JXO_F16:
        case JXO_BF16: return jxo_vec_dot_h16_f32(type, (const uint16_t*)(const void*)w, y, k);
        case JXO_Q4_0: return dot_q4_0_f32(w, y, k);
        case JXO_Q8_0: return dot_q8_0_f32(w, y, k);
        case JXO_Q4_K: return jxo_vec_dot_q4_K_f32(w, y, k);
        case JXO_Q5_0:
        case JXO_Q5_K: return dot_deq_f32(type, w, y, k);
        case JXO_Q6_K: return dot_q6_K_f32(w, y, k);
        default: abort();
    }
}

/* --------------------------------------------- Q8_0-activation dots -- */

/* int32 lane t of a 32-element block covers elements 4t..4t+3 (the
 * maddubs + madd(ones) reduction of the reference's dot kernels). */
static inline void lanes_q4_0(const uint8_t* blk, const uint8_t* yq, int32_t s[8]) {
    for (int t = 0; t < 8; ++t) {
        int32_t acc = 0;
        for (int e = 4 * t; e < 4 * t + 4; ++e) {
            int w = e < 16 ? (blk[2 + e] & 0x0F) - 8 : (blk[2 + e - 16] >> 4) - 8;
            acc += w * (int8_t)yq[2 + e];
        }
        s[t] = acc;
    }
}

static inline void lanes_q8_0(const uint8_t* blk, const uint8_t* yq, int32_t s[8]) {
    for (int t = 0; t < 8; ++t) {
        int32_t acc = 0;
        for (int e = 4 * t; e < 4 * t + 4; ++e) acc += (int8_t)blk[2 + e] * (int8_t)yq[2 + e];
        s[t] = acc;
    }
}

/* The 16-lane reduction _mm512_reduce_add_ps performs (GCC avx512fintrin.h):
 * halves, then quarters, then pairs. */
static inline float reduce16(const float a[16]) {
    float t3[8], t6[4];
    for (int i = 0; i < 8; ++i) t3[i] = a[8 + i] + a[i];
    for (int i = 0; i < 4; ++i) t6[i] = t3[4 + i] + t3[i];
    return (t6[0] + t6[2]) + (t6[1] + t6[3]);
}

/* vec_dot_q4_0_q8_0 (src/quant.cpp:3307-3348) and vec_dot_q8_0_q8_0
 * (3405-3439): acc_t = fma(dw*dx, lane_t, acc_t) per block, lanes summed in
 * order at the end.  AVX-512 variants (3359-3402, 3443-3474): two blocks per
 * step on 16 lanes, a tree reduction, and the AVX2 kernel for an odd last
 * block. */
static float dot_q4q8_32(int32_t type, const uint8_t* w, const uint8_t* y, int64_t nb) {
    const int bsz = type == JXO_Q4_0 ? 18 : 34;
    float acc[8] = {0};
    int32_t s[8];
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = w + i * bsz;
        const uint8_t* yq = y + i * 34;
        const float d = ld_f16(blk) * ld_f16(yq);
        if (type == JXO_Q4_0) lanes_q4_0(blk, yq, s); else lanes_q8_0(blk, yq, s);
        for (int t = 0; t < 8; ++t) acc[t] = fmaf(d, (float)s[t], acc[t]);
    }
    float total = 0.0f;
    for (int t = 0; t < 8; ++t) total += acc[t];
    return total;
}

static float dot_q4q8_32_avx512(int32_t type, const uint8_t* w, const uint8_t* y, int64_t nb) {
    const int bsz = type == JXO_Q4_0 ? 18 : 34;
    float acc[16] = {0};
    int32_t s0[8], s1[8];
    int64_t i = 0;
    for (; i + 1 < nb; i += 2) {
        const uint8_t *b0 = w + i * bsz, *b1 = w + (i + 1) * bsz;
        const uint8_t *y0 = y + i * 34, *y1 = y + (i + 1) * 34;
        const float d0 = ld_f16(b0) * ld_f16(y0);
        const float d1 = ld_f16(b1) * ld_f16(y1);
        if (type == JXO_Q4_0) { lanes_q4_0(b0, y0, s0); lanes_q4_0(b1, y1, s1); }
        else { lanes_q8_0(b0, y0, s0); lanes_q8_0(b1, y1, s1); }
        for (int t = 0; t < 8; ++t) {
            acc[t] = fmaf(d0, (float)s0[t], acc[t]);
            acc[8 + t] = fmaf(d1, (float)s1[t], acc[8 + t]);
        }
    }
    float total = reduce16(acc);
    if (i < nb) total += dot_q4q8_32(type, w + i * bsz, y + i * 34, nb - i);
    return total;
}

/* vec_dot_q4_K_q8_0 (src/quant.cpp:3477-3573), AVX-512 variant 3581-3645:
 * per sub-block pair, fma(d*sc*dy, dot) then fnmadd(dmin*m*dy, sum(y)). */
static float dot_q4K_q8(const uint8_t* x, const uint8_t* y, int64_t k, int32_t order) {
    const int64_t nb = k / 256;
    float acc[16] = {0};
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = x + i * 144;
        const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
        const uint8_t* scs = blk + 4;
        const uint8_t* q = blk + 16;
        const uint8_t* yb = y + i * 8 * 34;
        int is = 0;
        for (int j = 0; j < 4; ++j) {
            uint8_t s, m;
            scale_min_k4(is + 0, scs, &s, &m);
            const float d1 = d * (float)s, m1 = dmin * (float)m;
            scale_min_k4(is + 1, scs, &s, &m);
            const float d2 = d * (float)s, m2 = dmin * (float)m;
            const uint8_t* ya = yb + (2 * j) * 34;
            const uint8_t* yc = yb + (2 * j + 1) * 34;
            int32_t dot0[8], sum0[8], dot1[8], sum1[8];
            for (int t = 0; t < 8; ++t) {
                int32_t a = 0, b = 0, c = 0, e = 0;
                for (int l = 4 * t; l < 4 * t + 4; ++l) {
                    a += (q[l] & 0x0F) * (int8_t)ya[2 + l];
                    b += (int8_t)ya[2 + l];
                    c += (q[l] >> 4) * (int8_t)yc[2 + l];
                    e += (int8_t)yc[2 + l];
                }
                dot0[t] = a; sum0[t] = b; dot1[t] = c; sum1[t] = e;
            }
            const float dy0 = ld_f16(ya), dy1 = ld_f16(yc);
            if (order == JXO_ORDER_AVX512) {
                const float sd0 = d1 * dy0, sd1 = d2 * dy1, sm0 = m1 * dy0, sm1 = m2 * dy1;
                for (int t = 0; t < 8; ++t) {
                    acc[t] = fmaf(sd0, (float)dot0[t], acc[t]);
                    acc[8 + t] = fmaf(sd1, (float)dot1[t], acc[8 + t]);
                }
                for (int t = 0; t < 8; ++t) {
                    acc[t] = fmaf(-sm0, (float)sum0[t], acc[t]);
                    acc[8 + t] = fmaf(-sm1, (float)sum1[t], acc[8 + t]);
                }
            } else {
                const float a1 = d1 * dy0, b1 = m1 * dy0, a2 = d2 * dy1, b2 = m2 * dy1;
                for (int t = 0; t < 8; ++t) {
                    acc[t] = fmaf(a1, (float)dot0[t], acc[t]);
                    acc[t] = fmaf(-b1, (float)sum0[t], acc[t]);
                    acc[t] = fmaf(a2, (float)dot1[t], acc[t]);
                    acc[t] = fmaf(-b2, (float)sum1[t], acc[t]);
                }
            }
            q += 32;
            is += 2;
        }
    }
    float total;
    if (order == JXO_ORDER_AVX512) {
        total = reduce16(acc);
    } else {
        total = 0.0f;
        for (int t = 0; t < 8; ++t) total += acc[t];
    }
    const int64_t rem = k - nb * 256;
    if (rem > 0) {
        float deq[256], yf[256];
        dequant_q4_K(x + nb * 144, deq, 256);
        jxo_dequantize_row(JXO_Q8_0, y + nb * 8 * 34, yf, 256);
        total += jxo_vec_dot_f32(deq, yf, rem);
    }
    return total;
}

/* vec_dot_q5_K_q8_0 (src/quant.cpp:3648-3721; AVX2 only, no AVX-512 variant): as the Q4_K
 * AVX2 dot with 5-bit quants -- per 64-element chunk c, lane t of each 32-block takes the exact
 * integer dot of elements 4t..4t+3 and the sum of their activation quants, then
 * acc_t = fma(d1 dy0, dot0_t), fma(-(m1 dy0), sum0_t), fma(d2 dy1, dot1_t), fma(-(m2 dy1), sum1_t);
 * the 8 lanes summed in order; a partial last block as in dot_q4K_q8. */
static float dot_q5K_q8(const uint8_t* x, const uint8_t* y, int64_t k) {
    const int64_t nb = k / 256;
    float acc[8] = {0};
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = x + i * 176;
        const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
        const uint8_t* scs = blk + 4;
        const uint8_t* qh = blk + 16;
        const uint8_t* q = blk + 48;
        const uint8_t* yb = y + i * 8 * 34;
        for (int c = 0; c < 4; ++c) {
            uint8_t s, m;
            scale_min_k4(2 * c, scs, &s, &m);
            const float d1 = d * (float)s, m1 = dmin * (float)m;
            scale_min_k4(2 * c + 1, scs, &s, &m);
            const float d2 = d * (float)s, m2 = dmin * (float)m;
            const uint8_t* ya = yb + (2 * c) * 34;
            const uint8_t* yc = yb + (2 * c + 1) * 34;
            const float dy0 = ld_f16(ya), dy1 = ld_f16(yc);
            for (int t = 0; t < 8; ++t) {
                int32_t a = 0, b = 0, cc = 0, e = 0;
                for (int l = 4 * t; l < 4 * t + 4; ++l) {
                    const int q0 = (q[32 * c + l] & 0x0F) | (((qh[l] >> (2 * c)) & 1) << 4);
                    const int q1 = (q[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4);
                    a += q0 * (int8_t)ya[2 + l];
                    b += (int8_t)ya[2 + l];
                    cc += q1 * (int8_t)yc[2 + l];
                    e += (int8_t)yc[2 + l];
                }
                acc[t] = fmaf(d1 * dy0, (float)a, acc[t]);
                acc[t] = fmaf(-(m1 * dy0), (float)b, acc[t]);
                acc[t] = fmaf(d2 * dy1, (float)cc, acc[t]);
                acc[t] = fmaf(-(m2 * dy1), (float)e, acc[t]);
            }
        }
    }
    float total = 0.0f;
    for (int t = 0; t < 8; ++t) total += acc[t];
    const int64_t rem = k - nb * 256;
    if (rem > 0) {
        float deq[256], yf[256];
        dequant_q5_K(x + nb * 176, deq, 256);
        jxo_dequantize_row(JXO_Q8_0, y + nb * 8 * 34, yf, 256);
        total += jxo_vec_dot_f32(deq, yf, rem);
    }
    return total;
}

/* vec_dot_q6_K_q8_0 (src/quant.cpp:3723-3818; AVX2 only): per 128-element half n and quarter r
 * (the half's 32-block r), four int32 lanes s_r[t] = sc[8n + 2r] * (dot of elements 4t..4t+3)
 * + sc[8n + 2r + 1] * (dot of elements 16 + 4t..16 + 4t+3), exact; lanes 0-3 of acc take
 * fma(d * dy_0, s_0[t]) then fma(d * dy_2, s_2[t]), lanes 4-7 fma(d * dy_1, s_1[t]) then
 * fma(d * dy_3, s_3[t]); the 8 lanes summed in order; a partial last block dequantized. */
static float dot_q6K_q8(const uint8_t* x, const uint8_t* y, int64_t k) {
    const int64_t nb = k / 256;
    float acc[8] = {0};
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = x + i * 210;
        const float d = ld_f16(blk + 208);
        for (int n = 0; n < 2; ++n) {
            int32_t sr[4][4];
            float dy[4];
            for (int r = 0; r < 4; ++r) {
                const uint8_t* yq = y + (i * 8 + 4 * n + r) * 34;
                dy[r] = d * ld_f16(yq);
                const int sa = (int8_t)blk[192 + 8 * n + 2 * r], sb = (int8_t)blk[192 + 8 * n + 2 * r + 1];
                for (int t = 0; t < 4; ++t) {
                    int32_t a = 0, b = 0;
                    for (int l = 4 * t; l < 4 * t + 4; ++l) {
                        a += q6_val(blk, 128 * n + 32 * r + l) * (int8_t)yq[2 + l];
                        b += q6_val(blk, 128 * n + 32 * r + 16 + l) * (int8_t)yq[2 + 16 + l];
                    }
                    sr[r][t] = sa * a + sb * b;
                }
            }
            for (int t = 0; t < 4; ++t) {
                acc[t] = fmaf(dy[0], (float)sr[0][t], acc[t]);
                acc[4 + t] = fmaf(dy[1], (float)sr[1][t], acc[4 + t]);
            }
            for (int t = 0; t < 4; ++t) {
                acc[t] = fmaf(dy[2], (float)sr[2][t], acc[t]);
                acc[4 + t] = fmaf(dy[3], (float)sr[3][t], acc[4 + t]);
            }
        }
    }
    float total = 0.0f;
    for (int t = 0; t < 8; ++t) total += acc[t];
    const int64_t rem = k - nb * 256;
    if (rem > 0) {
        float deq[256], yf[256];
        dequant_q6_K(x + nb * 210, deq, 256);
        jxo_dequantize_row(JXO_Q8_0, y + nb * 8 * 34, yf, 256);
        total += jxo_vec_dot_f32(deq, yf, rem);
    }
    return total;
}

float jxo_vec_dot_q8(int32_t type, const uint8_t* w, const uint8_t* xq8, int64_t k, int32_t order) {
    if (type == JXO_Q4_K) return dot_q4K_q8(w, xq8, k, order);
    if (type == JXO_Q5_K) return dot_q5K_q8(w, xq8, k);
    if (type == JXO_Q6_K) return dot_q6K_q8(w, xq8, k);
    const int64_t nb = k / 32;
    if (order == JXO_ORDER_AVX512) return dot_q4q8_32_avx512(type, w, xq8, nb);
    return dot_q4q8_32(type, w, xq8, nb);
}

/* ----------------------------------------------------- matmul drivers -- */

static int supports_q8_act(int32_t type, int64_t cols) {
    /* supports_q8_activation (src/quant.cpp:3881-3893) */
    if (type == JXO_Q4_0 || type == JXO_Q8_0) return cols % 32 == 0;
    if (type == JXO_Q4_K || type == JXO_Q5_K || type == JXO_Q6_K) return cols % 256 == 0;
    return 0;
}

/* vec_dot_row_with_q8 (src/quant.cpp:3841-3879): the Q8_0-activation dot where a Q8_0 x
 * exists and the type/cols rule allows it, else the fp32-activation dot (vec_dot_quant_f32,
 * 3269-3305). */
static float row_dot(int32_t type, const uint8_t* row, const float* x, const uint8_t* xq8,
                     int64_t cols, int32_t order) {
    if (xq8 && type != JXO_F32 && type != JXO_Q5_0 && supports_q8_act(type, cols))
        return jxo_vec_dot_q8(type, row, xq8, cols, order);
    return jxo_vec_dot_quant_f32(type, row, x, cols);
}

/* matmul_quant_f32 (src/quant.cpp:3895-3922): Q8_0 activations iff rows >= 8
 * and the type/cols rule allows; rows are independent. */
void jxo_matmul_quant_f32(int32_t type, const uint8_t* W, const float* x, float* out,
                          int64_t rows, int64_t cols, int32_t order) {
    const int64_t rb = jxo_row_bytes(type, cols);
    uint8_t* xq = NULL;
    if (rows >= 8 && supports_q8_act(type, cols)) {
        xq = (uint8_t*)malloc((size_t)(cols / 32) * 34);
        jxo_quantize_row_q8_0(x, xq, cols);
    }
    int nth = g_threads;
#pragma omp parallel for schedule(static) if (rows >= 64) num_threads(nth > 0 ? nth : omp_get_max_threads())
    for (int64_t r = 0; r < rows; ++r) out[r] = row_dot(type, W + r * rb, x, xq, cols, order);
    free(xq);
}

/* matmul_swiglu_quant_f32 (src/quant.cpp:3970-4009): Q8_0 activations iff
 * exp_dim >= 8 and cols % 32 == 0; out = (g / (1 + exp(-g))) * u, or with
 * use_gelu (3999-4003) GELU-tanh(g) * u: inner = sqrt(2/pi) * (g + 0.044715 g^3),
 * whose inner sum the reference build contracts to one fma (GCC's default
 * -ffp-contract=fast with -mfma), then 0.5 g (1 + tanh(inner)) * u. */
void jxo_matmul_swiglu_quant_f32(int32_t gate_type, const uint8_t* Wg, int32_t up_type, const uint8_t* Wu,
                                 const float* x, float* out, int64_t exp_dim, int64_t cols, int32_t use_gelu,
                                 int32_t order) {
    const int64_t gb = jxo_row_bytes(gate_type, cols), ub = jxo_row_bytes(up_type, cols);
    uint8_t* xq = NULL;
    if (exp_dim >= 8 && cols % 32 == 0) {
        xq = (uint8_t*)malloc((size_t)(cols / 32) * 34);
        jxo_quantize_row_q8_0(x, xq, cols);
    }
    int nth = g_threads;
#pragma omp parallel for schedule(static) if (exp_dim >= 64) num_threads(nth > 0 ? nth : omp_get_max_threads())
    for (int64_t r = 0; r < exp_dim; ++r) {
        const float g = row_dot(gate_type, Wg + r * gb, x, xq, cols, order);
        const float u = row_dot(up_type, Wu + r * ub, x, xq, cols, order);
        if (use_gelu) {
            const float inner = 0.7978845608028654f * fmaf(0.044715f * g * g, g, g);
            out[r] = 0.5f * g * (1.0f + tanhf(inner)) * u;
        } else {
            out[r] = (g / (1.0f + expf(-g))) * u;
        }
    }
    free(xq);
}

/* matmul_qkv_quant_f32 (src/quant.cpp:3924-3968): x quantized once when the
 * given matrices (NULL ones skipped) hold 8 rows or more together and
 * cols % 32 == 0; each row then takes the Q8_0 dot where its type allows. */
void jxo_matmul_qkv_quant_f32(int32_t wq_type, const uint8_t* Wq, int64_t q_rows, float* q_out,
                              int32_t wk_type, const uint8_t* Wk, int64_t k_rows, float* k_out,
                              int32_t wv_type, const uint8_t* Wv, int64_t v_rows, float* v_out,
                              const float* x, int64_t cols, int32_t order) {
    const int64_t total = (Wq ? q_rows : 0) + (Wk ? k_rows : 0) + (Wv ? v_rows : 0);
    if (total <= 0) return;
    uint8_t* xq = NULL;
    if (total >= 8 && cols % 32 == 0) {
        xq = (uint8_t*)malloc((size_t)(cols / 32) * 34);
        jxo_quantize_row_q8_0(x, xq, cols);
    }
    const int32_t types[3] = {wq_type, wk_type, wv_type};
    const uint8_t* W[3] = {Wq, Wk, Wv};
    const int64_t rows[3] = {q_rows, k_rows, v_rows};
    float* outs[3] = {q_out, k_out, v_out};
    for (int m = 0; m < 3; ++m) {
        if (!W[m]) continue;
        const int64_t rb = jxo_row_bytes(types[m], cols);
        for (int64_t r = 0; r < rows[m]; ++r) outs[m][r] = row_dot(types[m], W[m] + r * rb, x, xq, cols, order);
    }
    free(xq);
}

/* ----------------------------------------------------------- routing -- */

/* select_experts_cache_aware (src/tier.cpp:124-198) with CACHE_ROUTE off:
 * order by logit descending, keep top_k, softmax over the kept logits
 * (exp(l - max), sequential sum, one reciprocal, multiply).  Exact ties are
 * ordered by expert index here; the reference's std::sort leaves their order
 * unspecified.  Returns the number of ordered expert pairs with exactly equal
 * logits (0 for the seeded inputs, checked by the tests), or -1 when top_k is
 * outside 1..256. */
int32_t jxo_select_experts(const float* logits, int32_t E, int32_t k, int32_t* ids, float* probs) {
    if (k > E) k = E;
    if (k < 1 || k > 256) return -1;
    int32_t ties = 0;
    for (int32_t e = 0; e < E; ++e) {
        int32_t rank = 0;
        for (int32_t f = 0; f < E; ++f) {
            if (logits[f] > logits[e] || (logits[f] == logits[e] && f < e)) rank++;
            if (f != e && logits[f] == logits[e]) ties++;
        }
        if (rank < k) ids[rank] = e;
    }
    float raw[256];
    for (int32_t i = 0; i < k; ++i) raw[i] = logits[ids[i]];
    float mx = raw[0];
    for (int32_t i = 1; i < k; ++i) mx = mx > raw[i] ? mx : raw[i];
    float sum = 0.0f;
    for (int32_t i = 0; i < k; ++i) {
        probs[i] = expf(raw[i] - mx);
        sum += probs[i];
    }
    const float inv = (sum > 0.0f) ? (1.0f / sum) : (1.0f / (float)k);
    for (int32_t i = 0; i < k; ++i) probs[i] *= inv;
    return ties;
}

/* Router GEMV (transformer.cpp:2589-2594 -> matmul_quant_f32(router type) -> vec_dot_f32 or the
 * F16 / BF16 dots), optional per-expert bias added after the GEMV, then top-k. */
void jxo_route(const jxo_moe_desc* L, const float* x, int32_t n_tok,
               float* logits, int32_t* topk_ids, float* topk_w) {
    const int32_t E = L->n_experts, d = L->d_model, k = L->top_k;
    for (int32_t t = 0; t < n_tok; ++t) {
        float* lg = logits + (int64_t)t * E;
        for (int32_t e = 0; e < E; ++e) {
            lg[e] = router_dot(L, e, x + (int64_t)t * d);
            if (L->router_bias) lg[e] = lg[e] + L->router_bias[e];
        }
        jxo_select_experts(lg, E, k, topk_ids + (int64_t)t * k, topk_w + (int64_t)t * k);
    }
}

/* MoETransformerEngine::rms_norm (src/transformer.cpp:67-73): ss in
 * vec_dot_f32's order, inv = 1 / sqrt(ss / size + eps), out = x * inv * w
 * (w NULL: weight 1); out may alias x. */
void jxo_rms_norm(float* out, const float* x, const float* weight, int64_t size, float eps) {
    const float ss = jxo_vec_dot_f32(x, x, size);
    const float inv = 1.0f / sqrtf((ss / (float)size) + eps);
    for (int64_t i = 0; i < size; ++i) out[i] = x[i] * inv * (weight ? weight[i] : 1.0f);
}

/* ------------------------------------------------------- MoE block -- */

/* One token through the MoE block (src/transformer.cpp:2589-2757, residual
 * excluded): routed experts in descending-logit order, accum += p * down
 * (contracted to an fma by the reference build), then the shared expert
 * (always SiLU-gated, 2741-2745) scaled by sigmoid(vec_dot_f32(gate_inp, x)) or 1. */
static void moe_token(const jxo_moe_desc* L, const float* x, float* out, int32_t* ids, float* probs,
                      float* logits, int32_t order, float* h, float* y) {
    const int32_t E = L->n_experts, d = L->d_model, Fd = L->d_ff, k = L->top_k;
    for (int32_t e = 0; e < E; ++e) {
        logits[e] = router_dot(L, e, x);
        if (L->router_bias) logits[e] = logits[e] + L->router_bias[e];
    }
    jxo_select_experts(logits, E, k, ids, probs);
    for (int32_t i = 0; i < d; ++i) out[i] = 0.0f;
    const int64_t gsl = (int64_t)Fd * jxo_row_bytes(L->gate_type, d);
    const int64_t usl = (int64_t)Fd * jxo_row_bytes(L->up_type, d);
    const int64_t dsl = (int64_t)d * jxo_row_bytes(L->down_type, Fd);
    for (int32_t s = 0; s < k; ++s) {
        const int64_t e = ids[s];
        jxo_matmul_swiglu_quant_f32(L->gate_type, L->gate + e * gsl, L->up_type, L->up + e * usl,
                                    x, h, Fd, d, L->activation, order);
        jxo_matmul_quant_f32(L->down_type, L->down + e * dsl, h, y, d, Fd, order);
        for (int32_t i = 0; i < d; ++i) out[i] = fmaf(probs[s], y[i], out[i]);
    }
    if (L->d_ff_shared > 0 && L->sh_gate && L->sh_up && L->sh_down) {
        const int32_t Fs = L->d_ff_shared;
        /* always SiLU: the shared expert's call (transformer.cpp:2741-2745) leaves use_gelu at its
         * default, false (quant.h:361), whatever the layer's activation */
        jxo_matmul_swiglu_quant_f32(L->sh_gate_type, L->sh_gate, L->sh_up_type, L->sh_up, x, h, Fs, d,
                                    0, order);
        jxo_matmul_quant_f32(L->sh_down_type, L->sh_down, h, y, d, Fs, order);
        float sh = 1.0f;
        if (L->sh_gate_inp) {
            const float g = jxo_vec_dot_f32(L->sh_gate_inp, x, d);
            sh = 1.0f / (1.0f + expf(-g));
        }
        for (int32_t i = 0; i < d; ++i) out[i] = fmaf(sh, y[i], out[i]);
    }
}

int32_t jxo_moe_forward(const jxo_moe_desc* L, const float* x, int32_t n_tok,
                        const int32_t* token_idx, int32_t n_sel,
                        float* out, int32_t* topk_ids, float* topk_w, float* logits, int32_t order) {
    const int32_t d = L->d_model, k = L->top_k, E = L->n_experts;
    int32_t fmax = L->d_ff > L->d_ff_shared ? L->d_ff : L->d_ff_shared;
    if (L->top_k > 256 || L->top_k < 1 || L->top_k > E) return -1;
    float* h = (float*)malloc(sizeof(float) * (size_t)fmax);
    float* y = (float*)malloc(sizeof(float) * (size_t)d);
    float* lg = (float*)malloc(sizeof(float) * (size_t)E);
    float* xn = (float*)malloc(sizeof(float) * (size_t)d);
    const int32_t cnt = token_idx ? n_sel : n_tok;
    for (int32_t i = 0; i < cnt; ++i) {
        const int32_t t = token_idx ? token_idx[i] : i;
        if (t < 0 || t >= n_tok) { free(h); free(y); free(lg); free(xn); return -2; }
        const float* xt = x + (int64_t)t * d;
        float* o = out + (int64_t)i * d;
        if (L->residual) /* the FFN step of forward_token (transformer.cpp:2585-2764) */
            jxo_rms_norm(xn, xt, L->ffn_norm, d, L->rms_eps);
        moe_token(L, L->residual ? xn : xt, o, topk_ids + (int64_t)i * k, topk_w + (int64_t)i * k, lg, order, h, y);
        if (L->residual) {
            if (L->post_ffw_norm) jxo_rms_norm(o, o, L->post_ffw_norm, d, L->rms_eps);
            for (int32_t j = 0; j < d; ++j) o[j] = xt[j] + o[j];
        }
        if (logits) memcpy(logits + (int64_t)i * E, lg, sizeof(float) * (size_t)E);
    }
    free(h);
    free(y);
    free(lg);
    free(xn);
    return 0;
}
