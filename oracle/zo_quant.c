/*
 * zo_quant.c -- CPU oracle: GGUF block decoders, row dots and elementwise math.
 *
 * TEST INFRASTRUCTURE ONLY (see zo.h).  Restates model/loader.zig and
 * model/quant_extra.zig of the reference; each function cites its source.
 * Built with -ffp-contract=off: every a*b+c below that is not written as
 * fmaf() is two rounded operations, as in the reference's strict float mode.
 */
#include "zo.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define SIMD 8 /* simd_lane_count, model/loader.zig:86 */

/* readF16AsF32 (model/loader.zig:4484-4488): exact binary16 -> binary32,
 * subnormals included. */
float zo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            float v = (float)mant * 0x1p-24f; /* exact: mant < 2^10 */
            return sign ? -v : v;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float rd_f16(const uint8_t *p) { return zo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static inline float rd_f32(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }

/* Sequential restatement of @reduce(.Add) over 8 lanes. */
static inline float reduce8(const float *v) {
    float s = v[0];
    for (int i = 1; i < SIMD; i++) s += v[i];
    return s;
}

/* tensorRowByteSize (model/loader.zig:3325-3389) for the types on the path. */
int zo_row_bytes(int type, size_t row_len, size_t *out) {
    switch (type) {
    case ZO_F32: *out = row_len * 4; return ZO_OK;
    case ZO_F16: *out = row_len * 2; return ZO_OK;
    case ZO_Q8_0: if (row_len % 32) return ZO_ERR_INVALID; *out = row_len / 32 * 34; return ZO_OK;
    case ZO_Q3_K: if (row_len % 256) return ZO_ERR_INVALID; *out = row_len / 256 * 110; return ZO_OK;
    case ZO_Q4_K: if (row_len % 256) return ZO_ERR_INVALID; *out = row_len / 256 * 144; return ZO_OK;
    case ZO_Q5_K: if (row_len % 256) return ZO_ERR_INVALID; *out = row_len / 256 * 176; return ZO_OK;
    case ZO_Q6_K: if (row_len % 256) return ZO_ERR_INVALID; *out = row_len / 256 * 210; return ZO_OK;
    case ZO_IQ4_XS: if (row_len % 256) return ZO_ERR_INVALID; *out = row_len / 256 * 136; return ZO_OK;
    default: return ZO_ERR_UNSUPPORTED;
    }
}

/* getScaleMinK4 (model/loader.zig:3814-3825). */
void zo_scale_min_k4(int j, const uint8_t *s, uint8_t *out) {
    if (j < 4) {
        out[0] = s[j] & 63;
        out[1] = s[j + 4] & 63;
    } else {
        out[0] = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        out[1] = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* ---------------- Q4_K ---------------- */

/* dequantizeRowQ4K (model/loader.zig:3647-3675). */
static void dequant_q4k(const uint8_t *row, size_t row_len, float *out) {
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 144;
        float d = rd_f16(blk), dmin = rd_f16(blk + 2);
        const uint8_t *sc = blk + 4, *q = blk + 16;
        float *o = out + b * 256;
        for (int g = 0; g < 4; g++) {
            uint8_t sm0[2], sm1[2];
            zo_scale_min_k4(2 * g, sc, sm0);
            zo_scale_min_k4(2 * g + 1, sc, sm1);
            float d1 = d * (float)sm0[0], m1 = dmin * (float)sm0[1];
            float d2 = d * (float)sm1[0], m2 = dmin * (float)sm1[1];
            for (int l = 0; l < 32; l++) o[64 * g + l] = d1 * (float)(q[l] & 0x0F) - m1;
            for (int l = 0; l < 32; l++) o[64 * g + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
            q += 32;
        }
    }
}

/* dotQ4KRow (model/loader.zig:3677-3726). */
static float dot_q4k(const uint8_t *row, size_t row_len, const float *x) {
    float sum = 0.0f;
    size_t off = 0;
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 144;
        float d = rd_f16(blk), dmin = rd_f16(blk + 2);
        const uint8_t *sc = blk + 4, *q = blk + 16;
        for (int g = 0; g < 4; g++) {
            uint8_t sm0[2], sm1[2];
            zo_scale_min_k4(2 * g, sc, sm0);
            zo_scale_min_k4(2 * g + 1, sc, sm1);
            float d1 = d * (float)sm0[0], m1 = dmin * (float)sm0[1];
            float d2 = d * (float)sm1[0], m2 = dmin * (float)sm1[1];
            float lqd = 0, lis = 0, hqd = 0, his = 0;
            for (int l = 0; l < 32; l += SIMD) {
                float pl[SIMD], ph[SIMD];
                const float *xl = x + off + l, *xh = x + off + 32 + l;
                for (int i = 0; i < SIMD; i++) {
                    pl[i] = (float)(q[l + i] & 0x0F) * xl[i];
                    ph[i] = (float)(q[l + i] >> 4) * xh[i];
                }
                lqd += reduce8(pl);
                lis += reduce8(xl);
                hqd += reduce8(ph);
                his += reduce8(xh);
            }
            sum = fmaf(d1, lqd, sum);
            sum = fmaf(-m1, lis, sum);
            sum = fmaf(d2, hqd, sum);
            sum = fmaf(-m2, his, sum);
            off += 64;
            q += 32;
        }
    }
    return sum;
}

/* ---------------- Q6_K ---------------- */

static inline int q6_value(const uint8_t *ql, const uint8_t *qh, int l, int which) {
    /* q1..q4 of dequantizeRowQ6K (model/loader.zig:3745-3748). */
    switch (which) {
    case 0: return ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
    case 1: return ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
    case 2: return ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
    default: return ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
    }
}

/* dequantizeRowQ6K (model/loader.zig:3728-3761). */
static void dequant_q6k(const uint8_t *row, size_t row_len, float *out) {
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 210;
        const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
        float d = rd_f16(blk + 208);
        float *o = out + b * 256;
        for (int half = 0; half < 2; half++) {
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                for (int w = 0; w < 4; w++) {
                    float s = d * (float)(int8_t)sc[is + 2 * w];
                    o[l + 32 * w] = s * (float)q6_value(ql, qh, l, w);
                }
            }
            o += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* dotQ6KRow (model/loader.zig:3763-3812). */
static float dot_q6k(const uint8_t *row, size_t row_len, const float *x) {
    float sum = 0.0f;
    size_t off = 0;
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 210;
        const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
        float d = rd_f16(blk + 208);
        for (int half = 0; half < 2; half++) {
            for (int g16 = 0; g16 < 2; g16++) {
                int l0 = g16 * 16;
                float s[4];
                for (int w = 0; w < 4; w++) s[w] = d * (float)(int8_t)sc[g16 + 2 * w];
                float qd[4] = {0, 0, 0, 0};
                for (int sub = 0; sub < 2; sub++) {
                    int base = l0 + sub * SIMD;
                    for (int w = 0; w < 4; w++) {
                        float p[SIMD];
                        for (int i = 0; i < SIMD; i++)
                            p[i] = (float)q6_value(ql, qh, base + i, w) * x[off + base + 32 * w + i];
                        qd[w] += reduce8(p);
                    }
                }
                for (int w = 0; w < 4; w++) sum = fmaf(s[w], qd[w], sum);
            }
            off += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
    return sum;
}

/* ---------------- Q8_0 ---------------- */

/* dequantizeRowQ8_0 (model/loader.zig:3589-3601). */
static void dequant_q8_0(const uint8_t *row, size_t row_len, float *out) {
    for (size_t b = 0; b < row_len / 32; b++) {
        const uint8_t *blk = row + b * 34;
        float d = rd_f16(blk);
        for (int i = 0; i < 32; i++) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
    }
}

/* dotQ8_0Row (model/loader.zig:3603-3617). */
static float dot_q8_0(const uint8_t *row, size_t row_len, const float *x) {
    float sum = 0.0f;
    for (size_t b = 0; b < row_len / 32; b++) {
        const uint8_t *blk = row + b * 34;
        float d = rd_f16(blk);
        for (int i = 0; i < 32; i++) sum = fmaf(d * (float)(int8_t)blk[2 + i], x[b * 32 + i], sum);
    }
    return sum;
}

/* ---------------- Q3_K ---------------- */

/* expandQ3KScales (model/quant_extra.zig:248-279). */
static void expand_q3k_scales(const uint8_t *raw, int32_t *out) {
    uint32_t aux[4];
    memcpy(&aux[0], raw, 4);
    memcpy(&aux[1], raw + 4, 4);
    memcpy(&aux[2], raw + 8, 4);
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
    for (int w = 0; w < 4; w++)
        for (int lane = 0; lane < 4; lane++) out[w * 4 + lane] = (int32_t)((aux[w] >> (8 * lane)) & 0xFF) - 32;
}

/* decodeQ3Value (model/quant_extra.zig:281-284). */
static inline int32_t q3_value(uint8_t q, int shift, uint8_t hm, uint8_t mask) {
    return (int32_t)((q >> shift) & 3) - ((hm & mask) ? 0 : 4);
}

/* dequantizeRowQ3K (model/quant_extra.zig:45-84). */
static void dequant_q3k(const uint8_t *row, size_t row_len, float *out) {
    size_t o = 0;
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 110;
        const uint8_t *hm = blk, *qs = blk + 32;
        int32_t sc[16];
        expand_q3k_scales(blk + 96, sc);
        float d_all = rd_f16(blk + 108);
        int qo = 0, si = 0;
        uint8_t mask = 1;
        for (int h = 0; h < 2; h++) {
            int shift = 0;
            for (int j = 0; j < 4; j++) {
                float dl0 = d_all * (float)sc[si++];
                for (int l = 0; l < 16; l++) out[o++] = dl0 * (float)q3_value(qs[qo + l], shift, hm[l], mask);
                float dl1 = d_all * (float)sc[si++];
                for (int l = 0; l < 16; l++) out[o++] = dl1 * (float)q3_value(qs[qo + 16 + l], shift, hm[16 + l], mask);
                shift += 2;
                mask = (uint8_t)(mask << 1);
            }
            qo += 32;
        }
    }
}

/* dotQ3KRow (model/quant_extra.zig:86-126). */
static float dot_q3k(const uint8_t *row, size_t row_len, const float *x) {
    float sum = 0.0f;
    size_t xi = 0;
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 110;
        const uint8_t *hm = blk, *qs = blk + 32;
        int32_t sc[16];
        expand_q3k_scales(blk + 96, sc);
        float d_all = rd_f16(blk + 108);
        int qo = 0, si = 0;
        uint8_t mask = 1;
        for (int h = 0; h < 2; h++) {
            int shift = 0;
            for (int j = 0; j < 4; j++) {
                float s0 = d_all * (float)sc[si++];
                for (int l = 0; l < 16; l++)
                    sum = fmaf(s0 * (float)q3_value(qs[qo + l], shift, hm[l], mask), x[xi++], sum);
                float s1 = d_all * (float)sc[si++];
                for (int l = 0; l < 16; l++)
                    sum = fmaf(s1 * (float)q3_value(qs[qo + 16 + l], shift, hm[16 + l], mask), x[xi++], sum);
                shift += 2;
                mask = (uint8_t)(mask << 1);
            }
            qo += 32;
        }
    }
    return sum;
}

/* ---------------- IQ4_XS ---------------- */

/* kvalues_iq4nl (model/quant_extra.zig:8). */
static const int8_t kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

static inline float iq4xs_dl(const uint8_t *blk, int ib) {
    /* model/quant_extra.zig:205-207 */
    float d = rd_f16(blk);
    uint16_t sh = (uint16_t)(blk[2] | (blk[3] << 8));
    int low = (blk[4 + ib / 2] >> (4 * (ib % 2))) & 0x0f;
    int high = (sh >> (2 * ib)) & 0x03;
    return d * (float)((low | (high << 4)) - 32);
}

/* dequantizeRowIQ4XS (model/quant_extra.zig:191-215). */
static void dequant_iq4xs(const uint8_t *row, size_t row_len, float *out) {
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 136;
        const uint8_t *qs = blk + 8;
        for (int ib = 0; ib < 8; ib++) {
            float dl = iq4xs_dl(blk, ib);
            float *o = out + b * 256 + ib * 32;
            for (int j = 0; j < 16; j++) {
                o[j] = dl * (float)kvalues_iq4nl[qs[j] & 0x0f];
                o[j + 16] = dl * (float)kvalues_iq4nl[qs[j] >> 4];
            }
            qs += 16;
        }
    }
}

/* dotIQ4XSRow (model/quant_extra.zig:217-246). */
static float dot_iq4xs(const uint8_t *row, size_t row_len, const float *x) {
    float sum = 0.0f;
    size_t xi = 0;
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 136;
        const uint8_t *qs = blk + 8;
        for (int ib = 0; ib < 8; ib++) {
            float dl = iq4xs_dl(blk, ib);
            for (int j = 0; j < 16; j++) sum = fmaf(dl * (float)kvalues_iq4nl[qs[j] & 0x0f], x[xi++], sum);
            for (int j = 0; j < 16; j++) sum = fmaf(dl * (float)kvalues_iq4nl[qs[j] >> 4], x[xi++], sum);
            qs += 16;
        }
    }
    return sum;
}

/* ---------------- Q5_K (known-answer pin only) ---------------- */

/* dequantizeRowQ5K (model/loader.zig:3461-3497). */
static void dequant_q5k(const uint8_t *row, size_t row_len, float *out) {
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 176;
        float d = rd_f16(blk), dmin = rd_f16(blk + 2);
        const uint8_t *sc = blk + 4, *qh = blk + 16, *qs = blk + 48;
        float *o = out + b * 256;
        uint8_t lo = 1, hi = 2;
        for (int g = 0; g < 4; g++) {
            uint8_t sm0[2], sm1[2];
            zo_scale_min_k4(2 * g, sc, sm0);
            zo_scale_min_k4(2 * g + 1, sc, sm1);
            float d1 = d * (float)sm0[0], m1 = dmin * (float)sm0[1];
            float d2 = d * (float)sm1[0], m2 = dmin * (float)sm1[1];
            for (int l = 0; l < 32; l++) {
                uint32_t q0 = (uint32_t)(qs[l] & 0x0F) + ((qh[l] & lo) ? 16u : 0u);
                uint32_t q1 = (uint32_t)(qs[l] >> 4) + ((qh[l] & hi) ? 16u : 0u);
                o[64 * g + l] = d1 * (float)q0 - m1;
                o[64 * g + 32 + l] = d2 * (float)q1 - m2;
            }
            qs += 32;
            lo = (uint8_t)(lo << 2);
            hi = (uint8_t)(hi << 2);
        }
    }
}

/* dotQ5KRow (model/loader.zig:3515-3567). */
static float dot_q5k(const uint8_t *row, size_t row_len, const float *x) {
    float sum = 0.0f;
    size_t off = 0;
    for (size_t b = 0; b < row_len / 256; b++) {
        const uint8_t *blk = row + b * 176;
        float d = rd_f16(blk), dmin = rd_f16(blk + 2);
        const uint8_t *sc = blk + 4, *qh = blk + 16, *qs = blk + 48;
        uint8_t lo = 1, hi = 2;
        for (int g = 0; g < 4; g++) {
            uint8_t sm0[2], sm1[2];
            zo_scale_min_k4(2 * g, sc, sm0);
            zo_scale_min_k4(2 * g + 1, sc, sm1);
            float d1 = d * (float)sm0[0], m1 = dmin * (float)sm0[1];
            float d2 = d * (float)sm1[0], m2 = dmin * (float)sm1[1];
            float lqd = 0, lis = 0, hqd = 0, his = 0;
            for (int l = 0; l < 32; l++) {
                uint32_t q0 = (uint32_t)(qs[l] & 0x0F) + ((qh[l] & lo) ? 16u : 0u);
                uint32_t q1 = (uint32_t)(qs[l] >> 4) + ((qh[l] & hi) ? 16u : 0u);
                lqd = fmaf((float)q0, x[off + l], lqd);
                lis += x[off + l];
                hqd = fmaf((float)q1, x[off + 32 + l], hqd);
                his += x[off + 32 + l];
            }
            sum = fmaf(d1, lqd, sum);
            sum = fmaf(-m1, lis, sum);
            sum = fmaf(d2, hqd, sum);
            sum = fmaf(-m2, his, sum);
            off += 64;
            qs += 32;
            lo = (uint8_t)(lo << 2);
            hi = (uint8_t)(hi << 2);
        }
    }
    return sum;
}

/* ---------------- dense rows ---------------- */

/* dotF32Row / dotF16Row (model/loader.zig:3619-3645). */
static float dot_dense(int type, const uint8_t *row, size_t n, const float *x) {
    float acc[SIMD] = {0};
    size_t i = 0;
    for (; i + SIMD <= n; i += SIMD)
        for (int j = 0; j < SIMD; j++) {
            float w = type == ZO_F32 ? rd_f32(row + 4 * (i + j)) : rd_f16(row + 2 * (i + j));
            acc[j] = acc[j] + w * x[i + j];
        }
    float sum = reduce8(acc);
    for (; i < n; i++) {
        float w = type == ZO_F32 ? rd_f32(row + 4 * i) : rd_f16(row + 2 * i);
        sum = fmaf(w, x[i], sum);
    }
    return sum;
}

int zo_dequantize_row(int type, const uint8_t *row, size_t row_len, float *out) {
    size_t bytes;
    int st = zo_row_bytes(type, row_len, &bytes);
    if (st) return st;
    switch (type) {
    case ZO_F32: for (size_t i = 0; i < row_len; i++) out[i] = rd_f32(row + 4 * i); break;
    case ZO_F16: for (size_t i = 0; i < row_len; i++) out[i] = rd_f16(row + 2 * i); break;
    case ZO_Q8_0: dequant_q8_0(row, row_len, out); break;
    case ZO_Q3_K: dequant_q3k(row, row_len, out); break;
    case ZO_Q4_K: dequant_q4k(row, row_len, out); break;
    case ZO_Q5_K: dequant_q5k(row, row_len, out); break;
    case ZO_Q6_K: dequant_q6k(row, row_len, out); break;
    case ZO_IQ4_XS: dequant_iq4xs(row, row_len, out); break;
    default: return ZO_ERR_UNSUPPORTED;
    }
    return ZO_OK;
}

static float dot_row_valid(int type, const uint8_t *row, size_t row_len, const float *x) {
    switch (type) {
    case ZO_F32:
    case ZO_F16: return dot_dense(type, row, row_len, x);
    case ZO_Q8_0: return dot_q8_0(row, row_len, x);
    case ZO_Q3_K: return dot_q3k(row, row_len, x);
    case ZO_Q4_K: return dot_q4k(row, row_len, x);
    case ZO_Q5_K: return dot_q5k(row, row_len, x);
    case ZO_Q6_K: return dot_q6k(row, row_len, x);
    case ZO_IQ4_XS: return dot_iq4xs(row, row_len, x);
    default: return 0.0f;
    }
}

int zo_dot_row(int type, const uint8_t *row, size_t row_len, const float *x, float *out) {
    size_t bytes;
    int st = zo_row_bytes(type, row_len, &bytes);
    if (st) return st;
    *out = dot_row_valid(type, row, row_len, x);
    return ZO_OK;
}

/* ---------------- elementwise ---------------- */

/* dotSimd (model/loader.zig:4133-4145). */
float zo_dot_simd(const float *a, const float *b, size_t n) {
    float acc[SIMD] = {0};
    size_t i = 0;
    for (; i + SIMD <= n; i += SIMD)
        for (int j = 0; j < SIMD; j++) acc[j] = acc[j] + a[i + j] * b[i + j];
    float sum = reduce8(acc);
    for (; i < n; i++) sum = fmaf(a[i], b[i], sum);
    return sum;
}

/* rmsNorm (model/loader.zig:3404-3426). */
void zo_rms_norm(float *out, const float *x, const float *w, size_t n, float eps, float off) {
    float ms = zo_dot_simd(x, x, n);
    ms /= (float)n;
    float scale = 1.0f / sqrtf(ms + eps);
    for (size_t i = 0; i < n; i++) out[i] = scale * x[i] * (w[i] + off);
}

/* rmsNormPerHeadWithOffset (model/loader.zig:1777-1812). */
void zo_rms_norm_per_head(float *out, const float *x, const float *w, size_t hc, size_t hd, float eps, float off) {
    for (size_t h = 0; h < hc; h++) {
        const float *hi = x + h * hd;
        float *ho = out + h * hd;
        float ms = 0.0f;
        for (size_t i = 0; i < hd; i++) ms += hi[i] * hi[i];
        ms /= (float)hd;
        float scale = 1.0f / sqrtf(ms + eps);
        for (size_t i = 0; i < hd; i++) ho[i] = scale * hi[i] * (w[i] + off);
    }
}

/* applyRoPE / applyInterleavedRoPE / applyNeoxRoPE (model/loader.zig:3827-3866).
 * style 0 = interleaved pairs (2i, 2i+1), 1 = NeoX halves (i, i+n/2). */
void zo_apply_rope(float *v, size_t hc, size_t hd, size_t rope_dim, size_t pos, float base, int style) {
    size_t n_rot = rope_dim < hd ? rope_dim : hd;
    float p = (float)pos;
    for (size_t h = 0; h < hc; h++) {
        float *head = v + h * hd;
        if (style == 0) {
            for (size_t pair = 0; pair + 1 < n_rot; pair += 2) {
                float e = (float)pair / (float)n_rot;
                float theta = p / powf(base, e);
                float c = cosf(theta), s = sinf(theta);
                float x0 = head[pair], x1 = head[pair + 1];
                head[pair] = fmaf(x0, c, -x1 * s);
                head[pair + 1] = fmaf(x0, s, x1 * c);
            }
        } else {
            size_t half = n_rot / 2;
            for (size_t i = 0; i < half; i++) {
                float e = (float)(i * 2) / (float)n_rot;
                float theta = p / powf(base, e);
                float c = cosf(theta), s = sinf(theta);
                float x0 = head[i], x1 = head[i + half];
                head[i] = fmaf(x0, c, -x1 * s);
                head[i + half] = fmaf(x0, s, x1 * c);
            }
        }
    }
}

/* softmaxInPlace (model/loader.zig:4160-4170). */
void zo_softmax(float *v, size_t n) {
    float mx = v[0];
    for (size_t i = 1; i < n; i++) mx = fmaxf(mx, v[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    for (size_t i = 0; i < n; i++) v[i] /= sum;
}

/* argmax (model/loader.zig:3910-3920; sampling.zig:196-206): first maximum wins. */
uint32_t zo_argmax(const float *v, size_t n) {
    size_t best = 0;
    float bv = v[0];
    for (size_t i = 1; i < n; i++)
        if (v[i] > bv) {
            bv = v[i];
            best = i;
        }
    return (uint32_t)best;
}

/* siluInPlace / siluScalar (model/loader.zig:4004-4024). */
void zo_silu_in_place(float *v, size_t n) {
    for (size_t i = 0; i < n; i++) v[i] = v[i] / (1.0f + expf(-v[i]));
}

/* sigmoidScalar (model/loader.zig:4026-4033). */
float zo_sigmoid(float x) {
    if (x >= 0) return 1.0f / (1.0f + expf(-x));
    float e = expf(x);
    return e / (1.0f + e);
}

/* selectTopK (model/loader.zig:3953-3975): insertion by strict '>' so the lower
 * index wins ties. */
void zo_select_topk(const float *probs, size_t n, uint32_t *idx, float *w, size_t k) {
    for (size_t i = 0; i < k; i++) {
        idx[i] = 0;
        w[i] = -INFINITY;
    }
    for (size_t i = 0; i < n; i++) {
        size_t at = k;
        for (size_t s = 0; s < k; s++)
            if (probs[i] > w[s]) {
                at = s;
                break;
            }
        if (at == k) continue;
        for (size_t s = k - 1; s > at; s--) {
            w[s] = w[s - 1];
            idx[s] = idx[s - 1];
        }
        w[at] = probs[i];
        idx[at] = (uint32_t)i;
    }
}

/* normalizePositiveWeights (model/loader.zig:3977-3990). */
void zo_normalize_positive(float *w, size_t k) {
    float sum = 0.0f;
    for (size_t i = 0; i < k; i++)
        if (isfinite(w[i]) && w[i] > 0) sum += w[i];
    if (sum <= 0) {
        for (size_t i = 0; i < k; i++) w[i] = 0;
        return;
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < k; i++) w[i] = (isfinite(w[i]) && w[i] > 0) ? w[i] * inv : 0.0f;
}

/* computeAttention (model/loader.zig:1397-1438), one layer. */
void zo_attention(float *out, const float *q, const float *kc, const float *vc, size_t hc, size_t hkv,
                  size_t hd, size_t kv_dim, size_t pos, size_t ws, float *scores) {
    memset(out, 0, hc * hd * sizeof(float));
    size_t group = hc / hkv;
    float scale = 1.0f / sqrtf((float)hd);
    size_t count = pos - ws + 1;
    for (size_t h = 0; h < hc; h++) {
        const float *qh = q + h * hd;
        size_t kvo = (h / group) * hd;
        for (size_t t = ws; t <= pos; t++) scores[t - ws] = zo_dot_simd(qh, kc + t * kv_dim + kvo, hd) * scale;
        zo_softmax(scores, count);
        float *oh = out + h * hd;
        for (size_t t = ws; t <= pos; t++) {
            float w = scores[t - ws];
            const float *vh = vc + t * kv_dim + kvo;
            for (size_t i = 0; i < hd; i++) oh[i] = fmaf(w, vh[i], oh[i]);
        }
    }
}

/* ---------------- row-parallel matvec (MatVecWorkers) ---------------- */

/* workerRowRange (model/loader.zig:2011-2016). */
static void row_range(size_t wi, size_t parts, size_t rows, size_t *s, size_t *e) {
    size_t per = (rows + parts - 1) / parts;
    *s = wi * per < rows ? wi * per : rows;
    *e = *s + per < rows ? *s + per : rows;
}

typedef struct {
    int type;
    const uint8_t *bytes;
    size_t row_size, row_len, rows;
    const float *x;
    float *y;
    size_t worker, parts;
} mv_task;

static void *mv_run(void *arg) {
    mv_task *t = (mv_task *)arg;
    size_t s, e;
    row_range(t->worker, t->parts, t->rows, &s, &e);
    for (size_t r = s; r < e; r++) t->y[r] = dot_row_valid(t->type, t->bytes + r * t->row_size, t->row_len, t->x);
    return NULL;
}

/* Persistent helper pool restating MatVecWorkers (model/loader.zig:1943-2052):
 * helpers wait on a generation counter; the caller takes the last row range. */
typedef struct {
    pthread_mutex_t mu;
    pthread_cond_t ready, done;
    pthread_t *threads;
    size_t n;
    mv_task task;
    uint64_t gen;
    size_t active;
    int stop;
} mv_pool;

typedef struct {
    mv_pool *pool;
    size_t index;
} mv_arg;

static void *pool_main(void *arg) {
    mv_arg *a = (mv_arg *)arg;
    mv_pool *p = a->pool;
    uint64_t seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        while (!p->stop && seen == p->gen) pthread_cond_wait(&p->ready, &p->mu);
        if (p->stop) {
            pthread_mutex_unlock(&p->mu);
            free(a);
            return NULL;
        }
        seen = p->gen;
        mv_task t = p->task;
        pthread_mutex_unlock(&p->mu);
        t.worker = a->index;
        t.parts = p->n + 1;
        mv_run(&t);
        pthread_mutex_lock(&p->mu);
        if (--p->active == 0) pthread_cond_signal(&p->done);
        pthread_mutex_unlock(&p->mu);
    }
}

static mv_pool *g_pool = NULL;
static size_t g_pool_helpers = 0;
static pthread_mutex_t g_pool_mu = PTHREAD_MUTEX_INITIALIZER;

static mv_pool *pool_get(size_t helpers) {
    pthread_mutex_lock(&g_pool_mu);
    if (g_pool && g_pool_helpers != helpers) {
        mv_pool *p = g_pool;
        pthread_mutex_lock(&p->mu);
        p->stop = 1;
        pthread_cond_broadcast(&p->ready);
        pthread_mutex_unlock(&p->mu);
        for (size_t i = 0; i < p->n; i++) pthread_join(p->threads[i], NULL);
        free(p->threads);
        free(p);
        g_pool = NULL;
    }
    if (!g_pool && helpers > 0) {
        mv_pool *p = (mv_pool *)calloc(1, sizeof(mv_pool));
        pthread_mutex_init(&p->mu, NULL);
        pthread_cond_init(&p->ready, NULL);
        pthread_cond_init(&p->done, NULL);
        p->threads = (pthread_t *)calloc(helpers, sizeof(pthread_t));
        p->n = helpers;
        for (size_t i = 0; i < helpers; i++) {
            mv_arg *a = (mv_arg *)malloc(sizeof(mv_arg));
            a->pool = p;
            a->index = i;
            pthread_create(&p->threads[i], NULL, pool_main, a);
        }
        g_pool = p;
        g_pool_helpers = helpers;
    }
    mv_pool *r = g_pool;
    pthread_mutex_unlock(&g_pool_mu);
    return r;
}

/* Session.init's helper count (model/loader.zig:974-978). */
static size_t default_helpers(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    size_t h = (size_t)(n - 1);
    return h < 11 ? h : 11;
}

int zo_matvec(int type, const uint8_t *bytes, size_t rows, size_t cols, const float *x, float *y, int threads) {
    size_t row_size;
    int st = zo_row_bytes(type, cols, &row_size);
    if (st) return st;
    size_t helpers = threads <= 0 ? default_helpers() : (size_t)(threads - 1);
    mv_task t = {type, bytes, row_size, cols, rows, x, y, 0, 1};
    /* parallel_matvec_min_rows / parallel_matvec_min_work (model/loader.zig:87-88) */
    if (helpers > 0 && rows >= 2048 && rows * cols >= 4000000) {
        mv_pool *p = pool_get(helpers);
        pthread_mutex_lock(&p->mu);
        p->task = t;
        p->active = p->n;
        p->gen++;
        pthread_cond_broadcast(&p->ready);
        pthread_mutex_unlock(&p->mu);
        t.worker = p->n;
        t.parts = p->n + 1;
        mv_run(&t);
        pthread_mutex_lock(&p->mu);
        while (p->active != 0) pthread_cond_wait(&p->done, &p->mu);
        pthread_mutex_unlock(&p->mu);
        return ZO_OK;
    }
    mv_run(&t);
    return ZO_OK;
}
