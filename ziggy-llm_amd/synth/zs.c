/*
 * zs.c -- synthetic GGUF weights: seeded N(mean, std) rows and this build's own
 * quantizers for Q4_K, Q6_K, Q8_0, Q3_K, IQ4_XS, F16 and F32.
 *
 * The reference ships no f32 -> K-quant quantizer (runtime/llama_fixture.zig
 * only encodes exact 0/1 values and zero blocks), so these quantizers are this
 * build's own: simple one-pass min/max scaling, written from the block layouts
 * that the reference's decoders define (model/loader.zig:3589-3825,
 * model/quant_extra.zig:45-246).  What the parity tests pin is DECODE: the
 * bytes emitted here are decoded bit-exactly by both the CPU oracle and the HIP
 * kernels.  The quantizers are checked for round-trip error only.
 *
 * Rows are generated independently (per-row seeded xoshiro256** + Box-Muller),
 * so the fill is deterministic for any thread count.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { ZS_F32 = 0, ZS_F16 = 1, ZS_Q8_0 = 8, ZS_Q3_K = 11, ZS_Q4_K = 12, ZS_Q6_K = 14, ZS_IQ4_XS = 23 };

/* ---------------- binary16 ---------------- */

static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float a;
        memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint16_t)nearbyintf(a * 0x1p24f));
    }
    uint32_t mant = ax & 0x7fffffu, exp = (ax >> 23) - 112u;
    uint32_t hm = mant >> 13, rem = mant & 0x1fffu, hv = (exp << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) hv++;
    return (uint16_t)(sign | hv);
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, bits;
    if (exp == 0) {
        float v = (float)mant * 0x1p-24f;
        return sign ? -v : v;
    }
    if (exp == 31) bits = sign | 0x7f800000u | (mant << 13);
    else bits = sign | ((exp + 112u) << 23) | (mant << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* ---------------- quantizers (one block each) ---------------- */

static void quant_q8_0(const float *x, uint8_t *b) {
    float amax = 0;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    uint16_t dh = f32_to_f16(amax / 127.0f);
    float d = f16_to_f32(dh), id = d != 0 ? 1.0f / d : 0.0f;
    put16(b, dh);
    for (int i = 0; i < 32; i++) b[2 + i] = (uint8_t)(int8_t)clampi((int)lrintf(x[i] * id), -127, 127);
}

static void quant_q4_k(const float *x, uint8_t *b) {
    float scale[8], minv[8], maxs = 0, maxm = 0;
    for (int j = 0; j < 8; j++) {
        float mn = 0, mx = x[32 * j];
        for (int i = 0; i < 32; i++) {
            mn = fminf(mn, x[32 * j + i]);
            mx = fmaxf(mx, x[32 * j + i]);
        }
        scale[j] = (mx - mn) / 15.0f;
        minv[j] = -mn;
        maxs = fmaxf(maxs, scale[j]);
        maxm = fmaxf(maxm, minv[j]);
    }
    uint16_t dh = f32_to_f16(maxs / 63.0f), mh = f32_to_f16(maxm / 63.0f);
    float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
    int sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0 ? clampi((int)lrintf(scale[j] / d), 0, 63) : 0;
        m[j] = dmin > 0 ? clampi((int)lrintf(minv[j] / dmin), 0, 63) : 0;
    }
    memset(b, 0, 144);
    put16(b, dh);
    put16(b + 2, mh);
    uint8_t *s = b + 4;
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t *qs = b + 16;
    for (int j = 0; j < 8; j++) {
        float ds = d * (float)sc[j], mm = dmin * (float)m[j];
        for (int i = 0; i < 32; i++) {
            int q = ds > 0 ? clampi((int)lrintf((x[32 * j + i] + mm) / ds), 0, 15) : 0;
            int g = j / 2;
            if (j % 2 == 0) qs[32 * g + i] |= (uint8_t)q;
            else qs[32 * g + i] |= (uint8_t)(q << 4);
        }
    }
}

static void quant_q6_k(const float *x, uint8_t *b) {
    float scale[16], maxs = 0;
    for (int g = 0; g < 16; g++) {
        float amax = 0;
        for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(x[16 * g + i]));
        scale[g] = amax / 31.0f;
        maxs = fmaxf(maxs, scale[g]);
    }
    uint16_t dh = f32_to_f16(maxs / 127.0f);
    float d = f16_to_f32(dh);
    memset(b, 0, 210);
    uint8_t *ql = b, *qh = b + 128, *sc = b + 192;
    int sci[16];
    for (int g = 0; g < 16; g++) {
        sci[g] = d > 0 ? clampi((int)lrintf(scale[g] / d), -128, 127) : 0;
        sc[g] = (uint8_t)(int8_t)sci[g];
    }
    for (int v = 0; v < 256; v++) {
        float ds = d * (float)sci[v / 16];
        int q = ds != 0 ? clampi((int)lrintf(x[v] / ds), -32, 31) : 0;
        int u = q + 32, h = v / 128, r = v % 128, w = r / 32, l = r % 32;
        uint8_t lo = (uint8_t)(u & 0xF), hi = (uint8_t)((u >> 4) & 3);
        int qli = 64 * h + l + ((w & 1) ? 32 : 0);
        if (w < 2) ql[qli] |= lo;
        else ql[qli] |= (uint8_t)(lo << 4);
        qh[32 * h + l] |= (uint8_t)(hi << (2 * w));
    }
    put16(b + 208, dh);
}

static void quant_q3_k(const float *x, uint8_t *b) {
    float scale[16], maxs = 0;
    for (int g = 0; g < 16; g++) {
        float am = 0, xm = 0;
        for (int i = 0; i < 16; i++)
            if (fabsf(x[16 * g + i]) > am) {
                am = fabsf(x[16 * g + i]);
                xm = x[16 * g + i];
            }
        scale[g] = -xm / 4.0f; /* the largest magnitude maps to q = -4 */
        maxs = fmaxf(maxs, fabsf(scale[g]));
    }
    uint16_t dh = f32_to_f16(maxs / 31.0f);
    float d = f16_to_f32(dh);
    int sv[16];
    memset(b, 0, 110);
    uint8_t *hm = b, *qs = b + 32, *raw = b + 96;
    for (int g = 0; g < 16; g++) sv[g] = (d > 0 ? clampi((int)lrintf(scale[g] / d), -32, 31) : 0) + 32;
    for (int v = 0; v < 256; v++) {
        float ds = d * (float)(sv[v / 16] - 32);
        int q = ds != 0 ? clampi((int)lrintf(x[v] / ds), -4, 3) : 0;
        int u = q + 4, h = v / 128, r = v % 128, j = r / 32, s = (r % 32) / 16, l = r % 16;
        qs[32 * h + 16 * s + l] |= (uint8_t)((u & 3) << (2 * j));
        if (u >> 2) hm[16 * s + l] |= (uint8_t)(1u << (4 * h + j));
    }
    for (int k = 0; k < 4; k++) {
        raw[k] = (uint8_t)((sv[k] & 0xF) | ((sv[8 + k] & 0xF) << 4));
        raw[4 + k] = (uint8_t)((sv[4 + k] & 0xF) | ((sv[12 + k] & 0xF) << 4));
        raw[8 + k] = (uint8_t)((sv[k] >> 4) | ((sv[4 + k] >> 4) << 2) | ((sv[8 + k] >> 4) << 4) | ((sv[12 + k] >> 4) << 6));
    }
    put16(b + 108, dh);
}

static const int8_t kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

static void quant_iq4_xs(const float *x, uint8_t *b) {
    float dl[8], maxd = 0;
    for (int ib = 0; ib < 8; ib++) {
        float am = 0, xm = 0;
        for (int i = 0; i < 32; i++)
            if (fabsf(x[32 * ib + i]) > am) {
                am = fabsf(x[32 * ib + i]);
                xm = x[32 * ib + i];
            }
        dl[ib] = -xm / 127.0f; /* the largest magnitude maps to kvalues[0] = -127 */
        maxd = fmaxf(maxd, fabsf(dl[ib]));
    }
    uint16_t dh = f32_to_f16(maxd / 32.0f);
    float d = f16_to_f32(dh);
    memset(b, 0, 136);
    put16(b, dh);
    uint16_t sh = 0;
    uint8_t *qs = b + 8;
    for (int ib = 0; ib < 8; ib++) {
        int ls = (d > 0 ? clampi((int)lrintf(dl[ib] / d), -32, 31) : 0) + 32;
        b[4 + ib / 2] |= (uint8_t)((ls & 0xF) << (4 * (ib % 2)));
        sh |= (uint16_t)(((ls >> 4) & 3) << (2 * ib));
        float dq = d * (float)(ls - 32);
        for (int i = 0; i < 32; i++) {
            int best = 0;
            float be = INFINITY;
            for (int k = 0; k < 16; k++) {
                float e = fabsf(x[32 * ib + i] - dq * (float)kvalues_iq4nl[k]);
                if (e < be) {
                    be = e;
                    best = k;
                }
            }
            if (i < 16) qs[16 * ib + i] |= (uint8_t)best;
            else qs[16 * ib + i - 16] |= (uint8_t)(best << 4);
        }
    }
    put16(b + 2, sh);
}

static int block_geom(int type, int *values, int *bytes) {
    switch (type) {
    case ZS_F32: *values = 1; *bytes = 4; return 0;
    case ZS_F16: *values = 1; *bytes = 2; return 0;
    case ZS_Q8_0: *values = 32; *bytes = 34; return 0;
    case ZS_Q3_K: *values = 256; *bytes = 110; return 0;
    case ZS_Q4_K: *values = 256; *bytes = 144; return 0;
    case ZS_Q6_K: *values = 256; *bytes = 210; return 0;
    case ZS_IQ4_XS: *values = 256; *bytes = 136; return 0;
    default: return -1;
    }
}

/* Quantizes one row of `cols` values into `dst` (cols must be a block multiple). */
int zs_quantize_row(int type, const float *x, uint64_t cols, uint8_t *dst) {
    int nv, nb;
    if (block_geom(type, &nv, &nb) || cols % (uint64_t)nv) return -1;
    for (uint64_t i = 0; i < cols / (uint64_t)nv; i++) {
        const float *xb = x + i * (uint64_t)nv;
        uint8_t *bb = dst + i * (uint64_t)nb;
        switch (type) {
        case ZS_F32: memcpy(bb, xb, 4); break;
        case ZS_F16: put16(bb, f32_to_f16(*xb)); break;
        case ZS_Q8_0: quant_q8_0(xb, bb); break;
        case ZS_Q3_K: quant_q3_k(xb, bb); break;
        case ZS_Q4_K: quant_q4_k(xb, bb); break;
        case ZS_Q6_K: quant_q6_k(xb, bb); break;
        case ZS_IQ4_XS: quant_iq4_xs(xb, bb); break;
        }
    }
    return 0;
}

int zs_row_bytes(int type, uint64_t cols, uint64_t *out) {
    int nv, nb;
    if (block_geom(type, &nv, &nb) || cols % (uint64_t)nv) return -1;
    *out = cols / (uint64_t)nv * (uint64_t)nb;
    return 0;
}

/* ---------------- seeded normal rows ---------------- */

static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
typedef struct {
    uint64_t s[4];
} xoshiro;
static inline uint64_t xo_next(xoshiro *r) {
    uint64_t *s = r->s, result = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return result;
}

/* Fills x[0..n) with N(mean, std) values for row `row` of a tensor seeded `seed`. */
void zs_normal_row(uint64_t seed, uint64_t row, float mean, float std, float *x, uint64_t n) {
    uint64_t sm = seed ^ (row * 0xD1B54A32D192ED03ull);
    xoshiro r;
    for (int i = 0; i < 4; i++) r.s[i] = splitmix64(&sm);
    for (uint64_t i = 0; i < n; i += 2) {
        double u1 = ((double)(xo_next(&r) >> 11) + 0.5) * 0x1p-53;
        double u2 = (double)(xo_next(&r) >> 11) * 0x1p-53;
        float rad = sqrtf(-2.0f * logf((float)u1)), th = (float)(6.283185307179586 * u2);
        x[i] = mean + std * rad * cosf(th);
        if (i + 1 < n) x[i + 1] = mean + std * rad * sinf(th);
    }
}

typedef struct {
    uint8_t *dst;
    int type;
    uint64_t rows, cols, seed, row_bytes;
    float mean, std;
    int worker, workers, status;
} fill_job;

static void *fill_main(void *arg) {
    fill_job *j = (fill_job *)arg;
    float *x = (float *)malloc((size_t)j->cols * sizeof(float));
    if (!x) {
        j->status = -2;
        return NULL;
    }
    uint64_t per = (j->rows + (uint64_t)j->workers - 1) / (uint64_t)j->workers;
    uint64_t r0 = (uint64_t)j->worker * per, r1 = r0 + per < j->rows ? r0 + per : j->rows;
    for (uint64_t r = r0; r < r1; r++) {
        if (j->std == 0.0f)
            for (uint64_t i = 0; i < j->cols; i++) x[i] = j->mean;
        else
            zs_normal_row(j->seed, r, j->mean, j->std, x, j->cols);
        if (zs_quantize_row(j->type, x, j->cols, j->dst + r * j->row_bytes)) j->status = -1;
    }
    free(x);
    return NULL;
}

/* Fills a whole tensor: rows x cols values N(mean, std) (std == 0 -> constant
 * `mean`), quantized to `type`, written row-major into dst.  threads <= 0
 * selects 8. Returns 0 on success. */
int zs_fill_tensor(uint8_t *dst, int type, uint64_t rows, uint64_t cols, uint64_t seed, float mean, float std,
                   int threads) {
    uint64_t rb;
    if (zs_row_bytes(type, cols, &rb)) return -1;
    int nt = threads > 0 ? threads : 8;
    if ((uint64_t)nt > rows) nt = (int)rows;
    if (nt < 1) nt = 1;
    pthread_t *th = (pthread_t *)calloc((size_t)nt, sizeof(pthread_t));
    fill_job *jobs = (fill_job *)calloc((size_t)nt, sizeof(fill_job));
    if (!th || !jobs) {
        free(th);
        free(jobs);
        return -2;
    }
    for (int i = 0; i < nt; i++) {
        jobs[i] = (fill_job){dst, type, rows, cols, seed, rb, mean, std, i, nt, 0};
        pthread_create(&th[i], NULL, fill_main, &jobs[i]);
    }
    int st = 0;
    for (int i = 0; i < nt; i++) {
        pthread_join(th[i], NULL);
        if (jobs[i].status) st = jobs[i].status;
    }
    free(th);
    free(jobs);
    return st;
}
