/* lg_encode.c -- host-side weight encoders fp32 -> GGUF block formats, and
 * seeded synthetic tensors.
 *
 * The reference ships no weight quantizers (only the activation quantizers
 * of fast/lil_math.cpp:329-394), so synthetic models are encoded here.  The
 * block layouts are the GGUF ones the reference reads (fast/lil_gguf.h:64-113)
 * and every encoder is the exact inverse of the reference's dequant index map
 * (fast/lil_math.cpp:93-298), which tests check by dequantizing.
 *
 * Q8_0 uses the reference's own activation formula (d = amax*(1/127),
 * q = roundf(x*127/amax)); the K and Q1 encoders are plain min/max fits (no
 * iterative search): valid blocks, not the best possible ones.
 *
 * Random tensors come from a counter-based generator keyed on (seed, stream,
 * element index), so a tensor is identical for any thread count.
 */
#define _GNU_SOURCE
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/ligguf_encode.h"

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* IEEE binary32 -> binary16, round to nearest even; overflow -> inf */
static uint16_t h16(float f)
{
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return sign | 0x7E00u;
    if (ax >= 0x477FF000u) return sign | 0x7C00u;
    if (ax < 0x38800000u) {
        float a; memcpy(&a, &ax, 4);
        return sign | (uint16_t)rintf(a * 16777216.0f);
    }
    uint32_t r = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3FFu);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return sign | (uint16_t)r;
}

static float f16v(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t u;
    float f;
    if (e == 0u) { f = (float)m * 5.9604644775390625e-8f; return sign ? -f : f; }
    u = sign | ((e + 112u) << 23) | (m << 13);
    memcpy(&f, &u, 4);
    return f;
}

static void put16(uint8_t* p, uint16_t v) { memcpy(p, &v, 2); }

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* nearest integer of a non-negative or negative float, ties away from zero */
static int rnd(float f) { return (int)roundf(f); }

/* ---- counter-based normal generator ---- */
static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* uniform in (0,1) from 24 random bits */
static inline float u01f(uint64_t k) { return ((float)(mix64(k) >> 40) + 0.5f) * 5.9604644775390625e-8f; }

static inline uint64_t stream_key(uint64_t seed, uint64_t stream) { return mix64(seed * 0x9E3779B97F4A7C15ull + stream); }

/* N(0,1) pair number `pair` of a stream: Box-Muller on two counters; element
 * 2*pair takes the cosine branch, 2*pair+1 the sine branch */
static inline void gauss_pair(uint64_t key, uint64_t pair, float* z0, float* z1)
{
    const uint64_t base = key ^ (pair * 0xD1B54A32D192ED03ull);
    const float u1 = u01f(base * 2 + 1), u2 = u01f(base * 2 + 2);
    const float r = sqrtf(-2.0f * logf(u1));
    float sn, cs;
    sincosf(6.28318530717958648f * u2, &sn, &cs);
    *z0 = r * cs;
    *z1 = r * sn;
}

/* n values of a stream starting at element `first` (even) */
static void gauss_run(uint64_t key, uint64_t first, float* out, int64_t n, float sigma)
{
    for (int64_t j = 0; j + 1 < n; j += 2) {
        float z0, z1;
        gauss_pair(key, (first + (uint64_t)j) >> 1, &z0, &z1);
        out[j] = sigma * z0;
        out[j + 1] = sigma * z1;
    }
    if (n & 1) {
        float z0, z1;
        gauss_pair(key, (first + (uint64_t)n - 1) >> 1, &z0, &z1);
        out[n - 1] = sigma * z0;
    }
}

static inline uint32_t ubits(uint64_t seed, uint64_t stream, uint64_t i)
{
    return (uint32_t)(mix64(mix64(seed ^ 0xA0761D6478BD642Full) + stream * 0xE7037ED1A0B428DBull + i) >> 32);
}

void lge_fill_normal(uint64_t seed, uint64_t stream, float* out, int64_t n, float sigma)
{
    const uint64_t key = stream_key(seed, stream);
    const int64_t chunk = 1 << 16;
    #pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < (n + chunk - 1) / chunk; c++) {
        const int64_t b = c * chunk, e = b + chunk < n ? b + chunk : n;
        gauss_run(key, (uint64_t)b, out + b, e - b, sigma);
    }
}

/* ---- block encoders (x: 32/128/256 floats -> one block) ---- */

static void enc_q8_0(const float* x, uint8_t* b)
{
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) { const float a = fabsf(x[j]); if (amax < a) amax = a; }
    const float d = amax * (1.0f / 127.0f);
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    put16(b, h16(d));
    for (int j = 0; j < 32; j++) b[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

/* Q1_0 / Q1_G: sign bits, scale = mean |x| */
static void enc_q1(const float* x, int g, uint8_t* b)
{
    double s = 0.0;
    for (int j = 0; j < g; j++) s += fabs(x[j]);
    put16(b, h16((float)(s / g)));
    memset(b + 2, 0, (size_t)g / 8);
    for (int j = 0; j < g; j++) if (x[j] >= 0.0f) b[2 + (j >> 3)] |= (uint8_t)(1u << (j & 7));
}

/* Q4_K / Q5_K 6-bit scale/min packing, the inverse of get_scale_min_k4
 * (fast/lil_math.cpp:129-138) */
static void pack_k4_scales(const int* sc, const int* mn, uint8_t* s)
{
    memset(s, 0, 12);
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            s[j] |= (uint8_t)(sc[j] & 63);
            s[j + 4] |= (uint8_t)(mn[j] & 63);
        } else {
            s[j + 4] |= (uint8_t)((sc[j] & 15) | ((mn[j] & 15) << 4));
            s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
            s[j] |= (uint8_t)((mn[j] >> 4) << 6);
        }
    }
}

/* shared fit for the asymmetric formats: nsub groups of len values with
 * levels 0..qmax; scales/mins quantized to smax levels */
static void fit_asym(const float* x, int nsub, int len, int qmax, int smax,
                     float* d_out, float* dmin_out, int* sc, int* mn, int* q)
{
    float scl[16], mnf[16], maxs = 0.0f, maxm = 0.0f;
    for (int s = 0; s < nsub; s++) {
        float lo = x[s * len], hi = x[s * len];
        for (int j = 1; j < len; j++) { const float v = x[s * len + j]; if (v < lo) lo = v; if (v > hi) hi = v; }
        if (lo > 0.0f) lo = 0.0f;
        scl[s] = (hi - lo) / (float)qmax;
        mnf[s] = -lo;
        if (scl[s] > maxs) maxs = scl[s];
        if (mnf[s] > maxm) maxm = mnf[s];
    }
    const uint16_t dh = h16(maxs / (float)smax), mh = h16(maxm / (float)smax);
    const float d = f16v(dh), dmin = f16v(mh);
    *d_out = d; *dmin_out = dmin;
    for (int s = 0; s < nsub; s++) {
        sc[s] = d > 0.0f ? clampi(rnd(scl[s] / d), 0, smax) : 0;
        mn[s] = dmin > 0.0f ? clampi(rnd(mnf[s] / dmin), 0, smax) : 0;
        const float ds = d * (float)sc[s], ms = dmin * (float)mn[s];
        for (int j = 0; j < len; j++) {
            const float v = x[s * len + j];
            q[s * len + j] = ds > 0.0f ? clampi(rnd((v + ms) / ds), 0, qmax) : 0;
        }
    }
}

static void enc_q4_k(const float* x, uint8_t* b)
{
    float d, dmin; int sc[8], mn[8], q[256];
    fit_asym(x, 8, 32, 15, 63, &d, &dmin, sc, mn, q);
    put16(b, h16(d)); put16(b + 2, h16(dmin));
    pack_k4_scales(sc, mn, b + 4);
    uint8_t* qs = b + 16;
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++)
            qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

static void enc_q5_k(const float* x, uint8_t* b)
{
    float d, dmin; int sc[8], mn[8], q[256];
    fit_asym(x, 8, 32, 31, 63, &d, &dmin, sc, mn, q);
    put16(b, h16(d)); put16(b + 2, h16(dmin));
    pack_k4_scales(sc, mn, b + 4);
    uint8_t* qh = b + 16;
    uint8_t* qs = b + 48;
    memset(qh, 0, 32);
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
            const int a = q[64 * c + l], h = q[64 * c + 32 + l];
            qs[32 * c + l] = (uint8_t)((a & 15) | ((h & 15) << 4));
            qh[l] |= (uint8_t)(((a >> 4) & 1) << (2 * c));
            qh[l] |= (uint8_t)(((h >> 4) & 1) << (2 * c + 1));
        }
}

static void enc_q2_k(const float* x, uint8_t* b)
{
    float d, dmin; int sc[16], mn[16], q[256];
    fit_asym(x, 16, 16, 3, 15, &d, &dmin, sc, mn, q);
    uint8_t* scales = b;
    uint8_t* qs = b + 16;
    for (int g = 0; g < 16; g++) scales[g] = (uint8_t)(sc[g] | (mn[g] << 4));
    memset(qs, 0, 64);
    /* value i = 128n + 32j + 16h + l -> qs[32n + 16h + l] bits 2j */
    for (int i = 0; i < 256; i++) {
        const int n = i >> 7, j = (i >> 5) & 3, h = (i >> 4) & 1, l = i & 15;
        qs[32 * n + 16 * h + l] |= (uint8_t)(q[i] << (2 * j));
    }
    put16(b + 80, h16(d)); put16(b + 82, h16(dmin));
}

static void enc_q3_k(const float* x, uint8_t* b)
{
    float gs[16], maxs = 0.0f;
    int sc6[16];
    for (int g = 0; g < 16; g++) {
        float amax = 0.0f, sv = 0.0f;
        for (int j = 0; j < 16; j++) { const float a = fabsf(x[16 * g + j]); if (a > amax) { amax = a; sv = x[16 * g + j]; } }
        /* signed group scale so that the largest-magnitude value lands on -4 */
        gs[g] = sv != 0.0f ? -sv / 4.0f : 0.0f;
        if (fabsf(gs[g]) > maxs) maxs = fabsf(gs[g]);
    }
    const uint16_t dh = h16(maxs / 31.0f);
    const float d = f16v(dh);
    uint8_t* hmask = b;
    uint8_t* qs = b + 32;
    uint8_t* scales = b + 96;
    memset(b, 0, 110);
    for (int g = 0; g < 16; g++) sc6[g] = d > 0.0f ? clampi(rnd(gs[g] / d), -32, 31) + 32 : 32;
    /* inverse of the aux shuffle: low nibble at byte g (g<8) or high nibble of
     * byte g-8, high two bits at byte 8+(g&3), bit 2*(g/4) */
    for (int g = 0; g < 16; g++) {
        const int lo = sc6[g] & 15, hi = sc6[g] >> 4;
        if (g < 8) scales[g] |= (uint8_t)lo; else scales[g - 8] |= (uint8_t)(lo << 4);
        scales[8 + (g & 3)] |= (uint8_t)(hi << (2 * (g >> 2)));
    }
    for (int i = 0; i < 256; i++) {
        const float ds = d * (float)(sc6[i >> 4] - 32);
        const int qv = ds != 0.0f ? clampi(rnd(x[i] / ds), -4, 3) : 0;
        const int n = i >> 7, j = (i >> 5) & 3, h = (i >> 4) & 1, l = i & 15;
        const int hb = qv >= 0;
        const int lo = hb ? qv : qv + 4;
        qs[32 * n + 16 * h + l] |= (uint8_t)(lo << (2 * j));
        if (hb) hmask[16 * h + l] |= (uint8_t)(1u << (4 * n + j));
    }
    put16(b + 108, dh);
}

static void enc_q6_k(const float* x, uint8_t* b)
{
    float gs[16], maxs = 0.0f;
    int sc[16];
    for (int g = 0; g < 16; g++) {
        float amax = 0.0f, sv = 0.0f;
        for (int j = 0; j < 16; j++) { const float a = fabsf(x[16 * g + j]); if (a > amax) { amax = a; sv = x[16 * g + j]; } }
        gs[g] = sv != 0.0f ? -sv / 32.0f : 0.0f;
        if (fabsf(gs[g]) > maxs) maxs = fabsf(gs[g]);
    }
    const uint16_t dh = h16(maxs / 127.0f);
    const float d = f16v(dh);
    uint8_t* ql = b;
    uint8_t* qh = b + 128;
    int8_t* scales = (int8_t*)(b + 192);
    memset(b, 0, 210);
    for (int g = 0; g < 16; g++) { sc[g] = d > 0.0f ? clampi(rnd(gs[g] / d), -128, 127) : 0; scales[g] = (int8_t)sc[g]; }
    /* value i = 128n + 32g + l: low nibble in ql[64n + l + 32(g&1)] at 4(g>>1),
     * high two bits in qh[32n + l] at 2g */
    for (int i = 0; i < 256; i++) {
        const float ds = d * (float)sc[i >> 4];
        const int qv = ds != 0.0f ? clampi(rnd(x[i] / ds), -32, 31) + 32 : 32;
        const int n = i >> 7, g = (i >> 5) & 3, l = i & 31;
        ql[64 * n + l + 32 * (g & 1)] |= (uint8_t)((qv & 15) << (4 * (g >> 1)));
        qh[32 * n + l] |= (uint8_t)((qv >> 4) << (2 * g));
    }
    put16(b + 208, dh);
}

int64_t lge_row_size(int type, int64_t n)
{
    switch (type) {
    case LGE_F32: return 4 * n;
    case LGE_F16: return 2 * n;
    case LGE_Q8_0: return n % 32 ? -1 : n / 32 * 34;
    case LGE_Q1_0: return n % 32 ? -1 : n / 32 * 6;
    case LGE_Q1_G: return n % 128 ? -1 : n / 128 * 18;
    case LGE_Q2_K: return n % 256 ? -1 : n / 256 * 84;
    case LGE_Q3_K: return n % 256 ? -1 : n / 256 * 110;
    case LGE_Q4_K: return n % 256 ? -1 : n / 256 * 144;
    case LGE_Q5_K: return n % 256 ? -1 : n / 256 * 176;
    case LGE_Q6_K: return n % 256 ? -1 : n / 256 * 210;
    default: return -1;
    }
}

static int block_len(int type)
{
    switch (type) {
    case LGE_Q8_0: case LGE_Q1_0: return 32;
    case LGE_Q1_G: return 128;
    case LGE_F32: case LGE_F16: return 1;
    default: return 256;
    }
}

/* encode one row of n floats */
static void enc_row(int type, const float* x, int64_t n, uint8_t* out)
{
    int64_t b;
    switch (type) {
    case LGE_F32: memcpy(out, x, (size_t)n * 4); return;
    case LGE_F16: for (b = 0; b < n; b++) put16(out + 2 * b, h16(x[b])); return;
    case LGE_Q8_0: for (b = 0; b < n / 32; b++) enc_q8_0(x + 32 * b, out + 34 * b); return;
    case LGE_Q1_0: for (b = 0; b < n / 32; b++) enc_q1(x + 32 * b, 32, out + 6 * b); return;
    case LGE_Q1_G: for (b = 0; b < n / 128; b++) enc_q1(x + 128 * b, 128, out + 18 * b); return;
    case LGE_Q2_K: for (b = 0; b < n / 256; b++) enc_q2_k(x + 256 * b, out + 84 * b); return;
    case LGE_Q3_K: for (b = 0; b < n / 256; b++) enc_q3_k(x + 256 * b, out + 110 * b); return;
    case LGE_Q4_K: for (b = 0; b < n / 256; b++) enc_q4_k(x + 256 * b, out + 144 * b); return;
    case LGE_Q5_K: for (b = 0; b < n / 256; b++) enc_q5_k(x + 256 * b, out + 176 * b); return;
    case LGE_Q6_K: for (b = 0; b < n / 256; b++) enc_q6_k(x + 256 * b, out + 210 * b); return;
    default: return;
    }
}

int lge_quantize(int type, const float* x, int64_t rows, int64_t cols, void* out)
{
    const int64_t rsz = lge_row_size(type, cols);
    if (rsz < 0 || rows < 0) return -1;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) enc_row(type, x + r * cols, cols, (uint8_t*)out + r * rsz);
    return 0;
}

int lge_random_tensor(int type, uint64_t seed, uint64_t stream, int64_t rows, int64_t cols, float sigma, void* out)
{
    const int64_t rsz = lge_row_size(type, cols);
    if (rsz < 0 || rows < 0 || block_len(type) <= 0 || (cols & 1)) return -1;
    const uint64_t key = stream_key(seed, stream);
    #pragma omp parallel
    {
        float* buf = (float*)malloc((size_t)cols * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            gauss_run(key, (uint64_t)(r * cols), buf, cols, sigma);
            enc_row(type, buf, cols, (uint8_t*)out + r * rsz);
        }
        free(buf);
    }
    return 0;
}

/* 1-bit tensors drawn directly: sign bits Bernoulli(0.5), fp16 group scale
 * |N(0, sigma)| (the Q1_G shape of the 1-bit Qwen3-8B workload) */
int lge_random_q1(int type, uint64_t seed, uint64_t stream, int64_t rows, int64_t cols, float sigma, void* out)
{
    const int g = type == LGE_Q1_0 ? 32 : (type == LGE_Q1_G ? 128 : 0);
    const int bs = g == 32 ? 6 : 18;
    if (!g || cols % g) return -1;
    const int64_t nb = rows * (cols / g);
    const uint64_t key = stream_key(seed, stream);
    #pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nb; b++) {
        uint8_t* blk = (uint8_t*)out + b * bs;
        float z0, z1;
        gauss_pair(key, (uint64_t)b, &z0, &z1);
        put16(blk, h16(fabsf(sigma * z0)));
        for (int k = 0; k < g / 32; k++) {
            const uint32_t w = ubits(seed, stream, (uint64_t)(b * 4 + k));
            memcpy(blk + 2 + 4 * k, &w, 4);
        }
    }
    return 0;
}
