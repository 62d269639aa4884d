/* lg_oracle.c -- CPU restatement of LiGGUF FAST's per-token decode path.
 * TEST INFRASTRUCTURE ONLY; see lg_oracle.h for the arithmetic contract and
 * what pins each function.  Built with -O2 -fno-fast-math -ffp-contract=off.
 */
#include "lg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* Block layouts: the GGUF on-disk format (fast/lil_gguf.h:64-119).    */
/* ------------------------------------------------------------------ */
#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t qs[32]; } b_q8_0;                                   /* 34 B  */
typedef struct { uint16_t d; uint8_t qs[4]; } b_q1_0;                                   /* 6 B   */
typedef struct { uint16_t d; uint8_t qs[16]; } b_q1_g;                                  /* 18 B  */
typedef struct { uint8_t scales[16]; uint8_t qs[64]; uint16_t d, dmin; } b_q2_k;        /* 84 B  */
typedef struct { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12]; uint16_t d; } b_q3_k; /* 110 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } b_q4_k;       /* 144 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } b_q5_k; /* 176 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } b_q6_k; /* 210 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } b_q8_k;                  /* 292 B */
#pragma pack(pop)

_Static_assert(sizeof(b_q8_0) == 34, "q8_0");
_Static_assert(sizeof(b_q1_0) == 6, "q1_0");
_Static_assert(sizeof(b_q1_g) == 18, "q1_g");
_Static_assert(sizeof(b_q2_k) == 84, "q2_k");
_Static_assert(sizeof(b_q3_k) == 110, "q3_k");
_Static_assert(sizeof(b_q4_k) == 144, "q4_k");
_Static_assert(sizeof(b_q5_k) == 176, "q5_k");
_Static_assert(sizeof(b_q6_k) == 210, "q6_k");
_Static_assert(sizeof(b_q8_k) == 292, "q8_k");

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ */
/* A1: IEEE binary16 <-> binary32.                                     */
/* The reference converts with bit tricks (fast/lil_math.cpp:37-76) and */
/* caches fp16->fp32 in a LUT (:78-81); both equal IEEE conversion with */
/* round-to-nearest-even for every finite |f| < 65520.  For |f| >=      */
/* 65520 the reference emits 0x7C00|mantissa-junk NaN patterns while    */
/* this restatement returns +-inf; NaN inputs map to sign|0x7E00 in     */
/* both, and fp16 NaNs widen to quiet fp32 NaNs in both.                */
/* ------------------------------------------------------------------ */
float or_fp16_to_fp32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    if (e == 31u) return u2f(sign | 0x7F800000u | (m ? 0x00400000u : 0u) | (m << 13)); /* NaNs come out quiet */
    if (e == 0u) {
        const float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t or_fp32_to_fp16(float f)
{
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return sign | 0x7E00u;           /* NaN */
    if (ax >= 0x477FF000u) return sign | 0x7C00u;          /* rounds past 65504 */
    if (ax < 0x38800000u) {                                /* below 2^-14: subnormal half */
        const float scaled = u2f(ax) * 16777216.0f;        /* |f| * 2^24, exact */
        return sign | (uint16_t)rintf(scaled);             /* RNE; 1024 -> min normal */
    }
    uint32_t r = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3FFu);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return sign | (uint16_t)r;
}

void or_f32_to_f16_row(const float* x, uint16_t* y, int64_t n)
{
    for (int64_t i = 0; i < n; i++) y[i] = or_fp32_to_fp16(x[i]);
}

#define H2F(h) or_fp16_to_fp32(h)

/* ------------------------------------------------------------------ */
/* Row sizes (fast/lil_gguf.cpp:190-225).                              */
/* ------------------------------------------------------------------ */
int64_t or_row_size(int type, int64_t n)
{
    switch (type) {
    case OR_F32: return 4 * n;
    case OR_F16: return 2 * n;
    case OR_Q8_0: return n % 32 ? -1 : (n / 32) * 34;
    case OR_Q1_0: return n % 32 ? -1 : (n / 32) * 6;
    case OR_Q1_G: return n % 128 ? -1 : (n / 128) * 18;
    case OR_Q2_K: return n % 256 ? -1 : (n / 256) * 84;
    case OR_Q3_K: return n % 256 ? -1 : (n / 256) * 110;
    case OR_Q4_K: return n % 256 ? -1 : (n / 256) * 144;
    case OR_Q5_K: return n % 256 ? -1 : (n / 256) * 176;
    case OR_Q6_K: return n % 256 ? -1 : (n / 256) * 210;
    default: return -1;
    }
}

/* ------------------------------------------------------------------ */
/* Integer view of one 256-value K-quant super-block: for value i the   */
/* unsigned/signed quant q[i], the integer scale of its group and, for  */
/* the min-carrying formats, the integer min of its group.  The value   */
/* is d*scale*q - dmin*min.  Index maps follow the reference dequant    */
/* loops (fast/lil_math.cpp:140-298).                                    */
/* ------------------------------------------------------------------ */
typedef struct {
    int q[256];
    int sc[256];
    int mn[256];
    float d, dmin;
    int has_min;
} kview;

/* 6-bit scale/min pair j of a Q4_K/Q5_K block (fast/lil_math.cpp:129-138) */
static void k4_scale_min(const uint8_t* s, int j, int* sc, int* m)
{
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* 6-bit scale g (0..15) of a Q3_K block, the aux-word shuffle of
 * fast/lil_math.cpp:187-192 written per scale: low nibble from byte g (g<8)
 * or the high nibble of byte g-8, two high bits from byte 8+(g&3) at bit
 * 2*(g/4). */
static int k3_scale(const uint8_t* s, int g)
{
    const int lo = g < 8 ? (s[g] & 15) : (s[g - 8] >> 4);
    const int hi = (s[8 + (g & 3)] >> (2 * (g >> 2))) & 3;
    return lo | (hi << 4);
}

static void kview_of(int type, const void* blk, kview* v)
{
    int i;
    v->has_min = 0;
    v->dmin = 0.0f;
    switch (type) {
    case OR_Q2_K: {
        const b_q2_k* b = (const b_q2_k*)blk;
        v->d = H2F(b->d); v->dmin = H2F(b->dmin); v->has_min = 1;
        for (i = 0; i < 256; i++) {
            const int n = i >> 7, j = (i >> 5) & 3, h = (i >> 4) & 1, l = i & 15;
            const uint8_t s = b->scales[i >> 4];
            v->q[i] = (b->qs[32 * n + 16 * h + l] >> (2 * j)) & 3;
            v->sc[i] = s & 15;
            v->mn[i] = s >> 4;
        }
        break;
    }
    case OR_Q3_K: {
        const b_q3_k* b = (const b_q3_k*)blk;
        v->d = H2F(b->d);
        for (i = 0; i < 256; i++) {
            const int n = i >> 7, j = (i >> 5) & 3, h = (i >> 4) & 1, l = i & 15;
            const int lo = (b->qs[32 * n + 16 * h + l] >> (2 * j)) & 3;
            const int hb = (b->hmask[16 * h + l] >> (4 * n + j)) & 1;
            v->q[i] = lo - (hb ? 0 : 4);
            v->sc[i] = k3_scale(b->scales, i >> 4) - 32;
            v->mn[i] = 0;
        }
        break;
    }
    case OR_Q4_K: {
        const b_q4_k* b = (const b_q4_k*)blk;
        v->d = H2F(b->d); v->dmin = H2F(b->dmin); v->has_min = 1;
        for (i = 0; i < 256; i++) {
            const int c = i >> 6, h = (i >> 5) & 1, l = i & 31;
            int sc, m;
            k4_scale_min(b->scales, 2 * c + h, &sc, &m);
            v->q[i] = (b->qs[32 * c + l] >> (4 * h)) & 15;
            v->sc[i] = sc;
            v->mn[i] = m;
        }
        break;
    }
    case OR_Q5_K: {
        const b_q5_k* b = (const b_q5_k*)blk;
        v->d = H2F(b->d); v->dmin = H2F(b->dmin); v->has_min = 1;
        for (i = 0; i < 256; i++) {
            const int c = i >> 6, h = (i >> 5) & 1, l = i & 31;
            int sc, m;
            k4_scale_min(b->scales, 2 * c + h, &sc, &m);
            v->q[i] = ((b->qs[32 * c + l] >> (4 * h)) & 15) + 16 * ((b->qh[l] >> (2 * c + h)) & 1);
            v->sc[i] = sc;
            v->mn[i] = m;
        }
        break;
    }
    case OR_Q6_K: {
        const b_q6_k* b = (const b_q6_k*)blk;
        v->d = H2F(b->d);
        for (i = 0; i < 256; i++) {
            const int n = i >> 7, g = (i >> 5) & 3, l = i & 31;
            const int lo = (b->ql[64 * n + l + 32 * (g & 1)] >> (4 * (g >> 1))) & 15;
            const int hi = (b->qh[32 * n + l] >> (2 * g)) & 3;
            v->q[i] = (lo | (hi << 4)) - 32;
            v->sc[i] = b->scales[i >> 4];
            v->mn[i] = 0;
        }
        break;
    }
    default:
        break;
    }
}

static int is_k(int t) { return t >= OR_Q2_K && t <= OR_Q6_K; }
static int is_q8_0_family(int t) { return t == OR_Q8_0 || t == OR_Q1_0 || t == OR_Q1_G; }
static int k_block_bytes(int t)
{
    switch (t) {
    case OR_Q2_K: return 84;
    case OR_Q3_K: return 110;
    case OR_Q4_K: return 144;
    case OR_Q5_K: return 176;
    case OR_Q6_K: return 210;
    default: return 0;
    }
}

/* ------------------------------------------------------------------ */
/* A3: dequantization.  Every product d*scale*q is exact in fp32 (at    */
/* most 24 significant bits); the only rounding is the final - dmin*m   */
/* of Q2_K/Q4_K/Q5_K, so this form is bit-identical to the reference's  */
/* loops (fast/lil_math.cpp:93-298) whatever the evaluation order.      */
/* ------------------------------------------------------------------ */
int or_dequantize_row(int type, const void* x, float* y, int64_t n)
{
    int64_t i, b;
    if (or_row_size(type, n) < 0) return -1;
    switch (type) {
    case OR_F32:
        memcpy(y, x, (size_t)n * 4);
        return 0;
    case OR_F16:
        for (i = 0; i < n; i++) y[i] = H2F(((const uint16_t*)x)[i]);
        return 0;
    case OR_Q8_0:
        for (b = 0; b < n / 32; b++) {
            const b_q8_0* blk = (const b_q8_0*)x + b;
            const float d = H2F(blk->d);
            for (i = 0; i < 32; i++) y[32 * b + i] = (float)blk->qs[i] * d;
        }
        return 0;
    case OR_Q1_0:
    case OR_Q1_G: {
        const int g = type == OR_Q1_0 ? 32 : 128;
        const int bs = type == OR_Q1_0 ? 6 : 18;
        for (b = 0; b < n / g; b++) {
            const uint8_t* blk = (const uint8_t*)x + b * bs;
            uint16_t dh; memcpy(&dh, blk, 2);
            const float d = H2F(dh);
            for (i = 0; i < g; i++) y[g * b + i] = ((blk[2 + (i >> 3)] >> (i & 7)) & 1) ? d : -d;
        }
        return 0;
    }
    default: {
        const int bb = k_block_bytes(type);
        kview v;
        for (b = 0; b < n / 256; b++) {
            kview_of(type, (const uint8_t*)x + b * bb, &v);
            for (i = 0; i < 256; i++) {
                const float dq = v.d * (float)v.sc[i] * (float)v.q[i];   /* exact */
                y[256 * b + i] = v.has_min ? dq - v.dmin * (float)v.mn[i] : dq;
            }
        }
        return 0;
    }
    }
}

/* ------------------------------------------------------------------ */
/* A2: activation quantizers, as the reference compiles them under      */
/* -Ofast (fast/Makefile:7).                                            */
/* quantize_q8_0 (fast/lil_math.cpp:329-351): the source computes       */
/*   d = amax/127, id = 1/d, qs = roundf(x*id)                          */
/* and -Ofast's reciprocal folding turns that into                      */
/*   d = amax * (1/127), id = 127/amax                                   */
/* (a textbook 1/d differs in ~2e-5 of blocks).                         */
/* ------------------------------------------------------------------ */
void or_quantize_q8_0(const float* x, int64_t n, void* y)
{
    const int64_t nb = n / 32;
    b_q8_0* out = (b_q8_0*)y;
    for (int64_t b = 0; b < nb; b++) {
        const float* p = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float a = fabsf(p[j]);
            if (amax < a) amax = a;
        }
        const float d = amax * (1.0f / 127.0f);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        out[b].d = or_fp32_to_fp16(d);
        for (int j = 0; j < 32; j++) out[b].qs[j] = (int8_t)roundf(p[j] * id);
    }
}

/* quantize_q8_K (fast/lil_math.cpp:353-394): the signed value of largest
 * magnitude (first index wins), iscale = -127/max, qs = min(127,
 * nearest_int(iscale*x)) with nearest_int = truncate(f -+ 0.5), 16-value
 * bsums, and d = 1/iscale, which -Ofast folds to max * (-1/127). */
void or_quantize_q8_K(const float* x, int64_t n, void* y)
{
    const int64_t nb = n / 256;
    b_q8_k* out = (b_q8_k*)y;
    for (int64_t b = 0; b < nb; b++) {
        const float* p = x + 256 * b;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 256; j++) {
            const float a = fabsf(p[j]);
            if (a > amax) { amax = a; max = p[j]; }
        }
        if (amax == 0.0f) {
            memset(&out[b], 0, sizeof(b_q8_k));
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < 256; j++) {
            const float f = iscale * p[j];
            int v = f < 0.0f ? (int)(f - 0.5f) : (int)(f + 0.5f);
            out[b].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int j = 0; j < 16; j++) s += out[b].qs[16 * g + j];
            out[b].bsums[g] = (int16_t)s;
        }
        out[b].d = max * (-1.0f / 127.0f);
    }
}

/* ------------------------------------------------------------------ */
/* A4: one row . quantized activation.  Integer parts are the           */
/* reference's sub-block sums (fast/lil_math.cpp:411-740): exact in     */
/* int64.  The floating combination is evaluated in double.             */
/* *abs_out gets the sum of |terms| for tolerance scaling.              */
/* ------------------------------------------------------------------ */
static double row_dot(int type, const uint8_t* w, int n, const void* xq, double* abs_out)
{
    double acc = 0.0, aacc = 0.0;
    int64_t b, i;
    if (type == OR_F32 || type == OR_F16) {
        const float* xf = (const float*)xq;
        for (i = 0; i < n; i++) {
            const double wv = type == OR_F32 ? (double)((const float*)w)[i] : (double)H2F(((const uint16_t*)w)[i]);
            const double t = wv * (double)xf[i];
            acc += t; aacc += fabs(t);
        }
    } else if (type == OR_Q8_0 || type == OR_Q1_0) {
        const b_q8_0* a = (const b_q8_0*)xq;
        const int bs = type == OR_Q8_0 ? 34 : 6;
        for (b = 0; b < n / 32; b++) {
            const uint8_t* blk = w + b * bs;
            uint16_t dh; memcpy(&dh, blk, 2);
            int64_t s = 0;
            for (i = 0; i < 32; i++) {
                const int q = type == OR_Q8_0 ? (int)(int8_t)blk[2 + i] : (((blk[2 + (i >> 3)] >> (i & 7)) & 1) ? 1 : -1);
                s += (int64_t)q * a[b].qs[i];
            }
            const double t = (double)H2F(dh) * (double)H2F(a[b].d) * (double)s;
            acc += t; aacc += fabs(t);
        }
    } else if (type == OR_Q1_G) {
        const b_q8_0* a = (const b_q8_0*)xq;
        for (b = 0; b < n / 128; b++) {
            const b_q1_g* blk = (const b_q1_g*)(w + b * 18);
            const double dw = H2F(blk->d);
            for (int k = 0; k < 4; k++) {
                const b_q8_0* ab = a + 4 * b + k;
                int64_t s = 0;
                for (i = 0; i < 32; i++) {
                    const int bit = 32 * k + (int)i;
                    s += (int64_t)(((blk->qs[bit >> 3] >> (bit & 7)) & 1) ? 1 : -1) * ab->qs[i];
                }
                const double t = dw * (double)H2F(ab->d) * (double)s;
                acc += t; aacc += fabs(t);
            }
        }
    } else if (is_k(type)) {
        const b_q8_k* a = (const b_q8_k*)xq;
        const int bb = k_block_bytes(type);
        kview v;
        for (b = 0; b < n / 256; b++) {
            kview_of(type, w + b * bb, &v);
            int64_t S = 0, M = 0;
            const double da = a[b].d;
            for (int g = 0; g < 16; g++) {
                int64_t Sg = 0;
                for (i = 16 * g; i < 16 * g + 16; i++) Sg += (int64_t)v.sc[i] * v.q[i] * a[b].qs[i];
                S += Sg;
                /* min of group g (Q2_K) or of sub-block g/2 (Q4_K/Q5_K) times
                 * the activation sum over those values: the reference uses the
                 * Q8_K bsums, which are exactly these sums */
                const int64_t Mg = v.has_min ? (int64_t)v.mn[16 * g] * a[b].bsums[g] : 0;
                M += Mg;
                /* tolerance scale: magnitudes per 16-value group, the finest
                 * unit any summation order combines */
                aacc += fabs(da * (double)v.d * (double)Sg) + fabs(da * (double)v.dmin * (double)Mg);
            }
            const double t1 = da * (double)v.d * (double)S;
            const double t2 = v.has_min ? da * (double)v.dmin * (double)M : 0.0;
            acc += t1 - t2;
        }
    }
    if (abs_out) *abs_out = aacc;
    return acc;
}

int or_matvec_q(int type, const void* w, uint32_t rsz, int n, int d, const void* xq, float* out, float* absout)
{
    if (or_row_size(type, n) < 0 || (int64_t)rsz < or_row_size(type, n)) return -1;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < d; r++) {
        double aa;
        const double v = row_dot(type, (const uint8_t*)w + (size_t)r * rsz, n, xq, &aa);
        out[r] = (float)v;
        if (absout) absout[r] = (float)aa;
    }
    return 0;
}

int or_matvec(int type, const void* w, uint32_t rsz, int n, int d, const float* x, float* out)
{
    void* xq = NULL;
    int rc;
    if (is_q8_0_family(type)) {
        xq = malloc((size_t)(n / 32) * sizeof(b_q8_0));
        or_quantize_q8_0(x, n, xq);
    } else if (is_k(type)) {
        xq = malloc((size_t)(n / 256) * sizeof(b_q8_k));
        or_quantize_q8_K(x, n, xq);
    }
    rc = or_matvec_q(type, w, rsz, n, d, xq ? xq : (const void*)x, out, NULL);
    free(xq);
    return rc;
}

/* ------------------------------------------------------------------ */
/* A6: x * w / sqrt(mean(x^2) + eps) (fast/lil_math.cpp:922-937).       */
/* ------------------------------------------------------------------ */
void or_rmsnorm(float* out, const float* x, const float* w, int n, float eps)
{
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const double s = 1.0 / sqrt(ss / n + (double)eps);
    for (int i = 0; i < n; i++) out[i] = (float)((double)x[i] * s * (double)w[i]);
}

/* ------------------------------------------------------------------ */
/* A7: adjacent-pair RoPE (fast/lil_math.cpp:901-920).  The angle is    */
/* the reference's fp32 product pos*freq[i/2]; rope_dim is clamped to   */
/* head_dim and made even.                                              */
/* ------------------------------------------------------------------ */
void or_rope(float* x, int n_heads, int head_dim, int rope_dim, int pos, const float* freq)
{
    int rd = rope_dim > head_dim ? head_dim : rope_dim;
    if (rd & 1) rd--;
    for (int h = 0; h < n_heads; h++) {
        float* v = x + (size_t)h * head_dim;
        for (int i = 0; i < rd; i += 2) {
            const float ang = (float)pos * freq[i >> 1];
            const double c = cos((double)ang), s = sin((double)ang);
            const double x0 = v[i], x1 = v[i + 1];
            v[i] = (float)(x0 * c - x1 * s);
            v[i + 1] = (float)(x0 * s + x1 * c);
        }
    }
}

/* ------------------------------------------------------------------ */
/* A10: SwiGLU, hb = silu(hb2) * hb (fast/ligguf_fast_qk.cpp:119-123).   */
/* ------------------------------------------------------------------ */
void or_swiglu(float* hb, const float* hb2, int n)
{
    for (int i = 0; i < n; i++) {
        const double g = hb2[i];
        hb[i] = (float)(g / (1.0 + exp(-g)) * (double)hb[i]);
    }
}

/* ------------------------------------------------------------------ */
/* A9: GQA decode attention (fast/ligguf_fast_qk.cpp:64-105).  Head h   */
/* reads KV head h/(n_heads/n_kv_heads); positions t < pos come from    */
/* the fp16 cache, t == pos from the fp32 k/v of this step.  Scores are */
/* scaled by 1/sqrt(head_dim) and softmaxed exactly (fast/lil_math.cpp: */
/* 964-976).                                                            */
/* ------------------------------------------------------------------ */
void or_attention(const float* q, const float* k, const float* v, const uint16_t* kc, const uint16_t* vc,
                  int n_heads, int n_kv_heads, int head_dim, int pos, float* out)
{
    const int kv_dim = n_kv_heads * head_dim;
    const int nrep = n_heads / n_kv_heads;
    const double scale = (double)(1.0f / sqrtf((float)head_dim));
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        const int kh = h / nrep;
        const float* qh = q + (size_t)h * head_dim;
        double* att = (double*)malloc(sizeof(double) * (size_t)(pos + 1));
        double* acc = (double*)calloc((size_t)head_dim, sizeof(double));
        double mx = -INFINITY, sum = 0.0;
        for (int t = 0; t <= pos; t++) {
            double s = 0.0;
            for (int i = 0; i < head_dim; i++) {
                const double kv = t == pos ? (double)k[kh * head_dim + i]
                                           : (double)H2F(kc[(size_t)t * kv_dim + kh * head_dim + i]);
                s += (double)qh[i] * kv;
            }
            att[t] = s * scale;
            if (att[t] > mx) mx = att[t];
        }
        for (int t = 0; t <= pos; t++) { att[t] = exp(att[t] - mx); sum += att[t]; }
        for (int t = 0; t <= pos; t++) {
            const double a = att[t] / sum;
            for (int i = 0; i < head_dim; i++) {
                const double vv = t == pos ? (double)v[kh * head_dim + i]
                                           : (double)H2F(vc[(size_t)t * kv_dim + kh * head_dim + i]);
                acc[i] += a * vv;
            }
        }
        for (int i = 0; i < head_dim; i++) out[(size_t)h * head_dim + i] = (float)acc[i];
        free(att);
        free(acc);
    }
}

int or_argmax(const float* x, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++) if (x[i] > x[best]) best = i;
    return best;
}

/* top-p / top-k sampling (sampler_topp, fast/ligguf_fast_qk.cpp:172-214):
 * softmax at temperature temp with a sequential float sum, a sort by p
 * descending then token ascending (cmp_sampler_ent_desc, :162-170), the
 * cutoff where the running sum reaches top (at most topk - 1), and the first
 * entry whose running sum reaches r01 * cum.  r01 stands for the
 * reference's (float)rand() / (float)RAND_MAX. */
typedef struct { float p; int tok; } or_samp;

static int or_samp_cmp(const void* pa, const void* pb)
{
    const or_samp* a = (const or_samp*)pa;
    const or_samp* b = (const or_samp*)pb;
    if (a->p != b->p) return a->p < b->p ? 1 : -1;
    return a->tok - b->tok;
}

int or_sampler_topp(const float* logits, int n, float temp, float topp, int topk, float r01)
{
    const int imax = or_argmax(logits, n);
    if (temp <= 0.0f) return imax;
    const float inv_temp = 1.0f / temp, maxlog = logits[imax];
    or_samp* s = (or_samp*)malloc((size_t)n * sizeof(or_samp));
    if (!s) return -1;
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        s[i].p = expf((logits[i] - maxlog) * inv_temp);
        s[i].tok = i;
        sum += s[i].p;
    }
    if (sum <= 0.0f) { free(s); return imax; }
    for (int i = 0; i < n; i++) s[i].p /= sum;
    qsort(s, (size_t)n, sizeof(or_samp), or_samp_cmp);
    float top = topp <= 0.0f ? s[0].p : topp;
    if (top > 1.0f) top = 1.0f;
    const int k = (topk <= 0 || topk > n) ? n : topk;
    float cum = 0.0f;
    int cut = 0;
    for (; cut < k; cut++) {
        cum += s[cut].p;
        if (cum >= top) break;
    }
    if (cut >= k) cut = k - 1;
    const float r = r01 * cum;
    float pcum = 0.0f;
    int tok = s[cut].tok;
    for (int i = 0; i <= cut; i++) {
        pcum += s[i].p;
        if (pcum >= r) { tok = s[i].tok; break; }
    }
    free(s);
    return tok;
}

/* ------------------------------------------------------------------ */
/* A12: the per-token step (fast/ligguf_fast_qk.cpp:24-144).            */
/* ------------------------------------------------------------------ */
struct or_state {
    or_model m;
    int pos;
    float *x, *xb, *xb2, *hb, *hb2, *q, *k, *v, *logits, *tmp;
    uint16_t *kc, *vc;
    float* trace;   /* NULL, or [4*n_layers+1][max(n_embed, n_ff)] for the next step only */
    /* next step only: quantized activations to use in place of the step's own
     * at each quantization point k whose form force_forms[k] is set */
    const uint8_t* force;
    size_t force_stride;
    const int* force_forms;
};

or_state* or_state_new(const or_model* m)
{
    or_state* s = (or_state*)calloc(1, sizeof(or_state));
    const int wide = m->n_ff > m->n_embed ? m->n_ff : m->n_embed;
    s->m = *m;
    s->x = (float*)calloc((size_t)m->n_embed, 4);
    s->xb = (float*)calloc((size_t)wide, 4);
    s->xb2 = (float*)calloc((size_t)m->n_embed, 4);
    s->hb = (float*)calloc((size_t)m->n_ff, 4);
    s->hb2 = (float*)calloc((size_t)m->n_ff, 4);
    s->q = (float*)calloc((size_t)m->n_heads * m->head_dim, 4);
    s->k = (float*)calloc((size_t)m->kv_dim, 4);
    s->v = (float*)calloc((size_t)m->kv_dim, 4);
    s->logits = (float*)calloc((size_t)m->vocab_size, 4);
    s->tmp = (float*)calloc((size_t)wide, 4);
    s->kc = (uint16_t*)calloc((size_t)m->n_layers * m->n_context * m->kv_dim, 2);
    s->vc = (uint16_t*)calloc((size_t)m->n_layers * m->n_context * m->kv_dim, 2);
    return s;
}

void or_state_free(or_state* s)
{
    if (!s) return;
    free(s->x); free(s->xb); free(s->xb2); free(s->hb); free(s->hb2); free(s->q); free(s->k); free(s->v);
    free(s->logits); free(s->tmp); free(s->kc); free(s->vc);
    free(s);
}

void or_state_trace(or_state* s, float* trace) { s->trace = trace; }

/* the float vector inference() quantizes at point k of the step (before
 * quantize_q8_K / quantize_q8_0, fast/ligguf_fast_qk.cpp:39,108,116,126,140) */
static void trace_vec(or_state* s, float* tr, int k, const float* v, int n)
{
    if (!tr) return;
    const int wide = s->m.n_ff > s->m.n_embed ? s->m.n_ff : s->m.n_embed;
    memcpy(tr + (size_t)k * wide, v, (size_t)n * 4);
}

int or_state_pos(const or_state* s) { return s->pos; }
void or_state_set_pos(or_state* s, int pos) { s->pos = pos; }

static void mv(const or_weight* w, const float* x, float* out)
{
    or_matvec(w->type, w->data, w->rsz, w->cols, w->rows, x, out);
}

void or_state_force(or_state* s, const void* acts, size_t stride, const int* forms)
{
    s->force = (const uint8_t*)acts;
    s->force_stride = stride;
    s->force_forms = forms;
}

/* mv() at quantization point k.  When the step forces that point in the
 * weight's activation form (Q8_K for the K-quants, Q8_0 for the Q8_0 family:
 * fast/ligguf_fast_qk.cpp:39-41) the matvec reads the given blocks instead of
 * quantizing x.  A Q8_K block's bsums are the 16-value sums of its quants
 * (quantize_q8_K, fast/lil_math.cpp:329-361), so they are recomputed from
 * the given quants rather than taken from the caller. */
static void mv_at(const or_state* s, const uint8_t* force, int k, const or_weight* w, const float* x, float* out)
{
    const int f = force ? s->force_forms[k] : 0;
    const uint8_t* a = force ? force + (size_t)k * s->force_stride : NULL;
    if (f == OR_Q8_K && is_k(w->type)) {
        const int nb = w->cols / 256;
        b_q8_k* q = (b_q8_k*)malloc((size_t)nb * sizeof(b_q8_k));
        memcpy(q, a, (size_t)nb * sizeof(b_q8_k));
        for (int b = 0; b < nb; b++)
            for (int g = 0; g < 16; g++) {
                int sum = 0;
                for (int i = 0; i < 16; i++) sum += q[b].qs[16 * g + i];
                q[b].bsums[g] = (int16_t)sum;
            }
        or_matvec_q(w->type, w->data, w->rsz, w->cols, w->rows, q, out, NULL);
        free(q);
    } else if (f == OR_Q8_0 && is_q8_0_family(w->type)) {
        or_matvec_q(w->type, w->data, w->rsz, w->cols, w->rows, a, out, NULL);
    } else {
        mv(w, x, out);
    }
}

int or_inference(or_state* s, int tok, float* logits)
{
    const or_model* m = &s->m;
    const int pos = s->pos;
    const int hd = m->head_dim, kvd = m->kv_dim, ne = m->n_embed;
    if (pos < 0 || pos >= m->n_context || tok < 0 || tok >= m->token_embd.rows) return -1;
    s->pos++;
    float* tr = s->trace;   /* one step only */
    const uint8_t* fc = s->force;
    s->trace = NULL;
    s->force = NULL;

    or_dequantize_row(m->token_embd.type, (const uint8_t*)m->token_embd.data + (size_t)tok * m->token_embd.rsz, s->x, ne);

    for (int l = 0; l < m->n_layers; l++) {
        const or_layer* L = &m->layers[l];
        or_rmsnorm(s->xb, s->x, L->att_norm, ne, m->rms_epsilon);
        trace_vec(s, tr, 4 * l, s->xb, ne);
        mv_at(s, fc, 4 * l, &L->att_q, s->xb, s->q);
        mv_at(s, fc, 4 * l, &L->att_k, s->xb, s->k);
        mv_at(s, fc, 4 * l, &L->att_v, s->xb, s->v);
        if (m->arch == 1) {
            for (int h = 0; h < m->n_heads; h++) or_rmsnorm(s->q + h * hd, s->q + h * hd, L->att_q_norm, hd, m->rms_epsilon);
            for (int h = 0; h < m->n_kv_heads; h++) or_rmsnorm(s->k + h * hd, s->k + h * hd, L->att_k_norm, hd, m->rms_epsilon);
        }
        or_rope(s->q, m->n_heads, hd, m->rope_dim, pos, m->rope_freq);
        or_rope(s->k, m->n_kv_heads, hd, m->rope_dim, pos, m->rope_freq);

        const size_t loff = (size_t)l * m->n_context * kvd;
        or_f32_to_f16_row(s->k, s->kc + loff + (size_t)pos * kvd, kvd);
        or_f32_to_f16_row(s->v, s->vc + loff + (size_t)pos * kvd, kvd);

        or_attention(s->q, s->k, s->v, s->kc + loff, s->vc + loff, m->n_heads, m->n_kv_heads, hd, pos, s->xb);

        trace_vec(s, tr, 4 * l + 1, s->xb, ne);
        mv_at(s, fc, 4 * l + 1, &L->att_out, s->xb, s->xb2);
        for (int j = 0; j < ne; j++) s->x[j] += s->xb2[j];

        or_rmsnorm(s->xb, s->x, L->ffn_norm, ne, m->rms_epsilon);
        trace_vec(s, tr, 4 * l + 2, s->xb, ne);
        mv_at(s, fc, 4 * l + 2, &L->ffn_up, s->xb, s->hb);
        mv_at(s, fc, 4 * l + 2, &L->ffn_gate, s->xb, s->hb2);
        or_swiglu(s->hb, s->hb2, m->n_ff);
        trace_vec(s, tr, 4 * l + 3, s->hb, m->n_ff);
        mv_at(s, fc, 4 * l + 3, &L->ffn_down, s->hb, s->xb);
        for (int j = 0; j < ne; j++) s->x[j] += s->xb[j];
    }

    or_rmsnorm(s->x, s->x, m->output_norm, ne, m->rms_epsilon);
    trace_vec(s, tr, 4 * m->n_layers, s->x, ne);
    mv_at(s, fc, 4 * m->n_layers, &m->output, s->x, s->logits);
    if (logits) memcpy(logits, s->logits, (size_t)m->vocab_size * 4);
    return 0;
}

void or_state_kv_write(or_state* s, int layer, int p0, int np, const uint16_t* k, const uint16_t* v)
{
    const size_t off = (size_t)layer * s->m.n_context * s->m.kv_dim + (size_t)p0 * s->m.kv_dim;
    const size_t cnt = (size_t)np * s->m.kv_dim;
    if (k) memcpy(s->kc + off, k, cnt * 2);
    if (v) memcpy(s->vc + off, v, cnt * 2);
}

void or_state_kv(const or_state* s, int layer, int p0, int np, uint16_t* k, uint16_t* v)
{
    const size_t off = (size_t)layer * s->m.n_context * s->m.kv_dim + (size_t)p0 * s->m.kv_dim;
    const size_t cnt = (size_t)np * s->m.kv_dim;
    if (k) memcpy(k, s->kc + off, cnt * 2);
    if (v) memcpy(v, s->vc + off, cnt * 2);
}

/* ------------------------------------------------------------------ */
/* (f)4: BERT sentence embedding (fast/vdb.cpp:123-245).               */
/* Token / position / type rows are dequantized and summed in fp32 as  */
/* the reference does (:162-165); matrix products go through           */
/* or_matvec (Q8_0 activations for Q8_0/Q1 weights, fp32 for F32/F16,  */
/* fast/lil_math.cpp:748-776); biases, residuals, attention, GELU,     */
/* pooling and the L2 norm are evaluated in double and rounded once.   */
/* ------------------------------------------------------------------ */
void or_layernorm(float* out, const float* x, const float* w, const float* b, int n, float eps)
{
    /* the reference's own double accumulation (fast/lil_math.cpp:948-962) */
    double mean = 0.0, var = 0.0;
    for (int i = 0; i < n; i++) mean += x[i];
    mean /= n;
    for (int i = 0; i < n; i++) {
        const double d = x[i] - mean;
        var += d * d;
    }
    var /= n;
    const float scale = 1.0f / sqrtf((float)(var + (double)eps));
    for (int i = 0; i < n; i++) out[i] = (float)(((double)x[i] - mean) * (double)scale * (double)w[i] + (double)b[i]);
}

static float or_gelu1(float v)
{
    /* gelu (fast/lil_math.cpp:978-984) with its float constants */
    const double c0 = (double)0.7978845608f, c1 = (double)0.044715f, d = v;
    return (float)(0.5 * d * (1.0 + tanh(c0 * (d + c1 * d * d * d))));
}

int or_bert_embed(const or_bert* m, const int* toks_in, int ntok_in, float* out)
{
    return or_bert_embed_traced(m, toks_in, ntok_in, out, NULL);
}

int or_bert_embed_traced(const or_bert* m, const int* toks_in, int ntok_in, float* out, float* trace)
{
    const int ne = m->n_embed, nff = m->n_ff, nh = m->n_heads, hd = ne / nh;
    int raw = ntok_in;
    if (raw > m->n_context - 2) raw = m->n_context - 2;      /* toks.resize(n_context - 2), :135 */
    const int T = raw + 2;
    int* toks = (int*)malloc((size_t)T * sizeof(int));
    toks[0] = m->tok_cls;                                     /* :136-137 */
    for (int i = 0; i < raw; i++) toks[1 + i] = toks_in[i];
    toks[T - 1] = m->tok_sep;
    for (int i = 0; i < T; i++)
        if (toks[i] < 0 || toks[i] >= m->vocab_size) { free(toks); return -1; }

    float* x = (float*)malloc((size_t)T * ne * 4);
    float* q = (float*)malloc((size_t)T * ne * 4);
    float* k = (float*)malloc((size_t)T * ne * 4);
    float* v = (float*)malloc((size_t)T * ne * 4);
    float* ctx = (float*)malloc((size_t)T * ne * 4);
    float* r0 = (float*)malloc((size_t)ne * 4);
    float* r1 = (float*)malloc((size_t)ne * 4);
    float* r2 = (float*)malloc((size_t)ne * 4);
    float* hf = (float*)malloc((size_t)nff * 4);
    double* att = (double*)malloc((size_t)T * sizeof(double));
    double* acc = (double*)malloc((size_t)hd * sizeof(double));

    /* embeddings + layernorm (:155-168) */
    or_dequantize_row(m->tok_types.type, m->tok_types.data, r2, ne);
    for (int t = 0; t < T; t++) {
        or_dequantize_row(m->tok_embd.type, (const uint8_t*)m->tok_embd.data + (size_t)toks[t] * m->tok_embd.rsz, r0, ne);
        or_dequantize_row(m->pos_embd.type, (const uint8_t*)m->pos_embd.data + (size_t)t * m->pos_embd.rsz, r1, ne);
        for (int i = 0; i < ne; i++) r0[i] = r0[i] + r1[i] + r2[i];
        or_layernorm(x + (size_t)t * ne, r0, m->emb_norm_w, m->emb_norm_b, ne, m->eps);
    }
    const double scale = (double)(1.0f / sqrtf((float)hd));
    const int wmax = ne > nff ? ne : nff;
#define OR_TRACE(l, s, t, src, n) \
    if (trace) memcpy(trace + (((size_t)(l) * 4 + (s)) * T + (t)) * wmax, (src), (size_t)(n) * 4)
    for (int l = 0; l < m->n_layers; l++) {
        const or_bert_layer* L = &m->layers[l];
        /* q, k, v (:173-187) */
        for (int t = 0; t < T; t++) {
            const float* xt = x + (size_t)t * ne;
            OR_TRACE(l, 0, t, xt, ne);
            or_matvec(L->attn_q.type, L->attn_q.data, L->attn_q.rsz, ne, ne, xt, q + (size_t)t * ne);
            or_matvec(L->attn_k.type, L->attn_k.data, L->attn_k.rsz, ne, ne, xt, k + (size_t)t * ne);
            or_matvec(L->attn_v.type, L->attn_v.data, L->attn_v.rsz, ne, ne, xt, v + (size_t)t * ne);
            for (int i = 0; i < ne; i++) {
                q[(size_t)t * ne + i] = (float)((double)q[(size_t)t * ne + i] + L->attn_q_bias[i]);
                k[(size_t)t * ne + i] = (float)((double)k[(size_t)t * ne + i] + L->attn_k_bias[i]);
                v[(size_t)t * ne + i] = (float)((double)v[(size_t)t * ne + i] + L->attn_v_bias[i]);
            }
        }
        /* bidirectional attention per head (:189-212) */
        for (int t = 0; t < T; t++)
            for (int h = 0; h < nh; h++) {
                const float* qh = q + (size_t)t * ne + h * hd;
                double mx = -INFINITY, sum = 0.0;
                for (int u = 0; u < T; u++) {
                    const float* kh = k + (size_t)u * ne + h * hd;
                    double s = 0.0;
                    for (int d = 0; d < hd; d++) s += (double)qh[d] * kh[d];
                    att[u] = s * scale;
                    if (att[u] > mx) mx = att[u];
                }
                for (int u = 0; u < T; u++) { att[u] = exp(att[u] - mx); sum += att[u]; }
                for (int d = 0; d < hd; d++) acc[d] = 0.0;
                for (int u = 0; u < T; u++) {
                    const float* vh = v + (size_t)u * ne + h * hd;
                    const double p = att[u] / sum;
                    for (int d = 0; d < hd; d++) acc[d] += p * vh[d];
                }
                for (int d = 0; d < hd; d++) ctx[(size_t)t * ne + h * hd + d] = (float)acc[d];
            }
        /* att_out + bias + residual, layernorm; up + bias, gelu; down + bias
         * + residual, layernorm (:214-232) */
        for (int t = 0; t < T; t++) {
            float* xt = x + (size_t)t * ne;
            OR_TRACE(l, 1, t, ctx + (size_t)t * ne, ne);
            or_matvec(L->attn_out.type, L->attn_out.data, L->attn_out.rsz, ne, ne, ctx + (size_t)t * ne, r1);
            for (int i = 0; i < ne; i++) r1[i] = (float)((double)r1[i] + L->attn_out_bias[i] + xt[i]);
            or_layernorm(r0, r1, L->attn_norm_w, L->attn_norm_b, ne, m->eps);
            OR_TRACE(l, 2, t, r0, ne);
            or_matvec(L->ffn_up.type, L->ffn_up.data, L->ffn_up.rsz, ne, nff, r0, hf);
            for (int i = 0; i < nff; i++) hf[i] = or_gelu1((float)((double)hf[i] + L->ffn_up_bias[i]));
            OR_TRACE(l, 3, t, hf, nff);
            or_matvec(L->ffn_down.type, L->ffn_down.data, L->ffn_down.rsz, nff, ne, hf, r1);
            for (int i = 0; i < ne; i++) r1[i] = (float)((double)r1[i] + L->ffn_down_bias[i] + r0[i]);
            or_layernorm(xt, r1, L->ffn_norm_w, L->ffn_norm_b, ne, m->eps);
        }
    }
#undef OR_TRACE
    /* mean over the tokens, l2norm (:237-244, fast/lil_math.cpp:939-946) */
    double ss = 0.0;
    for (int i = 0; i < ne; i++) {
        double s = 0.0;
        for (int t = 0; t < T; t++) s += x[(size_t)t * ne + i];
        r0[i] = (float)(s / T);
        ss += (double)r0[i] * r0[i];
    }
    for (int i = 0; i < ne; i++) out[i] = ss > 0.0 ? (float)(r0[i] / sqrt(ss)) : r0[i];

    free(toks); free(x); free(q); free(k); free(v); free(ctx); free(r0); free(r1); free(r2); free(hf); free(att); free(acc);
    return 0;
}

/* vdb_query's loop (fast/vdb.cpp:352-368): similarity of each fp16 row
 * (vec_dot_f16_f32, in double, rounded once), rows below thr skipped, and
 * the reference's strict-greater insertion into the k best */
int or_vdb_search(const uint16_t* vecs, int n, int dim, const float* emb, float thr, int k, int* idx, float* sim)
{
    float best[64];
    int bi[64];
    if (k <= 0 || k > 64) return -1;
    for (int i = 0; i < k; i++) { best[i] = -1e30f; bi[i] = -1; }
    for (int r = 0; r < n; r++) {
        double s = 0.0;
        for (int d = 0; d < dim; d++) s += (double)or_fp16_to_fp32(vecs[(size_t)r * dim + d]) * emb[d];
        const float sf = (float)s;
        if (!(sf >= thr)) continue;
        for (int j = 0; j < k; j++) {
            if (sf <= best[j]) continue;
            for (int u = k - 1; u > j; u--) { best[u] = best[u - 1]; bi[u] = bi[u - 1]; }
            best[j] = sf;
            bi[j] = r;
            break;
        }
    }
    int cnt = 0;
    for (int j = 0; j < k; j++) {
        if (bi[j] < 0) continue;
        idx[cnt] = bi[j];
        sim[cnt] = best[j];
        cnt++;
    }
    return cnt;
}
