/* lg_fmt.h -- per-format weight slot loaders and integer dot products of the
 * gfx950 matvecs (the per-format dots of fast/arch_avx2.h:83-435 and
 * fast/lil_math.cpp:396-740), shared by the standalone matvec kernel and the
 * persistent decode kernel.
 *
 * A row of n values is cut into "slots" of 64 values (K-quants, Q1_G) or 32
 * values (Q8_0, Q1_0, F16, F32).  Fmt<T>::load_w reads the weight bytes of
 * one slot of one row with 128-bit loads straight from the GGUF row;
 * Fmt<T>::load_act reads the matching slice of the quantized activation;
 * Fmt<T>::dot returns the slot's contribution: the reference's exact integer
 * sub-block sums (v_dot4_i32_i8) combined in fp32.
 */
#pragma once

#include "lg_common.h"
/* ------------------------------------------------------------------ */
/* Activation slices                                                    */
/* ------------------------------------------------------------------ */

/* 64 values of one Q8_K block as 4 runs of 16 (each run one bsums group) */
struct ActK {
    int a[16];
    float d;
    int bs[4];
};

/* run k of slot s starts at 64*(s&3) + 16k (contiguous: Q4_K/Q5_K) or at
 * 128*((s&3)>>1) + 16*(s&1) + 32k (strided: Q2_K/Q3_K/Q6_K) */
template <bool CONTIG>
__device__ __forceinline__ void load_actk(ActK& A, const uint8_t* __restrict__ xq, int slot)
{
    const uint8_t* b = xq + (size_t)(slot >> 2) * LG_BS_Q8_K;
    const int idx = slot & 3;
    A.d = lg_ld<float>(b);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int off = CONTIG ? 64 * idx + 16 * k : 128 * (idx >> 1) + 16 * (idx & 1) + 32 * k;
        const uint4 v = lg_ld<uint4>(b + 4 + off);
        A.a[4 * k + 0] = (int)v.x; A.a[4 * k + 1] = (int)v.y; A.a[4 * k + 2] = (int)v.z; A.a[4 * k + 3] = (int)v.w;
        A.bs[k] = lg_ld<int16_t>(b + 260 + 2 * (off >> 4));
    }
}

/* one Q8_0 block */
struct Act8 {
    int a[8];
    float d;
    int asum;
};

__device__ __forceinline__ void load_act8(Act8& A, const uint8_t* __restrict__ xq, int blk)
{
    const uint8_t* b = xq + (size_t)blk * LG_BS_Q8_0;
    A.d = lg_h2f(lg_ld16(b));
    const uint4 v0 = lg_ld<uint4>(b + 2), v1 = lg_ld<uint4>(b + 18);
    A.a[0] = (int)v0.x; A.a[1] = (int)v0.y; A.a[2] = (int)v0.z; A.a[3] = (int)v0.w;
    A.a[4] = (int)v1.x; A.a[5] = (int)v1.y; A.a[6] = (int)v1.z; A.a[7] = (int)v1.w;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s = lg_dot4(A.a[i], 0x01010101, s);
    A.asum = s;
}

/* 32 fp32 values (F16/F32 weights multiply the float activation) */
struct ActF {
    float a[32];
};

__device__ __forceinline__ void load_actf(ActF& A, const uint8_t* __restrict__ x, int slot)
{
    const float4* p = (const float4*)(x + (size_t)slot * 128);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 v = p[i];
        A.a[4 * i] = v.x; A.a[4 * i + 1] = v.y; A.a[4 * i + 2] = v.z; A.a[4 * i + 3] = v.w;
    }
}

__device__ __forceinline__ int byte_of(uint32_t w, int i) { return (int)((w >> (8 * i)) & 255u); }

/* byte j (0..15) of a uint4 */
__device__ __forceinline__ int byte16(const uint4& v, int j)
{
    const uint32_t w = j < 4 ? v.x : (j < 8 ? v.y : (j < 12 ? v.z : v.w));
    return byte_of(w, j & 3);
}

__device__ __forceinline__ void words8(const uint4& a, const uint4& b, uint32_t w[8])
{
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

/* ------------------------------------------------------------------ */
/* Formats                                                              */
/* ------------------------------------------------------------------ */
template <int T>
struct Fmt;

/* Q4_K (144 B: d, dmin, scales[12], qs[128]); slot (block b, pair c) =
 * sub-blocks 2c (low nibbles of qs[32c..32c+31]) and 2c+1 (high nibbles).
 * dot_q8_K_q4_K: fast/lil_math.cpp:582-616, fast/arch_avx2.h:272-323. */
template <>
struct Fmt<LG_Q4_K> {
    static constexpr int VALS = 64;
    using Act = ActK;
    struct W { uint4 h, q0, q1; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* xq, int s) { load_actk<true>(A, xq, s); }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* b = row + (size_t)(s >> 2) * LG_BS_Q4_K;
        const int c = s & 3;
        w.h = lg_ld<uint4>(b);
        w.q0 = lg_ld<uint4>(b + 16 + 32 * c);
        w.q1 = lg_ld<uint4>(b + 32 + 32 * c);
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int s)
    {
        const int c = s & 3;
        uint32_t q[8];
        words8(w.q0, w.q1, q);
        int dl = 0, dh = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            dl = lg_dot4((int)(q[i] & 0x0F0F0F0Fu), A.a[i], dl);
            dh = lg_dot4((int)((q[i] >> 4) & 0x0F0F0F0Fu), A.a[8 + i], dh);
        }
        /* get_scale_min_k4 (fast/lil_math.cpp:129-138) of sub-blocks 2c and
         * 2c+1 without a branch: the header's scales[12] are bytes 4..15
         * (y, z, w); v_perm_b32 gathers, at lane-constant positions e,
         * A4 = {y.e, y.e+1, z.e, z.e+1} and B4 = {w.e, w.e+1, w.e, w.e+1};
         * sub-blocks 0..3 take A4 & 63, sub-blocks 4..7 the low (sc) or high
         * (m) nibble of B4 with the top two bits of A4 above it */
        const uint32_t e = (uint32_t)(c & 1) * 2u;
        const uint32_t A4 = __builtin_amdgcn_perm(w.h.z, w.h.y, e | ((e + 1) << 8) | ((e + 4) << 16) | ((e + 5) << 24));
        const uint32_t B4 = __builtin_amdgcn_perm(w.h.w, w.h.w, e | ((e + 1) << 8) | (e << 16) | ((e + 1) << 24));
        const uint32_t lo = A4 & 0x3F3F3F3Fu;
        const uint32_t hi = ((A4 >> 2) & 0x30303030u) | (B4 & 0x00000F0Fu) | ((B4 >> 4) & 0x0F0F0000u);
        const uint32_t r = c < 2 ? lo : hi;
        const int sc0 = (int)(r & 0xFFu), sc1 = (int)((r >> 8) & 0xFFu);
        const int m0 = (int)((r >> 16) & 0xFFu), m1 = (int)(r >> 24);
        const float d = lg_h2f((uint16_t)(w.h.x & 0xffffu)), dmin = lg_h2f((uint16_t)(w.h.x >> 16));
        const int S = sc0 * dl + sc1 * dh;
        const int M = m0 * (A.bs[0] + A.bs[1]) + m1 * (A.bs[2] + A.bs[3]);
        return A.d * lg_fma2(d, (float)S, -dmin, (float)M);
    }
};

/* Q5_K (176 B: d, dmin, scales[12], qh[32], qs[128]): Q4_K plus bit 2c+h of
 * qh[l] as the fifth bit.  fast/lil_math.cpp:618-692, fast/arch_avx2.h:325-384 */
template <>
struct Fmt<LG_Q5_K> {
    static constexpr int VALS = 64;
    using Act = ActK;
    struct W { uint4 h, qh0, qh1, q0, q1; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* xq, int s) { load_actk<true>(A, xq, s); }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* b = row + (size_t)(s >> 2) * LG_BS_Q5_K;
        const int c = s & 3;
        w.h = lg_ld<uint4>(b);
        w.qh0 = lg_ld<uint4>(b + 16);
        w.qh1 = lg_ld<uint4>(b + 32);
        w.q0 = lg_ld<uint4>(b + 48 + 32 * c);
        w.q1 = lg_ld<uint4>(b + 64 + 32 * c);
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int s)
    {
        const int c = s & 3;
        uint32_t q[8], hb[8];
        words8(w.q0, w.q1, q);
        words8(w.qh0, w.qh1, hb);
        int dl = 0, dh = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | (((hb[i] >> (2 * c)) & 0x01010101u) << 4);
            const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((hb[i] >> (2 * c + 1)) & 0x01010101u) << 4);
            dl = lg_dot4((int)lo, A.a[i], dl);
            dh = lg_dot4((int)hi, A.a[8 + i], dh);
        }
        const int j0 = 2 * c, j1 = 2 * c + 1;
        int sc0, m0, sc1, m1;
        if (c < 2) {
            sc0 = byte16(w.h, 4 + j0) & 63; m0 = byte16(w.h, 8 + j0) & 63;
            sc1 = byte16(w.h, 4 + j1) & 63; m1 = byte16(w.h, 8 + j1) & 63;
        } else {
            sc0 = (byte16(w.h, 8 + j0) & 15) | ((byte16(w.h, j0) >> 6) << 4);
            m0 = (byte16(w.h, 8 + j0) >> 4) | ((byte16(w.h, 4 + j0) >> 6) << 4);
            sc1 = (byte16(w.h, 8 + j1) & 15) | ((byte16(w.h, j1) >> 6) << 4);
            m1 = (byte16(w.h, 8 + j1) >> 4) | ((byte16(w.h, 4 + j1) >> 6) << 4);
        }
        const float d = lg_h2f((uint16_t)(w.h.x & 0xffffu)), dmin = lg_h2f((uint16_t)(w.h.x >> 16));
        const int S = sc0 * dl + sc1 * dh;
        const int M = m0 * (A.bs[0] + A.bs[1]) + m1 * (A.bs[2] + A.bs[3]);
        return A.d * lg_fma2(d, (float)S, -dmin, (float)M);
    }
};

/* Q6_K (210 B: ql[128], qh[64], scales[16], d); slot (block, half n,
 * sixteen-run s) = values 128n + 32g + 16s + l', g = 0..3, l' < 16.
 * q - 32 is folded as sum(q*a) - 32*bsum (the AVX2 maddubs(m32s, q8) trick,
 * fast/arch_avx2.h:420-423).  fast/lil_math.cpp:694-740. */
template <>
struct Fmt<LG_Q6_K> {
    static constexpr int VALS = 64;
    using Act = ActK;
    struct W { uint4 a, b, h; uint2 sc; uint32_t d; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* xq, int s) { load_actk<false>(A, xq, s); }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* b = row + (size_t)(s >> 2) * LG_BS_Q6_K;
        const int n = (s & 3) >> 1, sh = s & 1;
        w.a = lg_ld<uint4>(b + 64 * n + 16 * sh);
        w.b = lg_ld<uint4>(b + 64 * n + 32 + 16 * sh);
        w.h = lg_ld<uint4>(b + 128 + 32 * n + 16 * sh);
        w.sc = lg_ld<uint2>(b + 192 + 8 * n);
        w.d = lg_ld16(b + 208);
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int s)
    {
        const int sh = s & 1;
        const uint32_t av[4] = {w.a.x, w.a.y, w.a.z, w.a.w};
        const uint32_t bv[4] = {w.b.x, w.b.y, w.b.z, w.b.w};
        const uint32_t hv[4] = {w.h.x, w.h.y, w.h.z, w.h.w};
        int S = 0;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int dg = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t lo4 = g == 0 ? av[i] : (g == 1 ? bv[i] : (g == 2 ? av[i] >> 4 : bv[i] >> 4));
                const uint32_t q = (lo4 & 0x0F0F0F0Fu) | (((hv[i] >> (2 * g)) & 0x03030303u) << 4);
                dg = lg_dot4((int)q, A.a[4 * g + i], dg);
            }
            dg -= 32 * A.bs[g];
            const int si = sh + 2 * g;  /* byte of scales[8n .. 8n+7] */
            const int sc = (int)(int8_t)(si < 4 ? byte_of(w.sc.x, si) : byte_of(w.sc.y, si - 4));
            S += sc * dg;
        }
        return A.d * lg_h2f((uint16_t)w.d) * (float)S;
    }
};

template <>
struct Fmt<LG_Q6_K_R> : Fmt<LG_Q6_K> {
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const int blk = s >> 2, n = (s & 3) >> 1, sh = s & 1, j = blk & 7;
        const uint8_t* g = row + (size_t)(blk >> 3) * (8 * LG_BS_Q6_K);
        w.a = *(const uint4*)(g + 128 * j + 64 * n + 16 * sh);
        w.b = *(const uint4*)(g + 128 * j + 64 * n + 32 + 16 * sh);
        w.h = *(const uint4*)(g + 1024 + 64 * j + 32 * n + 16 * sh);
        w.sc = *(const uint2*)(g + 1536 + 16 * j + 8 * n);
        w.d = *(const uint16_t*)(g + 1664 + 2 * j);
    }
};

/* Q2_K (84 B: scales[16], qs[64], d, dmin); slot (block, half n, h) =
 * values 128n + 32j + 16h + l, q = (qs[32n+16h+l] >> 2j) & 3.
 * fast/lil_math.cpp:539-580, fast/arch_avx2.h:160-212 */
template <>
struct Fmt<LG_Q2_K> {
    static constexpr int VALS = 64;
    using Act = ActK;
    struct W { uint4 sc, q; uint32_t dd; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* xq, int s) { load_actk<false>(A, xq, s); }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* b = row + (size_t)(s >> 2) * LG_BS_Q2_K;
        const int n = (s & 3) >> 1, h = s & 1;
        w.sc = lg_ld<uint4>(b);
        w.q = lg_ld<uint4>(b + 16 + 32 * n + 16 * h);
        w.dd = lg_ld<uint32_t>(b + 80);
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int s)
    {
        const int n = (s & 3) >> 1, h = s & 1;
        const uint32_t qv[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        /* scale bytes 8n + 2j + h: word 2n + j/2, byte (2j + h) & 3, picked
         * with masks and shifts (an index or a select between the uint4's
         * words made the compiler copy it to scratch and load it back) */
        const uint32_t mn = 0u - (uint32_t)n;
        const uint32_t s_lo = w.sc.x ^ ((w.sc.x ^ w.sc.z) & mn), s_hi = w.sc.y ^ ((w.sc.y ^ w.sc.w) & mn);
        int S = 0, M = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int dj = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) dj = lg_dot4((int)((qv[i] >> (2 * j)) & 0x03030303u), A.a[4 * j + i], dj);
            const int sb = (int)(((j >> 1 ? s_hi : s_lo) >> (8 * ((2 * j + h) & 3))) & 0xFFu);
            S += (sb & 15) * dj;
            M += (sb >> 4) * A.bs[j];
        }
        const float d = lg_h2f((uint16_t)(w.dd & 0xffffu)), dmin = lg_h2f((uint16_t)(w.dd >> 16));
        return A.d * lg_fma2(d, (float)S, -dmin, (float)M);
    }
};

/* Q3_K (110 B: hmask[32], qs[64], scales[12], d); slot (block, n, h);
 * q = ((qs >> 2j) & 3) - 4*(1 - hbit) folded as sum(u*a) - 4*bsum with
 * u = low2 | hbit<<2.  fast/lil_math.cpp:466-537, fast/arch_avx2.h:214-270 */
template <>
struct Fmt<LG_Q3_K> {
    static constexpr int VALS = 64;
    using Act = ActK;
    struct W { uint4 hm, q; uint32_t s0, s1, s2; uint32_t d; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* xq, int s) { load_actk<false>(A, xq, s); }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* b = row + (size_t)(s >> 2) * LG_BS_Q3_K;
        const int n = (s & 3) >> 1, h = s & 1;
        w.hm = lg_ld<uint4>(b + 16 * h);
        w.q = lg_ld<uint4>(b + 32 + 32 * n + 16 * h);
        w.s0 = lg_ld<uint32_t>(b + 96);
        w.s1 = lg_ld<uint32_t>(b + 100);
        w.s2 = lg_ld<uint32_t>(b + 104);
        w.d = lg_ld16(b + 108);
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int s)
    {
        const int n = (s & 3) >> 1, h = s & 1;
        const uint32_t qv[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        const uint32_t hv[4] = {w.hm.x, w.hm.y, w.hm.z, w.hm.w};
        int S = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int dj = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t u = ((qv[i] >> (2 * j)) & 0x03030303u) | (((hv[i] >> (4 * n + j)) & 0x01010101u) << 2);
                dj = lg_dot4((int)u, A.a[4 * j + i], dj);
            }
            dj -= 4 * A.bs[j];
            /* 6-bit scale g = 8n + 2j + h: low nibble of byte g (g < 8) or high
             * nibble of byte g-8, two high bits from byte 8+(g&3) at 2*(g/4) */
            const int g = 8 * n + 2 * j + h;
            const uint32_t lw = (g & 7) < 4 ? w.s0 : w.s1;
            const int lo = (g < 8) ? (byte_of(lw, g & 3) & 15) : (byte_of(lw, g & 3) >> 4);
            const int hi = (byte_of(w.s2, g & 3) >> (2 * (g >> 2))) & 3;
            S += ((lo | (hi << 4)) - 32) * dj;
        }
        return A.d * lg_h2f((uint16_t)w.d) * (float)S;
    }
};

/* Q8_0 (34 B: d, qs[32]) against a Q8_0 activation block.
 * dot_q8_0_q8_0: fast/lil_math.cpp:411-421, fast/arch_avx2.h:111-124 */
template <>
struct Fmt<LG_Q8_0> {
    static constexpr int VALS = 32;
    using Act = Act8;
    struct W { uint4 q0, q1; uint32_t d; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* xq, int s) { load_act8(A, xq, s); }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* b = row + (size_t)s * LG_BS_Q8_0;
        w.d = lg_ld16(b);
        w.q0 = lg_ld<uint4>(b + 2);
        w.q1 = lg_ld<uint4>(b + 18);
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int)
    {
        uint32_t q[8];
        words8(w.q0, w.q1, q);
        int S = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) S = lg_dot4((int)q[i], A.a[i], S);
        return lg_h2f((uint16_t)w.d) * A.d * (float)S;
    }
};

/* Q8_0 and Q6_K rows regrouped for aligned loads (an output head copy that
 * only the whole-step kernels read; lg_repack_rows).  Each run of 8 blocks
 * of a row becomes one group: Q8_0 (272 B) the 8 x 32 quants, then the 8
 * fp16 scales; Q6_K (1680 B) the 8 x 128 ql bytes, the 8 x 64 qh, the 8 x
 * 16 scales, the 8 fp16 d.  Groups, and so every 16-byte piece, are 16-byte
 * aligned when the row is; the values and the dot are the GGUF format's. */
template <>
struct Fmt<LG_Q8_0_R> : Fmt<LG_Q8_0> {
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* g = row + (size_t)(s >> 3) * (8 * LG_BS_Q8_0);
        const int j = s & 7;
        w.d = *(const uint16_t*)(g + 256 + 2 * j);
        w.q0 = *(const uint4*)(g + 32 * j);
        w.q1 = *(const uint4*)(g + 32 * j + 16);
    }
};

/* spread 4 bits to the low bit of 4 bytes */
__device__ __forceinline__ int bits4_to_bytes(uint32_t nib) { return (int)((nib * 0x00204081u) & 0x01010101u); }

/* Q1_0 (6 B: d, 32 sign bits): sum(+-a) = 2*sum_{bit=1}(a) - sum(a).
 * dot_q8_0_q1_0: fast/lil_math.cpp:423-438, fast/arch_avx2.h:126-139 */
template <>
struct Fmt<LG_Q1_0> {
    static constexpr int VALS = 32;
    using Act = Act8;
    struct W { uint32_t bits, d; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* xq, int s) { load_act8(A, xq, s); }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* b = row + (size_t)s * LG_BS_Q1_0;
        w.d = lg_ld16(b);
        w.bits = lg_ld<uint32_t>(b + 2);
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int)
    {
        int s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) s1 = lg_dot4(bits4_to_bytes((w.bits >> (4 * i)) & 15u), A.a[i], s1);
        return lg_h2f((uint16_t)w.d) * A.d * (float)(2 * s1 - A.asum);
    }
};

/* Q1_0 rows regrouped: each run of 8 blocks (48 B) holds the 8 x 4 bytes of
 * sign bits, then the 8 fp16 scales */
template <>
struct Fmt<LG_Q1_0_R> : Fmt<LG_Q1_0> {
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* g = row + (size_t)(s >> 3) * (8 * LG_BS_Q1_0);
        const int j = s & 7;
        w.d = *(const uint16_t*)(g + 32 + 2 * j);
        w.bits = *(const uint32_t*)(g + 4 * j);
    }
};

/* Q1_G (18 B: d, 128 sign bits); slot = half a block (64 values) against
 * two Q8_0 activation blocks: d * (da0*S0 + da1*S1).
 * dot_q8_0_q1_G: fast/lil_math.cpp:440-464, fast/arch_avx2.h:141-158 */
struct Act8x2 {
    Act8 b[2];
};

template <>
struct Fmt<LG_Q1_G> {
    static constexpr int VALS = 64;
    using Act = Act8x2;
    struct W { uint2 bits; uint32_t d; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* xq, int s)
    {
        load_act8(A.b[0], xq, 2 * s);
        load_act8(A.b[1], xq, 2 * s + 1);
    }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const uint8_t* b = row + (size_t)(s >> 1) * LG_BS_Q1_G;
        w.d = lg_ld16(b);
        w.bits = lg_ld<uint2>(b + 2 + 8 * (s & 1));
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int)
    {
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s0 = lg_dot4(bits4_to_bytes((w.bits.x >> (4 * i)) & 15u), A.b[0].a[i], s0);
            s1 = lg_dot4(bits4_to_bytes((w.bits.y >> (4 * i)) & 15u), A.b[1].a[i], s1);
        }
        const float sumi = lg_fma2(A.b[0].d, (float)(2 * s0 - A.b[0].asum), A.b[1].d, (float)(2 * s1 - A.b[1].asum));
        return lg_h2f((uint16_t)w.d) * sumi;
    }
};

/* Q1_G rows regrouped like Fmt<LG_Q8_0_R>: each run of 8 blocks (144 B)
 * holds the 8 x 16 bytes of sign bits, then the 8 fp16 scales */
template <>
struct Fmt<LG_Q1_G_R> : Fmt<LG_Q1_G> {
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const int blk = s >> 1, j = blk & 7;
        const uint8_t* g = row + (size_t)(blk >> 3) * (8 * LG_BS_Q1_G);
        w.d = *(const uint16_t*)(g + 128 + 2 * j);
        w.bits = *(const uint2*)(g + 16 * j + 8 * (s & 1));
    }
};

/* Q3_K rows regrouped like Fmt<LG_Q6_K_R>, 8 blocks (880 B) a group: the
 * 8 x 32 hmask bytes, the 8 x 64 qs, the 8 x 12 scale bytes, the 8 d.  (A
 * regrouped Q2_K measured no faster: 606 against 611 tok/s.) */
template <>
struct Fmt<LG_Q3_K_R> : Fmt<LG_Q3_K> {
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
        const int blk = s >> 2, n = (s & 3) >> 1, h = s & 1, j = blk & 7;
        const uint8_t* g = row + (size_t)(blk >> 3) * (8 * LG_BS_Q3_K);
        w.hm = *(const uint4*)(g + 32 * j + 16 * h);
        w.q = *(const uint4*)(g + 256 + 64 * j + 32 * n + 16 * h);
        const uint32_t* sc = (const uint32_t*)(g + 768 + 12 * j);
        w.s0 = sc[0];
        w.s1 = sc[1];
        w.s2 = sc[2];
        w.d = *(const uint16_t*)(g + 864 + 2 * j);
    }
};

/* F16 / F32 rows against the float activation (dot_f16_f32 / dot_f32,
 * fast/arch_avx2.h:83-109) */
template <>
struct Fmt<LG_F16> {
    static constexpr int VALS = 32;
    using Act = ActF;
    struct W { uint4 v[4]; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* x, int s) { load_actf(A, x, s); }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
#pragma unroll
        for (int i = 0; i < 4; i++) w.v[i] = lg_ld<uint4>(row + (size_t)s * 64 + 16 * i);
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int)
    {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t u[4] = {w.v[i].x, w.v[i].y, w.v[i].z, w.v[i].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                acc += lg_h2f((uint16_t)(u[k] & 0xffffu)) * A.a[8 * i + 2 * k];
                acc += lg_h2f((uint16_t)(u[k] >> 16)) * A.a[8 * i + 2 * k + 1];
            }
        }
        return acc;
    }
};

template <>
struct Fmt<LG_F32> {
    static constexpr int VALS = 32;
    using Act = ActF;
    struct W { float4 v[8]; };
    static __device__ __forceinline__ void load_act(Act& A, const uint8_t* x, int s) { load_actf(A, x, s); }
    static __device__ __forceinline__ void load_w(W& w, const uint8_t* row, int s)
    {
#pragma unroll
        for (int i = 0; i < 8; i++) w.v[i] = lg_ld<float4>(row + (size_t)s * 128 + 16 * i);
    }
    static __device__ __forceinline__ float dot(const W& w, const Act& A, int)
    {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++)
            acc += __builtin_fmaf(w.v[i].w, A.a[4 * i + 3],
                                  __builtin_fmaf(w.v[i].z, A.a[4 * i + 2],
                                                 lg_fma2(w.v[i].x, A.a[4 * i], w.v[i].y, A.a[4 * i + 1])));
        return acc;
    }
};

