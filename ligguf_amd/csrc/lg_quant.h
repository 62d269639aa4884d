/* lg_quant.h -- bit-exact dequantization of one weight value and the
 * activation quantizers (one wave per 256 values), shared by the per-op
 * kernels and the persistent decode kernel.
 */
#pragma once

#include <math.h>

#include "lg_common.h"

/* ------------------------------------------------------------------ */
/* Dequantization of one value (closed forms of fast/lil_math.cpp:93-298;*/
/* every product is exact in fp32, so the result is bit-identical).     */
/* ------------------------------------------------------------------ */
__device__ __forceinline__ int k4_sc(const uint8_t* s, int j)
{
    return j < 4 ? (s[j] & 63) : ((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
}

__device__ __forceinline__ int k4_mn(const uint8_t* s, int j)
{
    return j < 4 ? (s[j + 4] & 63) : ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
}

__device__ __forceinline__ int k3_sc(const uint8_t* s, int g)
{
    const int lo = g < 8 ? (s[g] & 15) : (s[g - 8] >> 4);
    const int hi = (s[8 + (g & 3)] >> (2 * (g >> 2))) & 3;
    return lo | (hi << 4);
}

__device__ __forceinline__ float lg_dq_value(int type, const uint8_t* row, int64_t i)
{
#pragma clang fp contract(off)
    switch (type) {
    case LG_F32: return lg_ld<float>(row + 4 * i);
    case LG_F16: return lg_h2f(lg_ld16(row + 2 * i));
    case LG_Q8_0: {
        const uint8_t* b = row + (i >> 5) * LG_BS_Q8_0;
        return (float)(int8_t)b[2 + (i & 31)] * lg_h2f(lg_ld16(b));
    }
    case LG_Q1_0: {
        const uint8_t* b = row + (i >> 5) * LG_BS_Q1_0;
        const float d = lg_h2f(lg_ld16(b));
        const int j = (int)(i & 31);
        return ((b[2 + (j >> 3)] >> (j & 7)) & 1) ? d : -d;
    }
    case LG_Q1_G: {
        const uint8_t* b = row + (i >> 7) * LG_BS_Q1_G;
        const float d = lg_h2f(lg_ld16(b));
        const int j = (int)(i & 127);
        return ((b[2 + (j >> 3)] >> (j & 7)) & 1) ? d : -d;
    }
    case LG_Q2_K: {
        const uint8_t* b = row + (i >> 8) * LG_BS_Q2_K;
        const int k = (int)(i & 255), n = k >> 7, j = (k >> 5) & 3, h = (k >> 4) & 1, l = k & 15;
        const int q = (b[16 + 32 * n + 16 * h + l] >> (2 * j)) & 3;
        const uint8_t s = b[k >> 4];
        const float d = lg_h2f(lg_ld16(b + 80)), dm = lg_h2f(lg_ld16(b + 82));
        return d * (float)(s & 15) * (float)q - dm * (float)(s >> 4);
    }
    case LG_Q3_K: {
        const uint8_t* b = row + (i >> 8) * LG_BS_Q3_K;
        const int k = (int)(i & 255), n = k >> 7, j = (k >> 5) & 3, h = (k >> 4) & 1, l = k & 15;
        const int lo = (b[32 + 32 * n + 16 * h + l] >> (2 * j)) & 3;
        const int hb = (b[16 * h + l] >> (4 * n + j)) & 1;
        const float d = lg_h2f(lg_ld16(b + 108));
        return d * (float)(k3_sc(b + 96, k >> 4) - 32) * (float)(lo - (hb ? 0 : 4));
    }
    case LG_Q4_K: {
        const uint8_t* b = row + (i >> 8) * LG_BS_Q4_K;
        const int k = (int)(i & 255), c = k >> 6, h = (k >> 5) & 1, l = k & 31;
        const int q = (b[16 + 32 * c + l] >> (4 * h)) & 15;
        const float d = lg_h2f(lg_ld16(b)), dm = lg_h2f(lg_ld16(b + 2));
        return d * (float)k4_sc(b + 4, 2 * c + h) * (float)q - dm * (float)k4_mn(b + 4, 2 * c + h);
    }
    case LG_Q5_K: {
        const uint8_t* b = row + (i >> 8) * LG_BS_Q5_K;
        const int k = (int)(i & 255), c = k >> 6, h = (k >> 5) & 1, l = k & 31;
        const int q = ((b[48 + 32 * c + l] >> (4 * h)) & 15) + 16 * ((b[16 + l] >> (2 * c + h)) & 1);
        const float d = lg_h2f(lg_ld16(b)), dm = lg_h2f(lg_ld16(b + 2));
        return d * (float)k4_sc(b + 4, 2 * c + h) * (float)q - dm * (float)k4_mn(b + 4, 2 * c + h);
    }
    case LG_Q6_K: {
        const uint8_t* b = row + (i >> 8) * LG_BS_Q6_K;
        const int k = (int)(i & 255), n = k >> 7, g = (k >> 5) & 3, l = k & 31;
        const int lo = (b[64 * n + l + 32 * (g & 1)] >> (4 * (g >> 1))) & 15;
        const int hi = (b[128 + 32 * n + l] >> (2 * g)) & 3;
        const float d = lg_h2f(lg_ld16(b + 208));
        return d * (float)(int8_t)b[192 + (k >> 4)] * (float)((lo | (hi << 4)) - 32);
    }
    default: return 0.0f;
    }
}

/* ------------------------------------------------------------------ */
/* Activation quantizers from registers.                               */
/* ------------------------------------------------------------------ */

/* Q8_K block from the wave's 256 values (lane l holds v[0..3] = values
 * 4l..4l+3; inactive values must be 0).  quantize_q8_K as the reference
 * compiles it (fast/lil_math.cpp:358-394 under -Ofast): first-index signed
 * max of |x|, iscale = -127/max, q = min(127, trunc(iscale*x -+ 0.5)),
 * 16-value bsums, d = max * (-1/127). */
/* one lane's share of a Q8_K block: its 4 quants packed, the 16-value sum
 * of its lane quad (bsums entry, in every lane of the quad) and the block
 * scale d */
struct Q8KLane {
    uint32_t packed;
    int bsum;
    float d;
};

__device__ __forceinline__ Q8KLane lg_q8k_lane(const float v[4])
{
#pragma clang fp contract(off)
    /* The signed value of the first element with the largest |x| -- the
     * strict '>' scan of the reference: amax by a wave max (exact), then
     * the lowest lane holding an element equal to it (ballot) and, within
     * that lane, the lowest such element; its value is read back from that
     * lane. */
    const float a0 = fabsf(v[0]), a1 = fabsf(v[1]), a2 = fabsf(v[2]), a3 = fabsf(v[3]);
    const float amax = lg_wave_max_nn(fmaxf(fmaxf(a0, a1), fmaxf(a2, a3)));
    const bool h0 = a0 == amax, h1 = a1 == amax, h2 = a2 == amax, h3 = a3 == amax;
    const float first = h0 ? v[0] : h1 ? v[1] : h2 ? v[2] : v[3];
    const unsigned long long hits = __ballot(h0 || h1 || h2 || h3);
    const int src = __builtin_ffsll((long long)hits) - 1;
    const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(first), src));
    /* amax == 0: every quant 0 and d = 0, as the reference's early out */
    const float iscale = amax != 0.0f ? -127.0f / mx : 0.0f;
    uint32_t packed = 0;
    int s = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float f = iscale * v[j];
        /* round half away from zero: f - 0.5 below zero, f + 0.5 otherwise
         * (-0 takes +0.5; both give 0) */
        int t = (int)(f + __builtin_copysignf(0.5f, f));
        t = t < 127 ? t : 127;
        s += t;
        packed |= (uint32_t)(t & 255) << (8 * j);
    }
    s = lg_group_isum<4>(s);
    Q8KLane r;
    r.packed = packed;
    r.bsum = s;
    r.d = amax != 0.0f ? mx * (-1.0f / 127.0f) : 0.0f;
    return r;
}

/* the block as quantize_q8_K lays it out: d, qs[256], bsums[16] */
__device__ __forceinline__ void lg_q8k_block(const float v[4], uint8_t* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const Q8KLane q = lg_q8k_lane(v);
    *(uint32_t*)(out + 4 + 4 * lane) = q.packed;
    if ((lane & 3) == 0) *(int16_t*)(out + 260 + 2 * (lane >> 2)) = (int16_t)q.bsum;
    if (lane == 0) *(float*)out = q.d;
}

/* one lane's 4 values of the wave's eight Q8_0 blocks (block = lane/8):
 * quantize_q8_0 as compiled (fast/lil_math.cpp:329-351 under -Ofast):
 * d = amax * (1/127), id = 127/amax, q = roundf(x*id); every lane of the
 * wave takes part (group maximum over 8 lanes) */
struct Q80Lane {
    uint32_t packed;   /* the lane's 4 int8 values */
    float d;           /* its block's scale, before the fp16 store */
};

__device__ __forceinline__ Q80Lane lg_q8_0_lane(const float v[4])
{
#pragma clang fp contract(off)
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float a = fabsf(v[j]);
        if (amax < a) amax = a;
    }
    amax = lg_group_max_nn<8>(amax);
    Q80Lane r;
    r.d = amax * (1.0f / 127.0f);
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    r.packed = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int q = (int)roundf(v[j] * id);
        r.packed |= (uint32_t)(q & 255) << (8 * j);
    }
    return r;
}

/* Eight Q8_0 blocks from the wave's 256 values (block = lane/8), or fewer
 * when nvalid < 256 */
__device__ __forceinline__ void lg_q8_0_blocks(const float v[4], uint8_t* __restrict__ out, int nvalid)
{
    const int lane = threadIdx.x & 63;
    const Q80Lane r = lg_q8_0_lane(v);
    const int blk = lane >> 3;
    if (32 * blk >= nvalid) return;
    uint8_t* b = out + LG_BS_Q8_0 * blk;
    __builtin_memcpy(b + 2 + 4 * (lane & 7), &r.packed, 4);
    if ((lane & 7) == 0) {
        const uint16_t dh = lg_f2h(r.d);
        __builtin_memcpy(b, &dh, 2);
    }
}

/* store the wave's 256 values in the requested activation format */
__device__ __forceinline__ void lg_emit(const float v[4], int qtype, uint8_t* out_q, int64_t chunk, int nvalid)
{
    const int lane = threadIdx.x & 63;
    if (qtype == LG_Q8_K) {
        lg_q8k_block(v, out_q + chunk * LG_BS_Q8_K);
    } else if (qtype == LG_Q8_0) {
        lg_q8_0_blocks(v, out_q + chunk * 8 * LG_BS_Q8_0, nvalid);
    } else if (qtype == LG_F32) {
        if (4 * lane < nvalid) *(float4*)((float*)out_q + chunk * 256 + 4 * lane) = make_float4(v[0], v[1], v[2], v[3]);
    }
}

