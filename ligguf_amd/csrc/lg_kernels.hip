/* lg_kernels.hip -- activation quantizers, dequantization, fused norms,
 * RoPE/KV write, SwiGLU, embedding gather and argmax for gfx950.
 *
 * Layout of the per-256 kernels: one wave (64 lanes) owns 256 consecutive
 * values, lane l holding values 4l..4l+3 (one float4), which is exactly one
 * Q8_K block (fast/lil_gguf.h:115-119) or eight Q8_0 blocks (8 lanes each).
 */
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

__device__ float lg_dq_value(int type, const uint8_t* row, int64_t i)
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

__global__ void k_dequantize(int type, const uint8_t* __restrict__ x, float* __restrict__ y, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = lg_dq_value(type, x, i);
}

/* embedding row tok (fast/ligguf_fast_qk.cpp:32); the token comes from the
 * device when tok_dev is given (graph-friendly decode loops) */
__global__ void k_embed(int type, const uint8_t* __restrict__ table, uint32_t rsz, const int* __restrict__ tok_dev,
                        int tok, int n, float* __restrict__ x)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int t = tok_dev ? *tok_dev : tok;
    if (i < n) x[i] = lg_dq_value(type, table + (size_t)t * rsz, i);
}

/* ------------------------------------------------------------------ */
/* Activation quantizers from registers.                               */
/* ------------------------------------------------------------------ */

/* Q8_K block from the wave's 256 values (lane l holds v[0..3] = values
 * 4l..4l+3; inactive values must be 0).  quantize_q8_K as the reference
 * compiles it (fast/lil_math.cpp:358-394 under -Ofast): first-index signed
 * max of |x|, iscale = -127/max, q = min(127, trunc(iscale*x -+ 0.5)),
 * 16-value bsums, d = max * (-1/127). */
__device__ void lg_q8k_block(const float v[4], uint8_t* __restrict__ out)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    float amax = 0.0f, mx = 0.0f;
    int idx = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float a = fabsf(v[j]);
        if (a > amax) { amax = a; mx = v[j]; idx = 4 * lane + j; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float oa = __shfl_xor(amax, o, 64);
        const float om = __shfl_xor(mx, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        if (oa > amax || (oa == amax && oi < idx)) { amax = oa; mx = om; idx = oi; }
    }
    uint32_t packed = 0;
    int s = 0;
    if (amax != 0.0f) {
        const float iscale = -127.0f / mx;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float f = iscale * v[j];
            int t = f < 0.0f ? (int)(f - 0.5f) : (int)(f + 0.5f);
            t = t < 127 ? t : 127;
            s += t;
            packed |= (uint32_t)(t & 255) << (8 * j);
        }
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    *(uint32_t*)(out + 4 + 4 * lane) = packed;
    if ((lane & 3) == 0) *(int16_t*)(out + 260 + 2 * (lane >> 2)) = (int16_t)s;
    if (lane == 0) *(float*)out = amax != 0.0f ? mx * (-1.0f / 127.0f) : 0.0f;
}

/* Eight Q8_0 blocks from the wave's 256 values (block = lane/8), or fewer
 * when nvalid < 256.  quantize_q8_0 as compiled (fast/lil_math.cpp:329-351
 * under -Ofast): d = amax * (1/127), id = 127/amax, q = roundf(x*id). */
__device__ void lg_q8_0_blocks(const float v[4], uint8_t* __restrict__ out, int nvalid)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float a = fabsf(v[j]);
        if (amax < a) amax = a;
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const int blk = lane >> 3;
    if (32 * blk >= nvalid) return;
    const float d = amax * (1.0f / 127.0f);
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    uint8_t* b = out + LG_BS_Q8_0 * blk;
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int q = (int)roundf(v[j] * id);
        packed |= (uint32_t)(q & 255) << (8 * j);
    }
    __builtin_memcpy(b + 2 + 4 * (lane & 7), &packed, 4);
    if ((lane & 7) == 0) {
        const uint16_t dh = lg_f2h(d);
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

/* one wave per 256 values */
__global__ __launch_bounds__(256) void k_quantize(const float* __restrict__ x, int64_t n, int qtype,
                                                  uint8_t* __restrict__ y)
{
    const int64_t chunk = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (chunk * 256 >= n) return;
    const int64_t base = chunk * 256 + 4 * lane;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (base < n) {
        const float4 t = *(const float4*)(x + base);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
    lg_emit(v, qtype, y, chunk, (int)min<int64_t>(256, n - chunk * 256));
}

/* ------------------------------------------------------------------ */
/* RMSNorm fused with the quantizer (fast/lil_math.cpp:922-929 then the */
/* quantize_q8_K/q8_0 of fast/ligguf_fast_qk.cpp:39,116,140).  Each     */
/* wave recomputes sum(x^2) over the whole vector (16 KB at dim 4096,   */
/* L2-resident) so that no second launch or grid sync is needed.        */
/* ------------------------------------------------------------------ */
__global__ __launch_bounds__(64) void k_rmsnorm_quant(const float* __restrict__ x, const float* __restrict__ w, int n,
                                                      float eps, int qtype, uint8_t* __restrict__ out_q,
                                                      float* __restrict__ out_f)
{
    const int lane = threadIdx.x;
    const int chunk = blockIdx.x;
    float ss = 0.0f;
    for (int i = 4 * lane; i < n; i += 256) {
        const float4 t = *(const float4*)(x + i);
        ss += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
    }
    ss = lg_group_sum<64>(ss);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    const int base = chunk * 256 + 4 * lane;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (base < n) {
        const float4 t = *(const float4*)(x + base);
        const float4 g = *(const float4*)(w + base);
        v[0] = t.x * scale * g.x; v[1] = t.y * scale * g.y; v[2] = t.z * scale * g.z; v[3] = t.w * scale * g.w;
        if (out_f) *(float4*)(out_f + base) = make_float4(v[0], v[1], v[2], v[3]);
    }
    if (out_q) lg_emit(v, qtype, out_q, chunk, min(256, n - chunk * 256));
}

/* SwiGLU hb = silu(hb2) * hb (fast/ligguf_fast_qk.cpp:119-123) fused with
 * the down-projection quantizer (:126) */
__global__ __launch_bounds__(256) void k_swiglu_quant(float* __restrict__ hb, const float* __restrict__ hb2, int n,
                                                      int qtype, uint8_t* __restrict__ out_q)
{
    const int chunk = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (chunk * 256 >= n) return;
    const int base = chunk * 256 + 4 * lane;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (base < n) {
        const float4 u = *(const float4*)(hb + base);
        const float4 g = *(const float4*)(hb2 + base);
        v[0] = (g.x / (1.0f + expf(-g.x))) * u.x;
        v[1] = (g.y / (1.0f + expf(-g.y))) * u.y;
        v[2] = (g.z / (1.0f + expf(-g.z))) * u.z;
        v[3] = (g.w / (1.0f + expf(-g.w))) * u.w;
        *(float4*)(hb + base) = make_float4(v[0], v[1], v[2], v[3]);
    }
    if (out_q) lg_emit(v, qtype, out_q, chunk, min(256, n - chunk * 256));
}

/* ------------------------------------------------------------------ */
/* Qwen3 QK RMSNorm + adjacent-pair RoPE + fp16 KV write.  One wave per */
/* head; lane l holds elements 4l..4l+3 of the head (head_dim <= 256,   */
/* multiple of 4), so each RoPE pair (2i, 2i+1) sits in one lane.       */
/* Waves 0..n_heads-1 take the Q heads, the next n_kv_heads the K heads */
/* (which also copy their V slice into the fp16 cache).                 */
/* ------------------------------------------------------------------ */
__global__ __launch_bounds__(256) void k_qk_norm_rope_kv(float* __restrict__ q, float* __restrict__ k,
                                                         const float* __restrict__ v, const float* __restrict__ qw,
                                                         const float* __restrict__ kw, int n_heads, int n_kv_heads,
                                                         int hd, int rope_dim, int pos,
                                                         const float* __restrict__ freq, float eps,
                                                         uint16_t* __restrict__ kc_row, uint16_t* __restrict__ vc_row)
{
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= n_heads + n_kv_heads) return;
    const bool is_q = wave < n_heads;
    const int h = is_q ? wave : wave - n_heads;
    float* p = (is_q ? q : k) + (size_t)h * hd;
    const float* nw = is_q ? qw : kw;
    const bool act = 4 * lane < hd;
    float e[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) {
        const float4 t = *(const float4*)(p + 4 * lane);
        e[0] = t.x; e[1] = t.y; e[2] = t.z; e[3] = t.w;
    }
    if (nw) {
        float ss = e[0] * e[0] + e[1] * e[1] + e[2] * e[2] + e[3] * e[3];
        ss = lg_group_sum<64>(ss);
        const float sc = 1.0f / sqrtf(ss / (float)hd + eps);
        if (act) {
            const float4 g = *(const float4*)(nw + 4 * lane);
            e[0] = e[0] * sc * g.x; e[1] = e[1] * sc * g.y; e[2] = e[2] * sc * g.z; e[3] = e[3] * sc * g.w;
        }
    }
    int rd = rope_dim < hd ? rope_dim : hd;
    rd &= ~1;
    if (act) {
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
            const int i = 4 * lane + j;
            if (i < rd) {
                const float ang = (float)pos * freq[i >> 1];
                float s, c;
                sincosf(ang, &s, &c);
                const float x0 = e[j], x1 = e[j + 1];
                e[j] = x0 * c - x1 * s;
                e[j + 1] = x0 * s + x1 * c;
            }
        }
        *(float4*)(p + 4 * lane) = make_float4(e[0], e[1], e[2], e[3]);
        if (!is_q) {
            const size_t o = (size_t)h * hd + 4 * lane;
            if (kc_row) {
                const uint32_t lo = (uint32_t)lg_f2h(e[0]) | ((uint32_t)lg_f2h(e[1]) << 16);
                const uint32_t hi = (uint32_t)lg_f2h(e[2]) | ((uint32_t)lg_f2h(e[3]) << 16);
                *(uint2*)(kc_row + o) = make_uint2(lo, hi);
            }
            if (vc_row) {
                const float4 t = *(const float4*)(v + o);
                const uint32_t lo = (uint32_t)lg_f2h(t.x) | ((uint32_t)lg_f2h(t.y) << 16);
                const uint32_t hi = (uint32_t)lg_f2h(t.z) | ((uint32_t)lg_f2h(t.w) << 16);
                *(uint2*)(vc_row + o) = make_uint2(lo, hi);
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* Greedy argmax, first index wins ties (fast/ligguf_fast_qk.cpp:146-160)*/
/* ------------------------------------------------------------------ */
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int n, int* __restrict__ out)
{
    __shared__ float sv[16];
    __shared__ int si[16];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float t = x[i];
        if (t > bv) { bv = t; bi = i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[w] = bv; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int j = 1; j < (int)(blockDim.x >> 6); j++)
            if (sv[j] > bv || (sv[j] == bv && si[j] < bi)) { bv = sv[j]; bi = si[j]; }
        *out = bi == 0x7fffffff ? 0 : bi;
    }
}

/* ------------------------------------------------------------------ */
/* launchers                                                            */
/* ------------------------------------------------------------------ */
static int qtype_ok(int qtype) { return qtype == LG_Q8_K || qtype == LG_Q8_0 || qtype == LG_F32; }

int lg_launch_quantize_q8_0(const float* x, int64_t n, void* y, hipStream_t s)
{
    if (n <= 0 || n % 32 || !x || !y) { lg_set_error("quantize_q8_0: n=%lld must be a positive multiple of 32", (long long)n); return LG_ERR_ARG; }
    const int64_t chunks = (n + 255) / 256;
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)((chunks + 3) / 4)), dim3(256), 0, s, x, n, (int)LG_Q8_0, (uint8_t*)y);
    return lg_check_launch("quantize_q8_0");
}

int lg_launch_quantize_q8_K(const float* x, int64_t n, void* y, hipStream_t s)
{
    if (n <= 0 || n % 256 || !x || !y) { lg_set_error("quantize_q8_K: n=%lld must be a positive multiple of 256", (long long)n); return LG_ERR_ARG; }
    const int64_t chunks = n / 256;
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)((chunks + 3) / 4)), dim3(256), 0, s, x, n, (int)LG_Q8_K, (uint8_t*)y);
    return lg_check_launch("quantize_q8_K");
}

int lg_launch_dequantize(int type, const void* x, float* y, int64_t n, hipStream_t s)
{
    if (lg_row_size(type, n) < 0 || type == LG_Q8_K) { lg_set_error("dequantize_row: type %d with n=%lld unsupported", type, (long long)n); return LG_ERR_TYPE; }
    if (!x || !y) { lg_set_error("dequantize_row: null pointer"); return LG_ERR_ARG; }
    hipLaunchKernelGGL(k_dequantize, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, type, (const uint8_t*)x, y, n);
    return lg_check_launch("dequantize_row");
}

int lg_launch_embed(int type, const uint8_t* table, uint32_t rsz, const int* tok_dev, int tok, int n, float* x,
                    hipStream_t s)
{
    hipLaunchKernelGGL(k_embed, dim3((n + 255) / 256), dim3(256), 0, s, type, table, rsz, tok_dev, tok, n, x);
    return lg_check_launch("embed");
}

int lg_launch_rmsnorm_quant(const float* x, const float* w, int n, float eps, int qtype, void* out_q, float* out_f,
                            hipStream_t s)
{
    if (n <= 0 || n % 32 || !x || !w || (!out_q && !out_f)) { lg_set_error("rmsnorm_quant: bad arguments (n=%d)", n); return LG_ERR_ARG; }
    if (out_q && (!qtype_ok(qtype) || (qtype == LG_Q8_K && n % 256))) { lg_set_error("rmsnorm_quant: qtype %d with n=%d unsupported", qtype, n); return LG_ERR_TYPE; }
    hipLaunchKernelGGL(k_rmsnorm_quant, dim3((n + 255) / 256), dim3(64), 0, s, x, w, n, eps, qtype, (uint8_t*)out_q, out_f);
    return lg_check_launch("rmsnorm_quant");
}

int lg_launch_swiglu_quant(float* hb, const float* hb2, int n, int qtype, void* out_q, hipStream_t s)
{
    if (n <= 0 || n % 32 || !hb || !hb2) { lg_set_error("swiglu_quant: bad arguments (n=%d)", n); return LG_ERR_ARG; }
    if (out_q && (!qtype_ok(qtype) || (qtype == LG_Q8_K && n % 256))) { lg_set_error("swiglu_quant: qtype %d with n=%d unsupported", qtype, n); return LG_ERR_TYPE; }
    const int chunks = (n + 255) / 256;
    hipLaunchKernelGGL(k_swiglu_quant, dim3((chunks + 3) / 4), dim3(256), 0, s, hb, hb2, n, qtype, (uint8_t*)out_q);
    return lg_check_launch("swiglu_quant");
}

int lg_launch_qk_norm_rope_kv(float* q, float* k, const float* v, const float* qw, const float* kw, int n_heads,
                              int n_kv_heads, int head_dim, int rope_dim, int pos, const float* freq, float eps,
                              uint16_t* kc_row, uint16_t* vc_row, hipStream_t s)
{
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim > 256 || head_dim % 4 || pos < 0 || !q || !k ||
        (rope_dim > 0 && !freq) || (vc_row && !v)) {
        lg_set_error("qk_norm_rope_kv: bad arguments (heads %d/%d, head_dim %d, pos %d)", n_heads, n_kv_heads, head_dim, pos);
        return LG_ERR_ARG;
    }
    const int waves = n_heads + n_kv_heads;
    hipLaunchKernelGGL(k_qk_norm_rope_kv, dim3((waves + 3) / 4), dim3(256), 0, s, q, k, v, qw, kw, n_heads, n_kv_heads,
                       head_dim, rope_dim, pos, freq, eps, kc_row, vc_row);
    return lg_check_launch("qk_norm_rope_kv");
}

int lg_launch_argmax(const float* x, int n, int* out, hipStream_t s)
{
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, x, n, out);
    return lg_check_launch("argmax");
}
