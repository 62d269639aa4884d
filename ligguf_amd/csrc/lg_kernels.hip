/* lg_kernels.hip -- activation quantizers, dequantization, fused norms,
 * RoPE/KV write, SwiGLU, embedding gather and argmax for gfx950.
 *
 * Layout of the per-256 kernels: one wave (64 lanes) owns 256 consecutive
 * values, lane l holding values 4l..4l+3 (one float4), which is exactly one
 * Q8_K block (fast/lil_gguf.h:115-119) or eight Q8_0 blocks (8 lanes each).
 */
#include <math.h>

#include "lg_common.h"
#include "lg_quant.h"
#include "lg_rope.h"

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
/* L2-resident) so that no second launch or grid sync is needed, in the */
/* order of the whole-step kernels' build: the 256-value chunks in 8    */
/* interleaved groups (chunk % 8), lane partials in chunk order, one    */
/* lg_wave_sum per group, the group sums added in group order.          */
/* ------------------------------------------------------------------ */
__global__ __launch_bounds__(64) void k_rmsnorm_quant(const float* __restrict__ x, const float* __restrict__ w, int n,
                                                      float eps, int qtype, uint8_t* __restrict__ out_q,
                                                      float* __restrict__ out_f)
{
    const int lane = threadIdx.x;
    const int chunk = blockIdx.x;
    const float ss = lg_sumsq_chunked(x, n, lane);
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
    lg_qk_norm_rope_kv_wave(wave, q, k, v, qw, kw, n_heads, n_kv_heads, hd, rope_dim, pos, freq, eps, kc_row, vc_row);
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

/* ------------------------------------------------------------------ */
/* HBM read probe (measurement only): every byte of a buffer read once, */
/* each workgroup streaming its own contiguous slab (measured faster    */
/* than a grid-stride sweep: 6.2 against 5.4-5.9 TB/s), 16 B per lane   */
/* per load, eight loads in flight per lane; the result is folded into  */
/* a value stored only when it takes one particular value, so the loads */
/* cannot be dropped and nothing is written.                            */
/* ------------------------------------------------------------------ */
/* external linkage: a store to it is observable, so the loads stay */
__device__ uint32_t lg_read_sink[1024];

__global__ __launch_bounds__(512) void k_read_probe(const uint4* __restrict__ p, size_t n16)
{
    constexpr int U = 8, T = 512;
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t b0 = (size_t)blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
    size_t i = b0 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (U - 1) * T < b1; i += U * T) {
        uint4 a[U];
#pragma unroll
        for (int u = 0; u < U; u++) a[u] = p[i + u * T];
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= a[u].x ^ a[u].y ^ a[u].z ^ a[u].w;
    }
    for (; i < b1; i += T) {
        const uint4 a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9E3779B9u) lg_read_sink[blockIdx.x & 1023] = acc;
}

int lg_launch_read_probe(const void* buf, size_t bytes, hipStream_t s)
{
    if (!buf || bytes < 16 || bytes % 16 || ((uintptr_t)buf & 15)) {
        lg_set_error("read probe: %zu bytes at %p (16-byte aligned multiples of 16 bytes)", bytes, buf);
        return LG_ERR_ARG;
    }
    int dev = 0, ncu = 0;
    LG_HIP_CHECK(hipGetDevice(&dev));
    LG_HIP_CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    hipLaunchKernelGGL(k_read_probe, dim3(ncu * 4), dim3(512), 0, s, (const uint4*)buf, bytes / 16);
    return lg_check_launch("read probe");
}
